#!/usr/bin/env bash
# Compiles the parts of the reference's CPU path that build from their own
# sources with the system compiler (no CUDA headers, no stand-ins), straight
# from /root/reference, into oracle/_ref/ (git-ignored; the built files are used in place):
#   gaussian_codebook   src/gaussian_codebook.cpp (its own main(): prints the
#                       Lloyd-Max 8-level design that produced kK3Codebook)
#   ref_layouts         src/tq_turbo_mse_layout.cpp + src/tq_layout.cpp with
#                       oracle/ref_layout_driver.cpp
#   ref_legacy_layouts  src/tq_layout.cpp + src/tq_dense_layout.cpp with
#                       oracle/ref_legacy_layout_driver.cpp (every field)
# Everything else on the path includes <cuda_runtime.h>/<cuda_fp16.h> and is
# not buildable here.  Silently does nothing when /root/reference is absent.
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
ref="${TQ_REFERENCE_DIR:-/root/reference}"
[ -d "$ref/src" ] || { echo "build_ref: $ref absent, skipping"; exit 0; }
mkdir -p "$here/_ref"
g++ -O2 -std=c++17 -o "$here/_ref/gaussian_codebook" "$ref/src/gaussian_codebook.cpp"
g++ -O2 -std=c++17 -I"$ref/include" -o "$here/_ref/ref_layouts" \
    "$here/ref_layout_driver.cpp" "$ref/src/tq_turbo_mse_layout.cpp" "$ref/src/tq_layout.cpp"
g++ -O2 -std=c++17 -I"$ref/include" -o "$here/_ref/ref_legacy_layouts" \
    "$here/ref_legacy_layout_driver.cpp" "$ref/src/tq_layout.cpp" "$ref/src/tq_dense_layout.cpp"
echo "build_ref: ok"
