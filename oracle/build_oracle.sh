#!/usr/bin/env bash
# Builds the CPU oracle (test infrastructure) into oracle/libtq_oracle.so.
# Strict IEEE: no -ffast-math, no FMA contraction (fmaf() only where written).
set -euo pipefail
here="$(cd "$(dirname "$0")" && pwd)"
gcc -O3 -march=x86-64-v3 -std=gnu99 -ffp-contract=off -fno-math-errno -fPIC -shared \
    -Wall -Wextra -Wno-unused-parameter \
    -o "$here/libtq_oracle.so.tmp" "$here/tq_oracle.c" -lm -lpthread
mv "$here/libtq_oracle.so.tmp" "$here/libtq_oracle.so"
