"""Build recipe for libturboquant.so (gfx950) and the CPU oracle.

``python -m turborag_amd.build`` (or ``__graft_entry__.build()``) compiles
every HIP/C++ source under ``turborag_amd/csrc`` with hipcc into
``build/libturboquant.so`` — the path the reference's ctypes wrapper loads
(tq_backend/turboquant_wrapper.py:16) — plus the oracle (test infrastructure)
and, when the reference tree is mounted, the reference's own buildable CPU
sources into ``oracle/_ref``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "turborag_amd" / "csrc"
BUILD = ROOT / "build"
OBJ = BUILD / "obj"
LIB = BUILD / "libturboquant.so"

ARCH = os.environ.get("TQ_OFFLOAD_ARCH", "gfx950")

# -ffp-contract=off: float expressions are evaluated exactly as written (the
# bit-exact codec paths depend on it; kernels call fmaf() where they want FMA).
# Packed FP32 instructions (v_pk_add/mul/fma_f32) are disabled: some of their
# forms have given wrong results on these GPUs, with no error.
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]

SOURCES = ["tq_capi.cpp", "tq_pool.cpp", "tq_loader.cpp", "tq_store.cpp", "tq_launch_cxx.cpp",
           "tq_codec.hip", "tq_legacy.hip", "tq_attention.hip", "tq_noalloc.hip"]


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise FileNotFoundError("hipcc not found")


def _compile(src: Path, hipcc: str) -> Path:
    obj = OBJ / (src.name + ".o")
    cmd = [hipcc, "-x", "hip", *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build_library(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(4, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_oracle(verbose: bool = True) -> None:
    subprocess.run(["bash", str(ROOT / "oracle" / "build_oracle.sh")], check=True)
    r = subprocess.run(["bash", str(ROOT / "oracle" / "build_ref.sh")], capture_output=True,
                       text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle/_ref build failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print("built oracle" + (" + oracle/_ref" if "ok" in r.stdout else ""))


def build_all(verbose: bool = True) -> None:
    build_library(verbose)
    build_oracle(verbose)


if __name__ == "__main__":
    build_all()
    sys.exit(0)
