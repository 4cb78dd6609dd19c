"""The host C++ of libturboquant (C ABI validation, page allocator and block
table, layer loader, on-disk store readers) built for the CPU with
AddressSanitizer and UndefinedBehaviorSanitizer, then run: the C-ABI host
checks and a seeded mutation fuzz of the .meta / fp16 .bin / .bin footer /
manifest readers (tests/sanitize/host_fuzz.cpp).  Device launchers are
stand-ins that throw (tests/sanitize/launch_stubs.cpp), so no GPU is used.
The first sanitizer report or failed check ends the run."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "turborag_amd" / "csrc"
SAN = ROOT / "tests" / "sanitize"
HOST_SOURCES = ["tq_capi.cpp", "tq_pool.cpp", "tq_loader.cpp", "tq_store.cpp", "tq_launch_cxx.cpp"]


@pytest.fixture(scope="module")
def host_fuzz(tmp_path_factory):
    gxx = shutil.which("g++")
    hip_inc = Path("/opt/rocm/include")
    hip_lib = Path("/opt/rocm/lib")
    if not gxx or not (hip_lib / "libamdhip64.so").exists():
        pytest.skip("needs g++ and the ROCm runtime library")
    out = tmp_path_factory.mktemp("sanitize") / "host_fuzz"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__",
           f"-I{hip_inc}", f"-I{ROOT / 'include'}", f"-I{CSRC}",
           str(SAN / "host_fuzz.cpp"), str(SAN / "launch_stubs.cpp"),
           *[str(CSRC / s) for s in HOST_SOURCES],
           f"-L{hip_lib}", "-lamdhip64", f"-Wl,-rpath,{hip_lib}", "-lpthread", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, f"sanitizer build failed:\n{r.stderr[-4000:]}"
    return out


def _run(exe, *args, timeout=300):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True,
                       timeout=timeout, env=env)
    assert r.returncode == 0, f"rc {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-6000:]}"
    return r.stdout


def test_c_abi_host_paths_under_sanitizers(host_fuzz):
    assert "abi ok" in _run(host_fuzz, "abi")


@pytest.mark.parametrize("seed", [1, 2])
def test_store_readers_mutation_fuzz(host_fuzz, tmp_path, seed):
    out = _run(host_fuzz, "fuzz", seed, 30000, tmp_path)
    assert "fuzz ok" in out
