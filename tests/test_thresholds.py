"""Decision thresholds of the wide pack's nearest-level search.

The pack finds the nearest K3 / V4 level by a binary search over thresholds
T_i = the smallest fp32 x with |x - c_i| < |x - c_(i-1)| (fp32 arithmetic),
which the library computes at compile time (``thr::thresholds`` in
``tq_device.h``).  Here the thresholds are derived independently in numpy
float32, the search over them is checked against the reference's rule (the
first minimum of the fp32 distances, ``nearest_*_idx`` in
src/cuda/tq_turbo_prod_kernels.cu:39-59) on every float near each threshold
and on a spread over the clamped domain, and the compiled tables are checked
equal to the numpy derivation.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest


REPO = Path(__file__).resolve().parent.parent
f32 = np.float32


def _closer(x, a, b):
    return np.abs(f32(x) - f32(b)) < np.abs(f32(x) - f32(a))


def _thresholds(levels):
    """Bisection over floats: closer() false at lo, true at hi, until adjacent."""
    out = [f32(0)]
    for a, b in zip(levels[:-1], levels[1:]):
        lo, hi = f32(a), f32(b)
        while np.nextafter(lo, f32(np.inf)) != hi:
            m = f32((lo + hi) * f32(0.5))
            if _closer(m, a, b):
                hi = m
            else:
                lo = m
        assert _closer(hi, a, b) and not _closer(lo, a, b)
        out.append(hi)
    return np.array(out, f32)


def _search(x, T):
    """The kernel's branchless binary search: #{i >= 1 : x >= T[i]}."""
    n = len(T)
    idx = np.zeros(x.shape, np.int64)
    s = n // 2
    while s >= 1:
        idx += np.where(x >= T[idx + s], s, 0)
        s //= 2
    return idx


def _argmin_first(x, levels):
    return np.argmin(np.abs(x[:, None] - levels[None, :]), axis=1)


def _floats_around(t, radius):
    """Every float within `radius` ulps of t (ordered bit patterns)."""
    b = np.array([t], f32).view(np.int32)[0].astype(np.int64)
    key = b if b >= 0 else -(b & 0x7FFFFFFF)
    keys = np.arange(key - radius, key + radius + 1)
    bits = np.where(keys >= 0, keys, (-keys) | 0x80000000).astype(np.uint32)
    return bits.view(f32)


@pytest.mark.parametrize("name,bound", [("k3", 2.5), ("v4", 2.75)])
def test_search_equals_first_argmin(oracle, name, bound):
    levels = getattr(oracle, name)
    T = _thresholds(levels)
    assert np.all(np.diff(T[1:]) > 0)
    xs = [_floats_around(t, 1 << 15) for t in T[1:]]
    # ~4M floats spread over the clamped domain by bit pattern, both signs
    pos = np.linspace(0, np.array([bound], f32).view(np.int32)[0], 1 << 21).astype(np.int32)
    xs += [pos.view(f32), (pos | np.int32(-0x80000000)).view(f32)]
    xs += [np.array([0.0, -0.0, bound, -bound, np.nan], f32)]
    x = np.concatenate(xs)
    x = x[np.isnan(x) | (np.abs(x) <= bound)]
    got = _search(x, T)
    want = _argmin_first(x, levels)
    want[np.isnan(x)] = 0  # every comparison with NaN is false: the scan keeps index 0
    assert np.array_equal(got, want)


def test_compiled_tables_match(oracle, tmp_path):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not shutil.which(hipcc):
        pytest.skip("hipcc not available")
    src = tmp_path / "thr.hip"
    src.write_text(
        '#include "tq_device.h"\n#include <cstdio>\nusing namespace tq::dev;\n'
        "int main() {\n"
        "  constexpr auto a = thr::thresholds(kK3);\n"
        "  constexpr auto b = thr::thresholds(kV4);\n"
        '  for (int i = 1; i < 8; ++i) printf("%a\\n", a.t[i]);\n'
        '  for (int i = 1; i < 16; ++i) printf("%a\\n", b.t[i]);\n'
        "}\n")
    exe = tmp_path / "thr"
    subprocess.run([hipcc, "-std=c++17", "-O1", "--offload-arch=gfx950",
                    f"-I{REPO / 'include'}", f"-I{REPO / 'turborag_amd' / 'csrc'}",
                    str(src), "-o", str(exe)], check=True, capture_output=True, timeout=300)
    vals = [float.fromhex(v) for v in subprocess.run(
        [str(exe)], check=True, capture_output=True, text=True, timeout=60).stdout.split()]
    assert np.array_equal(np.array(vals[:7], f32), _thresholds(oracle.k3)[1:])
    assert np.array_equal(np.array(vals[7:], f32), _thresholds(oracle.v4)[1:])
