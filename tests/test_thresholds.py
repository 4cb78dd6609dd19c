"""Decision thresholds of the wide pack's nearest-level search.

The pack finds the nearest K3 / V4 level of a clamped x from thresholds
T_i = the smallest fp32 x with |x - c_i| < |x - c_(i-1)| (fp32 arithmetic):
the count #{i : x >= T_i}, read as first[g] + (x >= T[first[g] + 1]) for the
grid cell g = (int)(8x + off) with first[g] = #{i : cell(T_i) < g}.  The
library computes T and the grid at compile time (``thr::`` and
``kPackTables`` in ``tq_device.h``).  Here both are derived independently in
numpy float32, the grid search is checked against the reference's rule (the
first minimum of the fp32 distances, ``nearest_*_idx`` in
src/cuda/tq_turbo_prod_kernels.cu:39-59) on every float near each threshold
and each cell edge and on a spread over the clamped domain, and the compiled
tables are checked equal to the numpy derivation.
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


GRID = {"k3": (2.5, 20.0, 41), "v4": (2.75, 22.0, 45)}  # clamp bound, offset, cells


def _cell(x, off):
    # 8x is exact, so this is the kernel's fma(x, 8, off) rounded once
    return (x.astype(f32) * f32(8) + f32(off)).astype(f32).astype(np.int64)


def _grid(T, off, cells):
    ct = _cell(T[1:], off)
    assert np.all(np.diff(ct) > 0) and ct.min() >= 0 and ct.max() < cells  # one per cell
    return np.array([(ct < g).sum() for g in range(cells)], np.int64)


def _search(x, T, first, off):
    """The kernel's grid search: first[g] + (x >= T[first[g] + 1]), T[n] = +inf."""
    Tp = np.append(T, f32(np.inf))
    l = first[_cell(x, off)]
    return l + (x >= Tp[l + 1])


def _argmin_first(x, levels):
    return np.argmin(np.abs(x[:, None] - levels[None, :]), axis=1)


def _floats_around(t, radius):
    """Every float within `radius` ulps of t (ordered bit patterns)."""
    b = np.array([t], f32).view(np.int32)[0].astype(np.int64)
    key = b if b >= 0 else -(b & 0x7FFFFFFF)
    keys = np.arange(key - radius, key + radius + 1)
    bits = np.where(keys >= 0, keys, (-keys) | 0x80000000).astype(np.uint32)
    return bits.view(f32)


@pytest.mark.parametrize("name", ["k3", "v4"])
def test_search_equals_first_argmin(oracle, name):
    bound, off, cells = GRID[name]
    levels = getattr(oracle, name)
    T = _thresholds(levels)
    assert np.all(np.diff(T[1:]) > 0)
    first = _grid(T, off, cells)
    xs = [_floats_around(t, 1 << 15) for t in T[1:]]
    xs += [_floats_around(f32((g - off) / 8), 64) for g in range(cells)]  # cell edges
    # ~4M floats spread over the clamped domain by bit pattern, both signs
    pos = np.linspace(0, np.array([bound], f32).view(np.int32)[0], 1 << 21).astype(np.int32)
    xs += [pos.view(f32), (pos | np.int32(-0x80000000)).view(f32)]
    xs += [np.array([0.0, -0.0, bound, -bound, np.nan], f32)]
    x = np.concatenate(xs)
    nan = np.isnan(x)
    x = x[nan | (np.abs(x) <= bound)]
    nan = np.isnan(x)
    # NaN: every comparison is false, the scan keeps index 0; the kernel clamps
    # NaN to -bound first (fmin/fmax), whose index is 0 too
    want = _argmin_first(x, levels)
    want[nan] = 0
    x = np.where(nan, f32(-bound), x)
    assert np.array_equal(_search(x, T, first, off), want)


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
        "  constexpr PackTables p = thr::pack_tables();\n"
        '  for (int i = 1; i < 8; ++i) printf("%a\\n", a.t[i]);\n'
        '  for (int i = 1; i < 16; ++i) printf("%a\\n", b.t[i]);\n'
        '  for (int g = 0; g < kV4Cells; ++g) printf("%d\\n", p.v4_row[g] / 8);\n'
        '  for (int g = 0; g < kK3Cells; ++g) printf("%d\\n", p.k3_row[g] / 16);\n'
        '  for (int l = 0; l < 16; ++l) printf("%a %u\\n", p.v4[l].t, p.v4[l].code);\n'
        '  for (int l = 0; l < 8; ++l)\n'
        '    printf("%a %a %a %u\\n", p.k3[l].t, p.k3[l].lo, p.k3[l].hi, p.k3[l].code);\n'
        "}\n")
    exe = tmp_path / "thr"
    subprocess.run([hipcc, "-std=c++17", "-O1", "--offload-arch=gfx950",
                    f"-I{REPO / 'include'}", f"-I{REPO / 'turborag_amd' / 'csrc'}",
                    str(src), "-o", str(exe)], check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                         timeout=60).stdout.split()
    fl = lambda a: np.array([float.fromhex(v) for v in a], f32)  # noqa: E731
    T3, T4 = _thresholds(oracle.k3), _thresholds(oracle.v4)
    assert np.array_equal(fl(out[:7]), T3[1:])
    assert np.array_equal(fl(out[7:22]), T4[1:])
    n = 22
    assert [int(v) for v in out[n:n + 45]] == list(_grid(T4, 22.0, 45))
    n += 45
    assert [int(v) for v in out[n:n + 41]] == list(_grid(T3, 20.0, 41))
    n += 41
    v4 = out[n:n + 32]
    assert np.array_equal(fl(v4[0::2]), np.append(T4[1:], f32(np.inf)))
    assert [int(c) for c in v4[1::2]] == list(range(16))
    n += 32
    k3 = out[n:n + 32]
    assert np.array_equal(fl(k3[0::4]), np.append(T3[1:], f32(np.inf)))
    assert np.array_equal(fl(k3[1::4]), oracle.k3)
    assert np.array_equal(fl(k3[2::4]), np.append(oracle.k3[1:], oracle.k3[7]))
    assert [int(c) for c in k3[3::4]] == list(range(8))
