"""Decision tables of the wide pack's nearest-level search.

The pack finds codes from breakpoints instead of scanning the codebook:
T_i = the smallest fp32 x with |x - c_i| < |x - c_(i-1)| (fp32 arithmetic) is
where the reference's first-minimum scan moves from index i-1 to i.  A count
#{breakpoints <= x} is read as first[g] + (x >= B[first[g] + 1]) for the grid
cell g = (int)(8x + off) with first[g] = #{i : cell(B_i) < g}.

* V4: breakpoints T_1..T_15, x unclamped over |x| <= 12 (the clamp to +-2.75
  moves no code); NaN lands in cell 0, code 0.
* K3 (turbo_prod K, x clamped to +-2.5): breakpoints L_0 < T_1 < L_1 < ... <
  L_7; state m = #{B <= x} gives the nibble (m >> 1) | (m & 1) << 3 (code and
  residual sign, e = x - L >= 0 exactly when x >= L) and the level L_(m >> 1).

The library computes T and the tables at compile time (``thr::`` and
``kPackTables`` in ``tq_device.h``).  Here both are derived independently in
numpy float32, the searches are checked against the reference's rules (the
first minimum of the fp32 distances, ``nearest_*_idx`` in
src/cuda/tq_turbo_prod_kernels.cu:39-59, and the sign of the fp32 residual)
on every float near each breakpoint and each cell edge and on a spread over
the domain, and the compiled tables are checked equal to the derivation.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
f32 = np.float32
V4_OFF, V4_CELLS, V4_SPAN = 96.0, 193, 12.0
K3_OFF, K3_CELLS, K3_BOUND = 20.0, 41, 2.5


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


def _k3_points(levels, T):
    """L_0, T_1, L_1, ..., T_7, L_7."""
    pts = []
    for c in range(8):
        if c:
            pts.append(T[c])
        pts.append(levels[c])
    return np.array(pts, f32)


def _cell(x, off):
    # 8x is exact, so this is the kernel's fma(x, 8, off) rounded once; NaN -> 0
    y = (x.astype(f32) * f32(8) + f32(off)).astype(f32)
    return np.where(np.isnan(y), 0, y).astype(np.int64)


def _first(points, off, cells):
    ct = _cell(points, off)
    assert np.all(np.diff(ct) > 0) and ct.min() >= 0 and ct.max() < cells  # one per cell
    return np.array([(ct < g).sum() for g in range(cells)], np.int64)


def _count(x, points, first, off):
    """The kernel's grid search: first[g] + (x >= B[first[g] + 1]), B[n + 1] = +inf."""
    B = np.concatenate([[f32(0)], points, [f32(np.inf)]]).astype(f32)
    l = first[_cell(x, off)]
    return l + (x >= B[l + 1])


def _argmin_first(x, levels):
    return np.argmin(np.abs(x[:, None] - levels[None, :]), axis=1)


def _floats_around(t, radius):
    """Every float within `radius` ulps of t (ordered bit patterns)."""
    b = np.array([t], f32).view(np.int32)[0].astype(np.int64)
    key = b if b >= 0 else -(b & 0x7FFFFFFF)
    keys = np.arange(key - radius, key + radius + 1)
    bits = np.where(keys >= 0, keys, (-keys) | 0x80000000).astype(np.uint32)
    return bits.view(f32)


def _probe(points, off, cells, span):
    xs = [_floats_around(t, 1 << 15) for t in points]
    xs += [_floats_around(f32((g - off) / 8), 64) for g in range(cells)]  # cell edges
    pos = np.linspace(0, np.array([span], f32).view(np.int32)[0], 1 << 21).astype(np.int32)
    xs += [pos.view(f32), (pos | np.int32(-0x80000000)).view(f32)]
    xs += [np.array([0.0, -0.0, span, -span], f32)]
    x = np.concatenate(xs)
    return x[np.abs(x) <= span]


def test_v4_search_equals_clamped_first_argmin(oracle):
    T = _thresholds(oracle.v4)
    first = _first(T[1:], V4_OFF, V4_CELLS)
    x = np.concatenate([_probe(T[1:], V4_OFF, V4_CELLS, V4_SPAN), np.array([np.nan], f32)])
    # the reference clamps to +-2.75 first; a NaN compares false everywhere: index 0
    xc = np.clip(x, f32(-2.75), f32(2.75))
    want = _argmin_first(xc, oracle.v4)
    want[np.isnan(x)] = 0
    assert np.array_equal(_count(x, T[1:], first, V4_OFF), want)


def test_k3_state_equals_code_and_residual_sign(oracle):
    L = oracle.k3
    T = _thresholds(L)
    P = _k3_points(L, T)
    assert np.all(np.diff(P) > 0)
    first = _first(P, K3_OFF, K3_CELLS)
    x = _probe(P, K3_OFF, K3_CELLS, K3_BOUND)
    m = _count(x, P, first, K3_OFF)
    code = _argmin_first(x, L)
    e = (x - L[code]).astype(f32)
    assert np.array_equal(m >> 1, code)
    assert np.array_equal(m & 1, (e >= 0).astype(np.int64))


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
        '  for (int g = 0; g < kK3Cells; ++g) printf("%d\\n", p.k3_row[g] / 8);\n'
        '  for (int l = 0; l < 16; ++l) printf("%a %u\\n", p.v4[l].t, p.v4[l].code);\n'
        "  for (int m = 0; m < 16; ++m)\n"
        '    printf("%a %a %a %u %u\\n", p.k3a[m].b, p.k3a[m].lo, p.k3b[m].hi, p.k3b[m].nlo,'
        " p.k3c[m].nhi);\n"
        "}\n")
    exe = tmp_path / "thr"
    r = subprocess.run([hipcc, "-std=c++17", "-O1", "--offload-arch=gfx950",
                        f"-I{REPO / 'include'}", f"-I{REPO / 'turborag_amd' / 'csrc'}",
                        str(src), "-o", str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True,
                         timeout=60).stdout.split()
    fl = lambda a: np.array([float.fromhex(v) for v in a], f32)  # noqa: E731
    L3, L4 = oracle.k3, oracle.v4
    T3, T4 = _thresholds(L3), _thresholds(L4)
    P3 = _k3_points(L3, T3)
    n = 0
    assert np.array_equal(fl(out[n:n + 7]), T3[1:])
    n += 7
    assert np.array_equal(fl(out[n:n + 15]), T4[1:])
    n += 15
    assert [int(v) for v in out[n:n + V4_CELLS]] == list(_first(T4[1:], V4_OFF, V4_CELLS))
    n += V4_CELLS
    assert [int(v) for v in out[n:n + K3_CELLS]] == list(_first(P3, K3_OFF, K3_CELLS))
    n += K3_CELLS
    v4 = out[n:n + 32]
    assert np.array_equal(fl(v4[0::2]), np.append(T4[1:], f32(np.inf)))
    assert [int(c) for c in v4[1::2]] == list(range(16))
    n += 32
    k3 = out[n:n + 80]
    m = np.arange(16)
    m1 = np.minimum(m + 1, 15)
    assert np.array_equal(fl(k3[0::5]), np.append(P3, f32(np.inf)))
    assert np.array_equal(fl(k3[1::5]), L3[m >> 1])
    assert np.array_equal(fl(k3[2::5]), L3[m1 >> 1])
    nib = lambda s: (s >> 1) | ((s & 1) << 3)  # noqa: E731
    assert [int(c) for c in k3[3::5]] == list(nib(m))
    assert [int(c) for c in k3[4::5]] == list(nib(m1))
