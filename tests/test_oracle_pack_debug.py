"""Pins of the oracle's turbo_prod pack debug outputs (the reference pack
kernel's optional buffers, src/cuda/tq_turbo_prod_kernels.cu:216-217,
243-246) and of its boundary list, against things other than the oracle's
own formulas: a float64 Hadamard transform (scipy), a float64 RMS and clamp
recomputed in numpy, brute-force first-argmin over the codebooks, the code
nibbles of the oracle's own packed pages, and float neighbours
(np.nextafter) of every listed value."""
from __future__ import annotations

import numpy as np
import pytest
import scipy.linalg

from turborag_amd.synthetic import as_u16, kv_tokens_major

K3 = np.array([-2.1513, -1.34326, -0.755526, -0.244919, 0.244919, 0.755526, 1.34326, 2.1513],
              np.float32)
V4 = np.array([-2.7326, -2.0690, -1.6180, -1.2562, -0.9423, -0.6568, -0.3880, -0.1284,
               0.1284, 0.3880, 0.6568, 0.9423, 1.2562, 1.6180, 2.0690, 2.7326], np.float32)


def _first_argmin(x, book):
    """Index of the first codebook entry at minimal |x - c| (fp32 distances,
    the reference's strict '<' scan)."""
    d = np.abs(x[..., None].astype(np.float32) - book.astype(np.float32))
    return np.argmin(d, axis=-1).astype(np.int32)


@pytest.mark.parametrize("N,H,D", [(40, 2, 128), (31, 3, 64), (17, 1, 32)])
def test_debug_outputs_against_independent_math(oracle, N, H, D):
    k, v = kv_tokens_major(N, H, D, seed=700 + D)
    ku, vu = as_u16(k), as_u16(v)
    dbg = oracle.prod_pack_debug(ku, vu)
    Hd = scipy.linalg.hadamard(D).astype(np.float64)
    s = np.array([[(-1.0) ** (i + h) for i in range(D)] for h in range(H)])  # (-1)^(i+h)
    for name, src, clamp in (("k", ku, 2.5), ("v", vu, 2.75)):
        x = src.view(np.float16).astype(np.float64) * s[None]
        rot = (x @ Hd.T) / np.sqrt(D)
        got_rot = dbg[f"{name}_rot"].astype(np.float64)
        # fp32 butterfly sums of 128 terms: a few ulps of the row's largest value
        tol = 1e-5 * np.abs(rot).max(axis=-1, keepdims=True)
        assert np.all(np.abs(got_rot - rot) <= tol)
        # normalised values from the oracle's own rotated row, in float64
        r = got_rot
        rms = np.maximum(np.sqrt((r * r).sum(-1, keepdims=True) / D), 1e-8)
        nrm = np.clip(r / rms, -clamp, clamp)
        got_n = dbg[f"{name}n"].astype(np.float64)
        assert np.all(np.abs(got_n - nrm) <= 1e-6 * np.maximum(np.abs(nrm), 1.0))
        assert np.all(np.abs(got_n) <= clamp)
    # code indices: brute-force first argmin over the codebooks of the oracle's
    # normalised values (exact: same fp32 values in)
    assert np.array_equal(dbg["kidx"], _first_argmin(dbg["kn"], K3))
    assert np.array_equal(dbg["vidx"], _first_argmin(dbg["vn"], V4))


def test_debug_indices_are_the_packed_nibbles(oracle):
    N, H, D, B = 64, 2, 128, 16
    k, v = kv_tokens_major(N, H, D, seed=731)
    ku, vu = as_u16(k), as_u16(v)
    slots = np.arange(N, dtype=np.int32)
    pool = oracle.prod_pack(ku, vu, slots, N // B, B)
    lay = oracle.prod_layout(B, H, D)
    dbg = oracle.prod_pack_debug(ku, vu)
    for t in range(N):
        page, tib = divmod(int(slots[t]), B)
        for h in range(H):
            cell = tib * H + h
            base = page * lay.page_size
            k4 = pool[base + lay.k4_off + cell * lay.k4_bytes:][:D // 2]
            v4 = pool[base + lay.v4_off + cell * lay.v4_bytes:][:D // 2]
            kn = np.stack([k4 & 15, k4 >> 4], -1).reshape(-1)
            vn = np.stack([v4 & 15, v4 >> 4], -1).reshape(-1)
            assert np.array_equal(kn & 7, dbg["kidx"][t, h])
            assert np.array_equal(vn, dbg["vidx"][t, h])


@pytest.mark.parametrize("seed", [201, 202])  # config 2 layers 1 and 2: every kind flagged
def test_boundary_list_matches_counts_and_neighbours(oracle, seed):
    N, H, D = 8192, 2, 128
    k, v = kv_tokens_major(N, H, D, seed=seed)
    ku, vu = as_u16(k), as_u16(v)
    elem, kind, val = oracle.prod_boundary_list(ku, vu)
    counts = oracle.boundary_counts("turbo_prod", ku, vu)
    assert [int((kind == c).sum()) for c in range(3)] == list(counts)
    assert len(elem) > 0
    dbg = oracle.prod_pack_debug(ku, vu)
    flat_kn, flat_vn = dbg["kn"].reshape(-1), dbg["vn"].reshape(-1)
    up = np.nextafter(val, np.float32(np.inf))
    dn = np.nextafter(val, np.float32(-np.inf))
    for e, kd, x, u, d in zip(elem, kind, val, up, dn):
        if kd == 2:
            assert x == flat_vn[e]
            assert _first_argmin(np.array([u]), V4)[0] != _first_argmin(np.array([x]), V4)[0] or \
                _first_argmin(np.array([d]), V4)[0] != _first_argmin(np.array([x]), V4)[0]
        else:
            assert x == flat_kn[e]
            if kd == 0:
                c = _first_argmin(np.array([x]), K3)[0]
                assert _first_argmin(np.array([u]), K3)[0] != c or \
                    _first_argmin(np.array([d]), K3)[0] != c
            else:  # residual sign (x - level >= 0) flips between the neighbours
                lvl = K3[_first_argmin(np.array([x]), K3)[0]]
                assert (np.float32(u - lvl) >= 0) != (np.float32(d - lvl) >= 0)
