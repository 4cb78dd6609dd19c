"""Oracle pins for the kernels the reference compiles but does not export:
QJL-1b (src/cuda/tq_qjl_kernels.cu), the legacy INT4 and dense pages
(src/cuda/tq_pack_kernels.cu, tq_dequant_kernels.cu, tq_dense_kernels.cu) and
the GPU SDPA reference (src/cuda/tq_attention_ref_kernel.cu).

Pinned by: the reference's own layout factories built and run
(tests/golden/ref_legacy_layouts.txt), the QJL layout factory's arithmetic
(src/tq_qjl.cpp:7-35) worked by hand for one page,
float64 linear algebra (scipy's Hadamard matrix), numpy brute force
(rint half-to-even, argmin), hand-derived known answers, and the reference's
CPU SDPA (src/tq_attention_ref.cpp semantics)."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np
import pytest
from scipy.linalg import hadamard

GOLDEN = Path(__file__).resolve().parent / "golden"


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _h(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _f(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def _sign(D):  # QJL sign flip: (-1)^i (the turbo_prod hash without the head)
    return np.where(np.arange(D) % 2 == 0, 1.0, -1.0)


# ── layouts ──────────────────────────────────────────────────────────── #

def test_legacy_and_dense_layouts_match_reference_factories(oracle):
    lines = (GOLDEN / "ref_legacy_layouts.txt").read_text().strip().splitlines()
    n = 0
    for line in lines:
        if line.startswith("reject"):
            continue
        cfg, i4, dn = line.split(" | ")
        B, H, D, al, f32 = map(int, cfg.split())
        L = oracle.int4_layout(B, H, D, align=al, scale_fp32=bool(f32))
        got = [L.code_bytes, L.scale_bytes, L.k_codes_off, L.v_codes_off, L.k_scales_off,
               L.v_scales_off, L.k_codes_bytes, L.v_codes_bytes, L.k_scales_bytes,
               L.v_scales_bytes, L.page_size]
        assert got == list(map(int, i4.split())), line
        Dn = oracle.dense_layout(B, H, D, align=al)
        assert [Dn.elem_bytes, Dn.k_off, Dn.v_off, Dn.k_bytes, Dn.v_bytes, Dn.page_size] == \
            list(map(int, dn.split())), line
        n += 1
    assert n == 288


def test_legacy_layout_rejects_what_reference_rejects(oracle):
    lines = [l for l in (GOLDEN / "ref_legacy_layouts.txt").read_text().splitlines()
             if l.startswith("reject")]
    assert len(lines) == 3 and all(l.endswith("throws") for l in lines)
    assert oracle.int4_layout(16, 8, 128, nbits=8) is None
    assert oracle.int4_layout(16, 8, 128, group_size=64) is None
    assert oracle.int4_layout(16, 8, 128, nbits=2) is None


def test_qjl_layout_published_figures(oracle):
    # src/tq_qjl.cpp:7-35 by hand for B = 16, H = 2, D = 128 (32 token-heads):
    # k1 @0 (32 x 16 = 512), ks @512 (64), v4 @576 (32 x 64 = 2048), vs @2624 (64), page 2688
    L = oracle.qjl_layout(16, 2, 128)
    assert (L.k1_off, L.ks_off, L.v4_off, L.vs_off, L.page_size) == (0, 512, 576, 2624, 2688)
    assert (L.k1_bytes, L.v4_bytes, L.scale_bytes) == (16, 64, 2)
    # closed form over a grid: regions in order, 2-byte aligned
    for B in (1, 8, 16):
        for H in (1, 2, 8):
            for D in (2, 8, 64, 128):
                L = oracle.qjl_layout(B, H, D)
                th = B * H
                k1 = (D + 7) // 8
                ks = -(-(th * k1) // 2) * 2
                assert L.ks_off == ks and L.v4_off == ks + 2 * th
                vs = -(-(L.v4_off + th * (D // 2)) // 2) * 2
                assert L.vs_off == vs and L.page_size == vs + 2 * th


# ── QJL-1b ───────────────────────────────────────────────────────────── #

def _rotate64(x, D):
    return hadamard(D) @ (_sign(D) * x.astype(np.float64)) / np.sqrt(D)


def test_qjl_pack_known_answer_one_hot(oracle):
    D = 128
    k = np.zeros(D, np.float32)
    k[0] = 1.0
    v = np.zeros(D, np.float32)
    v[0] = 2.0
    r = oracle.qjl_pack_row(_h(k), _h(v))
    # s * e0 = e0, WHT(e0) = all ones, / sqrt(D): every coordinate 1/sqrt(D) > 0
    assert np.all(r["k1"] == 0xFF)
    assert _f([r["ks"]])[0] == np.float16(1.0 / np.sqrt(D))
    # V rotated = 2/sqrt(D) everywhere, rms = 2/sqrt(D): normalised 1.0 -> level 0.9423 (code 11)
    assert np.all(r["v4"] == (11 | (11 << 4)))
    assert _f([r["vs"]])[0] == np.float16(2.0 / np.sqrt(D))


@pytest.mark.parametrize("D", [8, 64, 128])
def test_qjl_pack_matches_float64_rotation(oracle, D):
    rng = np.random.default_rng(D)
    checked = 0
    for _ in range(40):
        k = rng.standard_normal(D).astype(np.float16)
        v = rng.standard_normal(D).astype(np.float16)
        r = oracle.qjl_pack_row(k.view(np.uint16), v.view(np.uint16))
        yk, yv = _rotate64(k.astype(np.float32), D), _rotate64(v.astype(np.float32), D)
        rk, rv = np.sqrt(np.mean(yk ** 2)), np.sqrt(np.mean(yv ** 2))
        bits = np.unpackbits(r["k1"], bitorder="little")[:D]
        clear = np.abs(yk) > 1e-5 * rk  # away from a rounding-decided sign
        assert np.array_equal(bits[clear], (yk[clear] >= 0).astype(np.uint8))
        assert abs(_f([r["ks"]])[0] - rk) <= 2 ** -10 * rk
        assert abs(_f([r["vs"]])[0] - rv) <= 2 ** -10 * rv
        # V codes: brute-force nearest level of clamp(y / rms), away from midpoints
        lv = np.array([oracle.lib.tqo_v4(i) for i in range(16)], np.float64)
        xn = np.clip(yv / rv, -2.75, 2.75)
        dist = np.abs(xn[:, None] - lv[None, :])
        srt = np.sort(dist, axis=1)
        ok = srt[:, 1] - srt[:, 0] > 1e-5
        nib = np.stack([r["v4"] & 0xF, r["v4"] >> 4], axis=1).reshape(-1)
        assert np.array_equal(nib[ok], np.argmin(dist, axis=1)[ok])
        checked += int(clear.sum() + ok.sum())
    assert checked > 40 * D


def test_qjl_dequant_is_inverse_rotation_of_codes(oracle):
    D, H, B, N = 128, 2, 16, 40
    rng = np.random.default_rng(3)
    k = rng.standard_normal((N, H, D)).astype(np.float16)
    v = rng.standard_normal((N, H, D)).astype(np.float16)
    slots = rng.permutation(48)[:N].astype(np.int32)
    pool = oracle.qjl_pack(k.view(np.uint16), v.view(np.uint16), slots, 3, B)
    ok, ov = oracle.qjl_dequant(pool, slots, H, D, B)
    L = oracle.qjl_layout(B, H, D)
    Hm = hadamard(D).astype(np.float64)
    lv = np.array([oracle.lib.tqo_v4(i) for i in range(16)], np.float64)
    for t in range(N):
        page, tib = divmod(int(slots[t]), B)
        for h in range(H):
            cell = tib * H + h
            base = page * L.page_size
            k1 = pool[base + L.k1_off + cell * 16: base + L.k1_off + cell * 16 + 16]
            ks = _f(pool[base + L.ks_off + 2 * cell: base + L.ks_off + 2 * cell + 2].view(np.uint16))[0]
            v4 = pool[base + L.v4_off + cell * 64: base + L.v4_off + cell * 64 + 64]
            vs = _f(pool[base + L.vs_off + 2 * cell: base + L.vs_off + 2 * cell + 2].view(np.uint16))[0]
            bk = np.where(np.unpackbits(k1, bitorder="little") == 1, 1.0, -1.0) * ks
            bv = lv[np.stack([v4 & 0xF, v4 >> 4], axis=1).reshape(-1)] * vs
            ek = _sign(D) * (Hm @ bk) / np.sqrt(D)
            ev = _sign(D) * (Hm @ bv) / np.sqrt(D)
            gk, gv = _f(ok[t, h]), _f(ov[t, h])
            assert np.all(np.abs(gk - ek) <= 2 ** -10 * np.abs(ek) + 1e-6)
            assert np.all(np.abs(gv - ev) <= 2 ** -10 * np.abs(ev) + 1e-6)


def test_qjl_attention_oracles(oracle):
    """fp64 oracle = softmax(q . k) v over the oracle's own float dequant (no
    1/sqrt(D): the QJL kernel's logit convention), and the kernel-order fp32
    restatement within 1e-3 of it."""
    D, H, B, N, Q = 128, 2, 16, 300, 3
    rng = np.random.default_rng(11)
    k = rng.standard_normal((N, H, D)).astype(np.float16)
    v = rng.standard_normal((N, H, D)).astype(np.float16)
    q = (0.05 * rng.standard_normal((Q, H, D))).astype(np.float16)
    slots = rng.permutation(320)[:N].astype(np.int32)
    slots[::17] = -1  # unmapped tokens are skipped
    pool = oracle.qjl_pack(k.view(np.uint16), v.view(np.uint16), slots, 20, B)
    o64 = oracle.qjl_attention_f64(q.view(np.uint16), pool, slots, B)
    o32 = _f(oracle.qjl_attention_f32(q.view(np.uint16), pool, slots, B))
    live = slots >= 0
    ok, ov = oracle.qjl_dequant(pool, np.where(live, slots, 0).astype(np.int32), H, D, B)
    K, V = _f(ok).astype(np.float64)[live], _f(ov).astype(np.float64)[live]
    qq = q.astype(np.float64)
    for qi in range(Q):
        for h in range(H):
            lg = K[:, h] @ qq[qi, h]
            w = np.exp(lg - lg.max())
            ref = (w / w.sum()) @ V[:, h]
            err = np.abs(o64[qi, h] - ref).max() / np.abs(ref).max()
            assert err < 3e-3, err  # fp16 rounding of the dequantized K/V
            err32 = np.abs(o32[qi, h] - o64[qi, h]).max() / np.abs(o64[qi, h]).max()
            assert err32 < 1e-3, err32


# ── legacy INT4 ──────────────────────────────────────────────────────── #

def test_int4_pack_row_against_numpy(oracle):
    rng = np.random.default_rng(5)
    for D in (2, 8, 64, 128):
        for trial in range(20):
            k = (rng.standard_normal(D) * (10 ** rng.uniform(-3, 2))).astype(np.float16)
            v = rng.standard_normal(D).astype(np.float16)
            r = oracle.int4_pack_row(k.view(np.uint16), v.view(np.uint16))
            for x, codes, sc in ((k, r["kc"], r["ks"]), (v, r["vc"], r["vs"])):
                xf = x.astype(np.float32)
                scale = np.maximum(np.float32(np.abs(xf).max()) / np.float32(7.0),
                                   np.float32(1e-8))
                q = np.clip(np.rint(xf / scale), -8, 7).astype(np.int64)  # rint: half to even
                want = ((q[0::2] & 0xF) | ((q[1::2] & 0xF) << 4)).astype(np.uint8)
                assert np.array_equal(codes, want)
                assert sc == int(np.float16(scale).view(np.uint16))


def test_int4_known_answers(oracle):
    # absmax 7 -> scale 1: values quantise to themselves; halves go to even
    k = np.array([7, -7, 0.5, 1.5, 2.5, -0.5, -2.5, 3], np.float32)
    r = oracle.int4_pack_row(_h(k), _h(np.zeros(8)))
    q = [7, -7, 0, 2, 2, 0, -2, 3]
    assert list(np.stack([r["kc"] & 0xF, r["kc"] >> 4], 1).reshape(-1)) == [x & 0xF for x in q]
    assert _f([r["ks"]])[0] == 1.0
    # all-zero V: scale floor 1e-8, codes 0
    assert np.all(r["vc"] == 0) and r["vs"] == int(np.float16(1e-8).view(np.uint16))


def test_int4_dequant_closed_form(oracle):
    D, H, B, N = 64, 2, 16, 30
    rng = np.random.default_rng(6)
    k = rng.standard_normal((N, H, D)).astype(np.float16)
    v = rng.standard_normal((N, H, D)).astype(np.float16)
    slots = rng.permutation(32)[:N].astype(np.int32)
    for f32 in (False, True):
        pool = oracle.int4_pack(k.view(np.uint16), v.view(np.uint16), slots, 2, B, scale_fp32=f32)
        ok, ov = oracle.int4_dequant(pool, slots, H, D, B, scale_fp32=f32)
        for t in range(N):
            for h in range(H):
                r = oracle.int4_pack_row(k[t, h].view(np.uint16), v[t, h].view(np.uint16))
                nib = np.stack([r["kc"] & 0xF, r["kc"] >> 4], 1).reshape(-1).astype(np.int64)
                q = np.where(nib >= 8, nib - 16, nib).astype(np.float32)
                want = (q * _f([r["ks"]])[0]).astype(np.float16).view(np.uint16)
                assert np.array_equal(ok[t, h], want)


# ── GPU SDPA reference ───────────────────────────────────────────────── #

def test_sdpa_gpu_ref_against_cpu_reference(oracle):
    """The GPU kernel's algorithm (tree-reduced logits, two passes) against
    the reference's CPU SDPA (src/tq_attention_ref.cpp) per head, and its
    logits against float64."""
    Q, H, N, D = 3, 2, 257, 64
    rng = np.random.default_rng(8)
    q = rng.standard_normal((Q, H, D)).astype(np.float16)
    k = rng.standard_normal((N, H, D)).astype(np.float16)
    v = rng.standard_normal((N, H, D)).astype(np.float16)
    out, lg = oracle.sdpa_gpu_ref(q.view(np.uint16), k.view(np.uint16), v.view(np.uint16))
    for qi in range(Q):
        for h in range(H):
            cpu = np.zeros(D, np.float32)
            qh, kh, vh = (np.ascontiguousarray(a).view(np.uint16) for a in (q[qi, h], k[:, h], v[:, h]))
            oracle.lib.tqo_sdpa_single_head(_ptr(qh), _ptr(kh), _ptr(vh), N, D, _ptr(cpu))
            got = _f(out[qi, h])
            assert np.abs(got - cpu).max() <= 1e-3 * np.abs(cpu).max() + 1e-3
            l64 = k[:, h].astype(np.float64) @ q[qi, h].astype(np.float64) / np.sqrt(D)
            assert np.abs(lg[qi, h] - l64).max() <= 1e-5 * np.abs(l64).max()
