"""GPU parity: libturboquant.so (through the C ABI) against the CPU oracle on
identical seeded inputs.

Bar: packed codes, scales and dequantized halves
bit-exact; attention output within max rel err 1e-3 of the exact oracle,
where rel err = max|o - r| / max|r| per (query row, kv head).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, gqa_rows, kv_tokens_major, permuted_slots, query

pytestmark = pytest.mark.gpu

ATT_TOL = 1e-3


def _cfg(tq, H, D, B=16):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    return cfg, tq.make_layout_for(cfg), tq.make_mse_layout_for(cfg)


def _case(N, H, D, B, seed, slot_kind):
    k, v = kv_tokens_major(N, H, D, seed=seed)
    if slot_kind == "arange":
        slots = torch.arange(N, dtype=torch.int32)
    elif slot_kind == "perm":
        slots = permuted_slots(N, B, seed=seed + 1, num_pages=(N + B - 1) // B + 5)
    else:  # "holes": every 5th token unmapped (slot -1), others permuted
        slots = permuted_slots(N, B, seed=seed + 1)
        slots[::5] = -1
    num_pages = int(slots.max().item()) // B + 1 if N else 1
    return k, v, slots, num_pages


CASES = [
    # N, H, D, B, seed, slots
    (1143, 2, 128, 16, 101, "arange"),      # config 1 shape (ragged last page)
    (700, 2, 128, 16, 7, "perm"),
    (257, 8, 64, 16, 8, "holes"),
    (37, 1, 32, 8, 9, "perm"),
    (50, 3, 16, 7, 10, "perm"),              # non-power-of-two block size
    (9, 2, 2, 4, 11, "arange"),              # smallest head_dim
]


@pytest.mark.parametrize("N,H,D,B,seed,slot_kind", CASES)
def test_prod_pack_dequant_bit_exact(tq, oracle, cuda, N, H, D, B, seed, slot_kind):
    print(f"[prod codec] N={N} H={H} D={D} B={B} slots={slot_kind}", flush=True)
    k, v, slots, pages = _case(N, H, D, B, seed, slot_kind)
    cfg, lp, _ = _cfg(tq, H, D, B)
    pool = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lp, cfg)
    torch.cuda.synchronize()
    want = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    got = pool.cpu().numpy()
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} pool bytes differ, first at {bad[:8]}"

    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.dequant(pool, slots.to(cuda), ok, ov, lp, cfg)
    torch.cuda.synchronize()
    wk, wv = oracle.prod_dequant(want, slots.numpy(), H, D, B)
    live = slots.numpy() >= 0
    assert np.array_equal(as_u16(ok)[live], wk[live])
    assert np.array_equal(as_u16(ov)[live], wv[live])


@pytest.mark.parametrize("N,H,D,B,seed,slot_kind", CASES)
def test_mse_pack_dequant_bit_exact(tq, oracle, cuda, N, H, D, B, seed, slot_kind):
    print(f"[mse codec] N={N} H={H} D={D} B={B} slots={slot_kind}", flush=True)
    k, v, slots, pages = _case(N, H, D, B, seed, slot_kind)
    cfg, _, lm = _cfg(tq, H, D, B)
    pool = torch.zeros(pages * lm.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.mse_pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lm, cfg)
    torch.cuda.synchronize()
    want = oracle.mse_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B, fused_pairsum=True)
    got = pool.cpu().numpy()
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} pool bytes differ, first at {bad[:8]}"
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.mse_dequant(pool, slots.to(cuda), ok, ov, lm, cfg)
    torch.cuda.synchronize()
    wk, wv = oracle.mse_dequant(want, slots.numpy(), H, D, B)
    live = slots.numpy() >= 0
    assert np.array_equal(as_u16(ok)[live], wk[live])
    assert np.array_equal(as_u16(ov)[live], wv[live])


def _special_rows(N, H, D, seed):
    """Seeded K/V whose first rows hold non-finite and extreme fp16 values:
    +-inf, NaN, all zeros, +-65504, fp16 subnormals, a single spike."""
    k, v = kv_tokens_major(N, H, D, seed=seed)
    specials = []
    for t in (k, v):
        f = t.float()
        f[0, 0, 3] = float("inf")
        f[1, 0, 0] = float("-inf")
        f[2, 0, 5] = float("nan")
        f[3] = 0.0
        f[4, 0] = 65504.0
        f[4, -1, ::2] = -65504.0
        f[5, 0] = 2.0 ** -24 * torch.arange(1, D + 1, dtype=torch.float32)
        f[6, 0] = 0.0
        f[6, 0, D // 2] = 1.0
        f[7, :, :] = float("nan")
        specials.append(f.half())
    return specials[0], specials[1]


def _scale_mask(pool_len, page_size, regions):
    """True at the bytes of the fp16 scale fields (offset, length per page)."""
    m = np.zeros(pool_len, bool)
    for p0 in range(0, pool_len, page_size):
        for off, n in regions:
            m[p0 + off: p0 + off + n] = True
    return m


def _equal_nan_scales(got, want, scale_mask):
    """Codes bit-exact; scale fields bit-exact or NaN in both (the NaN payload an
    fp32 -> fp16 conversion produces is the platform's own)."""
    diff = got != want
    assert not np.any(diff & ~scale_mask), "code bytes differ"
    g16, w16 = got.view(np.uint16), want.view(np.uint16)
    bad = np.flatnonzero(g16 != w16)
    nan = lambda h: ((h & 0x7C00) == 0x7C00) & ((h & 0x03FF) != 0)  # noqa: E731
    assert np.all(nan(g16[bad]) & nan(w16[bad])), f"scale halves differ at {bad[:8]}"


@pytest.mark.parametrize("D", [128, 64, 32])
def test_pack_non_finite_and_extreme_rows(tq, oracle, cuda, D):
    print(f"[codec specials] D={D}", flush=True)
    N, H, B = 40, 2, 16
    k, v = _special_rows(N, H, D, seed=120 + D)
    slots = permuted_slots(N, B, seed=121)
    pages = int(slots.max()) // B + 1
    cfg, lp, lm = _cfg(tq, H, D, B)
    sb = B * H * 2
    pool = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lp, cfg)
    want = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    _equal_nan_scales(pool.cpu().numpy(), want, _scale_mask(
        want.size, lp.page_size_bytes, [(lp.k_scales_offset, sb), (lp.k_residual_scales_offset, sb),
                                        (lp.v_scales_offset, sb)]))
    pool = torch.zeros(pages * lm.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.mse_pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lm, cfg)
    want = oracle.mse_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B, fused_pairsum=True)
    _equal_nan_scales(pool.cpu().numpy(), want, _scale_mask(
        want.size, lm.page_size_bytes, [(lm.k_norms_offset, sb), (lm.v_norms_offset, sb)]))


def _rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max over (row, head) of max|o - r| / max|r|."""
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    den = np.maximum(np.abs(r).max(axis=1), 1e-30)
    return float((np.abs(g - r).max(axis=1) / den).max())


ATT_CASES = [
    # Q rows, H, D, N, B, seed
    (8, 2, 128, 1000, 16, 31),     # GQA 16/2 decode
    (1, 2, 128, 1, 16, 32),        # single token
    (16, 2, 128, 4097, 16, 33),
    (3, 8, 64, 513, 16, 34),
    (2, 1, 32, 77, 8, 35),
]


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("Q,H,D,N,B,seed", ATT_CASES)
def test_attention_vs_exact_oracle(tq, oracle, cuda, scheme, Q, H, D, N, B, seed):
    print(f"[attention {scheme}] Q={Q} H={H} D={D} N={N}", flush=True)
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    q = kv_tokens_major(Q, H, D, seed=seed + 2)[0]
    cfg, lp, lm = _cfg(tq, H, D, B)
    if scheme == "turbo_prod":
        pool_np = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
        ref = oracle.prod_attention_f64(as_u16(q), pool_np, slots.numpy(), B)
    else:
        pool_np = oracle.mse_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
        ref = oracle.mse_attention_f64(as_u16(q), pool_np, slots.numpy(), B)
    pool = torch.from_numpy(pool_np).to(cuda)
    out = torch.zeros(Q, H, D, dtype=torch.float16, device=cuda)
    fn = tq.fused_attn_output if scheme == "turbo_prod" else tq.mse_fused_attn_output
    fn(q.to(cuda), pool, slots.to(cuda), out, lp if scheme == "turbo_prod" else lm, cfg, Q, N)
    torch.cuda.synchronize()
    err = _rel_err(out.cpu().float().numpy(), ref)
    print(f"    rel err {err:.3e}", flush=True)
    assert err < ATT_TOL


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("Q,H,D,N,seed", [(8, 2, 128, 3000, 51), (3, 2, 64, 700, 52)])
def test_attention_skips_unmapped_tokens(tq, oracle, cuda, scheme, Q, H, D, N, seed):
    """Slots < 0 (unmapped tokens) are excluded from the softmax: every 7th
    token unmapped, and one split range with no mapped token at all."""
    print(f"[attention holes {scheme}] Q={Q} H={H} D={D} N={N}", flush=True)
    B = 16
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    q = kv_tokens_major(Q, H, D, seed=seed + 2)[0]
    cfg, lp, lm = _cfg(tq, H, D, B)
    if scheme == "turbo_prod":
        pool_np = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    else:
        pool_np = oracle.mse_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    slots[::7] = -1
    slots[256:600] = -1
    ref = (oracle.prod_attention_f64 if scheme == "turbo_prod" else oracle.mse_attention_f64)(
        as_u16(q), pool_np, slots.numpy(), B)
    out = torch.zeros(Q, H, D, dtype=torch.float16, device=cuda)
    fn = tq.fused_attn_output if scheme == "turbo_prod" else tq.mse_fused_attn_output
    fn(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), out,
       lp if scheme == "turbo_prod" else lm, cfg, Q, N)
    torch.cuda.synchronize()
    err = _rel_err(out.cpu().float().numpy(), ref)
    print(f"    rel err {err:.3e}", flush=True)
    assert err < ATT_TOL


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_attention_empty_context_is_zero(tq, cuda, scheme):
    """num_kv_tokens == 0: l = 0 -> 1/l taken as 1, output +-0 (:562)."""
    cfg, lp, lm = _cfg(tq, 2, 128)
    q = torch.randn(2, 2, 128, dtype=torch.float16, device=cuda)
    out = torch.full((2, 2, 128), 7.0, dtype=torch.float16, device=cuda)
    pool = torch.zeros(4288 * 2, dtype=torch.uint8, device=cuda)
    slots = torch.zeros(1, dtype=torch.int32, device=cuda)
    fn = tq.fused_attn_output if scheme == "turbo_prod" else tq.mse_fused_attn_output
    fn(q, pool, slots, out, lp if scheme == "turbo_prod" else lm, cfg, 2, 0)
    torch.cuda.synchronize()
    assert torch.all(out.float() == 0.0)


def test_gqa_decode_matches_sdpa_over_dequant(tq, oracle, cuda):
    """Config-4 shape at 2K context: GPU fused attention vs SDPA
    (src/tq_attention_ref.cpp semantics) over the GPU-dequantized KV, per q
    head (16 q heads / 2 kv heads).  Bound 3e-3: fp16 rounding of the
    dequantized KV alone contributes ~1e-3 on outlier-heavy data."""
    N, H, D = 2048, 2, 128
    k, v = kv_tokens_major(N, H, D, seed=402)
    slots = permuted_slots(N, 16, seed=401)
    cfg, lp, _ = _cfg(tq, H, D)
    pool = torch.zeros((N // 16) * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lp, cfg)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.dequant(pool, slots.to(cuda), ok, ov, lp, cfg)
    qh = query(16, D, seed=400)
    qa = gqa_rows(qh, H)
    out = torch.zeros(8, H, D, dtype=torch.float16, device=cuda)
    tq.fused_attn_output(qa.to(cuda), pool, slots.to(cuda), out, lp, cfg, 8, N)
    torch.cuda.synchronize()
    okn, ovn = as_u16(ok), as_u16(ov)
    for j in range(16):
        h, g = j // 8, j % 8
        sd = oracle.sdpa_single_head(as_u16(qh[j]), okn[:, h].copy(), ovn[:, h].copy())
        o = out[g, h].cpu().float().numpy()
        assert np.abs(o - sd).max() / np.abs(sd).max() < 3e-3, j


@pytest.mark.parametrize("Q,H,D,N,B,seed", [(8, 2, 128, 1000, 16, 41), (3, 8, 64, 300, 16, 42),
                                            (1, 2, 128, 1, 16, 43),
                                            (8, 2, 128, 32768, 16, 44),   # the bench's shape
                                            (9, 2, 128, 32768 + 77, 16, 45),  # ragged tile, 2 row groups
                                            (5, 1, 128, 777, 16, 46),     # one kv head
                                            (16, 8, 128, 1500, 12, 47),   # 8 heads, 12-token pages
                                            (24, 2, 128, 4099, 32, 48)])  # 3 row groups
def test_logits_vs_oracle(tq, oracle, cuda, Q, H, D, N, B, seed):
    print(f"[logits] Q={Q} H={H} D={D} N={N}", flush=True)
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    q = kv_tokens_major(Q, H, D, seed=seed + 2)[0]
    cfg, lp, _ = _cfg(tq, H, D, B)
    pool_np = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    _, ref64 = oracle.prod_attention_f64(as_u16(q), pool_np, slots.numpy(), B, want_logits=True)
    ref32 = oracle.prod_logits(as_u16(q), pool_np, slots.numpy(), B)
    logits = torch.zeros(Q * H * N, dtype=torch.float32, device=cuda)
    tq.fused_attn_logits(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), logits,
                         lp, cfg, Q, N)
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(Q, H, N).astype(np.float64)
    scale = np.abs(ref64).max(axis=-1, keepdims=True) + 1e-30
    assert (np.abs(got - ref64) / scale).max() < 1e-5
    assert (np.abs(ref32 - ref64) / scale).max() < 1e-5


def test_logits_unmapped_tokens_are_neg_inf(tq, oracle, cuda):
    Q, H, D, N, B = 4, 2, 128, 300, 16
    k, v = kv_tokens_major(N, H, D, seed=61)
    slots = permuted_slots(N, B, seed=62)
    pages = int(slots.max()) // B + 1
    q = kv_tokens_major(Q, H, D, seed=63)[0]
    cfg, lp, _ = _cfg(tq, H, D, B)
    pool_np = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    slots[::5] = -1
    ref32 = oracle.prod_logits(as_u16(q), pool_np, slots.numpy(), B)
    logits = torch.zeros(Q * H * N, dtype=torch.float32, device=cuda)
    tq.fused_attn_logits(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), logits,
                         lp, cfg, Q, N)
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(Q, H, N)
    hole = slots.numpy() < 0
    assert np.all(np.isneginf(got[:, :, hole])) and np.all(np.isneginf(ref32[:, :, hole]))
    live = ~hole
    scale = np.abs(ref32[:, :, live]).max(axis=-1, keepdims=True)
    assert (np.abs(got[:, :, live] - ref32[:, :, live]) / scale).max() < 1e-5


# ---- full-size properties (32K-token layers), sampled against the oracle ---

def test_full_size_prod_codec_sampled(tq, oracle, cuda):
    """Config 2/3 shape: 32768 tokens, 2 heads, D=128, shuffled pages.  The
    GPU packs the whole layer; the oracle re-packs 1500 random tokens into
    their own slots and every byte of those cells must agree; the GPU
    dequant of those tokens must equal the oracle's, bit for bit."""
    N, H, D, B = 32768, 2, 128, 16
    k, v = kv_tokens_major(N, H, D, seed=300)
    slots = permuted_slots(N, B, seed=301)
    cfg, lp, _ = _cfg(tq, H, D, B)
    pool = torch.zeros((N // B) * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lp, cfg)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.dequant(pool, slots.to(cuda), ok, ov, lp, cfg)
    torch.cuda.synchronize()
    got_pool = pool.cpu().numpy()
    pick = np.random.default_rng(7).choice(N, 1500, replace=False)
    sub_slots = slots.numpy()[pick]
    ref_pool = oracle.prod_pack(as_u16(k)[pick], as_u16(v)[pick], sub_slots, N // B, B)
    mask = np.zeros_like(ref_pool, dtype=bool)
    L = oracle.prod_layout(B, H, D)
    for s in sub_slots:
        page, tib = divmod(int(s), B)
        base = page * L.page_size
        for h in range(H):
            c = tib * H + h
            for off, n in ((L.k4_off, 64), (L.v4_off, 64), (L.ks_off, 2), (L.kres_off, 2),
                           (L.vs_off, 2)):
                stride = 64 if n == 64 else 2
                mask[base + off + c * stride: base + off + c * stride + n] = True
    assert np.array_equal(got_pool[mask], ref_pool[mask])
    wk, wv = oracle.prod_dequant(got_pool, sub_slots, H, D, B)
    assert np.array_equal(as_u16(ok)[pick], wk)
    assert np.array_equal(as_u16(ov)[pick], wv)


def test_full_size_attention_32k(tq, oracle, cuda):
    """Config 4: GQA 16/2, D=128, 32768 tokens on shuffled pages."""
    N, H, D, B = 32768, 2, 128, 16
    k, v = kv_tokens_major(N, H, D, seed=402)
    slots = permuted_slots(N, B, seed=401)
    qa = gqa_rows(query(16, D, seed=400), H)
    cfg, lp, lm = _cfg(tq, H, D, B)
    for scheme in ("turbo_prod", "turbo_mse"):
        if scheme == "turbo_prod":
            pool = torch.zeros((N // B) * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
            tq.pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lp, cfg)
            out = torch.zeros(8, H, D, dtype=torch.float16, device=cuda)
            tq.fused_attn_output(qa.to(cuda), pool, slots.to(cuda), out, lp, cfg, 8, N)
            torch.cuda.synchronize()
            ref = oracle.prod_attention_f64(as_u16(qa), pool.cpu().numpy(), slots.numpy(), B)
        else:
            pool = torch.zeros((N // B) * lm.page_size_bytes, dtype=torch.uint8, device=cuda)
            tq.mse_pack(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lm, cfg)
            out = torch.zeros(8, H, D, dtype=torch.float16, device=cuda)
            tq.mse_fused_attn_output(qa.to(cuda), pool, slots.to(cuda), out, lm, cfg, 8, N)
            torch.cuda.synchronize()
            ref = oracle.mse_attention_f64(as_u16(qa), pool.cpu().numpy(), slots.numpy(), B)
        err = _rel_err(out.cpu().float().numpy(), ref)
        print(f"[32K {scheme}] rel err {err:.3e}", flush=True)
        assert err < ATT_TOL
