"""GPU parity for the reference's unexported kernels against the CPU oracle:
QJL-1b pack / dequant bit-exact and fused attention within 1e-3 of the fp64
oracle; legacy INT4 pack / dequant bit-exact (fp16 and fp32 scale cells);
dense store / load exact; the GPU SDPA reference within 1e-3 of the
reference kernel's algorithm (logits within 1e-5)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, kv_tokens_major

pytestmark = pytest.mark.gpu
ATT_TOL = 1e-3


def _cfg(tq, H, D, B, scale_fp32=False):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size, cfg.group_size = H, D, B, D
    cfg.scale_type = 1 if scale_fp32 else 0
    return cfg


def _slots(N, B, seed, holes=False):
    pages = (N + B - 1) // B + 1
    rng = np.random.default_rng(seed)
    s = rng.permutation(pages * B)[:N].astype(np.int32)
    if holes:
        s[::7] = -1
    return s, pages


def _rel_err(got, ref):
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max())


@pytest.mark.parametrize("N,H,D,B", [(1000, 2, 128, 16), (333, 4, 64, 16), (77, 2, 16, 8),
                                     (50, 3, 4, 16), (40, 2, 2, 4)])
def test_qjl_pack_dequant_bit_exact(tq, oracle, cuda, N, H, D, B):
    print(f"[qjl pack/dequant] N={N} H={H} D={D} B={B}", flush=True)
    cfg = _cfg(tq, H, D, B)
    lay = tq.make_qjl_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=40 + D)
    slots, pages = _slots(N, B, 41 + D, holes=True)
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    st = torch.from_numpy(slots).to(cuda)
    tq.qjl_pack(k.to(cuda), v.to(cuda), st, pool, lay, cfg)
    ref = oracle.qjl_pack(as_u16(k), as_u16(v), slots, pages, B)
    assert np.array_equal(pool.cpu().numpy(), ref)
    ok = torch.full((N, H, D), 7.0, dtype=torch.float16, device=cuda)
    ov = torch.full_like(ok, 7.0)
    tq.qjl_dequant(pool, st, ok, ov, lay, cfg)
    rk, rv = oracle.qjl_dequant(ref, slots, H, D, B)
    live = slots >= 0
    assert np.array_equal(as_u16(ok)[live], rk[live])
    assert np.array_equal(as_u16(ov)[live], rv[live])
    assert np.all(ok.cpu().float().numpy()[~live] == 7.0)  # unmapped tokens untouched


@pytest.mark.parametrize("Q,N,H,D", [(8, 3000, 2, 128), (2, 1, 2, 128), (3, 513, 4, 64),
                                     (1, 0, 2, 128)])
def test_qjl_attention(tq, oracle, cuda, Q, N, H, D):
    print(f"[qjl attention] Q={Q} N={N} H={H} D={D}", flush=True)
    B = 16
    cfg = _cfg(tq, H, D, B)
    lay = tq.make_qjl_layout_for(cfg)
    k, v = kv_tokens_major(max(N, 1), H, D, seed=60)
    slots, pages = _slots(max(N, 1), B, 61, holes=N > 100)
    st = torch.from_numpy(slots[:N].copy()).to(cuda) if N else torch.zeros(1, dtype=torch.int32,
                                                                            device=cuda)
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.qjl_pack(k.to(cuda), v.to(cuda), torch.from_numpy(slots).to(cuda), pool, lay, cfg)
    g = torch.Generator().manual_seed(62)
    q = (0.1 * torch.randn(Q, H, D, generator=g)).half()
    out = torch.full((Q, H, D), 3.0, dtype=torch.float16, device=cuda)
    tq.qjl_fused_attn_output(q.to(cuda), pool, st, out, lay, cfg, Q, N)
    got = out.cpu().float().numpy()
    if N == 0:
        assert np.all(got == 0.0)
        return
    ref = oracle.qjl_attention_f64(as_u16(q), pool.cpu().numpy(), slots[:N], B)
    assert _rel_err(got, ref) < ATT_TOL


@pytest.mark.parametrize("scale_fp32", [False, True])
@pytest.mark.parametrize("N,H,D,B", [(1000, 2, 128, 16), (200, 8, 64, 16), (31, 2, 2, 8)])
def test_int4_pack_dequant_bit_exact(tq, oracle, cuda, N, H, D, B, scale_fp32):
    print(f"[int4] N={N} H={H} D={D} fp32 scales={scale_fp32}", flush=True)
    cfg = _cfg(tq, H, D, B, scale_fp32)
    lay = tq.make_int4_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=70 + D)
    slots, pages = _slots(N, B, 71, holes=True)
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    st = torch.from_numpy(slots).to(cuda)
    tq.int4_pack(k.to(cuda), v.to(cuda), st, pool, lay, cfg)
    ref = oracle.int4_pack(as_u16(k), as_u16(v), slots, pages, B, scale_fp32=scale_fp32)
    assert np.array_equal(pool.cpu().numpy(), ref)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.int4_dequant(pool, st, ok, ov, lay, cfg)
    rk, rv = oracle.int4_dequant(ref, slots, H, D, B, scale_fp32=scale_fp32)
    live = slots >= 0
    assert np.array_equal(as_u16(ok)[live], rk[live])
    assert np.array_equal(as_u16(ov)[live], rv[live])


@pytest.mark.parametrize("N,H,D,B", [(1000, 2, 128, 16), (45, 3, 2, 4)])
def test_dense_store_load(tq, oracle, cuda, N, H, D, B):
    cfg = _cfg(tq, H, D, B)
    lay = tq.make_dense_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=80)
    slots, pages = _slots(N, B, 81, holes=True)
    st = torch.from_numpy(slots).to(cuda)
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.dense_store(k.to(cuda), v.to(cuda), st, pool, lay, cfg)
    # expected page bytes, placed by the layout's cell arithmetic
    want = np.zeros(pages * lay.page_size_bytes, np.uint8)
    ku, vu = as_u16(k), as_u16(v)
    for t in range(N):
        if slots[t] < 0:
            continue
        page, tib = divmod(int(slots[t]), B)
        for h in range(H):
            o = page * lay.page_size_bytes + (tib * H + h) * D * 2
            want[o + lay.k_offset: o + lay.k_offset + 2 * D] = ku[t, h].view(np.uint8)
            want[o + lay.v_offset: o + lay.v_offset + 2 * D] = vu[t, h].view(np.uint8)
    assert np.array_equal(pool.cpu().numpy(), want)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    tq.dense_load(pool, st, ok, ov, lay, cfg)
    live = slots >= 0
    assert np.array_equal(as_u16(ok)[live], ku[live])
    assert np.array_equal(as_u16(ov)[live], vu[live])


@pytest.mark.parametrize("Q,N,H,D", [(4, 2000, 2, 128), (3, 257, 4, 64), (2, 1, 2, 32),
                                     (1, 0, 2, 128)])
def test_attention_ref(tq, oracle, cuda, Q, N, H, D):
    print(f"[sdpa ref] Q={Q} N={N} H={H} D={D}", flush=True)
    cfg = _cfg(tq, H, D, 16)
    g = torch.Generator().manual_seed(90)
    q = torch.randn(Q, H, D, generator=g).half()
    k = torch.randn(max(N, 1), H, D, generator=g).half()
    v = torch.randn(max(N, 1), H, D, generator=g).half()
    out = torch.full((Q, H, D), 3.0, dtype=torch.float16, device=cuda)
    lg = torch.zeros(Q * H * max(N, 1), dtype=torch.float32, device=cuda)
    tq.attention_ref(q.to(cuda), k.to(cuda), v.to(cuda), out, lg, cfg, Q, N)
    got = out.cpu().float().numpy()
    if N == 0:
        assert np.all(got == 0.0)
        return
    ro, rl = oracle.sdpa_gpu_ref(as_u16(q), as_u16(k[:N]), as_u16(v[:N]))
    ref = ro.view(np.float16).astype(np.float32)
    assert _rel_err(got, ref) < ATT_TOL
    glg = lg.cpu().numpy().reshape(Q, H, N)
    assert np.abs(glg - rl).max() <= 1e-5 * max(np.abs(rl).max(), 1.0)
