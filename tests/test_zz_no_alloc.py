"""The allocation-free turbo_prod attention entry
(tq_launch_turbo_prod_fused_attention_output_noalloc), called through the C
ABI, against the allocating entry (tq_launch_turbo_prod_fused_attention_output)
on the same inputs: identical outputs (same kernels), on two calls in a row
with the second one smaller, under graph capture, and a launch too large for
the static scratch rejected with rc -2."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, gqa_rows, kv_tokens_major, permuted_slots, query

pytestmark = pytest.mark.gpu


def _case(oracle, N, seed, Q=8, H=2, D=128, B=16):
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    pool = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    q = gqa_rows(query(Q * H, D, seed=seed + 2), H)
    ref = oracle.prod_attention_f64(as_u16(q), pool, slots.numpy(), B)
    return q, pool, slots, ref


def _cfg(tq, H=2, D=128):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    return cfg, tq.make_layout_for(cfg)


def _rel(got, ref):
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.abs(r).max(axis=1)).max())


def test_noalloc_matches_allocating_entry_twice_smaller_second(tq, oracle, cuda):
    cfg, lp = _cfg(tq)
    oracle.nthreads = 16
    for n, seed in ((32768, 90), (3000, 91)):  # the second call smaller
        print(f"[noalloc] N={n}", flush=True)
        q, pool, slots, ref = _case(oracle, n, seed)
        q, pool_d, slots_d = q.to(cuda), torch.from_numpy(pool).to(cuda), slots.to(cuda)
        a = torch.full((8, 2, 128), 9.0, dtype=torch.float16, device=cuda)
        b = torch.full_like(a, 9.0)
        tq.fused_attn_output(q, pool_d, slots_d, a, lp, cfg, 8, n)
        rc = tq.lib.tq_launch_turbo_prod_fused_attention_output_noalloc(
            ctypes.c_void_p(q.data_ptr()), ctypes.cast(pool_d.data_ptr(), ctypes.POINTER(ctypes.c_uint8)),
            ctypes.cast(slots_d.data_ptr(), ctypes.POINTER(ctypes.c_int32)),
            ctypes.c_void_p(b.data_ptr()), ctypes.byref(lp), ctypes.byref(cfg), 8, n, None)
        torch.cuda.synchronize()
        assert rc == 0, tq.lib.tq_last_error()
        assert np.array_equal(as_u16(a), as_u16(b))
        assert _rel(b.cpu().float().numpy(), ref) < 1e-3


def test_noalloc_under_graph_capture(tq, oracle, cuda):
    cfg, lp = _cfg(tq)
    q, pool, slots, ref = _case(oracle, 5000, 92)
    q, pool_d, slots_d = q.to(cuda), torch.from_numpy(pool).to(cuda), slots.to(cuda)
    want = torch.empty(8, 2, 128, dtype=torch.float16, device=cuda)
    tq.fused_attn_output(q, pool_d, slots_d, want, lp, cfg, 8, 5000)
    out = torch.zeros_like(want)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # eager first call on this device (resolves the array)
        tq.fused_attn_output_noalloc(q, pool_d, slots_d, out, lp, cfg, 8, 5000,
                                     stream=side.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        tq.fused_attn_output_noalloc(q, pool_d, slots_d, out, lp, cfg, 8, 5000,
                                     stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(7.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(as_u16(out), as_u16(want)), rep
    del g


def test_noalloc_scratch_boundary(tq, oracle, cuda):
    """One kv head and 16 tokens (one split per row group): 1,008 row groups
    need 1,008 split partials of 4,160 bytes (4,193,280 of the 4,194,304
    scratch bytes) and are accepted, equal to the allocating entry and the
    oracle; 1,009 (4,197,440 bytes) are refused with rc -2 and the output
    untouched."""
    cfg, lp = _cfg(tq, H=1)
    N, B = 16, 16
    k, v = kv_tokens_major(N, 1, 128, seed=95)
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    pool = torch.zeros(lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    tq.pack(k.to(cuda), v.to(cuda), slots, pool, lp, cfg)
    for groups, ok in ((1008, True), (1009, False)):
        print(f"[noalloc boundary] row groups={groups}", flush=True)
        Q = 8 * groups
        q = query(Q, 128, seed=96).reshape(Q, 1, 128).to(cuda)
        out = torch.full((Q, 1, 128), 3.0, dtype=torch.float16, device=cuda)
        if not ok:
            with pytest.raises(RuntimeError, match="split-K scratch"):
                tq.fused_attn_output_noalloc(q, pool, slots, out, lp, cfg, Q, N)
            torch.cuda.synchronize()
            assert torch.all(out == 3.0)  # nothing ran
            continue
        tq.fused_attn_output_noalloc(q, pool, slots, out, lp, cfg, Q, N)
        want = torch.zeros_like(out)
        tq.fused_attn_output(q, pool, slots, want, lp, cfg, Q, N)
        torch.cuda.synchronize()
        assert np.array_equal(as_u16(out), as_u16(want))
        ref = oracle.prod_attention_f64(as_u16(q.cpu()), pool.cpu().numpy(), slots.cpu().numpy(),
                                        B)
        assert _rel(out.cpu().float().numpy(), ref) < 1e-3


def test_noalloc_rejects_launch_beyond_scratch(tq, cuda):
    """1000 row groups of 8 rows x 2 kv heads need 2,000 split partials of
    4,160 bytes: more than the 4 MiB scratch -> rc -2, nothing launched."""
    cfg, lp = _cfg(tq)
    Q, N = 8 * 1000, 16
    q = torch.zeros(Q, 2, 128, dtype=torch.float16, device=cuda)
    pool = torch.zeros(lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    out = torch.full_like(q, 3.0)
    with pytest.raises(RuntimeError, match="split-K scratch"):
        tq.fused_attn_output_noalloc(q, pool, slots, out, lp, cfg, Q, N)
    torch.cuda.synchronize()
    assert torch.all(out == 3.0)  # nothing ran
