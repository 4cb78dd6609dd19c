"""The workload configurations at their stated shapes, against the CPU oracle.

* Config 5: one serving step of 32 sequences, lengths U[1024, 32768]
  (seed 500), 1-8 new tokens each (seed 501), both schemes.  The whole page
  pool after the append (every prefill and appended cell, and the zero bytes
  of unused pages) equals the oracle's pack of the same tokens into the same
  slots; sampled row groups (the longest and the shortest sequence's last
  position included) against the fp64 oracle attention.
* Dequant at 32768 tokens x 2 heads, both schemes, and at N*H beyond one
  pass of the persistent dequant grid (40000 x 2, 16384 x 8).
* Matrix-core attention with 8 kv heads at head_dim 128, and single-query
  decode (num_queries = 1, the reference store's call) at 32K context.
* Config 2's 36-layer pack as one launch, and the multi-layer dequant.
* The attention workspace: growth, retirement, stream cycling and graphs.

Bars: pools and dequantized halves bit-exact; attention max rel err per
(row, head) <= 1e-3 against the fp64 oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.batched import PagedBatch
from turborag_amd.synthetic import (as_u16, gqa_rows, kv_tokens_major, permuted_slots, query,
                                    uniform_ints)

pytestmark = pytest.mark.gpu
ATT_TOL = 1e-3


def _rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max())


def _cfg(tq, H, D, B=16):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    return cfg, tq.make_layout_for(cfg), tq.make_mse_layout_for(cfg)


# ── config 5 ────────────────────────────────────────────────────────── #

@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_config5_batched_step_full_shape(tq, oracle, cuda, scheme):
    lens = uniform_ints(500, 32, 1024, 32768)
    widths = uniform_ints(501, 32, 1, 8)
    print(f"[config 5 {scheme}] {int(lens.sum())} prefill tokens, {int(widths.sum())} new",
          flush=True)
    oracle.nthreads = 16
    b = PagedBatch(tq, scheme, lens, widths, seed=500, device=cuda)
    new = b.append_new_tokens(seed=503)
    query_t, row_seq, row_len = b.decode_rows(seed=504)
    out = torch.zeros_like(query_t)
    b.attention(query_t, row_seq, row_len, b.block_tables(), out)
    torch.cuda.synchronize()
    pool = b.pool.cpu().numpy()

    # Every cell: the oracle packs each sequence's prefill and new tokens
    # into the slots the block table gave them.
    keys, vals, slots = [], [], []
    for s, (L, w) in enumerate(zip(b.lens, b.widths)):
        sl = b.slots_of(s, L + w)
        keys += [b.kv[s][0], new[s][0]]
        vals += [b.kv[s][1], new[s][1]]
        slots.append(sl)
    k_all, v_all = torch.cat(keys), torch.cat(vals)
    pages = pool.size // b.layout.page_size_bytes
    pack = oracle.prod_pack if scheme == "turbo_prod" else oracle.mse_pack
    want = pack(as_u16(k_all), as_u16(v_all), np.concatenate(slots), pages, b.B)
    bad = np.flatnonzero(pool != want)
    assert bad.size == 0, f"{bad.size} pool bytes differ, first at {bad[:8]}"

    # Attention of sampled row groups (sequence, position).
    groups = [(s, j) for s in range(b.S) for j in range(b.widths[s])]
    first_row = {}
    r = 0
    for g in groups:
        first_row[g] = r
        r += 8
    longest, shortest = int(np.argmax(lens)), int(np.argmin(lens))
    pick = {(longest, b.widths[longest] - 1), (shortest, b.widths[shortest] - 1)}
    rng = np.random.default_rng(77)
    for i in rng.choice(len(groups), size=16, replace=False):
        pick.add(groups[int(i)])
    q_np = as_u16(query_t)
    got = out.cpu().float().numpy()
    f64 = oracle.prod_attention_f64 if scheme == "turbo_prod" else oracle.mse_attention_f64
    worst = 0.0
    for (s, j) in sorted(pick):
        rows = slice(first_row[(s, j)], first_row[(s, j)] + 8)
        ref = f64(q_np[rows].copy(), want, b.slots_of(s, b.lens[s] + j + 1), b.B)
        worst = max(worst, _rel_err(got[rows], ref))
    print(f"    {len(pick)} row groups, worst rel err {worst:.3e}", flush=True)
    assert worst < ATT_TOL
    b.close()


# ── dequant at full size and past one grid pass ─────────────────────── #

@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("N,H", [(32768, 2), (40000, 2), (16384, 8)])
def test_dequant_large_vs_oracle(tq, oracle, cuda, scheme, N, H):
    """32768 x 2 is config 3's layer; 40000 x 2 and 16384 x 8 exceed the
    65536 rows one pass of the persistent grid covers, so every wave walks
    more than one row group."""
    D, B = 128, 16
    print(f"[dequant {scheme}] N={N} H={H}", flush=True)
    oracle.nthreads = 16
    k, v = kv_tokens_major(N, H, D, seed=310 + H)
    slots = permuted_slots(N, B, seed=311, num_pages=N // B + 3)
    pages = int(slots.max()) // B + 1
    cfg, lp, lm = _cfg(tq, H, D, B)
    prod = scheme == "turbo_prod"
    lay = lp if prod else lm
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    (tq.pack if prod else tq.mse_pack)(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lay, cfg)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    (tq.dequant if prod else tq.mse_dequant)(pool, slots.to(cuda), ok, ov, lay, cfg)
    torch.cuda.synchronize()
    want = (oracle.prod_pack if prod else oracle.mse_pack)(as_u16(k), as_u16(v), slots.numpy(),
                                                           pages, B)
    assert np.array_equal(pool.cpu().numpy(), want)
    wk, wv = (oracle.prod_dequant if prod else oracle.mse_dequant)(want, slots.numpy(), H, D, B)
    assert np.array_equal(as_u16(ok), wk)
    assert np.array_equal(as_u16(ov), wv)


# ── attention shapes ─────────────────────────────────────────────────── #

@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("Q,H,N,seed", [
    (8, 8, 3000, 41),      # 8 kv heads, one row group each (matrix-core path)
    (16, 8, 5000, 42),     # two row groups per kv head
    (5, 4, 777, 43),       # a partial row group
    (1, 2, 32768, 44),     # single-query decode at 32K (cag_store.py:284, num_queries = 1)
    (8, 2, 32768, 45),     # config 4: GQA 16/2 at 32K
])
def test_attention_d128_shapes(tq, oracle, cuda, scheme, Q, H, N, seed):
    D, B = 128, 16
    print(f"[attention {scheme}] Q={Q} H={H} N={N}", flush=True)
    oracle.nthreads = 16
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    q = kv_tokens_major(Q, H, D, seed=seed + 2)[0]
    cfg, lp, lm = _cfg(tq, H, D, B)
    prod = scheme == "turbo_prod"
    pool_np = (oracle.prod_pack if prod else oracle.mse_pack)(as_u16(k), as_u16(v),
                                                              slots.numpy(), pages, B)
    ref = (oracle.prod_attention_f64 if prod else oracle.mse_attention_f64)(
        as_u16(q), pool_np, slots.numpy(), B)
    out = torch.zeros(Q, H, D, dtype=torch.float16, device=cuda)
    fn = tq.fused_attn_output if prod else tq.mse_fused_attn_output
    fn(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), out, lp if prod else lm,
       cfg, Q, N)
    torch.cuda.synchronize()
    err = _rel_err(out.cpu().float().numpy(), ref)
    print(f"    rel err {err:.3e}", flush=True)
    assert err < ATT_TOL


def test_attention_more_row_groups_than_a_grid_dimension(tq, oracle, cuda):
    """65,537 row groups of one kv head: more than a grid's y/z dimension
    holds, so the split launch falls back to its one-dimensional grid.
    Sampled rows (the first and the last row group included) against the
    fp64 oracle."""
    Q, H, D, B, N = 65537 * 8, 1, 128, 16, 40
    print(f"[attention 1-D grid] Q={Q} H={H} N={N}", flush=True)
    k, v = kv_tokens_major(N, H, D, seed=46)
    slots = permuted_slots(N, B, seed=47)
    pages = int(slots.max()) // B + 1
    pool_np = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    q = torch.from_numpy(np.random.default_rng(48).standard_normal((Q, H, D)).astype(np.float16))
    cfg, lp, _ = _cfg(tq, H, D, B)
    out = torch.zeros(Q, H, D, dtype=torch.float16, device=cuda)
    tq.fused_attn_output(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), out, lp,
                         cfg, Q, N)
    torch.cuda.synchronize()
    rows = np.concatenate([np.arange(16), np.arange(Q - 16, Q),
                           np.random.default_rng(49).choice(Q, size=64, replace=False)])
    ref = oracle.prod_attention_f64(as_u16(q)[rows].copy(), pool_np, slots.numpy(), B)
    err = _rel_err(out.cpu().float().numpy()[rows], ref)
    print(f"    {rows.size} sampled rows, rel err {err:.3e}", flush=True)
    assert err < ATT_TOL
    # No kv tokens: the combine alone writes zeros, on its one-dimensional grid.
    out.fill_(1.0)
    tq.fused_attn_output(q.to(cuda), torch.from_numpy(pool_np).to(cuda), slots.to(cuda), out, lp,
                         cfg, Q, 0)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out)) == 0


# ── the attention workspace ──────────────────────────────────────────── #

def _att_case(oracle, N, seed, H=2, D=128, B=16, Q=8):
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=seed + 1)
    pages = int(slots.max()) // B + 1
    pool = oracle.prod_pack(as_u16(k), as_u16(v), slots.numpy(), pages, B)
    q = gqa_rows(query(Q * H, D, seed=seed + 2), H)
    ref = oracle.prod_attention_f64(as_u16(q), pool, slots.numpy(), B)
    return q, pool, slots, ref


def test_workspace_growth_retire_and_release(tq, oracle, cuda):
    """Small, large (the workspace grows and the old buffer is retired),
    small again, then after the retired buffer's kernels finished (freed on
    the next call), and after tq_workspace_release: every output right."""
    oracle.nthreads = 16
    cfg, lp, _ = _cfg(tq, 2, 128)
    cases = [_att_case(oracle, n, 60 + i) for i, n in enumerate((1000, 32768, 700))]
    dev = [(q.to(cuda), torch.from_numpy(p).to(cuda), s.to(cuda), ref) for q, p, s, ref in cases]
    stream = torch.cuda.Stream()
    order = [0, 1, 0, 2, 1, "release", 2, 1]
    with torch.cuda.stream(stream):
        for step in order:
            if step == "release":
                torch.cuda.synchronize()
                tq.release_workspaces()
                continue
            q, pool, slots, ref = dev[step]
            out = torch.zeros(8, 2, 128, dtype=torch.float16, device=cuda)
            tq.fused_attn_output(q, pool, slots, out, lp, cfg, 8, slots.numel(),
                                 stream=stream.cuda_stream)
            stream.synchronize()
            assert _rel_err(out.cpu().float().numpy(), ref) < ATT_TOL, step


def _hip():
    import ctypes
    lib = ctypes.CDLL("libamdhip64.so")
    lib.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    lib.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    return lib


def test_workspace_many_streams(tq, oracle, cuda):
    """70 distinct HIP streams (default priority), one call each with no
    synchronization in between: past 64 cached streams the least recently
    used buffers are evicted (freed, or retired behind an event on their
    stream while its kernels still run); every output stays right."""
    import ctypes
    cfg, lp, _ = _cfg(tq, 2, 128)
    q, pool, slots, ref = _att_case(oracle, 1200, 70)
    q, pool, slots = q.to(cuda), torch.from_numpy(pool).to(cuda), slots.to(cuda)
    torch.cuda.synchronize()
    hip = _hip()
    streams = []
    for _ in range(70):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        streams.append(h.value)
    outs = []
    try:
        for st in streams:
            out = torch.zeros(8, 2, 128, dtype=torch.float16, device=cuda)
            torch.cuda.synchronize()  # the zero fill (on torch's stream) before the call
            tq.fused_attn_output(q, pool, slots, out, lp, cfg, 8, 1200, stream=st)
            outs.append(out)
        torch.cuda.synchronize()
        for out in outs:
            assert _rel_err(out.cpu().float().numpy(), ref) < ATT_TOL
    finally:
        torch.cuda.synchronize()
        tq.release_workspaces()
        for st in streams:
            hip.hipStreamDestroy(st)


def test_workspace_eviction_during_capture(tq, oracle, cuda):
    """A graph is being captured on one stream while calls on 70 other HIP
    streams cycle the cache past its 64 streams (evictions with no device
    synchronization): the capture stays valid, its replays and every eager
    output equal the oracle."""
    import ctypes
    cfg, lp, _ = _cfg(tq, 2, 128)
    q, pool, slots, ref = _att_case(oracle, 1500, 90)
    q, pool, slots = q.to(cuda), torch.from_numpy(pool).to(cuda), slots.to(cuda)
    qb, poolb, slotsb, refb = _att_case(oracle, 3000, 91)
    qb, poolb, slotsb = qb.to(cuda), torch.from_numpy(poolb).to(cuda), slotsb.to(cuda)
    tq.release_workspaces()
    hip = _hip()
    streams = []
    for _ in range(70):
        h = ctypes.c_void_p()
        assert hip.hipStreamCreate(ctypes.byref(h)) == 0
        streams.append(h.value)
    cap = torch.cuda.Stream()
    out = torch.zeros(8, 2, 128, dtype=torch.float16, device=cuda)
    outs = [torch.zeros(8, 2, 128, dtype=torch.float16, device=cuda) for _ in streams]
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap, capture_error_mode="relaxed"):
            tq.fused_attn_output(q, pool, slots, out, lp, cfg, 8, 1500,
                                 stream=torch.cuda.current_stream().cuda_stream)
            for st, o in zip(streams, outs):  # eager, on other streams, mid-capture
                tq.fused_attn_output(qb, poolb, slotsb, o, lp, cfg, 8, 3000, stream=st)
        torch.cuda.synchronize()
        for o in outs:
            assert _rel_err(o.cpu().float().numpy(), refb) < ATT_TOL
        for rep in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert _rel_err(out.cpu().float().numpy(), ref) < ATT_TOL, rep
        del g
    finally:
        torch.cuda.synchronize()
        tq.release_workspaces()
        for st in streams:
            hip.hipStreamDestroy(st)


def test_workspace_kept_for_captured_graph(tq, oracle, cuda):
    """A graph captured on a stream keeps its workspace: a larger eager call
    on the same stream afterwards (the workspace grows) must not free it, so
    replays of the graph stay right."""
    cfg, lp, _ = _cfg(tq, 2, 128)
    q, pool, slots, ref = [x for x in _att_case(oracle, 2000, 80)]
    q, pool, slots = q.to(cuda), torch.from_numpy(pool).to(cuda), slots.to(cuda)
    qb, poolb, slotsb, refb = _att_case(oracle, 32768, 81)
    qb, poolb, slotsb = qb.to(cuda), torch.from_numpy(poolb).to(cuda), slotsb.to(cuda)
    tq.release_workspaces()
    side = torch.cuda.Stream()
    out = torch.zeros(8, 2, 128, dtype=torch.float16, device=cuda)
    outb = torch.zeros_like(out)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # the stream's workspace exists before the capture
        tq.fused_attn_output(q, pool, slots, out, lp, cfg, 8, 2000, stream=side.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        tq.fused_attn_output(q, pool, slots, out, lp, cfg, 8, 2000,
                             stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert _rel_err(out.cpu().float().numpy(), ref) < ATT_TOL, rep
        with torch.cuda.stream(side):  # grows the stream's workspace (eager)
            tq.fused_attn_output(qb, poolb, slotsb, outb, lp, cfg, 8, 32768,
                                 stream=side.cuda_stream)
        torch.cuda.synchronize()
        assert _rel_err(outb.cpu().float().numpy(), refb) < ATT_TOL, rep
    del g
    torch.cuda.synchronize()
    tq.release_workspaces()


# ── multi-layer dequant (tq_launch_*_dequant_kv_layers) ──────────────── #

def _layer_pools(tq, scheme, NL, N, H, D, B, cuda, seed):
    cfg, lp, lm = _cfg(tq, H, D, B)
    prod = scheme == "turbo_prod"
    lay = lp if prod else lm
    slots = permuted_slots(N, B, seed=seed).to(cuda)
    pages = (N + B - 1) // B
    pools = []
    for layer in range(NL):
        g = torch.Generator(device=cuda).manual_seed(seed + 1 + layer)
        k = torch.randn(N, H, D, generator=g, device=cuda).half()
        v = torch.randn(N, H, D, generator=g, device=cuda).half()
        pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
        (tq.pack if prod else tq.mse_pack)(k, v, slots, pool, lay, cfg)
        pools.append(pool)
    return cfg, lay, slots, pools


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("NL,N,H,head_major", [
    (36, 32768, 2, False),    # config 3: 36 layers x 32768 tokens, one launch
    (36, 32768, 2, True),     # ... into the cache layout [1, H, N, D]
    (70, 1000, 2, False),     # more than 64 layers: two launches
    (3, 777, 8, True),        # 8 kv heads, a ragged last page
])
def test_dequant_layers_vs_oracle(tq, oracle, cuda, scheme, NL, N, H, head_major):
    D, B = 128, 16
    print(f"[dequant_layers {scheme}] {NL} x {N} H={H} head_major={head_major}", flush=True)
    oracle.nthreads = 16
    cfg, lay, slots, pools = _layer_pools(tq, scheme, NL, N, H, D, B, cuda, seed=330 + NL)
    shape = (1, H, N, D) if head_major else (N, H, D)
    oks = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(NL)]
    ovs = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(NL)]
    tq.dequant_layers(scheme, pools, slots, oks, ovs, lay, cfg, N, head_major=head_major)
    torch.cuda.synchronize()
    fn = oracle.prod_dequant if scheme == "turbo_prod" else oracle.mse_dequant
    sl = slots.cpu().numpy()
    for layer in range(NL):
        wk, wv = fn(pools[layer].cpu().numpy(), sl, H, D, B)
        gk, gv = as_u16(oks[layer]), as_u16(ovs[layer])
        if head_major:
            gk, gv = gk[0].transpose(1, 0, 2), gv[0].transpose(1, 0, 2)
        assert np.array_equal(gk, wk), layer
        assert np.array_equal(gv, wv), layer


@pytest.mark.parametrize("scheme,NL,N,H,B,head_major", [
    ("turbo_prod", 3, 531, 2, 16, False),  # row-per-lane kernel, holes, ragged last group
    ("turbo_mse", 3, 531, 3, 7, True),     # ... 3 kv heads, 7-token blocks (division paths)
    ("turbo_prod", 2, 300, 3, 7, False),   # page not 16-byte aligned: the per-layer kernels
])
def test_dequant_layers_holes_and_geometry(tq, oracle, cuda, scheme, NL, N, H, B, head_major):
    """Unmapped tokens (slot -1) keep their output untouched; mapped ones are
    bit-exact against the oracle, with non-power-of-two heads and blocks; for
    the multi-layer entry and the one-layer entry."""
    D = 128
    print(f"[dequant_layers holes {scheme}] {NL} x {N} H={H} B={B} head_major={head_major}",
          flush=True)
    cfg, lp, lm = _cfg(tq, H, D, B)
    prod = scheme == "turbo_prod"
    lay = lp if prod else lm
    slots = permuted_slots(N, B, seed=350 + N)
    slots[::5] = -1
    pages = int(slots.max().item()) // B + 1
    pools = []
    for layer in range(NL):
        k, v = kv_tokens_major(N, H, D, seed=360 + layer)
        pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
        (tq.pack if prod else tq.mse_pack)(k.to(cuda), v.to(cuda), slots.to(cuda), pool, lay, cfg)
        pools.append(pool)
    shape = (1, H, N, D) if head_major else (N, H, D)
    oks = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(NL)]
    ovs = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(NL)]
    tq.dequant_layers(scheme, pools, slots.to(cuda), oks, ovs, lay, cfg, N,
                      head_major=head_major)
    torch.cuda.synchronize()
    fn = oracle.prod_dequant if prod else oracle.mse_dequant
    sl = slots.numpy()
    live = sl >= 0
    seven = np.float16(7.0).view(np.uint16)
    for layer in range(NL):
        wk, wv = fn(pools[layer].cpu().numpy(), sl, H, D, B)
        gk, gv = as_u16(oks[layer]), as_u16(ovs[layer])
        if head_major:
            gk, gv = gk[0].transpose(1, 0, 2), gv[0].transpose(1, 0, 2)
        assert np.array_equal(gk[live], wk[live]), layer
        assert np.array_equal(gv[live], wv[live]), layer
        assert np.all(gk[~live] == seven) and np.all(gv[~live] == seven), layer
    # the one-layer entry on layer 0 (its own kernel choice), same bar
    ok1 = torch.full(shape, 7.0, dtype=torch.float16, device=cuda)
    ov1 = torch.full(shape, 7.0, dtype=torch.float16, device=cuda)
    one = {(True, False): tq.dequant, (False, False): tq.mse_dequant,
           (True, True): tq.dequant_hnd, (False, True): tq.mse_dequant_hnd}[(prod, head_major)]
    one(pools[0], slots.to(cuda), ok1, ov1, lay, cfg, *((N,) if head_major else ()))
    torch.cuda.synchronize()
    wk, wv = fn(pools[0].cpu().numpy(), sl, H, D, B)
    gk, gv = as_u16(ok1), as_u16(ov1)
    if head_major:
        gk, gv = gk[0].transpose(1, 0, 2), gv[0].transpose(1, 0, 2)
    assert np.array_equal(gk[live], wk[live]) and np.array_equal(gv[live], wv[live])
    assert np.all(gk[~live] == seven) and np.all(gv[~live] == seven)


# ── multi-layer pack (config 2 in one launch) ───────────────────────── #

@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("NL,N,H,D,slot_kind", [
    (36, 8192, 2, 128, "arange"),    # config 2: 36 layers x 8192 tokens, the store's slots
    (36, 8192, 2, 128, "shuffled"),  # ... shuffled 16-token pages
    (70, 100, 2, 128, "shuffled"),   # more than 64 layers: two launches
    (3, 300, 8, 64, "shuffled"),     # head_dim 64, 8 kv heads, a ragged last page
])
def test_pack_layers_vs_oracle(tq, oracle, cuda, scheme, NL, N, H, D, slot_kind):
    """Every layer's pool from one tq_launch_*_pack_kv_layers call equals the
    oracle's pack of that layer (seeds 200 + layer, one shared slot map) and
    the per-layer entry's pool."""
    B = 16
    print(f"[pack_layers {scheme}] {NL} x {N} H={H} D={D} {slot_kind}", flush=True)
    oracle.nthreads = 16
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    prod = scheme == "turbo_prod"
    lay = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    slots = (torch.arange(N, dtype=torch.int32) if slot_kind == "arange"
             else permuted_slots(N, B, seed=402, num_pages=N // B + 3))
    pages = int(slots.max()) // B + 1
    kv = [kv_tokens_major(N, H, D, seed=200 + layer) for layer in range(NL)]
    keys = [k.to(cuda) for k, _ in kv]
    values = [v.to(cuda) for _, v in kv]
    pools = [torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
             for _ in range(NL)]
    sl = slots.to(cuda)
    tq.pack_layers(scheme, keys, values, sl, pools, lay, cfg)
    one = torch.zeros_like(pools[0])
    torch.cuda.synchronize()
    pack = oracle.prod_pack if prod else oracle.mse_pack
    for layer in range(NL):
        want = pack(as_u16(kv[layer][0]), as_u16(kv[layer][1]), slots.numpy(), pages, B)
        assert np.array_equal(pools[layer].cpu().numpy(), want), layer
        if layer in (0, NL - 1):  # the per-layer entry gives the same bytes
            one.zero_()
            (tq.pack if prod else tq.mse_pack)(keys[layer], values[layer], sl, one, lay, cfg)
            torch.cuda.synchronize()
            assert torch.equal(one, pools[layer]), layer


# ── debug-sync mode ──────────────────────────────────────────────────── #

def test_debug_sync_mode_runs_the_smoke_path():
    """TQ_DEBUG_SYNC=1 (the reference's TQ_DEBUG_SYNC build switch, as an
    environment variable): every launching entry synchronizes its stream;
    the smoke path (pack, dequant, attention against the oracle) still
    passes.  Run in a child process, since the switch is read once."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    env = dict(os.environ, TQ_DEBUG_SYNC="1")
    r = subprocess.run([sys.executable, "-c", "import __graft_entry__ as g; g.smoke()"],
                       cwd=root, env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "smoke ok" in r.stdout
