"""Seeded random geometries against the CPU oracle: every dequant kernel the
library picks (a whole row per lane for several layers, half a row per lane
for one layer, four lanes per row for other head dims, the generic kernel for
pages not 4-byte aligned), both schemes, both output layouts, unmapped tokens,
and attention (and turbo_prod logits) on the same pools.

Each case draws N in [1, 3000], H in {1, 2, 3, 4, 8}, a block size in
{1, 3, 7, 16, 32} and D in {32, 64, 128} (mostly 128) from the splitmix64
stream of the synthetic-input generator, so the cases are the same on every
machine.  Bars: pools and dequantized halves bit-exact (unmapped tokens keep
their output); attention within max rel err 1e-3 of the fp64 oracle;
turbo_prod logits within 1e-5 of the oracle's fp32 logits (-inf for unmapped
tokens).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, gqa_rows, kv_tokens_major, query, uniform_ints

pytestmark = pytest.mark.gpu

NCASES = 48
_HS = (1, 2, 3, 4, 8)
_BS = (1, 3, 7, 16, 32)
_DS = (32, 64, 128, 128, 128)


def _case(i: int):
    u = uniform_ints(9100 + i, 8, 0, 1 << 30)
    N = 1 + int(u[0] % 3000)
    H = _HS[int(u[1] % len(_HS))]
    B = _BS[int(u[2] % len(_BS))]
    D = _DS[int(u[3] % len(_DS))]
    scheme = "turbo_prod" if u[4] % 2 == 0 else "turbo_mse"
    holes = u[5] % 3 == 0
    head_major = u[6] % 2 == 1
    layers = 1 + int(u[7] % 3)
    return N, H, B, D, scheme, holes, head_major, layers


def _slots(N: int, B: int, seed: int, holes: bool) -> np.ndarray:
    pages = (N + B - 1) // B + 3
    perm = np.argsort(uniform_ints(seed, pages, 0, 1 << 30), kind="stable")[: (N + B - 1) // B]
    t = np.arange(N)
    s = (perm[t // B] * B + t % B).astype(np.int32)
    if holes:
        s[uniform_ints(seed + 1, N, 0, 4) == 0] = -1
    return s


@pytest.mark.parametrize("i", range(NCASES))
def test_random_geometry_pack_dequant_attention(tq, oracle, cuda, i):
    N, H, B, D, scheme, holes, head_major, L = _case(i)
    print(f"[random {i}] {scheme} N={N} H={H} B={B} D={D} holes={holes} "
          f"head_major={head_major} layers={L}", flush=True)
    prod = scheme == "turbo_prod"
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lay = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    sl = _slots(N, B, 9200 + i, holes)
    pages = int(sl.max()) // B + 1 if (sl >= 0).any() else 1
    slots = torch.from_numpy(sl).to(cuda)
    live = sl >= 0
    seven = np.float16(7.0).view(np.uint16)
    pack = tq.pack if prod else tq.mse_pack
    opack = oracle.prod_pack if prod else oracle.mse_pack
    odeq = oracle.prod_dequant if prod else oracle.mse_dequant
    pools, kvs = [], []
    for layer in range(L):
        k, v = kv_tokens_major(N, H, D, seed=9300 + 10 * i + layer)
        pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
        pack(k.to(cuda), v.to(cuda), slots, pool, lay, cfg)
        pools.append(pool)
        kvs.append((k, v))
    torch.cuda.synchronize()
    want_pools = [opack(as_u16(k), as_u16(v), sl, pages, B) for k, v in kvs]
    for layer in range(L):
        got = pools[layer].cpu().numpy()
        bad = np.flatnonzero(got != want_pools[layer])
        assert bad.size == 0, f"layer {layer}: {bad.size} pool bytes differ, first at {bad[:8]}"

    shape = (1, H, N, D) if head_major else (N, H, D)

    def check(ok, ov, layer):
        wk, wv = odeq(want_pools[layer], sl, H, D, B)
        gk, gv = as_u16(ok), as_u16(ov)
        if head_major:
            gk, gv = gk[0].transpose(1, 0, 2), gv[0].transpose(1, 0, 2)
        assert np.array_equal(gk[live], wk[live]) and np.array_equal(gv[live], wv[live]), layer
        assert np.all(gk[~live] == seven) and np.all(gv[~live] == seven), layer

    # one layer per call
    ok = torch.full(shape, 7.0, dtype=torch.float16, device=cuda)
    ov = torch.full(shape, 7.0, dtype=torch.float16, device=cuda)
    if head_major:
        (tq.dequant_hnd if prod else tq.mse_dequant_hnd)(pools[0], slots, ok, ov, lay, cfg, N)
    else:
        (tq.dequant if prod else tq.mse_dequant)(pools[0], slots, ok, ov, lay, cfg)
    torch.cuda.synchronize()
    check(ok, ov, 0)
    # every layer in one call
    oks = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(L)]
    ovs = [torch.full(shape, 7.0, dtype=torch.float16, device=cuda) for _ in range(L)]
    tq.dequant_layers(scheme, pools, slots, oks, ovs, lay, cfg, N, head_major=head_major)
    torch.cuda.synchronize()
    for layer in range(L):
        check(oks[layer], ovs[layer], layer)

    # attention over layer 0 (GQA 2 query rows per kv head), unless every token is unmapped
    if not live.any():
        return
    rows = 2
    qa = gqa_rows(query(rows * H, D, seed=9400 + i), H).contiguous()
    out = torch.empty(rows, H, D, dtype=torch.float16, device=cuda)
    att = tq.fused_attn_output if prod else tq.mse_fused_attn_output
    att(qa.to(cuda), pools[0], slots, out, lay, cfg, rows, N)
    torch.cuda.synchronize()
    fatt = oracle.prod_attention_f64 if prod else oracle.mse_attention_f64
    ref = fatt(as_u16(qa), want_pools[0], sl, B)
    g = out.cpu().float().numpy().reshape(-1, D).astype(np.float64)
    r = ref.reshape(-1, D)
    err = (np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max()
    assert err <= 1e-3, err

    # turbo_prod logits of 1-13 query rows over layer 0: within 1e-5 of the
    # oracle's reference-order fp32 logits per row, -inf for unmapped tokens
    if not prod:
        return
    Q = 1 + i % 13
    q = kv_tokens_major(Q, H, D, seed=9500 + i)[0]
    logits = torch.zeros(Q * H * N, dtype=torch.float32, device=cuda)
    tq.fused_attn_logits(q.to(cuda), pools[0], slots, logits, lay, cfg, Q, N)
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(Q, H, N)
    ref32 = oracle.prod_logits(as_u16(q), want_pools[0], sl, B)
    assert np.all(np.isneginf(got[:, :, ~live]))
    scale = np.abs(ref32[:, :, live]).max(axis=-1, keepdims=True) + 1e-30
    assert (np.abs(got[:, :, live] - ref32[:, :, live]) / scale).max() < 1e-5
