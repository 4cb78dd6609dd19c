"""Cache-layout dequant ([1, H, N, D], *_dequant_kv_hnd) and the
layer-pipelined loader (tq_load_*_layers) against the CPU oracle: pools are
packed on the GPU and checked against oracle.prod_pack / mse_pack byte for
byte, and every [1, H, N, D] output must equal the oracle's dequant of the
pool (oracle.prod_dequant / mse_dequant), transposed, bit for bit — with
shuffled pages, at small shapes and at config 3's full size (36 layers x
32768 tokens)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, kv_tokens_major, permuted_slots

pytestmark = pytest.mark.gpu


def _setup(tq, oracle, scheme, N, H, D, B, seed, cuda, slot_seed=None, check_pack=True):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    prod = scheme == "turbo_prod"
    layout = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=slot_seed if slot_seed is not None else seed + 1).to(cuda)
    pages = int(slots.max().item()) // B + 1
    pool = torch.zeros(pages * layout.page_size_bytes, dtype=torch.uint8, device=cuda)
    (tq.pack if prod else tq.mse_pack)(k.to(cuda), v.to(cuda), slots, pool, layout, cfg)
    if check_pack:
        torch.cuda.synchronize()
        want = (oracle.prod_pack if prod else oracle.mse_pack)(
            as_u16(k), as_u16(v), slots.cpu().numpy(), pages, B)
        assert np.array_equal(pool.cpu().numpy(), want)
    return cfg, layout, slots, pool


def _oracle_hnd(oracle, scheme, pool, slots, cfg):
    """The oracle's dequant of the pool, as [H, N, D] fp16 bit patterns."""
    fn = oracle.prod_dequant if scheme == "turbo_prod" else oracle.mse_dequant
    wk, wv = fn(pool.cpu().numpy(), slots.cpu().numpy(), cfg.num_kv_heads, cfg.head_dim,
                cfg.block_size)
    return wk.transpose(1, 0, 2), wv.transpose(1, 0, 2)


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("N,H,D,B", [(4100, 2, 128, 16), (777, 4, 64, 16), (300, 2, 16, 8)])
def test_dequant_hnd_matches_oracle(tq, oracle, cuda, scheme, N, H, D, B):
    print(f"[dequant hnd {scheme}] N={N} H={H} D={D}", flush=True)
    cfg, layout, slots, pool = _setup(tq, oracle, scheme, N, H, D, B, 70, cuda)
    hk = torch.full((1, H, N, D), 3.0, dtype=torch.float16, device=cuda)
    hv = torch.full_like(hk, 3.0)
    fn = tq.dequant_hnd if scheme == "turbo_prod" else tq.mse_dequant_hnd
    fn(pool, slots, hk, hv, layout, cfg, N)
    torch.cuda.synchronize()
    wk, wv = _oracle_hnd(oracle, scheme, pool, slots, cfg)
    assert np.array_equal(as_u16(hk[0]), wk)
    assert np.array_equal(as_u16(hv[0]), wv)


def test_dequant_hnd_leaves_unmapped_tokens(tq, oracle, cuda):
    N, H, D, B = 500, 2, 128, 16
    cfg, layout, slots, pool = _setup(tq, oracle, "turbo_prod", N, H, D, B, 71, cuda)
    holes = slots.clone()
    holes[::9] = -1
    hk = torch.full((1, H, N, D), 3.0, dtype=torch.float16, device=cuda)
    hv = torch.full_like(hk, 3.0)
    tq.dequant_hnd(pool, holes, hk, hv, layout, cfg, N)
    torch.cuda.synchronize()
    live = (holes >= 0).cpu().numpy()
    wk, _ = _oracle_hnd(oracle, "turbo_prod", pool, slots, cfg)
    assert np.array_equal(as_u16(hk[0])[:, live], wk[:, live])
    assert np.all(hk[0][:, ~torch.from_numpy(live).to(cuda)].float().cpu().numpy() == 3.0)


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("pinned,two_streams", [(True, True), (False, True), (True, False)])
def test_load_layers_matches_oracle(tq, oracle, cuda, scheme, pinned, two_streams):
    print(f"[load_layers {scheme}] pinned={pinned} two_streams={two_streams}", flush=True)
    NL, N, H, D, B = 5, 3000, 2, 128, 16
    host, dev_pools, oks, ovs = [], [], [], []
    cfg = layout = slots = None
    for layer in range(NL):
        # one slot mapping for every layer (the loader takes one, as a document's layers share it)
        cfg, layout, slots, pool = _setup(tq, oracle, scheme, N, H, D, B, 80 + 7 * layer, cuda,
                                          slot_seed=79)
        hp = pool.cpu()
        host.append(hp.pin_memory() if pinned else hp)
        dev_pools.append(torch.zeros_like(pool))
        oks.append(torch.zeros(1, H, N, D, dtype=torch.float16, device=cuda))
        ovs.append(torch.zeros(1, H, N, D, dtype=torch.float16, device=cuda))
    torch.cuda.synchronize()
    compute = torch.cuda.current_stream()
    copy = torch.cuda.Stream() if two_streams else compute
    tq.load_layers(scheme, host, dev_pools, slots, oks, ovs, layout, cfg, N,
                   copy_stream=copy.cuda_stream, compute_stream=compute.cuda_stream)
    torch.cuda.synchronize()
    for layer in range(NL):
        assert torch.equal(dev_pools[layer].cpu(), host[layer])
        wk, wv = _oracle_hnd(oracle, scheme, host[layer], slots, cfg)
        assert np.array_equal(as_u16(oks[layer][0]), wk), layer
        assert np.array_equal(as_u16(ovs[layer][0]), wv), layer


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_load_layers_config3_full_size(tq, oracle, cuda, scheme):
    """Config 3: 36 layers x 32768 tokens (2 kv heads, head_dim 128, one
    shuffled page table) from pinned host pages through the loader into
    [1, H, N, D]; every layer's output against the oracle's dequant of its
    pages.  The pages are packed on the GPU from device-drawn K/V; layers 0
    and 35 have their pages checked against the oracle's pack."""
    NL, N, H, D, B = 36, 32768, 2, 128, 16
    print(f"[load_layers config 3 {scheme}] {NL} x {N}", flush=True)
    oracle.nthreads = 16
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    prod = scheme == "turbo_prod"
    layout = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    slots = permuted_slots(N, B, seed=301).to(cuda)
    pages = N // B
    host, dev_pools, oks, ovs = [], [], [], []
    for layer in range(NL):
        g = torch.Generator(device=cuda).manual_seed(300 + layer)
        k = torch.randn(N, H, D, generator=g, device=cuda).half()
        v = torch.randn(N, H, D, generator=g, device=cuda).half()
        pool = torch.zeros(pages * layout.page_size_bytes, dtype=torch.uint8, device=cuda)
        (tq.pack if prod else tq.mse_pack)(k, v, slots, pool, layout, cfg)
        if layer in (0, NL - 1):
            torch.cuda.synchronize()
            want = (oracle.prod_pack if prod else oracle.mse_pack)(
                as_u16(k), as_u16(v), slots.cpu().numpy(), pages, B)
            assert np.array_equal(pool.cpu().numpy(), want), layer
        host.append(pool.cpu().pin_memory())
        dev_pools.append(torch.empty_like(pool))
        oks.append(torch.empty(1, H, N, D, dtype=torch.float16, device=cuda))
        ovs.append(torch.empty(1, H, N, D, dtype=torch.float16, device=cuda))
        del k, v, pool
    torch.cuda.synchronize()
    copy = torch.cuda.Stream()
    compute = torch.cuda.current_stream()
    tq.load_layers(scheme, host, dev_pools, slots, oks, ovs, layout, cfg, N,
                   copy_stream=copy.cuda_stream, compute_stream=compute.cuda_stream)
    torch.cuda.synchronize()
    for layer in range(NL):
        wk, wv = _oracle_hnd(oracle, scheme, host[layer], slots, cfg)
        assert np.array_equal(as_u16(oks[layer][0]), wk), layer
        assert np.array_equal(as_u16(ovs[layer][0]), wv), layer
    print("    36 layers bit-exact", flush=True)
