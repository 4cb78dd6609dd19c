"""Cache-layout dequant and the layer-pipelined loader, against the ABI's own
[N, H, D] dequant (itself bit-exact against the oracle in
test_gpu_parity.py): the [1, H, N, D] output must equal its permutation bit
for bit, and the loader must reproduce a per-layer copy + dequant."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, kv_tokens_major, permuted_slots

pytestmark = pytest.mark.gpu


def _setup(tq, scheme, N, H, D, B, seed, cuda, slot_seed=None):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    prod = scheme == "turbo_prod"
    layout = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=seed)
    slots = permuted_slots(N, B, seed=slot_seed if slot_seed is not None else seed + 1).to(cuda)
    pages = int(slots.max().item()) // B + 1
    pool = torch.zeros(pages * layout.page_size_bytes, dtype=torch.uint8, device=cuda)
    (tq.pack if prod else tq.mse_pack)(k.to(cuda), v.to(cuda), slots, pool, layout, cfg)
    return cfg, layout, slots, pool


def _nhd(tq, scheme, pool, slots, layout, cfg, N, cuda):
    H, D = cfg.num_kv_heads, cfg.head_dim
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    (tq.dequant if scheme == "turbo_prod" else tq.mse_dequant)(pool, slots, ok, ov, layout, cfg)
    return ok, ov


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("N,H,D,B", [(4100, 2, 128, 16), (777, 4, 64, 16), (300, 2, 16, 8)])
def test_dequant_hnd_is_permuted_nhd(tq, cuda, scheme, N, H, D, B):
    print(f"[dequant hnd {scheme}] N={N} H={H} D={D}", flush=True)
    cfg, layout, slots, pool = _setup(tq, scheme, N, H, D, B, 70, cuda)
    ok, ov = _nhd(tq, scheme, pool, slots, layout, cfg, N, cuda)
    hk = torch.full((1, H, N, D), 3.0, dtype=torch.float16, device=cuda)
    hv = torch.full_like(hk, 3.0)
    fn = tq.dequant_hnd if scheme == "turbo_prod" else tq.mse_dequant_hnd
    fn(pool, slots, hk, hv, layout, cfg, N)
    torch.cuda.synchronize()
    assert np.array_equal(as_u16(hk[0]), as_u16(ok.permute(1, 0, 2)))
    assert np.array_equal(as_u16(hv[0]), as_u16(ov.permute(1, 0, 2)))


def test_dequant_hnd_leaves_unmapped_tokens(tq, cuda):
    N, H, D, B = 500, 2, 128, 16
    cfg, layout, slots, pool = _setup(tq, "turbo_prod", N, H, D, B, 71, cuda)
    ok, ov = _nhd(tq, "turbo_prod", pool, slots, layout, cfg, N, cuda)
    holes = slots.clone()
    holes[::9] = -1
    hk = torch.full((1, H, N, D), 3.0, dtype=torch.float16, device=cuda)
    hv = torch.full_like(hk, 3.0)
    tq.dequant_hnd(pool, holes, hk, hv, layout, cfg, N)
    torch.cuda.synchronize()
    live = (holes >= 0).cpu().numpy()
    assert np.array_equal(as_u16(hk[0])[:, live], as_u16(ok.permute(1, 0, 2))[:, live])
    assert np.all(hk[0][:, ~torch.from_numpy(live).to(cuda)].float().cpu().numpy() == 3.0)


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("pinned,two_streams", [(True, True), (False, True), (True, False)])
def test_load_layers_matches_per_layer_dequant(tq, cuda, scheme, pinned, two_streams):
    print(f"[load_layers {scheme}] pinned={pinned} two_streams={two_streams}", flush=True)
    NL, N, H, D, B = 5, 3000, 2, 128, 16
    refs, host, dev_pools, oks, ovs = [], [], [], [], []
    cfg = layout = slots = None
    for layer in range(NL):
        # one slot mapping for every layer (the loader takes one, as a document's layers share it)
        cfg, layout, slots, pool = _setup(tq, scheme, N, H, D, B, 80 + 7 * layer, cuda,
                                          slot_seed=79)
        ok, ov = _nhd(tq, scheme, pool, slots, layout, cfg, N, cuda)
        refs.append((ok.permute(1, 0, 2).contiguous(), ov.permute(1, 0, 2).contiguous()))
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
        assert np.array_equal(as_u16(oks[layer][0]), as_u16(refs[layer][0])), layer
        assert np.array_equal(as_u16(ovs[layer][0]), as_u16(refs[layer][1])), layer
