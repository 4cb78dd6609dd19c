"""Layers at the row kernels' limit.  The buffer-store dequant kernels take
up to 2^23 - 1 (token, head) rows (their descriptors cover num_rows * 256
output bytes, below the 2^31 offset that marks a skipped row): 4,194,303
tokens x 2 kv heads = 8,388,606 rows run on them with output offsets up to
2^31 - 512, and 4,194,320 tokens (8,388,640 rows) go to the stream kernel,
for the one-layer and the multi-layer entries; the pack covers the whole
layer either way.  4,096 sampled tokens (the first and last, those around
2^22, and seeded random ones) are checked bit-exact against the oracle's pack
and dequant of the same K/V, which are per token: the oracle packs the
sample into its own compact slots.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, uniform_ints

pytestmark = pytest.mark.gpu

H, D, B = 2, 128, 16


def _sample(N: int) -> np.ndarray:
    fixed = np.array([0, 1, 15, 16, (1 << 22) - 2, (1 << 22) - 1, N - 2, N - 1])
    rnd = uniform_ints(9990, 4096 - fixed.size, 0, N - 1)
    idx = np.unique(np.concatenate([fixed, rnd])).astype(np.int64)
    idx = idx[(idx >= 0) & (idx < N)]  # (every index is a token of the layer)
    assert idx.size > 4000 and idx.max() < N
    return idx


@pytest.mark.parametrize("N", [(1 << 22) - 1, (1 << 22) + 16])
@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_dequant_at_row_kernel_limit(tq, oracle, cuda, scheme, N):
    print(f"[large] {scheme} N={N} H={H}: {N * H} rows", flush=True)
    prod = scheme == "turbo_prod"
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lay = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    g = torch.Generator(device=cuda)
    g.manual_seed(4242)
    k = torch.randn(N, H, D, generator=g, device=cuda, dtype=torch.float32).half()
    v = torch.randn(N, H, D, generator=g, device=cuda, dtype=torch.float32).half()
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    pages = (N + B - 1) // B
    pool = torch.zeros(pages * lay.page_size_bytes, dtype=torch.uint8, device=cuda)
    (tq.pack if prod else tq.mse_pack)(k, v, slots, pool, lay, cfg)
    ok = torch.empty(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.empty(N, H, D, dtype=torch.float16, device=cuda)
    (tq.dequant if prod else tq.mse_dequant)(pool, slots, ok, ov, lay, cfg)
    torch.cuda.synchronize()

    idx = _sample(N)
    ti = torch.from_numpy(idx).to(cuda)
    ks, vs = as_u16(k[ti].cpu()), as_u16(v[ti].cpu())
    n = idx.size
    compact = np.arange(n, dtype=np.int32)
    opack = oracle.prod_pack if prod else oracle.mse_pack
    odeq = oracle.prod_dequant if prod else oracle.mse_dequant
    want_pool = opack(ks, vs, compact, (n + B - 1) // B, B)
    wk, wv = odeq(want_pool, compact, H, D, B)
    gk, gv = as_u16(ok[ti].cpu()), as_u16(ov[ti].cpu())
    assert np.array_equal(gk, wk) and np.array_equal(gv, wv), "one-layer dequant"

    # the multi-layer entry over two layers (the same pool twice, separate outputs)
    del k, v
    ok2 = [torch.empty(N, H, D, dtype=torch.float16, device=cuda) for _ in range(2)]
    ov2 = [torch.empty(N, H, D, dtype=torch.float16, device=cuda) for _ in range(2)]
    tq.dequant_layers(scheme, [pool, pool], slots, ok2, ov2, lay, cfg, N)
    torch.cuda.synchronize()
    for layer in range(2):
        assert np.array_equal(as_u16(ok2[layer][ti].cpu()), wk), layer
        assert np.array_equal(as_u16(ov2[layer][ti].cpu()), wv), layer
