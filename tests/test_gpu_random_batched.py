"""Seeded random batched paged decode steps against the CPU oracle: 1-10
sequences of 1-2,500 tokens, 1-8 new tokens each, 1, 2, 4 or 8 kv heads
(8 GQA rows per kv head), blocks of 7, 16 or 32 tokens, both schemes.  Each
step appends the new tokens (one pack launch) and runs one paged-attention
launch; every row group is checked against the fp64 oracle over the
sequence's first L + j + 1 tokens (max rel err <= 1e-3), and the appended
cells against the oracle's pack of the same tokens into the same slots.

The cases come from the splitmix64 stream of the synthetic-input generator,
so they are the same on every machine; they exercise the device plan's units
(runs of up to four positions), the per-head work segments and the combine
over pieces at shapes the fixed tests do not reach.  Geometries whose pages
are not 16-byte aligned (turbo_prod pages are 134 bytes per token-head, so
block_size x kv heads not a multiple of 8) run on the generic split-K decode
and are checked the same way.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.batched import PagedBatch
from turborag_amd.synthetic import as_u16, uniform_ints

pytestmark = pytest.mark.gpu
NCASES = 24
ATT_TOL = 1e-3
_HS = (1, 2, 4, 8)
_BS = (7, 16, 32)


def _case(i: int):
    u = uniform_ints(9600 + i, 5, 0, 1 << 30)
    S = 1 + int(u[0] % 10)
    H = _HS[int(u[1] % len(_HS))]
    B = _BS[int(u[2] % len(_BS))]
    scheme = "turbo_prod" if u[3] % 2 == 0 else "turbo_mse"
    lens = [int(x) for x in uniform_ints(9700 + i, S, 1, 2500)]
    widths = [int(x) for x in uniform_ints(9800 + i, S, 1, 8)]
    return S, H, B, scheme, lens, widths


def _rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max())


@pytest.mark.parametrize("i", range(NCASES))
def test_random_batched_step(tq, oracle, cuda, i):
    S, H, B, scheme, lens, widths = _case(i)
    print(f"[random batched {i}] {scheme} H={H} B={B} lens={lens} widths={widths}", flush=True)
    b = PagedBatch(tq, scheme, lens, widths, kv_heads=H, q_heads=8 * H, block_size=B,
                   seed=9900 + i, device=cuda)
    b.append_new_tokens(seed=9950 + i)
    query, row_seq, row_len = b.decode_rows(seed=9970 + i)
    bt = b.block_tables()
    out = torch.zeros_like(query)
    b.attention(query, row_seq, row_len, bt, out)
    torch.cuda.synchronize()
    pool_np = b.pool.cpu().numpy()
    q_np = as_u16(query)
    got = out.cpu().float().numpy()
    f64 = oracle.prod_attention_f64 if scheme == "turbo_prod" else oracle.mse_attention_f64
    r, worst = 0, 0.0
    for s, (L, w) in enumerate(zip(lens, widths)):
        for j in range(w):
            ref = f64(q_np[r:r + 8].copy(), pool_np, b.slots_of(s, L + j + 1), B)
            worst = max(worst, _rel_err(got[r:r + 8], ref))
            r += 8
    print(f"    worst rel err {worst:.3e}", flush=True)
    assert worst < ATT_TOL
    # the appended cells: the oracle's pack of the step's new tokens into their slots
    k, v, slots = b._last_pack
    pack = oracle.prod_pack if scheme == "turbo_prod" else oracle.mse_pack
    want = pack(as_u16(k), as_u16(v), slots.cpu().numpy(), pool_np.size // b.layout.page_size_bytes,
                B, pool=pool_np.copy())
    assert np.array_equal(pool_np, want)
    b.close()
