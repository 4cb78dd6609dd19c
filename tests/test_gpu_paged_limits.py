"""The paged decode entry's int32 work-count limit: the plan counts each kv
head's work (every head has the same) as at most 4 * ceil(max_kv_len / 256)
+ 8 (a unit's setup) per row group in int32.  With max_kv_len = 2^23 (32,768
passes), 16,384 row groups reach 2^31 + 2^17 and are refused on the host
with the reason, leaving the output untouched; 16,383 row groups
(2^31 - 8) are accepted, with 8 kv heads, and sampled row groups equal the
slot-mapped entry over the same tokens.  Every input is valid for the rows' real kv length (10 tokens on
page 0), so a launch stays in bounds either way.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.batched import PagedBatch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("groups,accepted", [(16384, False), (16383, True)])
def test_paged_work_count_limit(tq, cuda, groups, accepted):
    print(f"[paged limit] row groups={groups}", flush=True)
    b = PagedBatch(tq, "turbo_prod", [64], [1], kv_heads=8, q_heads=64, block_size=16,
                   seed=530, device=cuda)
    H, D, L = 8, 128, 10
    rows = 8 * groups
    max_kv_len = 1 << 23
    gen = torch.Generator(device="cpu").manual_seed(groups)
    query = torch.randn(rows, H, D, generator=gen).half().to(cuda)
    row_seq = torch.zeros(rows, dtype=torch.int32, device=cuda)
    row_len = torch.full((rows,), L, dtype=torch.int32, device=cuda)
    tables = torch.zeros(1, max_kv_len // 16, dtype=torch.int32, device=cuda)  # every block: page 0
    out = torch.full((rows, H, D), 3.0, dtype=torch.float16, device=cuda)
    if not accepted:
        with pytest.raises(RuntimeError, match="too many rows"):
            tq.paged_attn_output("turbo_prod", query, b.pool, tables, row_seq, row_len, out,
                                 b.layout, b.cfg, max_kv_len)
        torch.cuda.synchronize()
        assert bool((out == 3.0).all())
        b.close()
        return
    tq.paged_attn_output("turbo_prod", query, b.pool, tables, row_seq, row_len, out, b.layout,
                         b.cfg, max_kv_len)
    slots = torch.arange(L, dtype=torch.int32, device=cuda)  # tokens 0 .. 9 of page 0
    for gi in (0, 1, groups // 2, groups - 1):
        r = slice(8 * gi, 8 * gi + 8)
        ref = torch.zeros(8, H, D, dtype=torch.float16, device=cuda)
        tq.fused_attn_output(query[r].contiguous(), b.pool, slots, ref, b.layout, b.cfg, 8, L)
        torch.cuda.synchronize()
        got, want = out[r].float().cpu().numpy(), ref.float().cpu().numpy()
        err = float(np.abs(got - want).max() / np.abs(want).max())
        assert err < 2e-3, gi
    b.close()
