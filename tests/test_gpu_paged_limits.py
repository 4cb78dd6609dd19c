"""The paged decode entry's int32 work-count limit: the plan counts work as
H * 4 * ceil(max_kv_len / 256) per row group in int32, so 4,096 row groups of
8 kv heads with max_kv_len = 2^23 (4,096 * 8 * 4 * 32,768 = 2^32) are refused
on the host with the reason, and the output is left untouched.  Every input
is valid for the rows' real kv length (10 tokens on page 0), so a launch would
stay in bounds even if the check were missing.
"""
from __future__ import annotations

import pytest
import torch

from turborag_amd.batched import PagedBatch

pytestmark = pytest.mark.gpu


def test_paged_work_count_limit_refused(tq, cuda):
    b = PagedBatch(tq, "turbo_prod", [64], [1], kv_heads=8, q_heads=64, block_size=16,
                   seed=530, device=cuda)
    H, D = 8, 128
    rows = 8 * 4096
    max_kv_len = 1 << 23
    query = torch.randn(rows, H, D, device=cuda).half()
    row_seq = torch.zeros(rows, dtype=torch.int32, device=cuda)
    row_len = torch.full((rows,), 10, dtype=torch.int32, device=cuda)
    tables = torch.zeros(1, max_kv_len // 16, dtype=torch.int32, device=cuda)  # every block: page 0
    out = torch.full((rows, H, D), 3.0, dtype=torch.float16, device=cuda)
    with pytest.raises(RuntimeError, match="too many rows"):
        tq.paged_attn_output("turbo_prod", query, b.pool, tables, row_seq, row_len, out,
                             b.layout, b.cfg, max_kv_len)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all())
    b.close()
