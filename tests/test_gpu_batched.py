"""Batched paged decode + append-quantize (one pack launch for every
sequence's new tokens, one paged-attention launch for all rows) against the
CPU oracle run per sequence and position with the per-token slot list the
reference would pass (fp64 attention; max rel err <= 1e-3)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from turborag_amd.batched import PagedBatch
from turborag_amd.synthetic import as_u16

pytestmark = pytest.mark.gpu
ATT_TOL = 1e-3


def _rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max())


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_batched_paged_decode_with_append(tq, oracle, cuda, scheme):
    lens, widths = [1500, 37, 2900, 700, 64], [3, 1, 4, 2, 1]
    print(f"[batched {scheme}] lens={lens} widths={widths}", flush=True)
    b = PagedBatch(tq, scheme, lens, widths, seed=510, device=cuda)
    b.append_new_tokens(seed=900)
    query, row_seq, row_len = b.decode_rows(seed=901)
    bt = b.block_tables()
    out = torch.zeros_like(query)
    b.attention(query, row_seq, row_len, bt, out)
    torch.cuda.synchronize()
    pool_np = b.pool.cpu().numpy()
    q_np = as_u16(query)
    got = out.cpu().float().numpy()
    f64 = oracle.prod_attention_f64 if scheme == "turbo_prod" else oracle.mse_attention_f64
    r = 0
    worst = 0.0
    for s, (L, w) in enumerate(zip(lens, widths)):
        for j in range(w):
            rows = slice(r, r + 8)
            ref = f64(q_np[rows].copy(), pool_np, b.slots_of(s, L + j + 1), 16)
            worst = max(worst, _rel_err(got[rows], ref))
            r += 8
    print(f"    worst rel err {worst:.3e}", flush=True)
    assert worst < ATT_TOL
    b.close()


def test_paged_rows_zero_length_and_padding(tq, oracle, cuda):
    """Rows with kv length 0 (padding inside an aligned group) give 0; the
    other rows of the group are unaffected."""
    b = PagedBatch(tq, "turbo_prod", [400], [1], seed=520, device=cuda)
    b.append_new_tokens(seed=904)
    query, row_seq, row_len = b.decode_rows(seed=902)
    row_len[3] = 0
    row_len[5] = 17
    out = torch.full_like(query, 5.0)
    b.attention(query, row_seq, row_len, b.block_tables(), out)
    torch.cuda.synchronize()
    got = out.cpu().float().numpy()
    assert np.all(got[3] == 0.0)
    pool_np = b.pool.cpu().numpy()
    q_np = as_u16(query)
    for r, n in ((0, 401), (5, 17)):
        ref = oracle.prod_attention_f64(q_np[r:r + 1].copy(), pool_np, b.slots_of(0, n), 16)
        assert _rel_err(got[r:r + 1], ref) < ATT_TOL
    b.close()


def test_paged_matches_slot_map_attention(tq, cuda):
    """One sequence, one position: the paged launch equals the reference-ABI
    fused_attention_output over the same tokens' slot map."""
    b = PagedBatch(tq, "turbo_prod", [5000], [1], seed=530, device=cuda)
    b.append_new_tokens(seed=905)
    query, row_seq, row_len = b.decode_rows(seed=903)
    out = torch.zeros_like(query)
    b.attention(query, row_seq, row_len, b.block_tables(), out)
    ref = torch.zeros_like(query)
    slots = torch.from_numpy(b.slots_of(0, 5001)).to(cuda)
    tq.fused_attn_output(query, b.pool, slots, ref, b.layout, b.cfg, 8, 5001)
    torch.cuda.synchronize()
    err = (out.float() - ref.float()).abs().max() / ref.float().abs().max()
    assert err.item() < 2e-3
    b.close()


def test_paged_many_sequences_against_slot_map_attention(tq, cuda):
    """Over a hundred row groups (the pairing of groups runs over several
    64-group chunks, with runs of odd and even length): every row group equals
    the reference-ABI fused_attention_output over its sequence's slot map."""
    rng = np.random.default_rng(540)
    lens = rng.integers(20, 700, size=41)
    widths = rng.integers(1, 6, size=41)
    print(f"[batched many] groups={int(widths.sum())}", flush=True)
    b = PagedBatch(tq, "turbo_prod", lens, widths, seed=541, device=cuda)
    b.append_new_tokens(seed=906)
    query, row_seq, row_len = b.decode_rows(seed=907)
    out = torch.zeros_like(query)
    b.attention(query, row_seq, row_len, b.block_tables(), out)
    r = 0
    worst = 0.0
    for s, (L, w) in enumerate(zip(lens, widths)):
        for j in range(w):
            n = int(L) + j + 1
            slots = torch.from_numpy(b.slots_of(s, n)).to(cuda)
            ref = torch.zeros_like(query[r:r + 8])
            tq.fused_attn_output(query[r:r + 8].contiguous(), b.pool, slots, ref, b.layout, b.cfg,
                                 8, n)
            torch.cuda.synchronize()
            err = ((out[r:r + 8].float() - ref.float()).abs().max() / ref.float().abs().max()).item()
            worst = max(worst, err)
            r += 8
    print(f"    worst rel diff {worst:.3e}", flush=True)
    assert worst < 2e-3
    b.close()


def test_paged_over_a_thousand_row_groups(tq, cuda):
    """More than 1024 row groups: the plan is built 1024 groups at a time, so
    runs of a sequence's positions and units of four positions straddle the
    window ends.  Every row group equals the reference-ABI
    fused_attention_output over its sequence's slot map."""
    rng = np.random.default_rng(550)
    lens = rng.integers(16, 300, size=300)
    widths = rng.integers(1, 9, size=300)
    groups = int(widths.sum())
    print(f"[batched >1024 groups] groups={groups}", flush=True)
    assert groups > 1100
    b = PagedBatch(tq, "turbo_prod", lens, widths, seed=551, device=cuda)
    b.append_new_tokens(seed=908)
    query, row_seq, row_len = b.decode_rows(seed=909)
    out = torch.zeros_like(query)
    b.attention(query, row_seq, row_len, b.block_tables(), out)
    ref = torch.zeros_like(query)
    r = 0
    for s, (L, w) in enumerate(zip(lens, widths)):
        for j in range(w):
            n = int(L) + j + 1
            slots = torch.from_numpy(b.slots_of(s, n)).to(cuda)
            tq.fused_attn_output(query[r:r + 8].contiguous(), b.pool, slots, ref[r:r + 8], b.layout,
                                 b.cfg, 8, n)
            r += 8
    torch.cuda.synchronize()
    o = out.float().reshape(-1, 8 * out.shape[1] * out.shape[2])
    e = ref.float().reshape(-1, 8 * out.shape[1] * out.shape[2])
    err = ((o - e).abs().amax(dim=1) / e.abs().amax(dim=1)).max().item()
    print(f"    worst rel diff {err:.3e}", flush=True)
    assert err < 2e-3
    b.close()


@pytest.mark.parametrize("scheme,H,D,B", [
    ("turbo_prod", 2, 128, 7),  # 1,876-byte pages: not 16-byte aligned
    ("turbo_prod", 1, 128, 7),  # 938-byte pages
    ("turbo_prod", 2, 64, 16),
    ("turbo_mse", 2, 64, 16),
    ("turbo_mse", 4, 32, 5),
    # aligned pages, D = 128: the matrix-core kernel
    ("turbo_prod", 2, 128, 16),
    ("turbo_mse", 2, 128, 16),
    ("turbo_prod", 8, 128, 32),
])
def test_paged_geometries(tq, oracle, cuda, scheme, H, D, B):
    """Geometries the matrix-core kernel does not take (unaligned pages, head
    dims other than 128) run on the generic split-K decode through the block
    table, the others on the matrix-core kernel: every row against the fp64
    oracle over its sequence's first row_kv_len tokens; a row of kv length 0
    gives 0 and a row whose length passes max_kv_len attends max_kv_len tokens,
    those past its sequence's pages unmapped (masked)."""
    lens, widths = [900, 33, 1500], [2, 1, 3]
    print(f"[paged geometry {scheme}] H={H} D={D} B={B}", flush=True)
    b = PagedBatch(tq, scheme, lens, widths, kv_heads=H, q_heads=8 * H, head_dim=D,
                   block_size=B, seed=560, device=cuda)
    b.append_new_tokens(seed=561)
    query, row_seq, row_len = b.decode_rows(seed=562)
    max_kv = max(L + w for L, w in zip(lens, widths))
    row_len[9] = 0
    # a row of sequence 1 (34 tokens) given a length past max_kv_len: it attends
    # max_kv_len positions, those past its pages unmapped (-1 in the block table;
    # the unwritten cells of its last page read as stored: zero bytes)
    row_len[17] = max_kv + 5
    out = torch.full_like(query, 7.0)
    b.attention(query, row_seq, row_len, b.block_tables(), out)
    torch.cuda.synchronize()
    got = out.cpu().float().numpy()
    pool_np = b.pool.cpu().numpy()
    q_np = as_u16(query)
    f64 = oracle.prod_attention_f64 if scheme == "turbo_prod" else oracle.mse_attention_f64
    seqs, lens_r = row_seq.cpu().numpy(), row_len.cpu().numpy()
    assert np.all(got[9] == 0.0)
    worst, worst_row = 0.0, -1
    for r in range(query.shape[0]):
        if r == 9:
            continue
        s = int(seqs[r])
        n = min(int(lens_r[r]), max_kv)
        blocks = np.asarray(b.table.blocks(s), dtype=np.int64)
        t = np.arange(n)
        mapped = t // B < blocks.size
        slots = np.where(mapped, blocks[np.minimum(t // B, blocks.size - 1)] * B + t % B,
                         -1).astype(np.int32)
        ref = f64(q_np[r:r + 1].copy(), pool_np, slots, B)
        e = _rel_err(got[r:r + 1], ref)
        if e > worst:
            worst, worst_row = e, r
    print(f"    worst rel err {worst:.3e} (row {worst_row})", flush=True)
    assert worst < ATT_TOL
    b.close()
