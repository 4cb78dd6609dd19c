"""The turbo_prod debug pack (tq_launch_turbo_prod_pack_kv_debug: the
reference's pack launcher with its six optional debug buffers,
include/tq_turbo_prod.cuh:51-65) through the C ABI: its pages equal both the
oracle's pack and the production entry's, and its rotated, normalised and
code-index outputs equal the oracle's (tq_oracle.c, tqo_prod_pack_row_debug)
bit for bit."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import as_u16, kv_tokens_major, permuted_slots

pytestmark = pytest.mark.gpu


def _cfg(tq, H, D, B):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    return cfg, tq.make_layout_for(cfg)


@pytest.mark.parametrize("N,H,D,B,holes", [(1000, 2, 128, 16, False), (333, 3, 64, 7, True),
                                           (97, 1, 32, 16, True), (8192, 2, 128, 16, False)])
def test_debug_pack_against_oracle(tq, oracle, cuda, N, H, D, B, holes):
    print(f"[pack debug] N={N} H={H} D={D} B={B} holes={holes}", flush=True)
    k, v = kv_tokens_major(N, H, D, seed=4000 + N)
    slots = permuted_slots(N, B, seed=4001 + N).numpy().copy()
    if holes:
        slots[::5] = -1  # skipped tokens: no page write, debug values still written
    pages = (N + B - 1) // B
    cfg, lp = _cfg(tq, H, D, B)
    ku, vu = as_u16(k), as_u16(v)
    kd, vd, sd = k.to(cuda), v.to(cuda), torch.from_numpy(slots).to(cuda)
    pool = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    out = tq.pack_debug(kd, vd, sd, pool, lp, cfg)
    prod = torch.zeros_like(pool)
    tq.pack(kd, vd, sd, prod, lp, cfg)
    torch.cuda.synchronize()
    want_pool = oracle.prod_pack(ku, vu, slots, pages, B)
    assert np.array_equal(pool.cpu().numpy(), want_pool)
    assert np.array_equal(prod.cpu().numpy(), want_pool)
    want = oracle.prod_pack_debug(ku, vu)
    for name in ("k_rot", "v_rot", "kn", "vn"):
        got = out[name].cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want[name].view(np.uint32)), name
    for name in ("kidx", "vidx"):
        assert np.array_equal(out[name].cpu().numpy(), want[name]), name


def test_debug_pack_null_buffers_and_alignment(tq, oracle, cuda):
    N, H, D, B = 64, 2, 128, 16
    k, v = kv_tokens_major(N, H, D, seed=4100)
    cfg, lp = _cfg(tq, H, D, B)
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    kd, vd = k.to(cuda), v.to(cuda)
    pool = torch.zeros(N // B * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    u8 = ctypes.POINTER(ctypes.c_uint8)
    i32 = ctypes.POINTER(ctypes.c_int32)
    args = [ctypes.c_void_p(kd.data_ptr()), ctypes.c_void_p(vd.data_ptr()),
            ctypes.cast(slots.data_ptr(), i32), ctypes.cast(pool.data_ptr(), u8),
            ctypes.byref(lp), ctypes.byref(cfg), N, None]
    # every debug buffer NULL: a plain pack
    rc = tq.lib.tq_launch_turbo_prod_pack_kv_debug(*args, None, None, None, None, None, None)
    torch.cuda.synchronize()
    assert rc == 0, tq.lib.tq_last_error()
    assert np.array_equal(pool.cpu().numpy(),
                          oracle.prod_pack(as_u16(k), as_u16(v), slots.cpu().numpy(), N // B, B))
    # only kn, at an offset that is not 8-byte aligned: refused before any launch
    buf = torch.zeros(N * H * D + 1, dtype=torch.float32, device=cuda)
    rc = tq.lib.tq_launch_turbo_prod_pack_kv_debug(*args, None, None,
                                                   ctypes.c_void_p(buf.data_ptr() + 4), None,
                                                   None, None)
    assert rc == -2
    assert b"aligned" in tq.lib.tq_last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(buf).item() == 0
