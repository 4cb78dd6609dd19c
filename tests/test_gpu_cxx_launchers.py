"""The reference's C-linkage C++ launchers (include/tq_turbo_prod.cuh:45-101;
this build's include/tq_turbo_prod_launch.h) on the GPU: each gives exactly
the results of the C entry it wraps (same kernels), and the pack's debug
buffers equal the debug entry's."""
from __future__ import annotations

import ctypes
from ctypes import c_int, c_void_p

import numpy as np
import pytest
import torch

from turborag_amd.synthetic import kv_tokens_major, permuted_slots, query

pytestmark = pytest.mark.gpu

P = c_void_p  # every pointer, reference (the config and layout) and stream


def _bind(lib):
    f = {}
    f["pack"] = lib.launch_tq_turbo_prod_pack_kv
    f["pack"].argtypes = [P, P, P, P, P, P, c_int, P, P, P, P, P, P, P]
    f["dequant"] = lib.launch_tq_turbo_prod_dequant_kv
    f["dequant"].argtypes = [P, P, P, P, P, P, c_int, P]
    f["logits"] = lib.launch_tq_turbo_prod_fused_attention_logits
    f["logits"].argtypes = [P, P, P, P, P, P, c_int, c_int, P]
    f["output"] = lib.launch_tq_turbo_prod_fused_attention_output
    f["output"].argtypes = [P, P, P, P, P, P, c_int, c_int, P]
    for g in f.values():
        g.restype = None
    return f


def test_cxx_launchers_equal_c_entries(tq, cuda):
    N, H, D, B, Q = 4096, 2, 128, 16, 8
    print(f"[cxx launchers] N={N} H={H}", flush=True)
    lib = ctypes.CDLL(str(tq.lib_path))
    f = _bind(lib)
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lp = tq.make_layout_for(cfg)
    k, v = kv_tokens_major(N, H, D, seed=7100)
    kd, vd = k.to(cuda), v.to(cuda)
    sd = permuted_slots(N, B, seed=7101).to(cuda)
    pages = N // B
    a = lambda t: c_void_p(t.data_ptr())  # noqa: E731
    cp, lpp = c_void_p(ctypes.addressof(cfg)), c_void_p(ctypes.addressof(lp))
    # pack, plain and with every debug buffer
    pool_c = torch.zeros(pages * lp.page_size_bytes, dtype=torch.uint8, device=cuda)
    pool_x = torch.zeros_like(pool_c)
    pool_d = torch.zeros_like(pool_c)
    tq.pack(kd, vd, sd, pool_c, lp, cfg)
    f["pack"](a(kd), a(vd), a(sd), a(pool_x), lpp, cp, N, None, None, None, None, None, None, None)
    dbg = {n: torch.zeros(N * H * D, dtype=dt, device=cuda)
           for n, dt in (("k_rot", torch.float32), ("v_rot", torch.float32), ("kn", torch.float32),
                         ("vn", torch.float32), ("kidx", torch.int32), ("vidx", torch.int32))}
    f["pack"](a(kd), a(vd), a(sd), a(pool_d), lpp, cp, N, None,
              *[a(dbg[n]) for n in ("k_rot", "v_rot", "kn", "vn", "kidx", "vidx")])
    want_dbg = tq.pack_debug(kd, vd, sd, torch.zeros_like(pool_c), lp, cfg)
    torch.cuda.synchronize()
    assert torch.equal(pool_x, pool_c) and torch.equal(pool_d, pool_c)
    for n in dbg:
        assert torch.equal(dbg[n].view(-1), want_dbg[n].reshape(-1)), n
    # dequant
    ok_c, ov_c = torch.empty_like(kd), torch.empty_like(vd)
    ok_x, ov_x = torch.empty_like(kd), torch.empty_like(vd)
    tq.dequant(pool_c, sd, ok_c, ov_c, lp, cfg)
    f["dequant"](a(pool_c), a(sd), a(ok_x), a(ov_x), lpp, cp, N, None)
    # logits and attention output (GQA 16/2 rows)
    from turborag_amd.synthetic import gqa_rows
    qa = gqa_rows(query(16, D, seed=7102), H).to(cuda)
    lg_c = torch.empty(Q * H * N, dtype=torch.float32, device=cuda)
    lg_x = torch.empty_like(lg_c)
    tq.fused_attn_logits(qa, pool_c, sd, lg_c, lp, cfg, Q, N)
    f["logits"](a(qa), a(pool_c), a(sd), a(lg_x), lpp, cp, Q, N, None)
    out_c = torch.empty(Q, H, D, dtype=torch.float16, device=cuda)
    out_x = torch.empty_like(out_c)
    tq.fused_attn_output(qa, pool_c, sd, out_c, lp, cfg, Q, N)
    f["output"](a(qa), a(pool_c), a(sd), a(out_x), lpp, cp, Q, N, None)
    torch.cuda.synchronize()
    assert torch.equal(ok_x, ok_c) and torch.equal(ov_x, ov_c)
    assert np.array_equal(lg_x.cpu().numpy().view(np.uint32), lg_c.cpu().numpy().view(np.uint32))
    assert torch.equal(out_x, out_c)
