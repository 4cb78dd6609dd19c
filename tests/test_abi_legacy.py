"""Host-side behaviour of the entries for the reference's unexported kernels
(QJL-1b, legacy INT4, dense pages, GPU SDPA reference): layout factories
against the oracle (itself pinned by the reference's factories), and the
argument errors decided before any HIP call."""
from __future__ import annotations

import ctypes
from ctypes import byref, c_int32, c_void_p

import pytest

from turborag_amd.turboquant_wrapper import TQDensePageLayout, TQPageLayout, TQQJLPageLayout


def _cfg(tq, H=2, D=128, B=16, align=256, scale_fp32=False):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size, cfg.page_alignment = H, D, B, align
    cfg.group_size = D
    cfg.scale_type = 1 if scale_fp32 else 0
    return cfg


def test_struct_sizes():
    # the reference structs: 5 size_t + 3 int (padded), 11 size_t, 6 size_t
    assert ctypes.sizeof(TQQJLPageLayout) == 56
    assert ctypes.sizeof(TQPageLayout) == 88
    assert ctypes.sizeof(TQDensePageLayout) == 48


@pytest.mark.parametrize("B,H,D", [(16, 2, 128), (8, 8, 64), (1, 1, 2), (32, 4, 16)])
def test_layout_factories_match_oracle(tq, oracle, B, H, D):
    for align in (1, 64, 256):
        for f32 in (False, True):
            cfg = _cfg(tq, H, D, B, align, f32)
            q = tq.make_qjl_layout_for(cfg)
            o = oracle.qjl_layout(B, H, D)
            assert (q.page_size_bytes, q.k1_codes_offset, q.k_scales_offset, q.v4_codes_offset,
                    q.v_scales_offset, q.k1_bytes_per_token_head, q.v4_bytes_per_token_head,
                    q.scale_bytes_per_token_head) == (o.page_size, o.k1_off, o.ks_off, o.v4_off,
                                                      o.vs_off, o.k1_bytes, o.v4_bytes,
                                                      o.scale_bytes)
            i = tq.make_int4_layout_for(cfg)
            o = oracle.int4_layout(B, H, D, align=align, scale_fp32=f32)
            assert (i.code_bytes_per_token_head, i.scale_bytes_per_token_head, i.k_codes_offset,
                    i.v_codes_offset, i.k_scales_offset, i.v_scales_offset, i.k_codes_bytes,
                    i.v_codes_bytes, i.k_scales_bytes, i.v_scales_bytes, i.page_size_bytes) == \
                (o.code_bytes, o.scale_bytes, o.k_codes_off, o.v_codes_off, o.k_scales_off,
                 o.v_scales_off, o.k_codes_bytes, o.v_codes_bytes, o.k_scales_bytes,
                 o.v_scales_bytes, o.page_size)
            d = tq.make_dense_layout_for(cfg)
            o = oracle.dense_layout(B, H, D, align=align)
            assert (d.elem_bytes, d.k_offset, d.v_offset, d.k_bytes, d.v_bytes,
                    d.page_size_bytes) == (o.elem_bytes, o.k_off, o.v_off, o.k_bytes, o.v_bytes,
                                           o.page_size)


def test_int4_layout_rejects_like_reference(tq):
    cfg = _cfg(tq)
    cfg.nbits = 8
    with pytest.raises(RuntimeError, match="Only int4"):
        tq.make_int4_layout_for(cfg)
    cfg = _cfg(tq)
    cfg.group_size = 64
    with pytest.raises(RuntimeError, match="group_size == head_dim"):
        tq.make_int4_layout_for(cfg)


def test_null_zero_negative_and_bad_layout(tq):
    L = tq.lib
    cfg = _cfg(tq)
    lq, li, ld = (tq.make_qjl_layout_for(cfg), tq.make_int4_layout_for(cfg),
                  tq.make_dense_layout_for(cfg))
    fake = c_void_p(0x1000)  # never dereferenced
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    u8 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_uint8))
    f32 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_float))
    nul = None
    # NULL arguments: -1
    assert L.tq_make_qjl_layout(nul, byref(lq)) == -1
    assert L.tq_make_int4_layout(byref(cfg), nul) == -1
    assert L.tq_make_dense_layout(nul, nul) == -1
    assert L.tq_launch_qjl_pack_kv(fake, nul, i32, u8, byref(lq), byref(cfg), 1, None) == -1
    assert L.tq_launch_qjl_dequant_kv(u8, i32, fake, nul, byref(lq), byref(cfg), 1, None) == -1
    assert L.tq_launch_qjl_fused_attention_output(fake, u8, nul, fake, byref(lq), byref(cfg), 1,
                                                  1, None) == -1
    assert L.tq_launch_int4_pack_kv(fake, fake, i32, u8, nul, byref(cfg), 1, None) == -1
    assert L.tq_launch_int4_dequant_kv(nul, i32, fake, fake, byref(li), byref(cfg), 1,
                                       None) == -1
    assert L.tq_launch_dense_store_kv(fake, fake, i32, nul, byref(ld), byref(cfg), 1, None) == -1
    assert L.tq_launch_dense_load_kv(u8, i32, fake, fake, byref(ld), nul, 1, None) == -1
    assert L.tq_launch_attention_ref(fake, fake, fake, fake, nul, byref(cfg), 1, 1, None) == -1
    # zero tokens / queries: nothing to do
    assert L.tq_launch_qjl_pack_kv(fake, fake, i32, u8, byref(lq), byref(cfg), 0, None) == 0
    assert L.tq_launch_int4_dequant_kv(u8, i32, fake, fake, byref(li), byref(cfg), 0, None) == 0
    assert L.tq_launch_dense_store_kv(fake, fake, i32, u8, byref(ld), byref(cfg), 0, None) == 0
    assert L.tq_launch_attention_ref(fake, fake, fake, fake, f32, byref(cfg), 0, 5, None) == 0
    # negative counts: -2
    assert L.tq_launch_qjl_dequant_kv(u8, i32, fake, fake, byref(lq), byref(cfg), -1, None) == -2
    assert b"negative" in L.tq_last_error()
    assert L.tq_launch_attention_ref(fake, fake, fake, fake, f32, byref(cfg), 1, -1, None) == -2
    # a layout built for another head_dim: -2
    other = tq.make_qjl_layout_for(_cfg(tq, D=64))
    assert L.tq_launch_qjl_pack_kv(fake, fake, i32, u8, byref(other), byref(cfg), 1, None) == -2
    assert b"layout" in L.tq_last_error()
    cfg64 = _cfg(tq, D=64)
    assert L.tq_launch_int4_pack_kv(fake, fake, i32, u8, byref(li), byref(cfg64), 1, None) == -2
    # head_dim outside [2, 128] or not a power of two: -2, the reference's message
    bad = _cfg(tq, D=256)
    assert L.tq_launch_attention_ref(fake, fake, fake, fake, f32, byref(bad), 1, 1, None) == -2
    assert b"head_dim > 128" in L.tq_last_error()
    bad = _cfg(tq, D=96)
    assert L.tq_launch_dense_load_kv(u8, i32, fake, fake, byref(tq.make_dense_layout_for(bad)),
                                     byref(bad), 1, None) == -2
    # misaligned fp16 buffers: -2
    odd = c_void_p(0x1002)
    assert L.tq_launch_qjl_pack_kv(odd, fake, i32, u8, byref(lq), byref(cfg), 1, None) == -2
    assert b"aligned" in L.tq_last_error()
