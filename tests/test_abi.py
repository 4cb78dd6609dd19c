"""The C ABI of build/libturboquant.so on the CPU: every symbol declared in
include/turboquant.h is exported; struct layouts match the reference's ctypes
mirror; host-only entry points and argument-error paths (which return before
any HIP call) behave like src/tq_capi.cpp; allocator / block-table
bookkeeping follows src/tq_allocator.cpp and src/tq_block_table.cpp."""
from __future__ import annotations

import ctypes
import re
from ctypes import byref, c_int, c_int32, c_void_p
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _declared_symbols() -> list[str]:
    text = (ROOT / "include" / "turboquant.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(lib_path):
    lib = ctypes.CDLL(str(lib_path))
    names = _declared_symbols()
    assert len(names) >= 23
    for n in names:
        assert hasattr(lib, n), n


def test_wrapper_binds_every_declared_symbol(tq):
    from turborag_amd.turboquant_wrapper import SIGNATURES
    assert sorted(SIGNATURES) == _declared_symbols()


def test_struct_sizes_match_reference_ctypes(tq):
    from turborag_amd.turboquant_wrapper import (TQConfig, TQTurbomsePageLayout,
                                                 TQTurboProdPageLayout)
    assert ctypes.sizeof(TQConfig) == 32
    assert ctypes.sizeof(TQTurboProdPageLayout) == 64
    assert ctypes.sizeof(TQTurbomsePageLayout) == 56
    assert TQTurboProdPageLayout.k4_bytes_per_token_head.offset == 48


def test_default_config(tq):
    cfg = tq.default_config()
    assert [getattr(cfg, f) for f, _ in cfg._fields_] == [16, 8, 128, 4, 128, 256, 0, 0]


@pytest.mark.parametrize("H,D,B", [(2, 128, 16), (8, 128, 16), (2, 64, 16), (1, 2, 1),
                                   (4, 32, 32), (2, 128, 7)])
def test_layouts_match_oracle(tq, oracle, H, D, B):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    lp = tq.make_layout_for(cfg)
    op = oracle.prod_layout(B, H, D)
    assert (lp.page_size_bytes, lp.k4_codes_offset, lp.k_residual_scales_offset,
            lp.k_scales_offset, lp.v4_codes_offset, lp.v_scales_offset,
            lp.k4_bytes_per_token_head, lp.v4_bytes_per_token_head,
            lp.scale_bytes_per_token_head) == \
        (op.page_size, op.k4_off, op.kres_off, op.ks_off, op.v4_off, op.vs_off, op.k4_bytes,
         op.v4_bytes, op.scale_bytes)
    lm = tq.make_mse_layout_for(cfg)
    om = oracle.mse_layout(B, H, D, cfg.nbits, cfg.page_alignment)
    assert (lm.code_bytes_per_token_head, lm.norm_bytes_per_token_head, lm.k_codes_offset,
            lm.v_codes_offset, lm.k_norms_offset, lm.v_norms_offset, lm.page_size_bytes) == \
        (om.code_bytes, om.norm_bytes, om.k_codes_off, om.v_codes_off, om.k_norms_off,
         om.v_norms_off, om.page_size)


def test_summary_ratios(tq):
    s = tq.summary()  # default cfg: H=8, D=128
    assert s["turbo_prod_compression_ratio_vs_fp16"] == round(16 * 8 * 128 * 4 / (16 * 8 * 134), 2)


# ---- error paths (no GPU call is reached) -------------------------------------

def _cfg_layout(tq, H=2, D=128, B=16):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    return cfg, tq.make_layout_for(cfg), tq.make_mse_layout_for(cfg)


def test_null_pointers_return_minus_one(tq):
    L = tq.lib
    cfg, lp, lm = _cfg_layout(tq)
    fake = c_void_p(0x1000)  # never dereferenced: the NULL check comes first
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    u8 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_uint8))
    f32 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_float))
    nul = None
    assert L.tq_make_default_config(nul) == -1
    assert L.tq_make_turbo_prod_layout(nul, byref(lp)) == -1
    assert L.tq_make_turbo_mse_layout(byref(cfg), nul) == -1
    assert L.tq_launch_turbo_prod_pack_kv(fake, nul, i32, u8, byref(lp), byref(cfg), 1, None) == -1
    assert L.tq_launch_turbo_prod_dequant_kv(u8, i32, fake, fake, nul, byref(cfg), 1, None) == -1
    # (the debug pack's six debug pointers may be NULL; the pack's own may not)
    assert L.tq_launch_turbo_prod_pack_kv_debug(fake, fake, i32, nul, byref(lp), byref(cfg), 1,
                                                None, fake, fake, fake, fake, fake, fake) == -1
    assert L.tq_launch_turbo_prod_fused_attention_logits(fake, u8, i32, nul, byref(lp),
                                                         byref(cfg), 1, 1, None) == -1
    assert L.tq_launch_turbo_prod_fused_attention_output(fake, u8, i32, fake, byref(lp), nul,
                                                         1, 1, None) == -1
    assert L.tq_launch_turbo_mse_pack_kv(fake, fake, nul, u8, byref(lm), byref(cfg), 1, None) == -1
    assert L.tq_launch_turbo_mse_dequant_kv(nul, i32, fake, fake, byref(lm), byref(cfg), 1,
                                            None) == -1
    assert L.tq_launch_turbo_mse_fused_attention_output(fake, u8, i32, nul, byref(lm),
                                                        byref(cfg), 1, 1, None) == -1
    assert L.tq_launch_turbo_prod_dequant_kv_hnd(u8, nul, fake, fake, byref(lp), byref(cfg), 1,
                                                 None) == -1
    assert L.tq_launch_turbo_mse_dequant_kv_hnd(u8, i32, fake, fake, byref(lm), nul, 1,
                                                None) == -1
    arr = (c_void_p * 1)(fake)
    assert L.tq_load_turbo_prod_layers(nul, arr, 8, 1, i32, 1, arr, arr, byref(lp), byref(cfg),
                                       None, None) == -1
    assert L.tq_load_turbo_mse_layers(arr, arr, 8, 1, i32, 1, arr, nul, byref(lm), byref(cfg),
                                      None, None) == -1


def test_loader_argument_errors_before_any_hip_call(tq):
    """Zero layers is a no-op; negative counts and bad layouts are rc -2,
    all decided on the host."""
    L = tq.lib
    cfg, lp, lm = _cfg_layout(tq)
    fake = c_void_p(0x1000)
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    arr = (c_void_p * 1)(fake)
    assert L.tq_load_turbo_prod_layers(arr, arr, 8, 0, i32, 16, arr, arr, byref(lp), byref(cfg),
                                       None, None) == 0
    assert L.tq_load_turbo_prod_layers(arr, arr, 8, -1, i32, 16, arr, arr, byref(lp),
                                       byref(cfg), None, None) == -2
    assert b"num_layers" in L.tq_last_error()
    bad = type(lp)()
    ctypes.memmove(byref(bad), byref(lp), ctypes.sizeof(lp))
    bad.k4_bytes_per_token_head = 32
    assert L.tq_load_turbo_prod_layers(arr, arr, 8, 1, i32, 16, arr, arr, byref(bad),
                                       byref(cfg), None, None) == -2
    assert L.tq_load_turbo_mse_layers(arr, arr, 8, 0, i32, 16, arr, arr, byref(lm), byref(cfg),
                                      None, None) == 0


def test_head_dim_errors_return_minus_two(tq):
    L = tq.lib
    fake = c_void_p(0x1000)
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    u8 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_uint8))
    for D, msg in ((256, "head_dim > 128 is not supported"), (96, "power of two")):
        cfg, lp, lm = _cfg_layout(tq, D=D)
        rc = L.tq_launch_turbo_prod_pack_kv(fake, fake, i32, u8, byref(lp), byref(cfg), 4, None)
        assert rc == -2 and msg in tq._last_cuda_error()
        rc = L.tq_launch_turbo_mse_dequant_kv(u8, i32, fake, fake, byref(lm), byref(cfg), 4, None)
        assert rc == -2 and msg in tq._last_cuda_error()
    with pytest.raises(RuntimeError, match=r"turbo_prod pack_kv CUDA error: .*head_dim"):
        tq._kernel_raise(-2, "turbo_prod", "pack_kv")


def test_grid_quirks(tq):
    """Reference behaviour kept: turbo_prod with num_tokens == 0 is a launch
    error (grid dim 0); turbo_mse with 0 tokens is a no-op returning 0."""
    L = tq.lib
    fake = c_void_p(0x1000)
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    u8 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_uint8))
    cfg, lp, lm = _cfg_layout(tq)
    assert L.tq_launch_turbo_prod_pack_kv(fake, fake, i32, u8, byref(lp), byref(cfg), 0, None) == -2
    assert "invalid configuration argument" in tq._last_cuda_error()
    assert L.tq_launch_turbo_mse_pack_kv(fake, fake, i32, u8, byref(lm), byref(cfg), 0, None) == 0
    assert L.tq_launch_turbo_mse_pack_kv(fake, fake, i32, u8, byref(lm), byref(cfg), -1, None) == -2


def test_mismatched_layout_rejected(tq):
    L = tq.lib
    fake = c_void_p(0x1000)
    i32 = ctypes.cast(fake, ctypes.POINTER(c_int32))
    u8 = ctypes.cast(fake, ctypes.POINTER(ctypes.c_uint8))
    cfg, lp, lm = _cfg_layout(tq, D=128)
    cfg64, _, _ = _cfg_layout(tq, D=64)
    rc = L.tq_launch_turbo_prod_dequant_kv(u8, i32, fake, fake, byref(lp), byref(cfg64), 4, None)
    assert rc == -2 and "layout does not match" in tq._last_cuda_error()


def test_wrapper_rejects_host_tensors(tq):
    import torch
    cfg, lp, _ = _cfg_layout(tq)
    k = torch.zeros(4, 2, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU tensor"):
        tq.pack(k, k, torch.arange(4, dtype=torch.int32), torch.zeros(4288, dtype=torch.uint8),
                lp, cfg)


def test_missing_library_raises():
    from turborag_amd.turboquant_wrapper import TurboQuantWrapper
    with pytest.raises(FileNotFoundError):
        TurboQuantWrapper("/nonexistent/libturboquant.so")


# ---- allocator / block table ----------------------------------------------------

def test_allocator_lifo_semantics(tq):
    from turborag_amd.turboquant_wrapper import BlockTable, PageAllocator

    class FakePool:  # bookkeeping never touches device memory
        def data_ptr(self):
            return 0x10000

    a = PageAllocator(tq, 4288, 4, device_pool=FakePool())
    assert a.device_pool_ptr() == 0x10000                          # the caller's pool, as given
    assert [a.alloc_block() for _ in range(4)] == [0, 1, 2, 3]   # free list [N-1..0]
    assert a.alloc_block() == -1                                   # empty -> -1
    a.free_block(2)
    a.free_block(0)
    assert a.alloc_block() == 0 and a.alloc_block() == 2           # LIFO
    a.close()

    a = PageAllocator(tq, 4288, 3, device_pool=FakePool())
    t = BlockTable(a, block_size=16)
    assert t.build_slot_map(7, 20) == list(range(0, 16)) + [16, 17, 18, 19]
    assert t.blocks(7) == [0, 1] and t.num_tokens(7) == 20
    # appending continues in the partially filled page, then allocates page 2
    assert t.build_slot_map(7, 13) == [20 + i for i in range(12)] + [32]
    assert t.blocks(7) == [0, 1, 2]
    with pytest.raises(RuntimeError, match="out of blocks"):
        t.build_slot_map(9, 1)
    with pytest.raises(KeyError):
        t.blocks(12345)
    t.free_sequence(7)
    assert a.num_free() == 3
    # pages 0, 1, 2 were pushed back in that order: LIFO hands out 2, then 1
    assert t.build_slot_map(8, 17) == [2 * 16 + i for i in range(16)] + [1 * 16]
    t.close()
    a.close()


def test_block_table_failed_append_leaves_sequence_unchanged(tq):
    from turborag_amd.turboquant_wrapper import BlockTable, PageAllocator

    class FakePool:
        def data_ptr(self):
            return 0x10000

    a = PageAllocator(tq, 4608, 2, device_pool=FakePool())
    t = BlockTable(a, 16)
    t.build_slot_map(1, 16)
    with pytest.raises(RuntimeError, match="out of blocks"):
        t.build_slot_map(1, 40)          # needs 3 more pages, only 1 free
    assert t.num_tokens(1) == 16 and t.blocks(1) == [0] and a.num_free() == 1


CXX_LAUNCHERS = ["make_tq_turbo_prod_page_layout", "launch_tq_turbo_prod_pack_kv",
                 "launch_tq_turbo_prod_dequant_kv", "launch_tq_turbo_prod_fused_attention_logits",
                 "launch_tq_turbo_prod_fused_attention_output"]


def test_cxx_launchers_declared_and_exported(lib_path):
    """The reference's C-linkage C++ launchers (include/tq_turbo_prod.cuh:45-101)
    are declared in include/tq_turbo_prod_launch.h and exported unmangled."""
    text = (ROOT / "include" / "tq_turbo_prod_launch.h").read_text()
    lib = ctypes.CDLL(str(lib_path))
    for n in CXX_LAUNCHERS:
        assert re.search(rf"\b{n}\s*\(", text), n
        assert hasattr(lib, n), n


@pytest.mark.parametrize("H,D,B", [(2, 128, 16), (3, 64, 7), (1, 2, 1)])
def test_cxx_layout_factory_matches_c_entry(tq, lib_path, H, D, B):
    from turborag_amd.turboquant_wrapper import TQTurboProdPageLayout
    lib = ctypes.CDLL(str(lib_path))
    f = lib.make_tq_turbo_prod_page_layout
    f.argtypes = [ctypes.c_void_p]  # const TQConfig& (a pointer in the ABI)
    f.restype = TQTurboProdPageLayout  # returned by value
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    got = f(ctypes.addressof(cfg))
    want = tq.make_layout_for(cfg)
    assert bytes(got) == bytes(want)
