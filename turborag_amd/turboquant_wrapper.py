"""TurboQuant Python wrapper over the gfx950 libturboquant.so.

Same class, method names, argument meaning and error behaviour as the
reference's ctypes wrapper (tq_backend/turboquant_wrapper.py:72-445), so the
reference's store code runs unchanged against this library; that file keeps
working as-is too, since the C ABI is identical.  Additions over the
reference: device/shape checks before each launch (a host pointer or a short
buffer would otherwise fault the GPU), and bindings for the page allocator and
block table.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int, c_int32, c_size_t, c_uint8, c_void_p
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent.parent
DEFAULT_LIB_PATH = ROOT / "build" / "libturboquant.so"


# --------------------------------------------------------------------------- #
# C-compatible structs (include/turboquant.h; reference :23-64)                #
# --------------------------------------------------------------------------- #

class TQConfig(ctypes.Structure):
    _fields_ = [
        ("block_size", c_int),
        ("num_kv_heads", c_int),
        ("head_dim", c_int),
        ("nbits", c_int),
        ("group_size", c_int),
        ("page_alignment", c_int),
        ("scale_type", c_int),
        ("quant_mode", c_int),
    ]


class TQTurboProdPageLayout(ctypes.Structure):
    """K interleaved nibble: bits[2:0] = 3-bit code, bit[3] = residual sign."""
    _fields_ = [
        ("page_size_bytes", c_size_t),
        ("k4_codes_offset", c_size_t),
        ("k_residual_scales_offset", c_size_t),
        ("k_scales_offset", c_size_t),
        ("v4_codes_offset", c_size_t),
        ("v_scales_offset", c_size_t),
        ("k4_bytes_per_token_head", c_int),
        ("v4_bytes_per_token_head", c_int),
        ("scale_bytes_per_token_head", c_int),
    ]


class TQTurbomsePageLayout(ctypes.Structure):
    _fields_ = [
        ("code_bytes_per_token_head", c_size_t),
        ("norm_bytes_per_token_head", c_size_t),
        ("k_codes_offset", c_size_t),
        ("v_codes_offset", c_size_t),
        ("k_norms_offset", c_size_t),
        ("v_norms_offset", c_size_t),
        ("page_size_bytes", c_size_t),
    ]


class TQQJLPageLayout(ctypes.Structure):
    """include/tq_qjl.cuh:21-33."""

    _fields_ = [
        ("page_size_bytes", c_size_t),
        ("k1_codes_offset", c_size_t),
        ("k_scales_offset", c_size_t),
        ("v4_codes_offset", c_size_t),
        ("v_scales_offset", c_size_t),
        ("k1_bytes_per_token_head", c_int),
        ("v4_bytes_per_token_head", c_int),
        ("scale_bytes_per_token_head", c_int),
    ]


class TQPageLayout(ctypes.Structure):
    """include/tq_layout.h:11-23 (the legacy INT4 page)."""

    _fields_ = [(n, c_size_t) for n in (
        "code_bytes_per_token_head", "scale_bytes_per_token_head", "k_codes_offset",
        "v_codes_offset", "k_scales_offset", "v_scales_offset", "k_codes_bytes", "v_codes_bytes",
        "k_scales_bytes", "v_scales_bytes", "page_size_bytes")]


class TQDensePageLayout(ctypes.Structure):
    """include/tq_dense_layout.h:5-12."""

    _fields_ = [(n, c_size_t) for n in (
        "elem_bytes", "k_offset", "v_offset", "k_bytes", "v_bytes", "page_size_bytes")]


class TQStoreFormat(ctypes.Structure):
    """Format record of the on-disk store (.bin footer, .meta keys)."""

    _fields_ = [
        ("version", c_int32),
        ("scheme", c_int32),  # 1 turbo_prod, 2 turbo_mse
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("block_size", c_int32),
        ("page_size_bytes", c_int32),
        ("num_pages", ctypes.c_int64),
        ("num_tokens", ctypes.c_int64),
    ]


# Every exported symbol and its ctypes signature (argtypes, restype).
_P = POINTER
_I64 = ctypes.c_int64
SIGNATURES: dict[str, tuple[list, object]] = {
    "tq_last_error": ([], ctypes.c_char_p),
    "tq_workspace_release": ([], c_int),
    "tq_make_default_config": ([_P(TQConfig)], c_int),
    "tq_make_turbo_prod_layout": ([_P(TQConfig), _P(TQTurboProdPageLayout)], c_int),
    "tq_make_turbo_mse_layout": ([_P(TQConfig), _P(TQTurbomsePageLayout)], c_int),
    "tq_launch_turbo_prod_pack_kv": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8),
                                      _P(TQTurboProdPageLayout), _P(TQConfig), c_int,
                                      c_void_p], c_int),
    "tq_launch_turbo_prod_pack_kv_debug": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8),
                                            _P(TQTurboProdPageLayout), _P(TQConfig), c_int,
                                            c_void_p] + [c_void_p] * 6, c_int),
    "tq_launch_turbo_prod_dequant_kv": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                         _P(TQTurboProdPageLayout), _P(TQConfig), c_int,
                                         c_void_p], c_int),
    "tq_launch_turbo_prod_fused_attention_logits": ([c_void_p, _P(c_uint8), _P(c_int32),
                                                     _P(c_float), _P(TQTurboProdPageLayout),
                                                     _P(TQConfig), c_int, c_int, c_void_p],
                                                    c_int),
    "tq_launch_turbo_prod_fused_attention_output": ([c_void_p, _P(c_uint8), _P(c_int32),
                                                     c_void_p, _P(TQTurboProdPageLayout),
                                                     _P(TQConfig), c_int, c_int, c_void_p],
                                                    c_int),
    "tq_launch_turbo_prod_fused_attention_output_noalloc": ([c_void_p, _P(c_uint8), _P(c_int32),
                                                             c_void_p, _P(TQTurboProdPageLayout),
                                                             _P(TQConfig), c_int, c_int,
                                                             c_void_p], c_int),
    "tq_launch_turbo_mse_pack_kv": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8),
                                     _P(TQTurbomsePageLayout), _P(TQConfig), c_int, c_void_p],
                                    c_int),
    "tq_launch_turbo_mse_dequant_kv": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                        _P(TQTurbomsePageLayout), _P(TQConfig), c_int,
                                        c_void_p], c_int),
    "tq_launch_turbo_mse_fused_attention_output": ([c_void_p, _P(c_uint8), _P(c_int32),
                                                    c_void_p, _P(TQTurbomsePageLayout),
                                                    _P(TQConfig), c_int, c_int, c_void_p],
                                                   c_int),
    # cache-layout dequant and layer loading (superset of the reference ABI)
    "tq_launch_turbo_prod_dequant_kv_hnd": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                             _P(TQTurboProdPageLayout), _P(TQConfig), c_int,
                                             c_void_p], c_int),
    "tq_launch_turbo_mse_dequant_kv_hnd": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                            _P(TQTurbomsePageLayout), _P(TQConfig), c_int,
                                            c_void_p], c_int),
    "tq_launch_turbo_prod_pack_kv_layers": ([_P(c_void_p), _P(c_void_p), _P(c_int32),
                                             _P(c_void_p), c_int, _P(TQTurboProdPageLayout),
                                             _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_turbo_mse_pack_kv_layers": ([_P(c_void_p), _P(c_void_p), _P(c_int32),
                                            _P(c_void_p), c_int, _P(TQTurbomsePageLayout),
                                            _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_turbo_prod_dequant_kv_layers": ([_P(c_void_p), _P(c_int32), _P(c_void_p),
                                                _P(c_void_p), c_int, _P(TQTurboProdPageLayout),
                                                _P(TQConfig), c_int, c_int, c_void_p], c_int),
    "tq_launch_turbo_mse_dequant_kv_layers": ([_P(c_void_p), _P(c_int32), _P(c_void_p),
                                               _P(c_void_p), c_int, _P(TQTurbomsePageLayout),
                                               _P(TQConfig), c_int, c_int, c_void_p], c_int),
    "tq_load_turbo_prod_layers": ([_P(c_void_p), _P(c_void_p), c_size_t, c_int, _P(c_int32),
                                   c_int, _P(c_void_p), _P(c_void_p), _P(TQTurboProdPageLayout),
                                   _P(TQConfig), c_void_p, c_void_p], c_int),
    "tq_load_turbo_mse_layers": ([_P(c_void_p), _P(c_void_p), c_size_t, c_int, _P(c_int32),
                                  c_int, _P(c_void_p), _P(c_void_p), _P(TQTurbomsePageLayout),
                                  _P(TQConfig), c_void_p, c_void_p], c_int),
    # batched decode over paged sequences (superset of the reference ABI)
    "tq_launch_turbo_prod_paged_attention": ([c_void_p, _P(c_uint8), _P(c_int32), c_int,
                                              _P(c_int32), _P(c_int32), c_void_p,
                                              _P(TQTurboProdPageLayout), _P(TQConfig), c_int,
                                              c_int, c_void_p], c_int),
    "tq_launch_turbo_mse_paged_attention": ([c_void_p, _P(c_uint8), _P(c_int32), c_int,
                                             _P(c_int32), _P(c_int32), c_void_p,
                                             _P(TQTurbomsePageLayout), _P(TQConfig), c_int,
                                             c_int, c_void_p], c_int),
    # page allocator / block table
    "tq_allocator_create": ([c_size_t, c_int, c_void_p, _P(c_void_p)], c_int),
    "tq_allocator_destroy": ([c_void_p], c_int),
    "tq_allocator_alloc_block": ([c_void_p, _P(c_int32)], c_int),
    "tq_allocator_free_block": ([c_void_p, c_int32], c_int),
    "tq_allocator_num_free": ([c_void_p, _P(c_int)], c_int),
    "tq_allocator_device_pool": ([c_void_p], c_void_p),
    "tq_block_table_create": ([c_void_p, c_int, _P(c_void_p)], c_int),
    "tq_block_table_destroy": ([c_void_p], c_int),
    "tq_block_table_build_slot_map": ([c_void_p, c_int32, c_int, _P(c_int32)], c_int),
    "tq_block_table_num_tokens": ([c_void_p, c_int32, _P(c_int)], c_int),
    "tq_block_table_blocks": ([c_void_p, c_int32, _P(c_int32), c_int, _P(c_int)], c_int),
    "tq_block_table_free_sequence": ([c_void_p, c_int32], c_int),
    # the reference's unexported kernels: QJL-1b, legacy INT4, dense, SDPA reference
    "tq_make_qjl_layout": ([_P(TQConfig), _P(TQQJLPageLayout)], c_int),
    "tq_launch_qjl_pack_kv": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8), _P(TQQJLPageLayout),
                               _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_qjl_dequant_kv": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                  _P(TQQJLPageLayout), _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_qjl_fused_attention_output": ([c_void_p, _P(c_uint8), _P(c_int32), c_void_p,
                                              _P(TQQJLPageLayout), _P(TQConfig), c_int, c_int,
                                              c_void_p], c_int),
    "tq_make_int4_layout": ([_P(TQConfig), _P(TQPageLayout)], c_int),
    "tq_launch_int4_pack_kv": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8), _P(TQPageLayout),
                                _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_int4_dequant_kv": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                   _P(TQPageLayout), _P(TQConfig), c_int, c_void_p], c_int),
    "tq_make_dense_layout": ([_P(TQConfig), _P(TQDensePageLayout)], c_int),
    "tq_launch_dense_store_kv": ([c_void_p, c_void_p, _P(c_int32), _P(c_uint8),
                                  _P(TQDensePageLayout), _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_dense_load_kv": ([_P(c_uint8), _P(c_int32), c_void_p, c_void_p,
                                 _P(TQDensePageLayout), _P(TQConfig), c_int, c_void_p], c_int),
    "tq_launch_attention_ref": ([c_void_p, c_void_p, c_void_p, c_void_p, _P(c_float),
                                 _P(TQConfig), c_int, c_int, c_void_p], c_int),
    # on-disk store (tq_backend/cag_store.py formats)
    "tq_store_sha256_hex": ([c_void_p, c_size_t, ctypes.c_char_p], c_int),
    "tq_store_key": ([ctypes.c_char_p, c_int, ctypes.c_char_p, ctypes.c_char_p, c_size_t], c_int),
    "tq_store_crc32c": ([c_void_p, c_size_t, _P(ctypes.c_uint32)], c_int),
    "tq_store_write_meta": ([ctypes.c_char_p, _I64, _P(c_int32), _I64, _P(TQStoreFormat)],
                            c_int),
    "tq_store_read_meta": ([ctypes.c_char_p, _P(_I64), _P(c_int32), _I64, _P(_I64),
                           _P(TQStoreFormat), _P(c_int)], c_int),
    "tq_store_write_pool": ([ctypes.c_char_p, c_void_p, c_size_t, _P(TQStoreFormat)], c_int),
    "tq_store_pool_info": ([ctypes.c_char_p, _P(c_size_t), _P(TQStoreFormat), _P(c_int)], c_int),
    "tq_store_read_pools": ([_P(ctypes.c_char_p), _P(c_void_p), c_size_t, c_int, c_int, c_int],
                            c_int),
    "tq_store_write_fp16": ([ctypes.c_char_p, _I64, c_void_p, _I64, _P(_I64), c_int], c_int),
    "tq_store_read_fp16": ([ctypes.c_char_p, _P(_I64), c_void_p, _I64, _P(_I64), _P(_I64), c_int,
                           _P(c_int)], c_int),
    "tq_store_manifest_update": ([ctypes.c_char_p, ctypes.c_char_p, c_int, ctypes.c_char_p, _I64],
                                 c_int),
    "tq_store_manifest_verify": ([ctypes.c_char_p, ctypes.c_char_p, c_int, ctypes.c_char_p],
                                 c_int),
}


class TurboQuantWrapper:
    """Wrapper around libturboquant.so.

    turbo_prod — K = 3-bit Lloyd-Max + 1-bit residual sign, V = 4-bit (3.82x vs fp16)
    turbo_mse  — 4-bit Gaussian-codebook K and V                     (3.56x vs fp16)
    """

    def __init__(self, lib_path: str | Path | None = None) -> None:
        path = Path(lib_path) if lib_path else DEFAULT_LIB_PATH
        if not path.exists():
            raise FileNotFoundError(
                f"libturboquant.so not found at {path}. "
                "Run:  python -m turborag_amd.build  first."
            )
        self.lib_path = path
        self._lib = ctypes.CDLL(str(path))
        self._bind_symbols()

    def _bind_symbols(self) -> None:
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(self._lib, name)
            fn.argtypes = argtypes
            fn.restype = restype

    @property
    def lib(self) -> ctypes.CDLL:
        return self._lib

    # ── errors (reference :177-189) ─────────────────────────────────── #

    def _last_cuda_error(self) -> str:
        raw = self._lib.tq_last_error()
        return raw.decode() if raw else ""

    def _kernel_raise(self, rc: int, scheme: str, op: str) -> None:
        if rc == -2:
            raise RuntimeError(f"{scheme} {op} CUDA error: {self._last_cuda_error()}")
        raise RuntimeError(f"{scheme} {op} failed (rc={rc})")

    # ── config / layout ─────────────────────────────────────────────── #

    def default_config(self) -> TQConfig:
        cfg = TQConfig()
        if self._lib.tq_make_default_config(ctypes.byref(cfg)) != 0:
            raise RuntimeError("tq_make_default_config failed")
        return cfg

    def make_layout_for(self, cfg: TQConfig) -> TQTurboProdPageLayout:
        layout = TQTurboProdPageLayout()
        if self._lib.tq_make_turbo_prod_layout(ctypes.byref(cfg), ctypes.byref(layout)) != 0:
            raise RuntimeError("tq_make_turbo_prod_layout failed")
        return layout

    def make_mse_layout_for(self, cfg: TQConfig) -> TQTurbomsePageLayout:
        layout = TQTurbomsePageLayout()
        if self._lib.tq_make_turbo_mse_layout(ctypes.byref(cfg), ctypes.byref(layout)) != 0:
            raise RuntimeError("tq_make_turbo_mse_layout failed")
        return layout

    # ── pointer helpers ─────────────────────────────────────────────── #

    @staticmethod
    def _vp(t: torch.Tensor) -> c_void_p:
        return c_void_p(t.data_ptr())

    @staticmethod
    def _i32p(t: torch.Tensor):
        return ctypes.cast(c_void_p(t.data_ptr()), POINTER(c_int32))

    @staticmethod
    def _u8p(t: torch.Tensor):
        return ctypes.cast(c_void_p(t.data_ptr()), POINTER(c_uint8))

    @staticmethod
    def _f32p(t: torch.Tensor):
        return ctypes.cast(c_void_p(t.data_ptr()), POINTER(c_float))

    @staticmethod
    def _check(scheme: str, op: str, **tensors: tuple[torch.Tensor, torch.dtype, int]) -> None:
        """Each tensor must live on a GPU, be contiguous, have the dtype and
        hold at least the given number of elements."""
        for name, (t, dtype, numel) in tensors.items():
            if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
                raise ValueError(f"{scheme} {op}: {name} must be a GPU tensor")
            if t.dtype != dtype:
                raise ValueError(f"{scheme} {op}: {name} must be {dtype}, got {t.dtype}")
            if not t.is_contiguous():
                raise ValueError(f"{scheme} {op}: {name} must be contiguous")
            if t.numel() < numel:
                raise ValueError(f"{scheme} {op}: {name} holds {t.numel()} elements, "
                                 f"needs {numel}")

    @staticmethod
    def _stream(stream: int) -> c_void_p:
        return c_void_p(int(stream) if stream else 0)

    # ── turbo_prod ──────────────────────────────────────────────────── #

    def pack(self, key, value, slot_mapping, page_pool, layout, cfg, stream: int = 0) -> None:
        N = key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check("turbo_prod", "pack_kv", key=(key, torch.float16, thd),
                    value=(value, torch.float16, thd), slot_mapping=(slot_mapping, torch.int32, N),
                    page_pool=(page_pool, torch.uint8, 0))
        rc = self._lib.tq_launch_turbo_prod_pack_kv(
            self._vp(key), self._vp(value), self._i32p(slot_mapping), self._u8p(page_pool),
            ctypes.byref(layout), ctypes.byref(cfg), N, self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "pack_kv")

    def pack_debug(self, key, value, slot_mapping, page_pool, layout, cfg,
                   stream: int = 0) -> dict:
        """pack() plus the reference pack kernel's debug buffers
        (include/tq_turbo_prod.cuh:60-65; tq_launch_turbo_prod_pack_kv_debug):
        k_rot, v_rot (rotated K/V), kn, vn (clamped normalised K/V) as fp32
        and kidx, vidx (code indices) as int32, each [N, H, D] on key's
        device."""
        N = key.shape[0]
        H, D = cfg.num_kv_heads, cfg.head_dim
        thd = N * H * D
        self._check("turbo_prod", "pack_kv", key=(key, torch.float16, thd),
                    value=(value, torch.float16, thd), slot_mapping=(slot_mapping, torch.int32, N),
                    page_pool=(page_pool, torch.uint8, 0))
        out = {n: torch.empty(N, H, D, dtype=torch.float32, device=key.device)
               for n in ("k_rot", "v_rot", "kn", "vn")}
        out.update({n: torch.empty(N, H, D, dtype=torch.int32, device=key.device)
                    for n in ("kidx", "vidx")})
        rc = self._lib.tq_launch_turbo_prod_pack_kv_debug(
            self._vp(key), self._vp(value), self._i32p(slot_mapping), self._u8p(page_pool),
            ctypes.byref(layout), ctypes.byref(cfg), N, self._stream(stream),
            *[self._vp(out[n]) for n in ("k_rot", "v_rot", "kn", "vn", "kidx", "vidx")])
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "pack_kv")
        return out

    def dequant(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                stream: int = 0) -> None:
        N = out_key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check("turbo_prod", "dequant_kv", page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, N),
                    out_key=(out_key, torch.float16, thd), out_value=(out_value, torch.float16, thd))
        rc = self._lib.tq_launch_turbo_prod_dequant_kv(
            self._u8p(page_pool), self._i32p(slot_mapping), self._vp(out_key),
            self._vp(out_value), ctypes.byref(layout), ctypes.byref(cfg), N,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "dequant_kv")

    def fused_attn_logits(self, query, page_pool, slot_mapping, logits, layout, cfg,
                          num_queries: int, num_kv_tokens: int, stream: int = 0) -> None:
        """Logit convention: <q, k> / sqrt(D) (what the reference kernel computes,
        src/cuda/tq_turbo_prod_kernels.cu:426)."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("turbo_prod", "fused_attn_logits",
                    query=(query, torch.float16, num_queries * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_kv_tokens),
                    logits=(logits, torch.float32, num_queries * H * num_kv_tokens))
        rc = self._lib.tq_launch_turbo_prod_fused_attention_logits(
            self._vp(query), self._u8p(page_pool), self._i32p(slot_mapping), self._f32p(logits),
            ctypes.byref(layout), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "fused_attn_logits")

    def fused_attn_output(self, query, page_pool, slot_mapping, output, layout, cfg,
                          num_queries: int, num_kv_tokens: int, stream: int = 0) -> None:
        """Online-softmax attention over the compressed pool; no KV rematerialisation."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("turbo_prod", "fused_attn_output",
                    query=(query, torch.float16, num_queries * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_kv_tokens),
                    output=(output, torch.float16, num_queries * H * D))
        rc = self._lib.tq_launch_turbo_prod_fused_attention_output(
            self._vp(query), self._u8p(page_pool), self._i32p(slot_mapping), self._vp(output),
            ctypes.byref(layout), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "fused_attn_output")

    def fused_attn_output_noalloc(self, query, page_pool, slot_mapping, output, layout, cfg,
                                  num_queries: int, num_kv_tokens: int, stream: int = 0) -> None:
        """fused_attn_output with its split-K partials in the library's static
        4 MiB device scratch (tq_launch_turbo_prod_fused_attention_output_noalloc):
        no device allocation; calls overlapping on one GPU race."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("turbo_prod", "fused_attn_output_noalloc",
                    query=(query, torch.float16, num_queries * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_kv_tokens),
                    output=(output, torch.float16, num_queries * H * D))
        rc = self._lib.tq_launch_turbo_prod_fused_attention_output_noalloc(
            self._vp(query), self._u8p(page_pool), self._i32p(slot_mapping), self._vp(output),
            ctypes.byref(layout), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_prod", "fused_attn_output_noalloc")

    # ── turbo_mse ───────────────────────────────────────────────────── #

    def mse_pack(self, key, value, slot_mapping, page_pool, layout, cfg, stream: int = 0) -> None:
        N = key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check("turbo_mse", "pack_kv", key=(key, torch.float16, thd),
                    value=(value, torch.float16, thd), slot_mapping=(slot_mapping, torch.int32, N),
                    page_pool=(page_pool, torch.uint8, 0))
        rc = self._lib.tq_launch_turbo_mse_pack_kv(
            self._vp(key), self._vp(value), self._i32p(slot_mapping), self._u8p(page_pool),
            ctypes.byref(layout), ctypes.byref(cfg), N, self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_mse", "pack_kv")

    def mse_dequant(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                    stream: int = 0) -> None:
        N = out_key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check("turbo_mse", "dequant_kv", page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, N),
                    out_key=(out_key, torch.float16, thd), out_value=(out_value, torch.float16, thd))
        rc = self._lib.tq_launch_turbo_mse_dequant_kv(
            self._u8p(page_pool), self._i32p(slot_mapping), self._vp(out_key),
            self._vp(out_value), ctypes.byref(layout), ctypes.byref(cfg), N,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_mse", "dequant_kv")

    def mse_fused_attn_output(self, query, page_pool, slot_mapping, output, layout, cfg,
                              num_queries: int, num_kv_tokens: int, stream: int = 0) -> None:
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("turbo_mse", "fused_attn_output",
                    query=(query, torch.float16, num_queries * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_kv_tokens),
                    output=(output, torch.float16, num_queries * H * D))
        rc = self._lib.tq_launch_turbo_mse_fused_attention_output(
            self._vp(query), self._u8p(page_pool), self._i32p(slot_mapping), self._vp(output),
            ctypes.byref(layout), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "turbo_mse", "fused_attn_output")

    # ── cache layout [1, H, N, D] and layer loading (this build) ────── #

    def _dequant_hnd(self, scheme, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                     num_tokens, stream):
        thd = num_tokens * cfg.num_kv_heads * cfg.head_dim
        self._check(scheme, "dequant_kv_hnd", page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_tokens),
                    out_key=(out_key, torch.float16, thd), out_value=(out_value, torch.float16, thd))
        fn = (self._lib.tq_launch_turbo_prod_dequant_kv_hnd if scheme == "turbo_prod"
              else self._lib.tq_launch_turbo_mse_dequant_kv_hnd)
        rc = fn(self._u8p(page_pool), self._i32p(slot_mapping), self._vp(out_key),
                self._vp(out_value), ctypes.byref(layout), ctypes.byref(cfg), num_tokens,
                self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "dequant_kv_hnd")

    def dequant_hnd(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                    num_tokens: int, stream: int = 0) -> None:
        """turbo_prod dequant straight into the cache layout [1, H, N, D]."""
        self._dequant_hnd("turbo_prod", page_pool, slot_mapping, out_key, out_value, layout,
                          cfg, num_tokens, stream)

    def mse_dequant_hnd(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                        num_tokens: int, stream: int = 0) -> None:
        self._dequant_hnd("turbo_mse", page_pool, slot_mapping, out_key, out_value, layout,
                          cfg, num_tokens, stream)

    def pack_layers(self, scheme: str, keys, values, slot_mapping, page_pools, layout, cfg,
                    stream: int = 0) -> None:
        """Pack every layer's K/V [N, H, D] fp16 (one shared slot mapping) into
        page_pools[l]; one launch per 64 layers at head_dim 64 and 128."""
        n = len(keys)
        if not (len(values) == len(page_pools) == n):
            raise ValueError("pack_layers: one key, value and pool per layer")
        num_tokens = keys[0].shape[0] if n else 0
        thd = num_tokens * cfg.num_kv_heads * cfg.head_dim
        for l in range(n):
            self._check(scheme, "pack_kv_layers", key=(keys[l], torch.float16, thd),
                        value=(values[l], torch.float16, thd),
                        slot_mapping=(slot_mapping, torch.int32, num_tokens),
                        page_pool=(page_pools[l], torch.uint8, 0))
            if keys[l].shape[0] != num_tokens:
                raise ValueError("pack_layers: every layer has the same number of tokens")
        arr = c_void_p * max(n, 1)
        ks = arr(*[t.data_ptr() for t in keys])
        vs = arr(*[t.data_ptr() for t in values])
        pools = arr(*[p.data_ptr() for p in page_pools])
        fn = (self._lib.tq_launch_turbo_prod_pack_kv_layers if scheme == "turbo_prod"
              else self._lib.tq_launch_turbo_mse_pack_kv_layers)
        rc = fn(ks, vs, self._i32p(slot_mapping), pools, n, ctypes.byref(layout),
                ctypes.byref(cfg), num_tokens, self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "pack_kv_layers")

    def dequant_layers(self, scheme: str, page_pools, slot_mapping, out_keys, out_values,
                       layout, cfg, num_tokens: int, head_major: bool = False,
                       stream: int = 0) -> None:
        """Dequant every layer's pool (one shared slot mapping) into
        out_keys[l] / out_values[l]: [N, H, D] fp16, or [1, H, N, D] with
        head_major; one launch per 64 layers at head_dim 128."""
        n = len(page_pools)
        if not (len(out_keys) == len(out_values) == n):
            raise ValueError("dequant_layers: one pool and two outputs per layer")
        thd = num_tokens * cfg.num_kv_heads * cfg.head_dim
        for l in range(n):
            self._check(scheme, "dequant_kv_layers", page_pool=(page_pools[l], torch.uint8, 0),
                        slot_mapping=(slot_mapping, torch.int32, num_tokens),
                        out_key=(out_keys[l], torch.float16, thd),
                        out_value=(out_values[l], torch.float16, thd))
        arr = c_void_p * max(n, 1)
        pools = arr(*[p.data_ptr() for p in page_pools])
        ks = arr(*[t.data_ptr() for t in out_keys])
        vs = arr(*[t.data_ptr() for t in out_values])
        fn = (self._lib.tq_launch_turbo_prod_dequant_kv_layers if scheme == "turbo_prod"
              else self._lib.tq_launch_turbo_mse_dequant_kv_layers)
        rc = fn(pools, self._i32p(slot_mapping), ks, vs, n, ctypes.byref(layout),
                ctypes.byref(cfg), num_tokens, int(head_major), self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "dequant_kv_layers")

    def load_layers(self, scheme: str, host_pools, device_pools, slot_mapping, out_keys,
                    out_values, layout, cfg, num_tokens: int, copy_stream: int = 0,
                    compute_stream: int = 0) -> None:
        """Copy each layer's pages host -> device and dequantize it into
        out_keys[l] / out_values[l] ([1, H, N, D] fp16), layer l's dequant
        overlapping layer l+1's copy (pinned host_pools overlap fully)."""
        L = len(host_pools)
        if not (len(device_pools) == len(out_keys) == len(out_values) == L):
            raise ValueError(f"{scheme} load_layers: per-layer lists differ in length")
        nbytes = host_pools[0].numel() if L else 0
        thd = num_tokens * cfg.num_kv_heads * cfg.head_dim
        for l in range(L):
            hp = host_pools[l]
            if hp.device.type != "cpu" or hp.dtype != torch.uint8 or not hp.is_contiguous() \
                    or hp.numel() != nbytes:
                raise ValueError(f"{scheme} load_layers: host_pools[{l}] must be a contiguous "
                                 f"CPU uint8 tensor of {nbytes} bytes")
            self._check(scheme, "load_layers", device_pool=(device_pools[l], torch.uint8, nbytes),
                        out_key=(out_keys[l], torch.float16, thd),
                        out_value=(out_values[l], torch.float16, thd))
        self._check(scheme, "load_layers", slot_mapping=(slot_mapping, torch.int32, num_tokens))
        arr = c_void_p * max(L, 1)
        hps = arr(*[t.data_ptr() for t in host_pools])
        dps = arr(*[t.data_ptr() for t in device_pools])
        oks = arr(*[t.data_ptr() for t in out_keys])
        ovs = arr(*[t.data_ptr() for t in out_values])
        fn = (self._lib.tq_load_turbo_prod_layers if scheme == "turbo_prod"
              else self._lib.tq_load_turbo_mse_layers)
        rc = fn(hps, dps, nbytes, L, self._i32p(slot_mapping), num_tokens, oks, ovs,
                ctypes.byref(layout), ctypes.byref(cfg), self._stream(copy_stream),
                self._stream(compute_stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "load_layers")

    def paged_attn_output(self, scheme: str, query, page_pool, block_tables, row_seq,
                          row_kv_len, output, layout, cfg, max_kv_len: int,
                          stream: int = 0) -> None:
        """One launch of decode attention for a batch of paged sequences.

        query / output [num_rows, H, D] fp16; row r belongs to sequence
        row_seq[r] (aligned groups of 8 rows share one) and attends its first
        row_kv_len[r] tokens; block_tables [num_seqs, max_blocks] int32 page
        ids.  head_dim 128."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        num_rows = query.shape[0]
        if block_tables.dim() != 2:
            raise ValueError(f"{scheme} paged_attn_output: block_tables must be [num_seqs, "
                             f"max_blocks]")
        self._check(scheme, "paged_attn_output", query=(query, torch.float16, num_rows * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    block_tables=(block_tables, torch.int32, block_tables.numel()),
                    row_seq=(row_seq, torch.int32, num_rows),
                    row_kv_len=(row_kv_len, torch.int32, num_rows),
                    output=(output, torch.float16, num_rows * H * D))
        fn = (self._lib.tq_launch_turbo_prod_paged_attention if scheme == "turbo_prod"
              else self._lib.tq_launch_turbo_mse_paged_attention)
        rc = fn(self._vp(query), self._u8p(page_pool), self._i32p(block_tables),
                block_tables.shape[1], self._i32p(row_seq), self._i32p(row_kv_len),
                self._vp(output), ctypes.byref(layout), ctypes.byref(cfg), num_rows, max_kv_len,
                self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "paged_attn_output")

    # ── the reference's unexported kernels ──────────────────────────── #
    # QJL-1b (include/tq_qjl.cuh), legacy INT4 (include/tq_layout.h), dense
    # (include/tq_dense_layout.h), GPU SDPA reference (include/tq_attention_ref.h).

    def _layout(self, fn: str, cls, cfg):
        layout = cls()
        rc = getattr(self._lib, fn)(ctypes.byref(cfg), ctypes.byref(layout))
        if rc != 0:
            raise RuntimeError(f"{fn} failed: {self._last_cuda_error()}")
        return layout

    def make_qjl_layout_for(self, cfg: TQConfig) -> TQQJLPageLayout:
        return self._layout("tq_make_qjl_layout", TQQJLPageLayout, cfg)

    def make_int4_layout_for(self, cfg: TQConfig) -> TQPageLayout:
        return self._layout("tq_make_int4_layout", TQPageLayout, cfg)

    def make_dense_layout_for(self, cfg: TQConfig) -> TQDensePageLayout:
        return self._layout("tq_make_dense_layout", TQDensePageLayout, cfg)

    def _store_pages(self, scheme, fn, key, value, slot_mapping, page_pool, layout, cfg, stream):
        N = key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check(scheme, "pack_kv", key=(key, torch.float16, thd),
                    value=(value, torch.float16, thd), slot_mapping=(slot_mapping, torch.int32, N),
                    page_pool=(page_pool, torch.uint8, 0))
        rc = getattr(self._lib, fn)(self._vp(key), self._vp(value), self._i32p(slot_mapping),
                                    self._u8p(page_pool), ctypes.byref(layout), ctypes.byref(cfg),
                                    N, self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "pack_kv")

    def _load_pages(self, scheme, fn, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                    stream):
        N = out_key.shape[0]
        thd = N * cfg.num_kv_heads * cfg.head_dim
        self._check(scheme, "dequant_kv", page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, N),
                    out_key=(out_key, torch.float16, thd), out_value=(out_value, torch.float16, thd))
        rc = getattr(self._lib, fn)(self._u8p(page_pool), self._i32p(slot_mapping),
                                    self._vp(out_key), self._vp(out_value), ctypes.byref(layout),
                                    ctypes.byref(cfg), N, self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, scheme, "dequant_kv")

    def qjl_pack(self, key, value, slot_mapping, page_pool, layout, cfg, stream: int = 0) -> None:
        self._store_pages("qjl", "tq_launch_qjl_pack_kv", key, value, slot_mapping, page_pool,
                          layout, cfg, stream)

    def qjl_dequant(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                    stream: int = 0) -> None:
        self._load_pages("qjl", "tq_launch_qjl_dequant_kv", page_pool, slot_mapping, out_key,
                         out_value, layout, cfg, stream)

    def qjl_fused_attn_output(self, query, page_pool, slot_mapping, output, layout, cfg,
                              num_queries: int, num_kv_tokens: int, stream: int = 0) -> None:
        """Logit convention <q, k> without 1/sqrt(D), as the QJL kernel
        (src/cuda/tq_qjl_kernels.cu:254)."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("qjl", "fused_attn_output", query=(query, torch.float16, num_queries * H * D),
                    page_pool=(page_pool, torch.uint8, 0),
                    slot_mapping=(slot_mapping, torch.int32, num_kv_tokens),
                    output=(output, torch.float16, num_queries * H * D))
        rc = self._lib.tq_launch_qjl_fused_attention_output(
            self._vp(query), self._u8p(page_pool), self._i32p(slot_mapping), self._vp(output),
            ctypes.byref(layout), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "qjl", "fused_attn_output")

    def int4_pack(self, key, value, slot_mapping, page_pool, layout, cfg, stream: int = 0) -> None:
        self._store_pages("int4", "tq_launch_int4_pack_kv", key, value, slot_mapping, page_pool,
                          layout, cfg, stream)

    def int4_dequant(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                     stream: int = 0) -> None:
        self._load_pages("int4", "tq_launch_int4_dequant_kv", page_pool, slot_mapping, out_key,
                         out_value, layout, cfg, stream)

    def dense_store(self, key, value, slot_mapping, page_pool, layout, cfg,
                    stream: int = 0) -> None:
        self._store_pages("dense", "tq_launch_dense_store_kv", key, value, slot_mapping,
                          page_pool, layout, cfg, stream)

    def dense_load(self, page_pool, slot_mapping, out_key, out_value, layout, cfg,
                   stream: int = 0) -> None:
        self._load_pages("dense", "tq_launch_dense_load_kv", page_pool, slot_mapping, out_key,
                         out_value, layout, cfg, stream)

    def attention_ref(self, query, key, value, output, logit_scratch, cfg, num_queries: int,
                      num_kv_tokens: int, stream: int = 0) -> None:
        """softmax(q k^T / sqrt(D)) V over contiguous fp16 K/V; logit_scratch
        (float32, num_queries * H * num_kv_tokens) receives the logits."""
        H, D = cfg.num_kv_heads, cfg.head_dim
        self._check("sdpa", "attention_ref", query=(query, torch.float16, num_queries * H * D),
                    key=(key, torch.float16, num_kv_tokens * H * D),
                    value=(value, torch.float16, num_kv_tokens * H * D),
                    output=(output, torch.float16, num_queries * H * D),
                    logit_scratch=(logit_scratch, torch.float32,
                                   num_queries * H * num_kv_tokens))
        rc = self._lib.tq_launch_attention_ref(
            self._vp(query), self._vp(key), self._vp(value), self._vp(output),
            self._f32p(logit_scratch), ctypes.byref(cfg), num_queries, num_kv_tokens,
            self._stream(stream))
        if rc != 0:
            self._kernel_raise(rc, "sdpa", "attention_ref")

    def release_workspaces(self) -> None:
        """Synchronize and free the attention entries' cached split-K
        workspaces (tq_workspace_release): for callers that cycle through
        many streams.  Graphs captured before must not be replayed after."""
        rc = self.lib.tq_workspace_release()
        if rc != 0:
            raise RuntimeError(f"tq_workspace_release failed: {self._last_cuda_error()}")

    # ── allocation helpers (reference :385-415) ─────────────────────── #

    def alloc_page_pool(self, num_tokens: int, layout, cfg) -> torch.Tensor:
        num_blocks = (num_tokens + cfg.block_size - 1) // cfg.block_size
        return torch.zeros(num_blocks * layout.page_size_bytes, device="cuda", dtype=torch.uint8)

    def alloc_mse_pool(self, num_tokens: int, layout, cfg) -> torch.Tensor:
        num_blocks = (num_tokens + cfg.block_size - 1) // cfg.block_size
        return torch.zeros(num_blocks * layout.page_size_bytes, device="cuda", dtype=torch.uint8)

    def fp16_bytes(self, num_tokens: int, cfg) -> int:
        """Bytes for both K and V in fp16."""
        return num_tokens * cfg.num_kv_heads * cfg.head_dim * 2 * 2

    def quant_bytes(self, num_tokens: int, layout, cfg) -> int:
        num_blocks = (num_tokens + cfg.block_size - 1) // cfg.block_size
        return num_blocks * layout.page_size_bytes

    def mse_bytes(self, num_tokens: int, layout, cfg) -> int:
        num_blocks = (num_tokens + cfg.block_size - 1) // cfg.block_size
        return num_blocks * layout.page_size_bytes

    @staticmethod
    def compute_mse(a: torch.Tensor, b: torch.Tensor) -> float:
        return torch.mean((a.float() - b.float()) ** 2).item()

    def summary(self) -> dict:
        cfg = self.default_config()
        prod = self.make_layout_for(cfg)
        mse_l = self.make_mse_layout_for(cfg)
        fp16_b = cfg.block_size * cfg.num_kv_heads * cfg.head_dim * 2 * 2
        return {
            "lib_path": str(self.lib_path),
            "config": {"block_size": cfg.block_size, "num_kv_heads": cfg.num_kv_heads,
                       "head_dim": cfg.head_dim, "nbits": cfg.nbits},
            "turbo_prod_compression_ratio_vs_fp16": round(fp16_b / prod.page_size_bytes, 2),
            "turbo_mse_compression_ratio_vs_fp16": round(fp16_b / mse_l.page_size_bytes, 2),
        }


# --------------------------------------------------------------------------- #
# Page allocator and block table                                               #
# --------------------------------------------------------------------------- #

class PageAllocator:
    """TQAllocator (src/tq_allocator.cpp): LIFO page ids 0, 1, 2, ...; -1 when empty.

    ``device_pool`` (a uint8 GPU tensor of num_pages * page_size bytes) is
    used as the pool when given; otherwise the library allocates it.
    """

    def __init__(self, tq: TurboQuantWrapper, page_size_bytes: int, num_pages: int,
                 device_pool: torch.Tensor | None = None) -> None:
        self._tq = tq
        self._keep = device_pool
        h = c_void_p()
        ptr = c_void_p(device_pool.data_ptr()) if device_pool is not None else c_void_p(0)
        rc = tq.lib.tq_allocator_create(page_size_bytes, num_pages, ptr, ctypes.byref(h))
        if rc != 0:
            tq._kernel_raise(rc, "allocator", "create")
        self.handle = h
        self.page_size_bytes = page_size_bytes
        self.num_pages = num_pages

    def alloc_block(self) -> int:
        b = c_int32()
        self._tq.lib.tq_allocator_alloc_block(self.handle, ctypes.byref(b))
        return int(b.value)

    def free_block(self, block: int) -> None:
        rc = self._tq.lib.tq_allocator_free_block(self.handle, int(block))
        if rc != 0:
            self._tq._kernel_raise(rc, "allocator", "free_block")

    def num_free(self) -> int:
        n = c_int()
        self._tq.lib.tq_allocator_num_free(self.handle, ctypes.byref(n))
        return int(n.value)

    def device_pool_ptr(self) -> int:
        return int(self._tq.lib.tq_allocator_device_pool(self.handle) or 0)

    def close(self) -> None:
        if self.handle:
            self._tq.lib.tq_allocator_destroy(self.handle)
            self.handle = c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class BlockTable:
    """TQBlockTable (src/tq_block_table.cpp): per-sequence pages and slot maps."""

    def __init__(self, alloc: PageAllocator, block_size: int = 16) -> None:
        self._alloc = alloc
        self._tq = alloc._tq
        h = c_void_p()
        rc = self._tq.lib.tq_block_table_create(alloc.handle, block_size, ctypes.byref(h))
        if rc != 0:
            self._tq._kernel_raise(rc, "block_table", "create")
        self.handle = h
        self.block_size = block_size

    def build_slot_map(self, seq_id: int, append_tokens: int) -> list[int]:
        out = (c_int32 * max(append_tokens, 1))()
        rc = self._tq.lib.tq_block_table_build_slot_map(self.handle, seq_id, append_tokens, out)
        if rc != 0:
            if rc == -2:
                raise RuntimeError(self._tq._last_cuda_error())
            self._tq._kernel_raise(rc, "block_table", "build_slot_map")
        return list(out[:append_tokens])

    def num_tokens(self, seq_id: int) -> int:
        n = c_int()
        rc = self._tq.lib.tq_block_table_num_tokens(self.handle, seq_id, ctypes.byref(n))
        if rc != 0:
            raise KeyError(seq_id)
        return int(n.value)

    def blocks(self, seq_id: int) -> list[int]:
        n = c_int()
        rc = self._tq.lib.tq_block_table_blocks(self.handle, seq_id, None, 0, ctypes.byref(n))
        if rc != 0:
            raise KeyError(seq_id)
        out = (c_int32 * max(n.value, 1))()
        self._tq.lib.tq_block_table_blocks(self.handle, seq_id, out, n.value, ctypes.byref(n))
        return list(out[:n.value])

    def free_sequence(self, seq_id: int) -> None:
        rc = self._tq.lib.tq_block_table_free_sequence(self.handle, seq_id)
        if rc != 0:
            raise KeyError(seq_id)

    def close(self) -> None:
        if self.handle:
            self._tq.lib.tq_block_table_destroy(self.handle)
            self.handle = c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
