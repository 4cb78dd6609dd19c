"""CPU oracle for the TurboCAG KV-compression path — TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this module, and only as the checker.  The product library
(``build/libturboquant.so``) never loads it.

The C code (``oracle/tq_oracle.c``) restates the reference's device-code
operation order; each function there cites the reference lines it follows.

Parity pins — what checks each oracle function against something other than
itself (tests/test_oracle.py unless noted):

* fp16 conversion  — numpy's float16 (IEEE RNE) on all 2^16 halves and on
  random/edge floats.
* sign_flip        — the closed form (-1)^(i+h) (the hash's bit 0), for all
  i < 128, h < 64.
* WHT              — scipy.linalg.hadamard(D) @ x in float64 (within fp32
  rounding), H.H = D.I, and the bit-exact pair-swap/negate identity
  WHT(s(.,h) * x) = +/-WHT(x)[j ^ 1] that the butterfly order implies.
* tree sum         — adversarial inputs where a sequential or pairwise-
  adjacent sum gives a different float32 than the halving tree.
* nearest codes    — numpy float32 brute force (np.argmin = first minimum).
* K3 codebook      — the reference's own src/gaussian_codebook.cpp built in
  oracle/_ref and run (prints the K3 literals), and this oracle's Lloyd-Max
  restatement; V4 — the 16-level Lloyd-Max design to 1.5e-4.
* layouts          — the reference's own src/tq_turbo_mse_layout.cpp and
  src/tq_layout.cpp built in oracle/_ref, over a grid of configs; turbo_prod
  layout by the closed form and the README's published VRAM figures
  (README.md:53-55,70-72: 302/324 MB at 32K x 36, 75/81 MB at 8K x 36).
* pack (turbo_prod) — hand-derived known-answer pages (all-zero and one-hot
  K/V, tests/test_known_answers.py), the reference test's relative-MSE bounds
  (tests/test_cag.py:212-215 of the reference), and idempotence of
  pack(dequant(pack(x))) away from boundary cases.
* pack (turbo_mse) — known-answer pages, relative-MSE bound, idempotence.
* dequant          — known-answer outputs of the hand-built pages and the
  linear-algebra identity dequant = s * H(decoded) / sqrt(D) in float64.
* attention        — fp64 oracle vs SDPA over the oracle's dequantized K/V
  (src/tq_attention_ref.cpp semantics) within 1e-3 relative, and the
  reference-order fp32 restatement within 1e-3 of the fp64 oracle.
* Lloyd-Max        — against the reference binary's printed output.

Parity unpinned (cannot be observed without NVIDIA hardware): the exact bits
of nvcc's rsqrtf(128.f) (this build uses the correctly rounded value), whether
nvcc contracted tq_turbo_mse_kernels.cu:108 into an FMA (the fused form is the
default here; the unfused form is available and their divergence is counted),
and CUDA expf ulps in the softmax (covered by the 1e-3 attention tolerance).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_double, c_float, c_int, c_longlong, c_size_t, c_uint16
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libtq_oracle.so"
REF_DIR = HERE / "_ref"

__all__ = ["Oracle", "ProdLayout", "MseLayout", "QjlLayout", "Int4Layout", "DenseLayout",
           "load", "REF_DIR"]


class ProdLayout(Structure):
    _fields_ = [("page_size", c_size_t), ("k4_off", c_size_t), ("kres_off", c_size_t),
                ("ks_off", c_size_t), ("v4_off", c_size_t), ("vs_off", c_size_t),
                ("k4_bytes", c_int), ("v4_bytes", c_int), ("scale_bytes", c_int)]


class MseLayout(Structure):
    _fields_ = [("code_bytes", c_size_t), ("norm_bytes", c_size_t), ("k_codes_off", c_size_t),
                ("v_codes_off", c_size_t), ("k_norms_off", c_size_t), ("v_norms_off", c_size_t),
                ("page_size", c_size_t)]


class QjlLayout(Structure):
    _fields_ = [("page_size", c_size_t), ("k1_off", c_size_t), ("ks_off", c_size_t),
                ("v4_off", c_size_t), ("vs_off", c_size_t), ("k1_bytes", c_int),
                ("v4_bytes", c_int), ("scale_bytes", c_int)]


class Int4Layout(Structure):
    _fields_ = [(n, c_size_t) for n in (
        "code_bytes", "scale_bytes", "k_codes_off", "v_codes_off", "k_scales_off", "v_scales_off",
        "k_codes_bytes", "v_codes_bytes", "k_scales_bytes", "v_scales_bytes", "page_size")]


class DenseLayout(Structure):
    _fields_ = [(n, c_size_t) for n in ("elem_bytes", "k_off", "v_off", "k_bytes", "v_bytes",
                                        "page_size")]


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _u16(a) -> np.ndarray:
    a = np.asarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    return np.ascontiguousarray(a, dtype=np.uint16)


class Oracle:
    """Thin numpy front end over liboracle (all arrays host, C-contiguous)."""

    def __init__(self, path: Path | str = LIB_PATH):
        if not Path(path).exists():
            raise FileNotFoundError(f"oracle library missing: {path} (run oracle/build_oracle.sh)")
        self.lib = ctypes.CDLL(str(path))
        L = self.lib
        vp = ctypes.c_void_p
        L.tqo_f2h.restype = c_uint16
        L.tqo_f2h.argtypes = [c_float]
        L.tqo_h2f.restype = c_float
        L.tqo_h2f.argtypes = [c_uint16]
        L.tqo_inv_sqrt_d.restype = c_float
        L.tqo_inv_sqrt_d.argtypes = [c_int]
        L.tqo_sign_flip.restype = c_float
        L.tqo_sign_flip.argtypes = [c_int, c_int]
        L.tqo_nearest_k3.restype = c_int
        L.tqo_nearest_k3.argtypes = [c_float]
        L.tqo_nearest_v4.restype = c_int
        L.tqo_nearest_v4.argtypes = [c_float]
        L.tqo_k3.restype = c_float
        L.tqo_k3.argtypes = [c_int]
        L.tqo_v4.restype = c_float
        L.tqo_v4.argtypes = [c_int]
        L.tqo_tree_sum.restype = c_float
        L.tqo_tree_sum.argtypes = [vp, c_int]
        L.tqo_wht.argtypes = [vp, c_int]
        L.tqo_make_prod_layout.argtypes = [c_int, c_int, c_int, POINTER(ProdLayout)]
        L.tqo_make_mse_layout.argtypes = [c_int, c_int, c_int, c_int, c_int, POINTER(MseLayout)]
        L.tqo_f2h_array.argtypes = [vp, vp, c_size_t]
        L.tqo_h2f_array.argtypes = [vp, vp, c_size_t]
        for name in ("tqo_prod_pack",):
            getattr(L, name).argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int,
                                         POINTER(ProdLayout), vp, c_int]
        L.tqo_prod_dequant.argtypes = [vp, vp, c_int, c_int, c_int, c_int, POINTER(ProdLayout),
                                       vp, vp, c_int]
        L.tqo_prod_logits_f32.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                          POINTER(ProdLayout), vp, c_int]
        L.tqo_prod_attention_f64.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                             POINTER(ProdLayout), vp, vp, c_int]
        L.tqo_prod_attention_f32.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                             POINTER(ProdLayout), vp, c_int]
        L.tqo_prod_pack_row.argtypes = [vp, vp, c_int, c_int, vp, vp, vp, vp, vp, vp, vp]
        L.tqo_prod_pack_row_debug.argtypes = [vp, vp, c_int, c_int] + [vp] * 11
        L.tqo_prod_pack_debug.argtypes = [vp, vp, c_int, c_int, c_int] + [vp] * 6 + [c_int]
        L.tqo_prod_boundary_list.argtypes = [vp, vp, c_int, c_int, c_int, vp, vp, vp, c_longlong]
        L.tqo_prod_boundary_list.restype = c_longlong
        L.tqo_mse_pack.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, POINTER(MseLayout),
                                   vp, c_int, c_int]
        L.tqo_mse_pack_row.argtypes = [vp, c_int, c_int, c_int, vp, vp, vp]
        L.tqo_mse_dequant.argtypes = [vp, vp, c_int, c_int, c_int, c_int, POINTER(MseLayout),
                                      vp, vp, c_int]
        L.tqo_mse_attention_f64.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                            POINTER(MseLayout), vp, c_int]
        L.tqo_mse_attention_f32.argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                            POINTER(MseLayout), vp, c_int]
        L.tqo_prod_boundary_count.argtypes = [vp, vp, c_int, c_int, c_int, POINTER(c_longlong)]
        L.tqo_mse_boundary_count.argtypes = [vp, vp, c_int, c_int, c_int, POINTER(c_longlong)]
        L.tqo_sdpa_single_head.argtypes = [vp, vp, vp, c_int, c_int, vp]
        L.tqo_make_qjl_layout.argtypes = [c_int, c_int, c_int, POINTER(QjlLayout)]
        L.tqo_make_int4_layout.argtypes = [c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                           POINTER(Int4Layout)]
        L.tqo_make_int4_layout.restype = c_int
        L.tqo_make_dense_layout.argtypes = [c_int, c_int, c_int, c_int, POINTER(DenseLayout)]
        L.tqo_qjl_pack_row.argtypes = [vp, vp, c_int, vp, vp, vp, vp]
        L.tqo_int4_pack_row.argtypes = [vp, vp, c_int, vp, vp, vp, vp]
        for name, lay in (("tqo_qjl_pack", QjlLayout), ("tqo_int4_pack", Int4Layout)):
            getattr(L, name).argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, POINTER(lay),
                                         vp, c_int]
        for name, lay in (("tqo_qjl_dequant", QjlLayout), ("tqo_int4_dequant", Int4Layout)):
            getattr(L, name).argtypes = [vp, vp, c_int, c_int, c_int, c_int, POINTER(lay), vp,
                                         vp, c_int]
        for name in ("tqo_qjl_attention_f64", "tqo_qjl_attention_f32"):
            getattr(L, name).argtypes = [vp, vp, vp, c_int, c_int, c_int, c_int, c_int,
                                         POINTER(QjlLayout), vp, c_int]
        L.tqo_sdpa_gpu_ref.argtypes = [vp, vp, vp, vp, vp, c_int, c_int, c_int, c_int, c_int]
        L.tqo_lloyd_max_gaussian.argtypes = [c_int, c_int, c_double, vp, vp]
        self.nthreads = int(os.environ.get("TQ_ORACLE_THREADS", "1"))

    # ---- scalars ---------------------------------------------------------
    def f2h(self, x: float) -> int:
        return int(self.lib.tqo_f2h(float(x)))

    def h2f(self, h: int) -> float:
        return float(self.lib.tqo_h2f(int(h)))

    def f2h_array(self, x) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.tqo_f2h_array(_p(x), _p(out), x.size)
        return out

    def h2f_array(self, h) -> np.ndarray:
        h = _u16(h)
        out = np.empty(h.shape, np.float32)
        self.lib.tqo_h2f_array(_p(h), _p(out), h.size)
        return out

    def inv_sqrt_d(self, D: int) -> float:
        return float(self.lib.tqo_inv_sqrt_d(D))

    def sign_flip(self, i: int, h: int) -> float:
        return float(self.lib.tqo_sign_flip(i, h))

    def nearest_k3(self, x: float) -> int:
        return int(self.lib.tqo_nearest_k3(float(x)))

    def nearest_v4(self, x: float) -> int:
        return int(self.lib.tqo_nearest_v4(float(x)))

    @property
    def k3(self) -> np.ndarray:
        return np.array([self.lib.tqo_k3(i) for i in range(8)], np.float32)

    @property
    def v4(self) -> np.ndarray:
        return np.array([self.lib.tqo_v4(i) for i in range(16)], np.float32)

    def wht(self, x) -> np.ndarray:
        x = np.array(x, dtype=np.float32, copy=True)
        self.lib.tqo_wht(_p(x), x.size)
        return x

    def tree_sum(self, r) -> float:
        r = np.ascontiguousarray(r, dtype=np.float32)
        return float(self.lib.tqo_tree_sum(_p(r), r.size))

    # ---- layouts -----------------------------------------------------------
    def prod_layout(self, block_size: int, H: int, D: int) -> ProdLayout:
        L = ProdLayout()
        self.lib.tqo_make_prod_layout(block_size, H, D, ctypes.byref(L))
        return L

    def mse_layout(self, block_size: int, H: int, D: int, nbits: int = 4,
                   align: int = 256) -> MseLayout:
        L = MseLayout()
        self.lib.tqo_make_mse_layout(block_size, H, D, nbits, align, ctypes.byref(L))
        return L

    @staticmethod
    def pool_bytes(num_pages: int, layout) -> int:
        return int(num_pages) * int(layout.page_size)

    # ---- turbo_prod ----------------------------------------------------------
    def prod_pack(self, key, value, slots, num_pages: int, block_size: int = 16,
                  pool: np.ndarray | None = None) -> np.ndarray:
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        L = self.prod_layout(block_size, H, D)
        if pool is None:
            pool = np.zeros(num_pages * L.page_size, np.uint8)
        self.lib.tqo_prod_pack(_p(key), _p(value), _p(slots), N, H, D, block_size,
                               ctypes.byref(L), _p(pool), self.nthreads)
        return pool

    def prod_pack_row(self, k, v, head: int):
        k, v = _u16(k), _u16(v)
        D = k.size
        k4 = np.zeros(D // 2, np.uint8)
        v4 = np.zeros(D // 2, np.uint8)
        sc = np.zeros(3, np.uint16)
        kn = np.zeros(D, np.float32)
        vn = np.zeros(D, np.float32)
        self.lib.tqo_prod_pack_row(_p(k), _p(v), head, D, _p(k4), _p(v4), _p(sc[0:]),
                                   _p(sc[1:]), _p(sc[2:]), _p(kn), _p(vn))
        return dict(k4=k4, v4=v4, ks=int(sc[0]), kres=int(sc[1]), vs=int(sc[2]), kn=kn, vn=vn)

    def prod_pack_debug(self, key, value) -> dict:
        """The reference pack kernel's debug buffers for K, V [N, H, D]
        (tq_turbo_prod_kernels.cu:216-217, 243-246): rotated K/V, clamped
        normalised K/V (fp32) and the K / V code indices (int32), each
        [N, H, D]."""
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        out = {n: np.zeros((N, H, D), np.float32) for n in ("k_rot", "v_rot", "kn", "vn")}
        out.update({n: np.zeros((N, H, D), np.int32) for n in ("kidx", "vidx")})
        self.lib.tqo_prod_pack_debug(_p(key), _p(value), N, H, D, _p(out["k_rot"]),
                                     _p(out["v_rot"]), _p(out["kn"]), _p(out["vn"]),
                                     _p(out["kidx"]), _p(out["vidx"]), self.nthreads)
        return out

    def prod_boundary_list(self, key, value, max_out: int = 1 << 16):
        """The values boundary_counts('turbo_prod') counts: (flat element
        index into [N, H, D], kind 0 K code / 1 K residual sign / 2 V code,
        normalised value)."""
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        elem = np.zeros(max_out, np.int64)
        kind = np.zeros(max_out, np.int32)
        val = np.zeros(max_out, np.float32)
        n = int(self.lib.tqo_prod_boundary_list(_p(key), _p(value), N * H, H, D, _p(elem),
                                                _p(kind), _p(val), max_out))
        n = min(n, max_out)
        return elem[:n], kind[:n], val[:n]

    def prod_dequant(self, pool, slots, H: int, D: int, block_size: int = 16):
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        N = slots.size
        L = self.prod_layout(block_size, H, D)
        ok = np.zeros((N, H, D), np.uint16)
        ov = np.zeros((N, H, D), np.uint16)
        self.lib.tqo_prod_dequant(_p(pool), _p(slots), N, H, D, block_size, ctypes.byref(L),
                                  _p(ok), _p(ov), self.nthreads)
        return ok, ov

    def prod_logits(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        N = slots.size
        L = self.prod_layout(block_size, H, D)
        out = np.zeros((Q, H, N), np.float32)
        self.lib.tqo_prod_logits_f32(_p(query), _p(pool), _p(slots), Q, N, H, D, block_size,
                                     ctypes.byref(L), _p(out), self.nthreads)
        return out

    def prod_attention_f64(self, query, pool, slots, block_size: int = 16,
                           want_logits: bool = False):
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        N = slots.size
        L = self.prod_layout(block_size, H, D)
        out = np.zeros((Q, H, D), np.float64)
        lg = np.zeros((Q, H, max(N, 1)), np.float64) if want_logits else None
        self.lib.tqo_prod_attention_f64(_p(query), _p(pool), _p(slots), Q, N, H, D, block_size,
                                        ctypes.byref(L), _p(out),
                                        _p(lg) if lg is not None else None, self.nthreads)
        return (out, lg[:, :, :N]) if want_logits else out

    def prod_attention_f32(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        L = self.prod_layout(block_size, H, D)
        out = np.zeros((Q, H, D), np.uint16)
        self.lib.tqo_prod_attention_f32(_p(query), _p(pool), _p(slots), Q, slots.size, H, D,
                                        block_size, ctypes.byref(L), _p(out), self.nthreads)
        return out

    # ---- turbo_mse -------------------------------------------------------------
    def mse_pack(self, key, value, slots, num_pages: int, block_size: int = 16,
                 fused_pairsum: bool = True, pool: np.ndarray | None = None) -> np.ndarray:
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        L = self.mse_layout(block_size, H, D)
        if pool is None:
            pool = np.zeros(num_pages * L.page_size, np.uint8)
        self.lib.tqo_mse_pack(_p(key), _p(value), _p(slots), N, H, D, block_size,
                              ctypes.byref(L), _p(pool), int(fused_pairsum), self.nthreads)
        return pool

    def mse_pack_row(self, x, head: int, fused_pairsum: bool = True):
        x = _u16(x)
        D = x.size
        codes = np.zeros(D // 2, np.uint8)
        norm = np.zeros(1, np.uint16)
        xn = np.zeros(D, np.float32)
        self.lib.tqo_mse_pack_row(_p(x), head, D, int(fused_pairsum), _p(codes), _p(norm),
                                  _p(xn))
        return dict(codes=codes, norm=int(norm[0]), xn=xn)

    def mse_dequant(self, pool, slots, H: int, D: int, block_size: int = 16):
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        N = slots.size
        L = self.mse_layout(block_size, H, D)
        ok = np.zeros((N, H, D), np.uint16)
        ov = np.zeros((N, H, D), np.uint16)
        self.lib.tqo_mse_dequant(_p(pool), _p(slots), N, H, D, block_size, ctypes.byref(L),
                                 _p(ok), _p(ov), self.nthreads)
        return ok, ov

    def mse_attention_f64(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        L = self.mse_layout(block_size, H, D)
        out = np.zeros((Q, H, D), np.float64)
        self.lib.tqo_mse_attention_f64(_p(query), _p(pool), _p(slots), Q, slots.size, H, D,
                                       block_size, ctypes.byref(L), _p(out), self.nthreads)
        return out

    def mse_attention_f32(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        L = self.mse_layout(block_size, H, D)
        out = np.zeros((Q, H, D), np.uint16)
        self.lib.tqo_mse_attention_f32(_p(query), _p(pool), _p(slots), Q, slots.size, H, D,
                                       block_size, ctypes.byref(L), _p(out), self.nthreads)
        return out

    # ---- QJL-1b, legacy INT4, dense, GPU SDPA reference ------------------------
    def qjl_layout(self, block_size: int, H: int, D: int) -> QjlLayout:
        L = QjlLayout()
        self.lib.tqo_make_qjl_layout(block_size, H, D, ctypes.byref(L))
        return L

    def int4_layout(self, block_size: int, H: int, D: int, nbits: int = 4,
                    group_size: int | None = None, align: int = 256,
                    scale_fp32: bool = False) -> Int4Layout | None:
        L = Int4Layout()
        rc = self.lib.tqo_make_int4_layout(block_size, H, D, nbits,
                                           D if group_size is None else group_size, align,
                                           int(scale_fp32), ctypes.byref(L))
        return L if rc == 0 else None

    def dense_layout(self, block_size: int, H: int, D: int, align: int = 256) -> DenseLayout:
        L = DenseLayout()
        self.lib.tqo_make_dense_layout(block_size, H, D, align, ctypes.byref(L))
        return L

    def qjl_pack_row(self, k, v):
        k, v = _u16(k), _u16(v)
        D = k.size
        k1 = np.zeros((D + 7) // 8, np.uint8)
        v4 = np.zeros(D // 2, np.uint8)
        sc = np.zeros(2, np.uint16)
        self.lib.tqo_qjl_pack_row(_p(k), _p(v), D, _p(k1), _p(v4), _p(sc[0:]), _p(sc[1:]))
        return dict(k1=k1, v4=v4, ks=int(sc[0]), vs=int(sc[1]))

    def int4_pack_row(self, k, v):
        k, v = _u16(k), _u16(v)
        D = k.size
        kc = np.zeros((D + 1) // 2, np.uint8)
        vc = np.zeros((D + 1) // 2, np.uint8)
        sc = np.zeros(2, np.uint16)
        self.lib.tqo_int4_pack_row(_p(k), _p(v), D, _p(kc), _p(vc), _p(sc[0:]), _p(sc[1:]))
        return dict(kc=kc, vc=vc, ks=int(sc[0]), vs=int(sc[1]))

    def _pack_any(self, fn, L, key, value, slots, num_pages, block_size, pool):
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        if pool is None:
            pool = np.zeros(num_pages * L.page_size, np.uint8)
        fn(_p(key), _p(value), _p(slots), N, H, D, block_size, ctypes.byref(L), _p(pool),
           self.nthreads)
        return pool

    def _dequant_any(self, fn, L, pool, slots, H, D, block_size):
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        N = slots.size
        ok = np.zeros((N, H, D), np.uint16)
        ov = np.zeros((N, H, D), np.uint16)
        fn(_p(pool), _p(slots), N, H, D, block_size, ctypes.byref(L), _p(ok), _p(ov),
           self.nthreads)
        return ok, ov

    def qjl_pack(self, key, value, slots, num_pages: int, block_size: int = 16, pool=None):
        _, H, D = np.shape(key)
        return self._pack_any(self.lib.tqo_qjl_pack, self.qjl_layout(block_size, H, D), key,
                              value, slots, num_pages, block_size, pool)

    def qjl_dequant(self, pool, slots, H: int, D: int, block_size: int = 16):
        return self._dequant_any(self.lib.tqo_qjl_dequant, self.qjl_layout(block_size, H, D),
                                 pool, slots, H, D, block_size)

    def int4_pack(self, key, value, slots, num_pages: int, block_size: int = 16, pool=None,
                  align: int = 256, scale_fp32: bool = False):
        _, H, D = np.shape(key)
        L = self.int4_layout(block_size, H, D, align=align, scale_fp32=scale_fp32)
        return self._pack_any(self.lib.tqo_int4_pack, L, key, value, slots, num_pages,
                              block_size, pool)

    def int4_dequant(self, pool, slots, H: int, D: int, block_size: int = 16, align: int = 256,
                     scale_fp32: bool = False):
        L = self.int4_layout(block_size, H, D, align=align, scale_fp32=scale_fp32)
        return self._dequant_any(self.lib.tqo_int4_dequant, L, pool, slots, H, D, block_size)

    def _qjl_att(self, fn, dtype, query, pool, slots, block_size):
        query = _u16(query)
        Q, H, D = query.shape
        slots = np.ascontiguousarray(slots, dtype=np.int32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        out = np.zeros((Q, H, D), dtype)
        fn(_p(query), _p(pool), _p(slots), Q, slots.size, H, D, block_size,
           ctypes.byref(self.qjl_layout(block_size, H, D)), _p(out), self.nthreads)
        return out

    def qjl_attention_f64(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        return self._qjl_att(self.lib.tqo_qjl_attention_f64, np.float64, query, pool, slots,
                             block_size)

    def qjl_attention_f32(self, query, pool, slots, block_size: int = 16) -> np.ndarray:
        return self._qjl_att(self.lib.tqo_qjl_attention_f32, np.uint16, query, pool, slots,
                             block_size)

    def sdpa_gpu_ref(self, query, key, value):
        """(fp16 output bits [Q,H,D], fp32 logits [Q,H,N]) of the GPU SDPA
        reference kernel's algorithm."""
        query, key, value = _u16(query), _u16(key), _u16(value)
        Q, H, D = query.shape
        N = key.shape[0]
        out = np.zeros((Q, H, D), np.uint16)
        lg = np.zeros((Q, H, max(N, 1)), np.float32)
        self.lib.tqo_sdpa_gpu_ref(_p(query), _p(key), _p(value), _p(out), _p(lg), Q, N, H, D,
                                  self.nthreads)
        return out, lg[:, :, :N]

    # ---- misc ------------------------------------------------------------------
    def boundary_counts(self, scheme: str, key, value) -> tuple[int, int, int]:
        key, value = _u16(key), _u16(value)
        N, H, D = key.shape
        c = (c_longlong * 3)()
        fn = self.lib.tqo_prod_boundary_count if scheme == "turbo_prod" else \
            self.lib.tqo_mse_boundary_count
        fn(_p(key), _p(value), N * H, H, D, c)
        return int(c[0]), int(c[1]), int(c[2])

    def sdpa_single_head(self, q, k_all, v_all) -> np.ndarray:
        q, k_all, v_all = _u16(q), _u16(k_all), _u16(v_all)
        D = q.size
        N = k_all.size // D
        out = np.zeros(D, np.float32)
        self.lib.tqo_sdpa_single_head(_p(q), _p(k_all), _p(v_all), N, D, _p(out))
        return out

    def lloyd_max(self, M: int, max_iter: int = 50, tol: float = 1e-12):
        lv = np.zeros(M, np.float64)
        th = np.zeros(M - 1, np.float64)
        self.lib.tqo_lloyd_max_gaussian(M, max_iter, tol, _p(lv), _p(th))
        return lv, th


_ORACLE: Oracle | None = None


def load() -> Oracle:
    """Process-wide oracle instance (builds nothing; see oracle/build_oracle.sh)."""
    global _ORACLE
    if _ORACLE is None:
        _ORACLE = Oracle()
    return _ORACLE
