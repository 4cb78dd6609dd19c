"""Known-answer pages derived by hand from the reference's operation order
(src/cuda/tq_turbo_prod_kernels.cu:180-259, tq_turbo_mse_kernels.cu:65-136),
checked on the oracle (CPU) and on the GPU library.

All-zero K and V: every rotated value is 0, so rms = max(0, 1e-8) = 1e-8,
which rounds to fp16 0x0000.  kn = 0 is equidistant from K3[3] = -0.244919
and K3[4]; the strict '<' keeps index 3; e = 0 - K3[3] > 0 -> sign 1, nibble
0xB, byte 0xBB.  The residual RMS is |K3[3]| = 0.244919 -> fp16 0x33D6.  V:
0 ties between V4[7] and V4[8] -> index 7 -> byte 0x77.  turbo_mse: the same
tie -> code 7 -> byte 0x77, norm 0.

One-hot x = e_0 (value 1.0 at index 0): head 0 has s_0 = +1, the WHT of e_0
is all ones, so every rotated element is +inv = RN(1/sqrt(128)) and
rms = sqrt(RN(inv^2)) = inv exactly (sqrt of a correctly rounded square) ->
fp16(0.0883883) = 0x2DA8.  kn = 1.0 -> K3[5] = 0.755526 (distance 0.2445 vs
0.3433 for K3[6]) -> code 5, e > 0 -> nibble 0xD, byte 0xDD; residual
0.244474 -> 0x33D3.  V: 1.0 -> V4[11] = 0.9423 -> byte 0xBB.  Head 1: s_0 =
-1, every element -inv, kn = -1 -> code 2, e < 0 -> nibble 0x2 (byte 0x22);
V -> V4[4] = -0.9423 -> byte 0x44.  turbo_mse one-hot: x/rms = +-1 -> codes
11 / 4 (bytes 0xBB / 0x44), norm 0x2DA8.
"""
from __future__ import annotations

import numpy as np
import pytest

D, H, B = 128, 2, 16

PROD_ZERO = dict(k=0xBB, v=0x77, ks=0x0000, kres=0x33D6, vs=0x0000)
PROD_ONEHOT = {0: dict(k=0xDD, v=0xBB, ks=0x2DA8, kres=0x33D3, vs=0x2DA8),
               1: dict(k=0x22, v=0x44, ks=0x2DA8, kres=0x33D3, vs=0x2DA8)}
MSE_ZERO = dict(k=0x77, v=0x77, kn=0x0000, vn=0x0000)
MSE_ONEHOT = {0: dict(k=0xBB, v=0xBB, kn=0x2DA8, vn=0x2DA8),
              1: dict(k=0x44, v=0x44, kn=0x2DA8, vn=0x2DA8)}


def _inputs(kind: str) -> np.ndarray:
    x = np.zeros((B, H, D), np.float16)
    if kind == "onehot":
        x[:, :, 0] = 1.0
    return x.view(np.uint16)


def _check_prod_page(page: np.ndarray, kind: str) -> None:
    from oracle.oracle import load
    L = load().prod_layout(B, H, D)
    for tib in range(B):
        for h in range(H):
            want = PROD_ZERO if kind == "zero" else PROD_ONEHOT[h]
            c = tib * H + h
            assert np.all(page[L.k4_off + c * 64: L.k4_off + c * 64 + 64] == want["k"])
            assert np.all(page[L.v4_off + c * 64: L.v4_off + c * 64 + 64] == want["v"])
            for key, off in (("ks", L.ks_off), ("kres", L.kres_off), ("vs", L.vs_off)):
                got = int(page[off + 2 * c]) | (int(page[off + 2 * c + 1]) << 8)
                assert got == want[key], (kind, tib, h, key, hex(got))


def _check_mse_page(page: np.ndarray, kind: str) -> None:
    from oracle.oracle import load
    L = load().mse_layout(B, H, D)
    for tib in range(B):
        for h in range(H):
            want = MSE_ZERO if kind == "zero" else MSE_ONEHOT[h]
            c = tib * H + h
            assert np.all(page[L.k_codes_off + c * 64: L.k_codes_off + c * 64 + 64] == want["k"])
            assert np.all(page[L.v_codes_off + c * 64: L.v_codes_off + c * 64 + 64] == want["v"])
            for key, off in (("kn", L.k_norms_off), ("vn", L.v_norms_off)):
                got = int(page[off + 2 * c]) | (int(page[off + 2 * c + 1]) << 8)
                assert got == want[key], (kind, tib, h, key, hex(got))
    # padding bytes of the 256-aligned regions stay zero
    assert not page[L.k_norms_off + 64: L.v_norms_off].any()
    assert not page[L.v_norms_off + 64:].any()


@pytest.mark.parametrize("kind", ["zero", "onehot"])
def test_oracle_known_pages(oracle, kind):
    x = _inputs(kind)
    slots = np.arange(B, dtype=np.int32)
    _check_prod_page(oracle.prod_pack(x, x, slots, num_pages=1), kind)
    _check_mse_page(oracle.mse_pack(x, x, slots, num_pages=1), kind)


def test_oracle_known_dequant(oracle):
    """Dequant of the one-hot page: K = (K3[5] + re) * ks in every rotated
    position (head 0), so the inverse WHT concentrates it back on index 0."""
    x = _inputs("onehot")
    slots = np.arange(B, dtype=np.int32)
    pool = oracle.prod_pack(x, x, slots, num_pages=1)
    ok, ov = oracle.prod_dequant(pool, slots, H, D)
    k = ok.view(np.float16).astype(np.float64)
    # every row is a scaled e_0: entries 1..127 are exactly 0 (all-equal input
    # to the WHT), entry 0 = 128 * y * inv
    assert np.all(k[:, :, 1:] == 0.0)
    y = (np.float32(0.755526) + np.float32(np.float16(0.244474))) * np.float32(np.float16(0.0883883))
    assert np.allclose(k[:, 0, 0], 128 * float(y) * 0.08838834764831845, rtol=2e-3)
    assert np.all(ov.view(np.float16)[:, :, 1:].astype(np.float32) == 0.0)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["zero", "onehot"])
def test_gpu_known_pages(tq, cuda, kind):
    import torch
    x = torch.from_numpy(_inputs(kind).view(np.float16)).to(cuda)
    slots = torch.arange(B, dtype=torch.int32, device=cuda)
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    lp = tq.make_layout_for(cfg)
    pool = tq.alloc_page_pool(B, lp, cfg)
    tq.pack(x, x, slots, pool, lp, cfg)
    lm = tq.make_mse_layout_for(cfg)
    mpool = tq.alloc_mse_pool(B, lm, cfg)
    tq.mse_pack(x, x, slots, mpool, lm, cfg)
    torch.cuda.synchronize()
    _check_prod_page(pool.cpu().numpy(), kind)
    _check_mse_page(mpool.cpu().numpy(), kind)
