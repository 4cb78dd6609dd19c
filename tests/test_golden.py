"""Committed golden fixtures (tests/golden/, written by make_fixtures.py).

Reference-produced data pins the oracle and the library without the reference
tree: the reference's own Lloyd-Max program output (src/gaussian_codebook.cpp)
and its turbo_mse layout factory (src/tq_turbo_mse_layout.cpp:7-28) over 144
configs.  The seeded oracle fixtures pin the oracle against regressions (CPU)
and are the fixed expected values of the GPU tests (bit-exact codes, scales
and dequantized halves; attention within 1e-3 of the fp64 result).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
K3_LITERALS = [-2.1513, -1.34326, -0.755526, -0.244919, 0.244919, 0.755526, 1.34326, 2.1513]
B, H, D = 16, 2, 128


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_reference_codebook_program_output(oracle):
    """The reference program's printed levels are the K3 literals, and this
    build's restatement of its Lloyd-Max design reproduces levels and
    thresholds."""
    text = (GOLDEN / "ref_gaussian_codebook.txt").read_text()
    levels = [float(x) for x in text.split("levels:")[1].split("thresholds:")[0].split()]
    thresholds = [float(x) for x in text.split("thresholds:")[1].split()]
    assert levels == K3_LITERALS
    assert np.array_equal(oracle.k3.astype(np.float32), np.float32(K3_LITERALS))
    mine_levels, mine_thr = oracle.lloyd_max(8)
    assert np.allclose(mine_levels, levels, atol=5e-6)
    assert np.allclose(mine_thr, thresholds, atol=5e-6)


def test_reference_mse_layouts(oracle, tq):
    """144 configs of the reference's turbo_mse layout factory: the oracle
    and the library's tq_make_turbo_mse_layout agree field for field."""
    from turborag_amd.turboquant_wrapper import TQConfig
    n = 0
    for line in (GOLDEN / "ref_layouts.txt").read_text().strip().splitlines():
        head, mse, _legacy = line.split("|")
        b, h, d, nbits, al = map(int, head.split())
        ref = list(map(int, mse.split()))
        L = oracle.mse_layout(b, h, d, nbits, al)
        assert [L.code_bytes, L.norm_bytes, L.k_codes_off, L.v_codes_off, L.k_norms_off,
                L.v_norms_off, L.page_size] == ref, line
        cfg = TQConfig(b, h, d, nbits, d, al, 0, 0)
        M = tq.make_mse_layout_for(cfg)
        assert [M.code_bytes_per_token_head, M.norm_bytes_per_token_head, M.k_codes_offset,
                M.v_codes_offset, M.k_norms_offset, M.v_norms_offset,
                M.page_size_bytes] == ref, line
        n += 1
    assert n == 144


def test_oracle_reproduces_prod_fixture(oracle):
    f = _load("prod_n37_h2_d128.npz")
    pool = oracle.prod_pack(f["key"], f["value"], f["slots"], f["pool"].size // 4288, B)
    assert np.array_equal(pool, f["pool"])
    dk, dv = oracle.prod_dequant(pool, f["slots"], H, D, B)
    assert np.array_equal(dk, f["dequant_key"]) and np.array_equal(dv, f["dequant_value"])
    assert np.array_equal(oracle.prod_logits(f["query"], pool, f["slots"], B), f["logits"])
    assert np.array_equal(oracle.prod_attention_f32(f["query"], pool, f["slots"], B),
                          f["attention_f32"])
    assert np.allclose(oracle.prod_attention_f64(f["query"], pool, f["slots"], B),
                       f["attention_f64"], rtol=0, atol=1e-12)


def test_oracle_reproduces_mse_fixture(oracle):
    f = _load("mse_n37_h2_d128.npz")
    pool = oracle.mse_pack(f["key"], f["value"], f["slots"], f["pool"].size // 4608, B)
    assert np.array_equal(pool, f["pool"])
    dk, dv = oracle.mse_dequant(pool, f["slots"], H, D, B)
    assert np.array_equal(dk, f["dequant_key"]) and np.array_equal(dv, f["dequant_value"])
    assert np.array_equal(oracle.mse_attention_f32(f["query"], pool, f["slots"], B),
                          f["attention_f32"])
    assert np.allclose(oracle.mse_attention_f64(f["query"], pool, f["slots"], B),
                       f["attention_f64"], rtol=0, atol=1e-12)


def _t16(a, dev):
    import torch
    return torch.from_numpy(a.view(np.int16)).view(torch.float16).to(dev)


def _rel_err(got, ref):
    g = got.reshape(-1, got.shape[-1]).astype(np.float64)
    r = ref.reshape(-1, ref.shape[-1]).astype(np.float64)
    return float((np.abs(g - r).max(axis=1) / np.maximum(np.abs(r).max(axis=1), 1e-30)).max())


@pytest.mark.gpu
@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_gpu_matches_fixture(tq, cuda, scheme):
    import torch

    from turborag_amd.synthetic import as_u16
    print(f"[golden {scheme}]", flush=True)
    f = _load("prod_n37_h2_d128.npz" if scheme == "turbo_prod" else "mse_n37_h2_d128.npz")
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim, cfg.block_size = H, D, B
    prod = scheme == "turbo_prod"
    layout = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    slots = torch.from_numpy(f["slots"]).to(cuda)
    N = f["slots"].size
    pool = torch.zeros(f["pool"].size, dtype=torch.uint8, device=cuda)
    (tq.pack if prod else tq.mse_pack)(_t16(f["key"], cuda), _t16(f["value"], cuda), slots,
                                       pool, layout, cfg)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    (tq.dequant if prod else tq.mse_dequant)(pool, slots, ok, ov, layout, cfg)
    out = torch.zeros(8, H, D, dtype=torch.float16, device=cuda)
    (tq.fused_attn_output if prod else tq.mse_fused_attn_output)(
        _t16(f["query"], cuda), pool, slots, out, layout, cfg, 8, N)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), f["pool"])
    assert np.array_equal(as_u16(ok), f["dequant_key"])
    assert np.array_equal(as_u16(ov), f["dequant_value"])
    assert _rel_err(out.cpu().float().numpy(), f["attention_f64"]) < 1e-3
    if prod:
        logits = torch.zeros(8 * H * N, dtype=torch.float32, device=cuda)
        tq.fused_attn_logits(_t16(f["query"], cuda), pool, slots, logits, layout, cfg, 8, N)
        torch.cuda.synchronize()
        got = logits.cpu().numpy().reshape(8, H, N).astype(np.float64)
        ref = f["logits"].astype(np.float64)
        assert (np.abs(got - ref) / (np.abs(ref).max(axis=-1, keepdims=True) + 1e-30)).max() < 1e-5
