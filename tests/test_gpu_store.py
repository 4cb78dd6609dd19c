"""CAGStore on the GPU: pack_document / load_document / load_as_kv_fp16 /
build_dynamic_cache through the C++ store entries and the layer-pipelined
loader, against the CPU oracle: pools equal oracle.prod_pack / mse_pack
byte for byte, loaded K/V equal oracle.prod_dequant / mse_dequant bit for
bit, attention within 1e-3 of the fp64 oracle.  Includes a store written the
way the reference writes it (raw .bin without footer, torch.save .meta, json
manifest), which must load unchanged."""
from __future__ import annotations

import hashlib
import json
import time

import numpy as np
import pytest
import torch

from turborag_amd.cag_store import CAGStore
from turborag_amd.synthetic import as_u16, kv_tokens_major

pytestmark = pytest.mark.gpu


def _layer_kv(layer, N, H, D, cuda):
    k, v = kv_tokens_major(N, H, D, seed=600 + layer)
    return k.to(cuda), v.to(cuda)


def _cache_kv(cache, layer):
    if hasattr(cache, "layers"):
        return cache.layers[layer].keys, cache.layers[layer].values
    return cache.key_cache[layer], cache.value_cache[layer]


def _dequant(oracle, scheme, pool, N, H, D):
    """The oracle's dequant of a pool with slots arange(N) (what the store's
    .meta holds), as fp16 bit patterns [N, H, D]."""
    slots = np.arange(N, dtype=np.int32)
    fn = oracle.prod_dequant if scheme == "turbo_prod" else oracle.mse_dequant
    return fn(pool.cpu().numpy(), slots, H, D, 16)


def _pack(tq, oracle, scheme, k, v, cuda):
    """The library's pack into a fresh pool (slots arange(N)), checked
    against the oracle's pack of the same K/V byte for byte."""
    N, H, D = k.shape
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    if scheme == "turbo_prod":
        lay = tq.make_layout_for(cfg)
        pool = tq.alloc_page_pool(N, lay, cfg)
        tq.pack(k, v, slots, pool, lay, cfg)
        want = oracle.prod_pack(as_u16(k), as_u16(v), slots.cpu().numpy(), (N + 15) // 16, 16)
    else:
        lay = tq.make_mse_layout_for(cfg)
        pool = tq.alloc_mse_pool(N, lay, cfg)
        tq.mse_pack(k, v, slots, pool, lay, cfg)
        want = oracle.mse_pack(as_u16(k), as_u16(v), slots.cpu().numpy(), (N + 15) // 16, 16)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), want)
    return pool


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("N,H,D", [(1000, 2, 128), (77, 4, 64)])
def test_store_roundtrip_and_dynamic_cache(tq, oracle, cuda, tmp_path, scheme, N, H, D):
    print(f"[store {scheme}] N={N} H={H} D={D}", flush=True)
    st = CAGStore(tmp_path, tq=tq)
    layers = 3
    pools = []
    for l in range(layers):
        k, v = _layer_kv(l, N, H, D, cuda)
        n = st.pack_document("doc", l, k, v, scheme)
        pools.append(_pack(tq, oracle, scheme, k, v, cuda))
        assert n == pools[-1].numel() + 64  # pages + footer
    torch.cuda.synchronize()
    for l in range(layers):
        pool, slots, n = st.load_document("doc", l, scheme, (H, D))
        assert n == N and torch.equal(slots.cpu(), torch.arange(N, dtype=torch.int32))
        assert torch.equal(pool.cpu(), pools[l].cpu())
        ok, ov = st.load_as_kv_fp16("doc", l, scheme, (H, D))
        rk, rv = _dequant(oracle, scheme, pools[l], N, H, D)
        assert np.array_equal(as_u16(ok), rk) and np.array_equal(as_u16(ov), rv)
    cache, doc_len = st.build_dynamic_cache("doc", layers + 2, scheme, (H, D))
    assert doc_len == N
    for l in range(layers):
        ck, cv = _cache_kv(cache, l)
        rk, rv = _dequant(oracle, scheme, pools[l], N, H, D)
        assert ck.shape == (1, H, N, D)
        assert np.array_equal(as_u16(ck[0]), rk.transpose(1, 0, 2))
        assert np.array_equal(as_u16(cv[0]), rv.transpose(1, 0, 2))


def test_reference_written_store_loads(tq, oracle, cuda, tmp_path):
    """Files exactly as cag_store.py:140-152 writes them: raw pool bytes,
    torch.save meta, manifest via json.dumps(indent=2)."""
    N, H, D, scheme = 500, 2, 128, "turbo_prod"
    h = hashlib.sha256(b"ref doc").hexdigest()
    manifest = {"v": 1, "entries": {"ref doc": {"sha256": h, "layers": {}}}}
    pools = []
    for l in range(2):
        k, v = _layer_kv(10 + l, N, H, D, cuda)
        pool = _pack(tq, oracle, scheme, k, v, cuda)
        pools.append(pool)
        key = f"{h[:16]}_L{l:02d}_{scheme}"
        (tmp_path / f"{key}.bin").write_bytes(pool.cpu().numpy().tobytes())
        torch.save({"num_tokens": N, "slots": torch.arange(N, dtype=torch.int32)},
                   tmp_path / f"{key}.meta")
        manifest["entries"]["ref doc"]["layers"][f"{l}::{scheme}"] = {
            "key": key, "num_tokens": N, "stored_at": time.time()}
    (tmp_path / "manifest.json").write_text(json.dumps(manifest, indent=2))
    st = CAGStore(tmp_path, tq=tq)
    cache, doc_len = st.build_dynamic_cache("ref doc", 2, scheme, (H, D))
    assert doc_len == N
    for l in range(2):
        ck, cv = _cache_kv(cache, l)
        rk, rv = _dequant(oracle, scheme, pools[l], N, H, D)
        assert np.array_equal(as_u16(ck[0]), rk.transpose(1, 0, 2))
        assert np.array_equal(as_u16(cv[0]), rv.transpose(1, 0, 2))


def test_fp16_scheme_roundtrip(tq, cuda, tmp_path):
    N, H, D = 123, 2, 64
    st = CAGStore(tmp_path, tq=tq)
    k, v = _layer_kv(20, N, H, D, cuda)
    st.pack_document("f", 0, k, v, "fp16")
    (gk, gv), slots, n = st.load_document("f", 0, "fp16", (H, D))
    assert n == N and torch.equal(gk, k) and torch.equal(gv, v)
    cache, doc_len = st.build_dynamic_cache("f", 1, "fp16", (H, D))
    ck, _ = _cache_kv(cache, 0)
    assert doc_len == N and torch.equal(ck[0], k.permute(1, 0, 2))


def test_fused_attention_from_store(tq, oracle, cuda, tmp_path):
    """CAGStore.fused_attention (one query row, cag_store.py:284-287) over a
    stored document, against the fp64 oracle over the stored pages."""
    N, H, D = 900, 2, 128
    st = CAGStore(tmp_path, tq=tq)
    k, v = _layer_kv(30, N, H, D, cuda)
    st.pack_document("a", 0, k, v, "turbo_prod")
    pool, slots, n = st.load_document("a", 0, "turbo_prod", (H, D))
    assert np.array_equal(pool.cpu().numpy(), oracle.prod_pack(
        as_u16(k), as_u16(v), np.arange(N, dtype=np.int32), (N + 15) // 16, 16))
    q = torch.randn(1, H, D, generator=torch.Generator().manual_seed(3)).half().to(cuda)
    out = st.fused_attention(q, pool, slots, n, "turbo_prod", (H, D))
    torch.cuda.synchronize()
    ref = oracle.prod_attention_f64(as_u16(q), pool.cpu().numpy(), slots.cpu().numpy(), 16)
    got = out.cpu().double().numpy().reshape(ref.shape)
    err = float((np.abs(got - ref).max(axis=-1) / np.abs(ref).max(axis=-1)).max())
    assert err < 1e-3
