"""CAGStore on the GPU: pack_document / load_document / load_as_kv_fp16 /
build_dynamic_cache through the C++ store entries and the layer-pipelined
loader, against the library's own pack and dequant (bit-exact against the
oracle in test_gpu_parity.py).  Includes a store written the way the
reference writes it (raw .bin without footer, torch.save .meta, json
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


def _dequant(tq, scheme, pool, N, H, D, cuda):
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    ok = torch.zeros(N, H, D, dtype=torch.float16, device=cuda)
    ov = torch.zeros_like(ok)
    if scheme == "turbo_prod":
        tq.dequant(pool, slots, ok, ov, tq.make_layout_for(cfg), cfg)
    else:
        tq.mse_dequant(pool, slots, ok, ov, tq.make_mse_layout_for(cfg), cfg)
    return ok, ov


def _pack(tq, scheme, k, v, cuda):
    N, H, D = k.shape
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    slots = torch.arange(N, dtype=torch.int32, device=cuda)
    if scheme == "turbo_prod":
        lay = tq.make_layout_for(cfg)
        pool = tq.alloc_page_pool(N, lay, cfg)
        tq.pack(k, v, slots, pool, lay, cfg)
    else:
        lay = tq.make_mse_layout_for(cfg)
        pool = tq.alloc_mse_pool(N, lay, cfg)
        tq.mse_pack(k, v, slots, pool, lay, cfg)
    return pool


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
@pytest.mark.parametrize("N,H,D", [(1000, 2, 128), (77, 4, 64)])
def test_store_roundtrip_and_dynamic_cache(tq, cuda, tmp_path, scheme, N, H, D):
    print(f"[store {scheme}] N={N} H={H} D={D}", flush=True)
    st = CAGStore(tmp_path, tq=tq)
    layers = 3
    pools = []
    for l in range(layers):
        k, v = _layer_kv(l, N, H, D, cuda)
        n = st.pack_document("doc", l, k, v, scheme)
        pools.append(_pack(tq, scheme, k, v, cuda))
        assert n == pools[-1].numel() + 64  # pages + footer
    torch.cuda.synchronize()
    for l in range(layers):
        pool, slots, n = st.load_document("doc", l, scheme, (H, D))
        assert n == N and torch.equal(slots.cpu(), torch.arange(N, dtype=torch.int32))
        assert torch.equal(pool.cpu(), pools[l].cpu())
        ok, ov = st.load_as_kv_fp16("doc", l, scheme, (H, D))
        rk, rv = _dequant(tq, scheme, pools[l], N, H, D, cuda)
        assert np.array_equal(as_u16(ok), as_u16(rk)) and np.array_equal(as_u16(ov), as_u16(rv))
    cache, doc_len = st.build_dynamic_cache("doc", layers + 2, scheme, (H, D))
    assert doc_len == N
    for l in range(layers):
        ck, cv = _cache_kv(cache, l)
        rk, rv = _dequant(tq, scheme, pools[l], N, H, D, cuda)
        assert ck.shape == (1, H, N, D)
        assert np.array_equal(as_u16(ck[0]), as_u16(rk.permute(1, 0, 2)))
        assert np.array_equal(as_u16(cv[0]), as_u16(rv.permute(1, 0, 2)))


def test_reference_written_store_loads(tq, cuda, tmp_path):
    """Files exactly as cag_store.py:140-152 writes them: raw pool bytes,
    torch.save meta, manifest via json.dumps(indent=2)."""
    N, H, D, scheme = 500, 2, 128, "turbo_prod"
    h = hashlib.sha256(b"ref doc").hexdigest()
    manifest = {"v": 1, "entries": {"ref doc": {"sha256": h, "layers": {}}}}
    pools = []
    for l in range(2):
        k, v = _layer_kv(10 + l, N, H, D, cuda)
        pool = _pack(tq, scheme, k, v, cuda)
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
        rk, rv = _dequant(tq, scheme, pools[l], N, H, D, cuda)
        assert np.array_equal(as_u16(ck[0]), as_u16(rk.permute(1, 0, 2)))
        assert np.array_equal(as_u16(cv[0]), as_u16(rv.permute(1, 0, 2)))


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


def test_fused_attention_from_store(tq, cuda, tmp_path):
    N, H, D = 900, 2, 128
    st = CAGStore(tmp_path, tq=tq)
    k, v = _layer_kv(30, N, H, D, cuda)
    st.pack_document("a", 0, k, v, "turbo_prod")
    pool, slots, n = st.load_document("a", 0, "turbo_prod", (H, D))
    q = torch.randn(1, H, D, generator=torch.Generator().manual_seed(3)).half().to(cuda)
    out = st.fused_attention(q, pool, slots, n, "turbo_prod", (H, D))
    ref = torch.zeros_like(q)
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = H, D
    tq.fused_attn_output(q, pool, slots, ref, tq.make_layout_for(cfg), cfg, 1, n)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
