"""The synthetic-input generator (turborag_amd/synthetic.py).

* splitmix64 against the published known answers of its reference C code
  (seed 1234567: the first five outputs).
* Box-Muller: every output pair satisfies z0^2 + z1^2 = -2 ln(1 - u1) and
  atan2(z1, z0) = 2 pi u2 (mod 2 pi) for the stream's own uniforms, so a
  swapped pair, a dropped factor or a wrong uniform fails.
* Fisher-Yates: a permutation, equal to the textbook loop written with the
  same uniforms.
* The workload tensors: layout ([H, N, D] drawn, [N, H, D] returned), the
  outlier channels scaled by exactly 8 before one fp16 rounding, and the
  SHA-256 of each spec input recorded in tests/golden/synthetic_sha256.json
  (machine-independent: no torch generator is involved).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import torch

from turborag_amd import synthetic as syn

GOLDEN = Path(__file__).resolve().parent / "golden" / "synthetic_sha256.json"


def test_splitmix64_known_answers():
    got = [int(x) for x in syn.splitmix64(1234567, 0, 5)]
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]
    # any slice of the stream is the same draws
    assert np.array_equal(syn.splitmix64(1234567, 3, 2), syn.splitmix64(1234567, 0, 5)[3:])


def test_uniforms_are_the_top_53_bits():
    x = syn.splitmix64(9, 0, 1000)
    u = syn.uniform53(9, 0, 1000)
    assert np.array_equal(u * 2.0 ** 53, (x >> np.uint64(11)).astype(np.float64))
    assert u.min() >= 0.0 and u.max() < 1.0


def test_box_muller_identities():
    n = 4096
    z = syn.normals(77, n).reshape(-1, 2)
    u = syn.uniform53(77, 0, n).reshape(-1, 2)
    r2 = -2.0 * np.log1p(-u[:, 0])
    np.testing.assert_allclose(z[:, 0] ** 2 + z[:, 1] ** 2, r2, rtol=1e-12, atol=1e-12)
    ang = np.mod(np.arctan2(z[:, 1], z[:, 0]), 2 * np.pi)
    want = np.mod(2 * np.pi * u[:, 1], 2 * np.pi)
    d = np.abs(ang - want)
    assert np.all(np.minimum(d, 2 * np.pi - d) < 1e-9)
    # chunked (threaded) generation equals one pass, and an odd count is a prefix
    big = syn.normals(5, 3 * syn._CHUNK + 6)
    assert np.array_equal(big[:1000], syn.normals(5, 1000))
    assert np.array_equal(big[2 * syn._CHUNK:2 * syn._CHUNK + 10],
                          syn.normals(5, 10, start=2 * syn._CHUNK))
    assert np.array_equal(syn.normals(5, 7), big[:7])


def test_normal_moments():
    z = syn.normals(123, 1 << 20)
    assert abs(z.mean()) < 5e-3 and abs(z.var() - 1.0) < 5e-3
    assert abs(np.mean(z ** 4) - 3.0) < 0.03


def test_fisher_yates_is_the_textbook_loop():
    for n, seed in ((1, 3), (2, 4), (10, 5), (2048, 401)):
        p = syn.fisher_yates(n, seed)
        assert sorted(p.tolist()) == list(range(n))
        want = list(range(n))
        u = syn.uniform53(seed, 0, max(n - 1, 0))
        for k, i in enumerate(range(n - 1, 0, -1)):
            j = int(u[k] * (i + 1))
            want[i], want[j] = want[j], want[i]
        assert p.tolist() == want


def test_uniform_ints_range():
    x = syn.uniform_ints(500, 10000, 1, 8)
    assert x.min() == 1 and x.max() == 8
    assert set(np.bincount(x)[1:] > 1000) == {True}


def test_kv_layout_and_outliers():
    N, H, D = 37, 2, 128
    k, v = syn.kv_tokens_major(N, H, D, seed=900)
    kh, vh = syn.kv_heads_major(N, H, D, seed=900)
    assert k.shape == (N, H, D) and k.dtype == torch.float16
    assert np.array_equal(k.numpy(), kh.transpose(1, 0, 2))
    assert np.array_equal(v.numpy(), vh.transpose(1, 0, 2))
    # K's normals first ([H, N, D] row-major), then V's; outliers x8 before rounding
    z = syn.normals(900, 2 * H * N * D)
    zk = z[:H * N * D].reshape(H, N, D)
    zv = z[H * N * D:].reshape(H, N, D)
    for h, chans in enumerate(syn.outlier_channels(H, D)):
        assert chans == sorted(syn.fisher_yates(D, 7000 + h)[:4].tolist())
        scale = np.ones(D)
        scale[chans] = 8.0
        assert np.array_equal(kh[h], (zk[h] * scale).astype(np.float16))
        assert np.array_equal(vh[h], (zv[h] * scale).astype(np.float16))


def test_slots_are_a_page_permutation():
    s = syn.permuted_slots(100, 16, seed=401, num_pages=9).numpy()
    pages = s.reshape(-1)[::16] // 16
    assert len(set(pages.tolist())) == len(pages) == 7
    assert np.array_equal(s % 16, np.arange(100) % 16)


def _sha(a) -> str:
    if isinstance(a, torch.Tensor):
        a = a.numpy()
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def spec_inputs() -> dict:
    """The spec's inputs whose SHA-256 the golden file records."""
    k, v = syn.kv_tokens_major(37, 2, 128, seed=900)
    k4, v4 = syn.kv_tokens_major(32768, 2, 128, seed=300)
    return {
        "kv_37x2x128_seed900_key": k, "kv_37x2x128_seed900_value": v,
        "kv_32768x2x128_seed300_key": k4, "kv_32768x2x128_seed300_value": v4,
        "query_16x128_seed400": syn.query(16, 128, seed=400),
        "slots_32768_b16_seed401": syn.permuted_slots(32768, 16, seed=401),
        "lens_seed500": syn.uniform_ints(500, 32, 1024, 32768),
        "widths_seed501": syn.uniform_ints(501, 32, 1, 8),
    }


def test_spec_inputs_match_recorded_sha256():
    want = json.loads(GOLDEN.read_text())
    got = {name: _sha(a) for name, a in spec_inputs().items()}
    assert got == want
