"""The disk-load latency harness (turborag_amd/ttft.py, the counterpart of
tq_backend/ttft_sim.py:90-147): the layer file it writes is the oracle's pack
of the same seeded tokens into slots 0..N-1, it is reused on the next call
(by the pinned path and by the reference's load steps), and a scheme without
pages gives 0."""
from __future__ import annotations

import numpy as np
import pytest

from turborag_amd.synthetic import as_u16, kv_tokens_major
from turborag_amd.ttft import sim_pool_path, simulate_disk_load_us

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("scheme", ["turbo_prod", "turbo_mse"])
def test_disk_load_file_and_timing(tq, oracle, cuda, tmp_path, scheme):
    N, H, D = 3000, 2, 128
    us = simulate_disk_load_us(tq, scheme, N, H, D, tmp_path, warmup=1, iters=3)
    assert us > 0.0
    path = sim_pool_path(tmp_path, scheme, N)
    k, v = kv_tokens_major(N, H, D, seed=700)
    pages = (N + 15) // 16
    pack = oracle.prod_pack if scheme == "turbo_prod" else oracle.mse_pack
    want = pack(as_u16(k), as_u16(v), np.arange(N, dtype=np.int32), pages, 16)
    got = np.frombuffer(path.read_bytes(), dtype=np.uint8)
    assert got.size == want.size and np.array_equal(got, want)
    mtime = path.stat().st_mtime_ns
    assert simulate_disk_load_us(tq, scheme, N, H, D, tmp_path, warmup=0, iters=1) > 0.0
    assert path.stat().st_mtime_ns == mtime  # reused, not rewritten
    # the reference's load steps on the same file (its figure, comparable
    # with the reference harness's)
    assert simulate_disk_load_us(tq, scheme, N, H, D, tmp_path, warmup=0, iters=2,
                                 mode="reference") > 0.0
    assert path.stat().st_mtime_ns == mtime
    with pytest.raises(ValueError):
        simulate_disk_load_us(tq, scheme, N, H, D, tmp_path, mode="mmap")
    assert simulate_disk_load_us(tq, "fp16", N, H, D, tmp_path) == 0.0
