"""Disk-load latency of one packed KV layer: the counterpart of the reference
harness's ``simulate_disk_load_us`` (tq_backend/ttft_sim.py:90-147), same
arguments.

The layer is packed once (seeded synthetic K/V of the requested shape, slots
0..N-1 as the reference's store writes them) and written as the raw page pool
``<store_dir>/_ttft_sim_<scheme>_<num_tokens>.bin`` (the reference's file
name and contents: the pool bytes, no footer); a file already there is
reused.  The result is the mean wall time of ``iters`` loads after ``warmup``
loads, in microseconds; the page cache usually holds the file after the first
read, as in the reference's measurement.  Two load paths:

- ``mode="pinned"`` (default, this build's path): the file's pool bytes are
  read straight into a pinned host buffer (``readinto``, no intermediate
  bytes object) and copied to the GPU with one asynchronous copy.  Faster
  than the reference's path, so its figure is not the reference's.
- ``mode="reference"``: the reference's steps (ttft_sim.py:134-138), timed
  the same way: the whole file read into a bytes object, the pool bytes
  copied into a bytearray, wrapped as a tensor and cloned, then a pageable
  host-to-device copy.  Its figure is the one comparable with the
  reference's.
"""
from __future__ import annotations

import time
from pathlib import Path

import torch

from turborag_amd.synthetic import kv_tokens_major
from turborag_amd.turboquant_wrapper import TurboQuantWrapper


def sim_pool_path(store_dir: str | Path, scheme: str, num_tokens: int) -> Path:
    return Path(store_dir) / f"_ttft_sim_{scheme}_{num_tokens}.bin"


def simulate_disk_load_us(tq: TurboQuantWrapper, scheme: str, num_tokens: int,
                          num_kv_heads: int, head_dim: int, store_dir: str | Path,
                          warmup: int = 3, iters: int = 20, mode: str = "pinned") -> float:
    """Mean µs to load one packed layer from its file into device memory
    (0.0 for a scheme without pages, as the reference returns); ``mode`` as
    in the module docstring."""
    if mode not in ("pinned", "reference"):
        raise ValueError(f"mode must be 'pinned' or 'reference', not {mode!r}")
    if scheme not in ("turbo_prod", "turbo_mse"):
        return 0.0
    cfg = tq.default_config()
    cfg.num_kv_heads, cfg.head_dim = num_kv_heads, head_dim
    prod = scheme == "turbo_prod"
    layout = tq.make_layout_for(cfg) if prod else tq.make_mse_layout_for(cfg)
    pool_bytes = (tq.quant_bytes if prod else tq.mse_bytes)(num_tokens, layout, cfg)
    path = sim_pool_path(store_dir, scheme, num_tokens)
    dev = torch.device("cuda")
    if not path.exists():
        k, v = kv_tokens_major(num_tokens, num_kv_heads, head_dim, seed=700)
        slots = torch.arange(num_tokens, dtype=torch.int32, device=dev)
        pool = torch.zeros(pool_bytes, dtype=torch.uint8, device=dev)
        (tq.pack if prod else tq.mse_pack)(k.to(dev), v.to(dev), slots, pool, layout, cfg)
        torch.cuda.synchronize()
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_bytes(pool.cpu().numpy().tobytes())

    if mode == "reference":
        def load() -> None:
            raw = path.read_bytes()
            pages = torch.frombuffer(bytearray(raw[:pool_bytes]), dtype=torch.uint8).clone()
            pages.to(dev, non_blocking=True)
            torch.cuda.synchronize()
    else:
        load = _pinned_loader(path, pool_bytes, dev)

    for _ in range(warmup):
        load()
    t0 = time.perf_counter()
    for _ in range(iters):
        load()
    return (time.perf_counter() - t0) / max(iters, 1) * 1e6


def _pinned_loader(path: Path, pool_bytes: int, dev):
    """One load of the pool bytes: file -> pinned host buffer -> device."""
    host = torch.empty(pool_bytes, dtype=torch.uint8, pin_memory=True)
    view = memoryview(host.numpy())
    dst = torch.empty(pool_bytes, dtype=torch.uint8, device=dev)

    def load() -> None:
        got = 0
        with path.open("rb", buffering=0) as f:
            while got < pool_bytes:
                n = f.readinto(view[got:])
                if not n:
                    raise ValueError(f"{path}: {got} bytes, expected {pool_bytes}")
                got += n
        dst.copy_(host, non_blocking=True)
        torch.cuda.synchronize()

    return load
