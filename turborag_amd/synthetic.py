"""Seeded synthetic Qwen2.5-3B-shaped inputs: one host generator for the
oracle, the GPU tests and the bench, independent of the torch build.

* PRNG: splitmix64 (Steele, Lea and Flood, "Fast splittable pseudorandom
  number generators", OOPSLA 2014; the constants of Vigna's public-domain
  splitmix64.c).  Draw i of a stream with seed s is mix(s + (i + 1) * gamma),
  so any slice of a stream is computed directly (vectorised, in chunks on
  several threads).
* Uniforms: the top 53 bits of a draw, u = (x >> 11) * 2^-53 in [0, 1); the
  Box-Muller radius uses 1 - u in (0, 1].
* Normals: Box-Muller in fp64 on consecutive draw pairs (u1, u2):
  sqrt(-2 ln(1 - u1)) * (cos 2 pi u2, sin 2 pi u2), in that order.
* K and V of one seed: K's normals in the HF layout [H, N, D] row-major,
  then V's from the same stream; x8 on each head's outlier channels in fp64,
  one round-to-nearest-even to fp16, then permuted to the ABI's [N, H, D].
* Outlier channels of kv head h: the first 4 entries of a Fisher-Yates
  shuffle of 0..D-1 with seed 7000 + h (the same for K and V, every token
  and layer).  Fisher-Yates step i (from n - 1 down to 1) swaps entry i
  with entry floor(u * (i + 1)) of the next uniform u.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

OUTLIER_CHANNELS = 4
OUTLIER_SCALE = 8.0

_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 20


def splitmix64(seed: int, start: int, n: int) -> np.ndarray:
    """Draws start .. start + n - 1 of the splitmix64 stream of `seed`."""
    with np.errstate(over="ignore"):
        z = (np.arange(start + 1, start + n + 1, dtype=np.uint64) * _GAMMA
             + np.uint64(seed & 0xFFFFFFFFFFFFFFFF))
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform53(seed: int, start: int, n: int) -> np.ndarray:
    """fp64 uniforms in [0, 1) from draws start .. start + n - 1."""
    return (splitmix64(seed, start, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def _normals_chunk(seed: int, start: int, n: int) -> np.ndarray:
    # start and n even: pairs (u1, u2) at draws (start + 2j, start + 2j + 1)
    u = uniform53(seed, start, n).reshape(-1, 2)
    r = np.sqrt(-2.0 * np.log1p(-u[:, 0]))
    t = 2.0 * np.pi * u[:, 1]
    out = np.empty((n // 2, 2), np.float64)
    out[:, 0] = r * np.cos(t)
    out[:, 1] = r * np.sin(t)
    return out.reshape(-1)


def normals(seed: int, n: int, start: int = 0) -> np.ndarray:
    """n standard normals (fp64) from draw `start` (even) of the stream."""
    if start % 2:
        raise ValueError("normals start at an even draw")
    m = n + (n & 1)
    if m <= _CHUNK:
        return _normals_chunk(seed, start, m)[:n]
    out = np.empty(m, np.float64)
    bounds = list(range(0, m, _CHUNK)) + [m]

    def job(i):
        a, b = bounds[i], bounds[i + 1]
        out[a:b] = _normals_chunk(seed, start + a, b - a)
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(job, range(len(bounds) - 1)))
    return out[:n]


def fisher_yates(n: int, seed: int) -> np.ndarray:
    """A permutation of 0..n-1 (int64): step i = n-1 .. 1 swaps entries i and
    floor(u_i * (i + 1)), u_i the stream's uniforms in order."""
    p = np.arange(n, dtype=np.int64)
    if n < 2:
        return p
    u = uniform53(seed, 0, n - 1)
    js = np.floor(u * np.arange(n, 1, -1, dtype=np.float64)).astype(np.int64)
    for k, i in enumerate(range(n - 1, 0, -1)):
        j = js[k]
        p[i], p[j] = p[j], p[i]
    return p


def uniform_ints(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform on [lo, hi] (inclusive): lo + floor(u * (hi - lo + 1))."""
    u = uniform53(seed, 0, n)
    return (lo + np.floor(u * (hi - lo + 1))).astype(np.int64)


def outlier_channels(num_kv_heads: int, head_dim: int) -> list[list[int]]:
    return [sorted(fisher_yates(head_dim, 7000 + h)[:OUTLIER_CHANNELS].tolist())
            for h in range(num_kv_heads)]


def _rne_fp16(x: np.ndarray) -> np.ndarray:
    """fp64 -> fp16, one round-to-nearest-even (numpy converts doubles to
    halves directly)."""
    return x.astype(np.float16)


def kv_heads_major(num_tokens: int, num_kv_heads: int = 2, head_dim: int = 128,
                   seed: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """K, V as fp16 numpy [H, N, D] (the HF layout the stream is drawn in)."""
    n = num_kv_heads * num_tokens * head_dim
    z = normals(seed, 2 * n)
    k = z[:n].reshape(num_kv_heads, num_tokens, head_dim)
    v = z[n:].reshape(num_kv_heads, num_tokens, head_dim)
    for h, chans in enumerate(outlier_channels(num_kv_heads, head_dim)):
        k[h][:, chans] *= OUTLIER_SCALE
        v[h][:, chans] *= OUTLIER_SCALE
    return _rne_fp16(k), _rne_fp16(v)


def kv_tokens_major(num_tokens: int, num_kv_heads: int = 2, head_dim: int = 128,
                    seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """K, V as fp16 torch [num_tokens, H, D] (the ABI's layout), on the CPU."""
    k, v = kv_heads_major(num_tokens, num_kv_heads, head_dim, seed)
    return (torch.from_numpy(np.ascontiguousarray(k.transpose(1, 0, 2))),
            torch.from_numpy(np.ascontiguousarray(v.transpose(1, 0, 2))))


def query(num_q_heads: int = 16, head_dim: int = 128, seed: int = 400) -> torch.Tensor:
    """fp16 query [num_q_heads, D] drawn N(0, 1)."""
    z = normals(seed, num_q_heads * head_dim).reshape(num_q_heads, head_dim)
    return torch.from_numpy(_rne_fp16(z))


def gqa_rows(q: torch.Tensor, num_kv_heads: int) -> torch.Tensor:
    """[Hq, D] -> the ABI's [Hq/Hkv, Hkv, D]: row g of kv head h is q head
    h*(Hq/Hkv) + g (q head j attends kv head j // (Hq/Hkv))."""
    hq, d = q.shape
    groups = hq // num_kv_heads
    return q.view(num_kv_heads, groups, d).permute(1, 0, 2).contiguous()


def permuted_slots(num_tokens: int, block_size: int = 16, seed: int = 401,
                   num_pages: int | None = None) -> torch.Tensor:
    """slot[t] = perm[t // B] * B + t % B for a Fisher-Yates permutation of
    the pages (seed)."""
    pages_needed = (num_tokens + block_size - 1) // block_size
    num_pages = num_pages or pages_needed
    perm = fisher_yates(num_pages, seed)[:pages_needed]
    t = np.arange(num_tokens)
    return torch.from_numpy((perm[t // block_size] * block_size + t % block_size)
                            .astype(np.int32))


def as_u16(t: torch.Tensor) -> np.ndarray:
    """fp16 torch tensor -> numpy uint16 bit patterns (host)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
