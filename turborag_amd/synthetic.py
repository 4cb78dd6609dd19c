"""Seeded synthetic Qwen2.5-3B-shaped KV (the workloads' input distribution).

K and V are drawn N(0, 1) per element; for each kv head h, 4 fixed outlier
channels (the first 4 of a seeded permutation of the head dim, seed 7000 + h)
are scaled by 8 — the same channels for K and V, every token and layer.  The
draw uses torch's CPU generator, so a (seed, shape) pair gives the same
halves on every machine with this torch build.
"""
from __future__ import annotations

import numpy as np
import torch

OUTLIER_CHANNELS = 4
OUTLIER_SCALE = 8.0


def outlier_channels(num_kv_heads: int, head_dim: int) -> list[list[int]]:
    out = []
    for h in range(num_kv_heads):
        g = torch.Generator().manual_seed(7000 + h)
        out.append(sorted(torch.randperm(head_dim, generator=g)[:OUTLIER_CHANNELS].tolist()))
    return out


def kv_tokens_major(num_tokens: int, num_kv_heads: int = 2, head_dim: int = 128,
                    seed: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """K, V as fp16 [num_tokens, H, D] (the ABI's layout), on the CPU."""
    g = torch.Generator().manual_seed(int(seed))
    k = torch.randn(num_tokens, num_kv_heads, head_dim, generator=g, dtype=torch.float32)
    v = torch.randn(num_tokens, num_kv_heads, head_dim, generator=g, dtype=torch.float32)
    for h, chans in enumerate(outlier_channels(num_kv_heads, head_dim)):
        k[:, h, chans] *= OUTLIER_SCALE
        v[:, h, chans] *= OUTLIER_SCALE
    return k.half().contiguous(), v.half().contiguous()


def query(num_q_heads: int = 16, head_dim: int = 128, seed: int = 400) -> torch.Tensor:
    """fp16 query [num_q_heads, D] drawn N(0, 1)."""
    g = torch.Generator().manual_seed(int(seed))
    return torch.randn(num_q_heads, head_dim, generator=g, dtype=torch.float32).half()


def gqa_rows(q: torch.Tensor, num_kv_heads: int) -> torch.Tensor:
    """[Hq, D] -> the ABI's [Hq/Hkv, Hkv, D]: row g of kv head h is q head
    h*(Hq/Hkv) + g (q head j attends kv head j // (Hq/Hkv))."""
    hq, d = q.shape
    groups = hq // num_kv_heads
    return q.view(num_kv_heads, groups, d).permute(1, 0, 2).contiguous()


def permuted_slots(num_tokens: int, block_size: int = 16, seed: int = 401,
                   num_pages: int | None = None) -> torch.Tensor:
    """slot[t] = perm[t // B] * B + t % B for a seeded permutation of pages."""
    pages_needed = (num_tokens + block_size - 1) // block_size
    num_pages = num_pages or pages_needed
    g = torch.Generator().manual_seed(int(seed))
    perm = torch.randperm(num_pages, generator=g)[:pages_needed]
    t = torch.arange(num_tokens)
    return (perm[t // block_size] * block_size + t % block_size).to(torch.int32)


def as_u16(t: torch.Tensor) -> np.ndarray:
    """fp16 torch tensor -> numpy uint16 bit patterns (host)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
