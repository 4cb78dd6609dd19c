"""Batched paged decode with append-quantize (a serving step over many
sequences), on the library's allocator, block table, pack and paged
attention entry points.

A ``PagedBatch`` holds S sequences in one page pool.  Pages come from the
library's LIFO allocator; the prefill is appended page by page in a seeded
random order of sequences, so every sequence's pages are scattered over the
pool.  One ``step`` appends w_s new tokens to every sequence (one pack
launch over all of them, slots from the block table) and runs decode
attention for 8 GQA rows per new token (one paged-attention launch), the
rows of new token j attending L_s + j + 1 tokens (causal over the new
tokens).  The reference does the same work with one pack call per sequence
and one fused_attention_output call per sequence and position, each with a
per-token slot map (tq_backend/turboquant_wrapper.py; the C5 serving
configuration).
"""
from __future__ import annotations

import numpy as np
import torch

from turborag_amd.synthetic import fisher_yates, gqa_rows, kv_tokens_major
from turborag_amd.synthetic import query as draw_query
from turborag_amd.turboquant_wrapper import BlockTable, PageAllocator, TurboQuantWrapper


class PagedBatch:
    def __init__(self, tq: TurboQuantWrapper, scheme: str, lens, widths, *, kv_heads: int = 2,
                 q_heads: int = 16, head_dim: int = 128, block_size: int = 16, seed: int = 500,
                 device: torch.device | None = None) -> None:
        self.tq, self.scheme = tq, scheme
        self.dev = device or torch.device("cuda", 0)
        self.lens = [int(x) for x in lens]
        self.widths = [int(x) for x in widths]
        self.S = len(self.lens)
        self.H, self.D, self.B = kv_heads, head_dim, block_size
        self.group = q_heads // kv_heads  # GQA rows per kv head and token
        cfg = tq.default_config()
        cfg.num_kv_heads, cfg.head_dim, cfg.block_size = kv_heads, head_dim, block_size
        self.cfg = cfg
        self.prod = scheme == "turbo_prod"
        self.layout = tq.make_layout_for(cfg) if self.prod else tq.make_mse_layout_for(cfg)
        B = block_size
        pages = sum((L + w + B - 1) // B for L, w in zip(self.lens, self.widths)) + self.S
        self.pool = torch.zeros(pages * self.layout.page_size_bytes, dtype=torch.uint8,
                                device=self.dev)
        self.alloc = PageAllocator(tq, self.layout.page_size_bytes, pages, device_pool=self.pool)
        self.table = BlockTable(self.alloc, B)
        self.max_blocks = max((L + w + B - 1) // B for L, w in zip(self.lens, self.widths))
        self.seed = seed
        self._prefill()

    # ── helpers ─────────────────────────────────────────────────────── #

    def _pack(self, k: torch.Tensor, v: torch.Tensor, slots: list[int]) -> None:
        self._last_pack = (k.to(self.dev), v.to(self.dev),
                           torch.tensor(slots, dtype=torch.int32, device=self.dev))
        self.repack()

    def repack(self, stream: int = 0) -> None:
        """Issue the last pack launch again (same tokens into the same slots:
        idempotent), e.g. to time the append of a step."""
        k, v, s = self._last_pack
        (self.tq.pack if self.prod else self.tq.mse_pack)(k, v, s, self.pool, self.layout,
                                                          self.cfg, stream=stream)

    def _prefill(self) -> None:
        """Every sequence's first L_s tokens, appended one page at a time in a
        seeded random order of sequences (scattered pages)."""
        self.kv = [kv_tokens_major(L, self.H, self.D, seed=self.seed + 3 + s)
                   for s, L in enumerate(self.lens)]
        pages = []
        for s, L in enumerate(self.lens):
            pages += [s] * ((L + self.B - 1) // self.B)
        todo = [pages[i] for i in fisher_yates(len(pages), self.seed + 2)]
        done = [0] * self.S
        keys, vals, slots = [], [], []
        for s in todo:
            n = min(self.B, self.lens[s] - done[s])
            slots += self.table.build_slot_map(s, n)
            keys.append(self.kv[s][0][done[s]:done[s] + n])
            vals.append(self.kv[s][1][done[s]:done[s] + n])
            done[s] += n
        self._pack(torch.cat(keys), torch.cat(vals), slots)

    def block_tables(self) -> torch.Tensor:
        bt = torch.full((self.S, self.max_blocks), -1, dtype=torch.int32)
        for s in range(self.S):
            b = self.table.blocks(s)
            bt[s, :len(b)] = torch.tensor(b, dtype=torch.int32)
        return bt.to(self.dev)

    def slots_of(self, s: int, n: int) -> np.ndarray:
        """The first n tokens' slots of sequence s (page * B + position)."""
        b = np.asarray(self.table.blocks(s), dtype=np.int64)
        t = np.arange(n)
        return (b[t // self.B] * self.B + t % self.B).astype(np.int32)

    # ── one serving step ───────────────────────────────────────────── #

    def append_new_tokens(self, seed: int) -> tuple[list, list]:
        """w_s new tokens per sequence, quantized into (newly allocated)
        pages with one pack launch; returns the new K/V per sequence."""
        keys, vals, slots, new = [], [], [], []
        for s, w in enumerate(self.widths):
            k, v = kv_tokens_major(w, self.H, self.D, seed=seed + s)
            slots += self.table.build_slot_map(s, w)
            keys.append(k)
            vals.append(v)
            new.append((k, v))
        self._pack(torch.cat(keys), torch.cat(vals), slots)
        return new

    def decode_rows(self, seed: int):
        """Query rows of the step: for sequence s and new token j, the 8 GQA
        rows of every kv head ([8, H, D]), attending L_s + j + 1 tokens."""
        q, row_seq, row_len = [], [], []
        for s, (L, w) in enumerate(zip(self.lens, self.widths)):
            for j in range(w):
                qh = draw_query(self.group * self.H, self.D, seed=seed + 1000 * s + j)
                q.append(gqa_rows(qh, self.H))
                row_seq += [s] * self.group
                row_len += [L + j + 1] * self.group
        query = torch.cat(q).contiguous().to(self.dev)
        return (query, torch.tensor(row_seq, dtype=torch.int32, device=self.dev),
                torch.tensor(row_len, dtype=torch.int32, device=self.dev))

    def attention(self, query, row_seq, row_len, block_tables, out, stream: int = 0) -> None:
        self.tq.paged_attn_output(self.scheme, query, self.pool, block_tables, row_seq, row_len,
                                  out, self.layout, self.cfg,
                                  max(L + w for L, w in zip(self.lens, self.widths)), stream)

    def close(self) -> None:
        self.table.close()
        self.alloc.close()
