"""Invariants of the paged step's work split (tq_attention.hip: Segments,
item_passes, the split kernel's item walk and attn_paged_combine_kernel),
restated in integer Python.

The split kernel gives workgroup s of G the work positions [bound(s),
bound(s + 1)) with bound(s) = floor(s * total / G), computed as q*s + floor(r*s
/ G); a unit's item h (one per kv head) holds n passes of weight w starting at
work position start + h*w*n, and a pass belongs to the segment holding its
first position.  Each workgroup writes one partial per (item, segment) piece
at slot item + segment; the combine finds an item's segments from its first
and last pass.  On random plans (weights 1, 3, 4, empty units, more segments
than work) this checks what the kernels rely on: the bound formula equals the
exact floor, the segment lookup inverts it, every pass of every item lands in
exactly one piece, no two pieces share a slot, and the combine visits exactly
the pieces the split kernel wrote."""
from __future__ import annotations

import numpy as np


def _bound(s, total, G):
    q, r = divmod(total, G)
    return q * s + (r * s) // G


def _segment_of(x, total, G):
    # the kernel's float estimate, then the +-1 correction
    g = int(np.float32(np.float32(x) + np.float32(1)) * np.float32(G) / np.float32(total)) - 1
    g = max(0, min(g, G - 1))
    while g + 1 < G and _bound(g + 1, total, G) <= x:
        g += 1
    while g > 0 and _bound(g, total, G) > x:
        g -= 1
    return g


def _passes(S, n, w, b0, b1):
    x0 = 0 if S >= b0 else (b0 - S + w - 1) // w
    x1 = 0 if S >= b1 else min(n, (b1 - S + w - 1) // w)
    return x0, x1


def test_paged_plan_pieces_partition_every_item():
    rng = np.random.default_rng(77)
    for _ in range(400):
        U = int(rng.integers(1, 40))
        H = int(rng.choice([1, 2, 4]))
        G = int(rng.choice([8, 64, 256, 512]))
        units, start = [], 0
        for _u in range(U):
            n = int(rng.choice([0, 1, 2, 17, 128, int(rng.integers(0, 300))]))
            w = int(rng.choice([1, 3, 4]))
            units.append((start, n, w))
            start += H * w * n
        total = start
        if total == 0:
            continue
        ends = [units[k + 1][0] if k + 1 < U else total for k in range(U)]
        for s in range(G + 1):
            assert _bound(s, total, G) == (s * total) // G
        for x in range(0, total, max(1, total // 97)):
            g = _segment_of(x, total, G)
            assert _bound(g, total, G) <= x < _bound(g + 1, total, G)
        written = {}
        for seg in range(G):  # the split kernel's walk
            b0, b1 = _bound(seg, total, G), _bound(seg + 1, total, G)
            if b0 >= b1:
                continue
            u = next(k for k in range(U) if units[k][0] <= b0 < ends[k])
            st, n, w = units[u]
            h = (b0 - st) // (w * n)
            while u < U:
                st, n, w = units[u]
                S = st + h * w * n
                if S >= b1:
                    break
                x0, x1 = _passes(S, n, w, b0, b1)
                if x0 < x1:
                    slot = u * H + h + seg
                    assert slot not in written
                    written[slot] = (u, h, x0, x1)
                h += 1
                if h == H:
                    h, u = 0, u + 1
        assert max(written) < U * H + G
        seen = 0
        for u, (st, n, w) in enumerate(units):  # the combine's view
            for h in range(H):
                S = st + h * w * n
                covered = []
                if n > 0:
                    lo = _segment_of(S, total, G)
                    hi = _segment_of(S + w * (n - 1), total, G)
                    for g in range(lo, hi + 1):
                        x0, x1 = _passes(S, n, w, _bound(g, total, G), _bound(g + 1, total, G))
                        if x0 < x1:
                            assert written[u * H + h + g] == (u, h, x0, x1)
                            covered += range(x0, x1)
                            seen += 1
                assert covered == list(range(n))
        assert seen == len(written)
