"""Invariants of the paged step's work split (tq_attention.hip: Segments,
item_passes, the split kernel's unit walk and attn_paged_combine_kernel),
restated in integer Python.

Every kv head has the same work: unit u holds n passes of weight w from work
position start (a per-head prefix sum), after a lead of positions that no
pass occupies (a unit's setup cost, 8 in the kernel's plan; 0 for a unit
without passes).  Each head's work is split into Gh
segments; workgroup s of a head takes the work positions [bound(s),
bound(s + 1)) with bound(s) = floor(s * total / Gh), computed as q*s +
floor(r*s / Gh), and a pass belongs to the segment holding its first
position.  Each workgroup writes one partial per (unit, segment) piece of its
head at slot (unit + segment) * H + head; the combine finds a unit's
segments from its first and last pass.  On random plans (weights 1, 3, 4,
empty units, more segments than work) this checks what the kernels rely on:
the bound formula equals the exact floor, the segment lookup inverts it,
every pass of every (unit, head) lands in exactly one piece, no two pieces
share a slot, slots stay below (units + Gh) * H, and the combine visits
exactly the pieces the split kernel wrote."""
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
        Gh = int(rng.choice([8, 64, 256, 512]))
        lead = int(rng.choice([0, 1, 8, 40]))
        units, start = [], 0
        for _u in range(U):
            n = int(rng.choice([0, 1, 2, 17, 128, int(rng.integers(0, 300))]))
            w = int(rng.choice([1, 3, 4]))
            start += lead if n > 0 else 0
            units.append((start, n, w))
            start += w * n
        total = start
        if total == 0:
            continue
        ends = [units[k + 1][0] if k + 1 < U else total for k in range(U)]
        for s in range(Gh + 1):
            assert _bound(s, total, Gh) == (s * total) // Gh
        for x in range(0, total, max(1, total // 97)):
            g = _segment_of(x, total, Gh)
            assert _bound(g, total, Gh) <= x < _bound(g + 1, total, Gh)
        written = {}
        for h in range(H):  # the split kernel's walk: workgroup (head h, segment seg)
            for seg in range(Gh):
                b0, b1 = _bound(seg, total, Gh), _bound(seg + 1, total, Gh)
                if b0 >= b1:
                    continue
                # (before the first unit's first pass: unit 0)
                u = next(k for k in range(U) if (k == 0 or units[k][0] <= b0) and b0 < ends[k])
                while u < U:
                    S, n, w = units[u]
                    if S >= b1:
                        break
                    x0, x1 = _passes(S, n, w, b0, b1)
                    if x0 < x1:
                        slot = (u + seg) * H + h
                        assert slot not in written
                        written[slot] = (u, h, x0, x1)
                    u += 1
        assert max(written) < (U + Gh) * H
        seen = 0
        for u, (S, n, w) in enumerate(units):  # the combine's view
            for h in range(H):
                covered = []
                if n > 0:
                    lo = _segment_of(S, total, Gh)
                    hi = _segment_of(S + w * (n - 1), total, Gh)
                    for g in range(lo, hi + 1):
                        x0, x1 = _passes(S, n, w, _bound(g, total, Gh), _bound(g + 1, total, Gh))
                        if x0 < x1:
                            assert written[(u + g) * H + h] == (u, h, x0, x1)
                            covered += range(x0, x1)
                            seen += 1
                assert covered == list(range(n))
        assert seen == len(written)
