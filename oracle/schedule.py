"""Brute-force counterparts of the tile scheduler. TEST INFRASTRUCTURE ONLY.

The scheduler lists the (sequence, query tile) tiles of a pack; a tile visits the aligned steps of ``bn`` keys that
hold any key one of its queries sees under the window rule (tests/test_gemma_blocks.py:28-43), so steps outside the
window, above the causal diagonal or in another sequence are never visited. Tiles longer than the pack's
per-workgroup share are split into parts over their steps; the items are ordered by their steps, longest first.
Here the steps are found by enumerating (query, key) pairs; ``split_plan`` restates the split rule (a part is at most
tau = max(8, ceil(sum of steps x head groups / concurrent workgroups)) steps) on top of them.
"""

from __future__ import annotations

from collections.abc import Sequence

from . import brute


def pairs(q_cu: Sequence[int], k_cu: Sequence[int], left: int, right: int,
          spans: Sequence[tuple[int, int]] = ()) -> int:
    """Allowed (query, key) pairs of a pack, counted pair by pair."""
    total = 0
    for qa, qb, ka, kb in zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:]):
        lq, lk = qb - qa, kb - ka
        for i in range(lq):
            qs = brute._span_of(qa + i, spans)
            for j in range(lk):
                ks = brute._span_of(qa + j - (lk - lq), spans)
                total += brute.sees(i, j, lq, lk, left, right, qs, ks)
    return total


def tile_steps(lq: int, lk: int, t: int, rows: int, bn: int, left: int, right: int) -> int:
    """Key steps of ``bn`` (aligned to the sequence's first key) between the first and the last key any query of
    tile ``t`` sees, plus one (the tile's store); 1 when it sees none."""
    seen = [j for i in range(t * rows, min(lq, (t + 1) * rows)) for j in range(lk)
            if brute.sees(i, j, lq, lk, left, right)]
    if not seen:
        return 1
    return (max(seen) // bn) - (min(seen) // bn) + 1 + 1


def work_list(q_cu: Sequence[int], k_cu: Sequence[int], rows: int, bn: int, left: int, right: int,
              clamp: int = 2047) -> list[tuple[int, int, int]]:
    """(cost, sequence, tile) of every tile, longest first, ties in sequence then tile order."""
    items = []
    for n, (qa, qb, ka, kb) in enumerate(zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:])):
        lq, lk = qb - qa, kb - ka
        for t in range(-(-lq // rows)):
            items.append((min(tile_steps(lq, lk, t, rows, bn, left, right), clamp), n, t))
    return sorted(items, key=lambda x: -x[0])


def split_plan(q_cu: Sequence[int], k_cu: Sequence[int], rows: int, bn: int, left: int, right: int, n_hg: int,
               conc: int) -> tuple[list[tuple[int, int, int, int]], list[tuple[int, int, int, int]]]:
    """(merges, items) of the plan: merges (sequence, tile, parts, first slot) of split tiles in tile order; items
    (sequence, tile, part, parts) longest first, ties in sequence, tile, part order."""
    tiles = []
    for n, (qa, qb, ka, kb) in enumerate(zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:])):
        lq, lk = qb - qa, kb - ka
        for t in range(-(-lq // rows)):
            tiles.append((n, t, tile_steps(lq, lk, t, rows, bn, left, right) - 1))
    total = sum(steps for _, _, steps in tiles) * n_hg
    tau = max(8, -(-total // conc))
    merges, items, slot = [], [], 0
    for n, t, steps in tiles:
        parts = -(-steps // tau) if steps > tau else 1
        cost = min(-(-steps // parts) + 1, 2047)
        if parts > 1:
            merges.append((n, t, parts, slot))
            slot += parts
        items.extend((cost, n, t, q, parts) for q in range(parts))
    items.sort(key=lambda x: -x[0])
    return merges, [(n, t, q, parts) for _, n, t, q, parts in items]
