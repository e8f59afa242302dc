"""Brute-force counterparts of the tile scheduler. TEST INFRASTRUCTURE ONLY.

The scheduler lists one work item per (sequence, query tile), ordered by the key steps the tile visits, longest
first; a tile visits the aligned steps of ``bn`` keys that hold any key one of its queries sees under the window rule
(tests/test_gemma_blocks.py:28-43), so steps outside the window, above the causal diagonal or in another sequence
are never visited. Here every quantity is found by enumerating (query, key) pairs.
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
