"""Float64 attention by explicit loops, for tiny packs. TEST INFRASTRUCTURE ONLY.

Every rule is stated pair by pair, independently of ``oracle.attention``'s vectorised masks and of torch's SDPA:
a query at sequence index i sits at key coordinate i + Lk - Lq (tests/test_gemma_blocks.py:37-39); it sees key j when
j is not after it by more than ``right`` and not before it by more than ``left`` (-1: unbounded), or when both lie in
the same image span (tests/test_gemma_images.py:127-131); query head h reads key/value head h // (H / Hkv)
(families/gemma/triton_attention.py:37); the weights are exp(scale * q.k - max) / sum, the output their mean of v.
"""

from __future__ import annotations

import math
from collections.abc import Sequence

import numpy as np


def sees(i: int, j: int, lq: int, lk: int, left: int, right: int, q_span: int = -1, k_span: int = -1) -> bool:
    """Does query i of a sequence see key j?"""
    at = i + (lk - lq)
    if q_span >= 0 and q_span == k_span:
        return True
    if right >= 0 and j > at + right:
        return False
    if left >= 0 and j < at - left:
        return False
    return True


def _span_of(row: int, spans: Sequence[tuple[int, int]]) -> int:
    for n, (s, e) in enumerate(spans):
        if s <= row < e:
            return n
    return -1


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, q_cu: Sequence[int], k_cu: Sequence[int], scale: float,
              left: int = -1, right: int = -1, spans: Sequence[tuple[int, int]] = ()) -> np.ndarray:
    """(Tq, H, D) float64."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    n_heads, n_kv = q.shape[1], k.shape[1]
    group = n_heads // n_kv
    out = np.zeros(q.shape, dtype=np.float64)
    for qa, qb, ka, kb in zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:]):
        lq, lk = qb - qa, kb - ka
        delta = lk - lq
        for i in range(lq):
            qs = _span_of(qa + i, spans)
            keys = []
            for j in range(lk):
                # key j lies in span n when the query row it is aligned with, qa + j - delta, does
                ks = _span_of(qa + j - delta, spans)
                if sees(i, j, lq, lk, left, right, qs, ks):
                    keys.append(j)
            if not keys:
                continue
            for h in range(n_heads):
                kv = h // group
                logits = [scale * float(np.dot(q[qa + i, h], k[ka + j, kv])) for j in keys]
                top = max(logits)
                w = [math.exp(x - top) for x in logits]
                total = math.fsum(w)
                acc = np.zeros(q.shape[2], dtype=np.float64)
                for wj, j in zip(w, keys):
                    acc += wj * v[ka + j, kv]
                out[qa + i, h] = acc / total
    return out
