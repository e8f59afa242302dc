"""Writes the golden fixtures in this directory (run from the repository root: python tests/golden/make_golden.py).

Two kinds of vectors, both small:

* ``mask_<name>.npz``: known answers for the mask contract. Queries are zero, so every visible key gets the same
  weight, and value row j of a sequence is the one-hot vector e_j: the output row of a query is 1/|S| on the keys S
  it sees and 0 elsewhere. Each case's S is written out below as a literal list, derived by hand from the reference's
  rules (varlen alignment i' = i + Lk - Lq and the window, tests/test_gemma_blocks.py:28-43; image spans,
  tests/test_gemma_images.py:127-131): a wrong alignment, window edge or span rule changes a listed set.
* ``random_<name>.npz``: seeded bf16-representable inputs and their float64 attention from ``oracle.brute`` (explicit
  loops, math.exp), pinning the vectorised oracle across torch versions and feeding the GPU kernel a committed case.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import brute  # noqa: E402

# (q_cu, k_cu, left, right, spans, visible key sets per query row in pack order, local to the row's sequence)
MASK_CASES = {
    # causal, window of two keys before, 4 queries aligned at the end of 6 keys: query 0 sits at key 2
    "window_bottom_right": ([0, 4], [0, 6], 2, 0, [],
                            [[0, 1, 2], [1, 2, 3], [2, 3, 4], [3, 4, 5]]),
    # more queries than keys, causal: the first two queries sit before key 0 and see nothing
    "causal_more_queries": ([0, 5], [0, 3], -1, 0, [],
                            [[], [], [0], [0, 1], [0, 1, 2]]),
    # bidirectional, two sequences with their own key bounds and an empty one between
    "bidirectional_bounds": ([0, 2, 2, 5], [0, 3, 3, 4], -1, -1, [],
                             [[0, 1, 2], [0, 1, 2], [0], [0], [0]]),
    # causal with one image span over rows 2-4: those rows see the whole span
    "span_causal": ([0, 8], [0, 8], -1, 0, [(2, 5)],
                    [[0], [0, 1], [0, 1, 2, 3, 4], [0, 1, 2, 3, 4], [0, 1, 2, 3, 4], [0, 1, 2, 3, 4, 5],
                     [0, 1, 2, 3, 4, 5, 6], [0, 1, 2, 3, 4, 5, 6, 7]]),
    # causal window of one key before, span over rows 3-5: the span adds keys after a query, never before the window
    "span_window": ([0, 7], [0, 7], 1, 0, [(3, 6)],
                    [[0], [0, 1], [1, 2], [2, 3, 4, 5], [3, 4, 5], [3, 4, 5], [5, 6]]),
    # a branch: 4 queries over 7 keys (3 shared, then its own 4, aligned at the end); a span on the branch's query
    # rows 4-5 covers its keys 4-5
    "span_branch": ([0, 3, 7], [0, 3, 10], -1, 0, [(4, 6)],
                    [[0], [0, 1], [0, 1, 2], [0, 1, 2, 3], [0, 1, 2, 3, 4, 5], [0, 1, 2, 3, 4, 5],
                     [0, 1, 2, 3, 4, 5, 6]]),
    # sliding window of 3 keys before, bidirectional to the right limited to 1 key after
    "two_sided_window": ([0, 6], [0, 6], 3, 1, [],
                         [[0, 1], [0, 1, 2], [0, 1, 2, 3], [0, 1, 2, 3, 4], [1, 2, 3, 4, 5], [2, 3, 4, 5]]),
}

# (q_cu, k_cu, heads, kv_heads, head_dim, scale, left, right, spans, seed)
RANDOM_CASES = {
    "causal_gqa": ([0, 37, 37, 100, 140], [0, 37, 37, 100, 140], 4, 2, 64, 0.125, -1, 0, [], 1),
    "window_spans": ([0, 90, 150], [0, 90, 150], 4, 2, 64, 0.125, 20, 0, [(10, 40), (100, 130)], 2),
    "branches_bidirectional": ([0, 50, 70, 95], [0, 50, 120, 195], 4, 1, 64, 0.2, -1, -1, [], 3),
    "large_logits": ([0, 60], [0, 60], 2, 1, 64, 8.0, -1, -1, [], 4),
}


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def mask_case(q_cu, k_cu, left, right, spans, sets):
    tq, tk = q_cu[-1], k_cu[-1]
    d = 16
    heads, kv_heads = 2, 1
    q = np.zeros((tq, heads, d), dtype=np.float32)
    k = np.zeros((tk, kv_heads, d), dtype=np.float32)
    v = np.zeros((tk, kv_heads, d), dtype=np.float32)
    for ka, kb in zip(k_cu[:-1], k_cu[1:]):
        for j in range(kb - ka):
            v[ka + j, 0, j] = 1.0
    want = np.zeros((tq, heads, d), dtype=np.float64)
    for row, keys in enumerate(sets):
        for j in keys:
            want[row, :, j] = 1.0 / len(keys)
    return dict(q=q, k=k, v=v, q_cu=np.array(q_cu), k_cu=np.array(k_cu), left=left, right=right,
                spans=np.array(spans, dtype=np.int64).reshape(-1, 2), scale=1.0, want=want)


def random_case(q_cu, k_cu, heads, kv_heads, head_dim, scale, left, right, spans, seed):
    rng = np.random.default_rng(seed)
    q = bf16_round(rng.standard_normal((q_cu[-1], heads, head_dim)).astype(np.float32))
    k = bf16_round(rng.standard_normal((k_cu[-1], kv_heads, head_dim)).astype(np.float32))
    v = bf16_round(rng.standard_normal((k_cu[-1], kv_heads, head_dim)).astype(np.float32))
    want = brute.attention(q, k, v, q_cu, k_cu, scale, left, right, spans)
    # inputs as raw bfloat16 bits (exact), expected outputs in float32 (far below the kernel's tolerance)
    bits = {name: (t.view(np.uint32) >> 16).astype(np.uint16) for name, t in (("q", q), ("k", k), ("v", v))}
    return dict(**{f"{n}_bf16": b for n, b in bits.items()}, q_cu=np.array(q_cu), k_cu=np.array(k_cu), left=left,
                right=right, spans=np.array(spans, dtype=np.int64).reshape(-1, 2), scale=scale,
                want=want.astype(np.float32))


def main() -> None:
    for name, case in MASK_CASES.items():
        np.savez_compressed(HERE / f"mask_{name}.npz", **mask_case(*case))
    for name, case in RANDOM_CASES.items():
        np.savez_compressed(HERE / f"random_{name}.npz", **random_case(*case))
    print(f"wrote {len(MASK_CASES) + len(RANDOM_CASES)} fixtures to {HERE}")


if __name__ == "__main__":
    main()
