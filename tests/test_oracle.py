"""The CPU oracle pinned before it judges the kernel: golden known answers (mask contract, float64 vectors), closed
forms (uniform weights, one-hot values, two keys, GQA head mapping, scale), and agreement of the vectorised torch
restatement with the pair-by-pair float64 loops on random packs, including empty sequences, branches (Lq != Lk),
windows on both sides and image spans."""

import math

import numpy as np
import pytest
import torch

import golden_io
from oracle import attention as oa
from oracle import brute


@pytest.mark.parametrize("name", golden_io.names("mask"))
def test_mask_known_answers(name):
    c = golden_io.load(name)
    got = oa.packed_attention(c["q"], c["k"], c["v"], c["q_cu"], c["k_cu"], c["scale"], c["left"], c["right"],
                              c["spans"], dtype=torch.float64)
    torch.testing.assert_close(got, c["want"], atol=1e-12, rtol=0)
    got_brute = brute.attention(c["q"].numpy(), c["k"].numpy(), c["v"].numpy(), c["q_cu"], c["k_cu"], c["scale"],
                                c["left"], c["right"], c["spans"])
    np.testing.assert_allclose(got_brute, c["want"].numpy(), atol=1e-12, rtol=0)


@pytest.mark.parametrize("name", golden_io.names("random"))
def test_random_golden_vectors(name):
    c = golden_io.load(name)
    got = oa.packed_attention(c["q"], c["k"], c["v"], c["q_cu"], c["k_cu"], c["scale"], c["left"], c["right"],
                              c["spans"], dtype=torch.float64)
    torch.testing.assert_close(got, c["want"], atol=1e-6, rtol=1e-6)


def _pack(q_lens, k_lens, heads, kv_heads, d, seed):
    g = torch.Generator().manual_seed(seed)
    q_cu = np.concatenate([[0], np.cumsum(q_lens)]).tolist()
    k_cu = np.concatenate([[0], np.cumsum(k_lens)]).tolist()
    q = torch.randn(q_cu[-1], heads, d, generator=g, dtype=torch.float64)
    k = torch.randn(k_cu[-1], kv_heads, d, generator=g, dtype=torch.float64)
    v = torch.randn(k_cu[-1], kv_heads, d, generator=g, dtype=torch.float64)
    return q, k, v, q_cu, k_cu


LAYOUTS = [
    # (q lengths, k lengths, left, right, spans as (sequence, start, end) local query rows)
    ([7, 0, 12], [7, 0, 12], -1, 0, []),
    ([5, 9], [11, 9], -1, 0, []),            # a branch: more keys than queries, aligned at the end
    ([9, 4], [9, 2], -1, 0, []),             # more queries than keys: leading queries see nothing
    ([13], [13], 3, 0, [(0, 4, 8)]),          # window with a span
    ([10, 6], [10, 6], 2, 2, [(0, 1, 3)]),    # two-sided window
    ([8, 8], [12, 8], -1, -1, [(1, 2, 6)]),   # bidirectional
    ([16], [16], 0, 0, [(0, 3, 9)]),          # a query sees only itself, and its span
]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("heads,kv_heads", [(4, 2), (3, 3), (6, 1)])
def test_vectorised_oracle_matches_the_loops(layout, heads, kv_heads):
    q_lens, k_lens, left, right, local_spans = layout
    q, k, v, q_cu, k_cu = _pack(q_lens, k_lens, heads, kv_heads, 8, seed=len(q_lens) + heads)
    spans = [(q_cu[s] + a, q_cu[s] + b) for s, a, b in local_spans]
    got = oa.packed_attention(q, k, v, q_cu, k_cu, 0.7, left, right, spans, dtype=torch.float64)
    want = brute.attention(q.numpy(), k.numpy(), v.numpy(), q_cu, k_cu, 0.7, left, right, spans)
    np.testing.assert_allclose(got.numpy(), want, atol=1e-12, rtol=1e-12)


def test_row_and_head_subsets_match_the_whole():
    q, k, v, q_cu, k_cu = _pack([30, 50], [40, 50], 4, 2, 8, seed=5)
    whole = oa.packed_attention(q, k, v, q_cu, k_cu, 0.5, 7, 0, [(40, 55)], dtype=torch.float64)
    rows = [0, 3, 29, 30, 45, 79]
    part = oa.packed_attention(q, k, v, q_cu, k_cu, 0.5, 7, 0, [(40, 55)], dtype=torch.float64, rows=rows,
                               heads=[1, 2])
    torch.testing.assert_close(part, whole[rows][:, [1, 2]], atol=1e-12, rtol=0)


def test_zero_queries_average_the_visible_values():
    """q = 0: every visible key weighs the same, so a causal query at i outputs the mean of v[0..i]."""
    q, k, v, q_cu, k_cu = _pack([20], [20], 2, 1, 4, seed=6)
    got = oa.packed_attention(torch.zeros_like(q), k, v, q_cu, k_cu, 1.0, -1, 0, dtype=torch.float64)
    want = torch.cumsum(v[:, 0], 0) / torch.arange(1, 21, dtype=torch.float64)[:, None]
    torch.testing.assert_close(got[:, 0], want, atol=1e-12, rtol=0)
    torch.testing.assert_close(got[:, 1], want, atol=1e-12, rtol=0)


def test_two_keys_give_a_logistic_weight():
    """One query over two keys: weight of key 1 is sigmoid(scale * q.(k1 - k0))."""
    q = torch.tensor([[[1.0, 2.0]]], dtype=torch.float64)
    k = torch.tensor([[[0.5, -1.0]], [[2.0, 0.25]]], dtype=torch.float64)
    v = torch.tensor([[[1.0, 0.0]], [[0.0, 1.0]]], dtype=torch.float64)
    scale = 0.3
    w1 = 1 / (1 + math.exp(-scale * (1.0 * (2.0 - 0.5) + 2.0 * (0.25 + 1.0))))
    got = oa.packed_attention(q, k, v, [0, 1], [0, 2], scale, dtype=torch.float64)
    torch.testing.assert_close(got[0, 0], torch.tensor([1 - w1, w1], dtype=torch.float64), atol=1e-15, rtol=0)


def test_gqa_query_head_reads_its_group_key_value_head():
    """Value head g is the constant g + 1: query head h must output h // (H / Hkv) + 1."""
    heads, kv_heads = 8, 2
    q, k, _, q_cu, k_cu = _pack([9], [9], heads, kv_heads, 4, seed=7)
    v = torch.stack([torch.full((9, 4), g + 1.0, dtype=torch.float64) for g in range(kv_heads)], 1)
    got = oa.packed_attention(q, k, v, q_cu, k_cu, 1.0, -1, 0, dtype=torch.float64)
    for h in range(heads):
        torch.testing.assert_close(got[:, h], torch.full((9, 4), h // 4 + 1.0, dtype=torch.float64))


def test_scale_multiplies_the_logits():
    """Scaling q by a and the scale by 1/a leaves the output unchanged; negative scales flip the weights."""
    q, k, v, q_cu, k_cu = _pack([11], [11], 2, 1, 8, seed=8)
    a = oa.packed_attention(q, k, v, q_cu, k_cu, 0.4, -1, -1, dtype=torch.float64)
    b = oa.packed_attention(q * 4, k, v, q_cu, k_cu, 0.1, -1, -1, dtype=torch.float64)
    c = oa.packed_attention(-q, k, v, q_cu, k_cu, -0.4, -1, -1, dtype=torch.float64)
    torch.testing.assert_close(a, b, atol=1e-12, rtol=0)
    torch.testing.assert_close(a, c, atol=1e-12, rtol=0)


@pytest.mark.parametrize("left,right", [(-1, 0), (4, 0), (-1, -1)])
def test_negative_and_zero_scales_under_masks(left, right):
    q, k, v, q_cu, k_cu = _pack([12, 9], [12, 9], 4, 2, 8, seed=9)
    for scale in (-0.3, 0.0):
        got = oa.packed_attention(q, k, v, q_cu, k_cu, scale, left, right, dtype=torch.float64)
        want = brute.attention(q.numpy(), k.numpy(), v.numpy(), q_cu, k_cu, scale, left, right)
        np.testing.assert_allclose(got.numpy(), want, atol=1e-12, rtol=1e-12)


def test_a_planted_mask_mistake_is_caught():
    """The checks above must reject a plausible oracle bug: alignment at the start instead of the end of the keys."""
    c = golden_io.load("mask_window_bottom_right")
    lq, lk = 4, 6
    wrong = torch.arange(lq)[:, None]  # i' = i, the top-left alignment
    j = torch.arange(lk)[None, :]
    mask = (j <= wrong) & (j >= wrong - 2)
    w = mask / mask.sum(-1, keepdim=True)
    assert not torch.allclose(w.double(), c["want"][:, 0, :lk])
