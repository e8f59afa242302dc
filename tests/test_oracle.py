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


# ---- the fused prologue / gate restatement (oracle/prologue.py)

def test_prologue_norms_match_the_transformers_modules():
    """Gemma4RMSNorm (with and without a weight) and Qwen3_5RMSNorm, the modules the reference's fused norms restate
    (families/gemma/fused.py:21-25, families/qwen/fused.py:17-19), give the same bf16 values."""
    from transformers.models.gemma4.modeling_gemma4 import Gemma4RMSNorm
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5RMSNorm

    from oracle import prologue

    torch.manual_seed(21)
    x = (torch.randn(64, 4, 128) * 3).bfloat16()
    g = Gemma4RMSNorm(128, eps=1e-6)
    q = Qwen3_5RMSNorm(128, eps=1e-6)
    plain = Gemma4RMSNorm(128, eps=1e-6, with_scale=False)
    with torch.no_grad():
        g.weight.copy_(torch.randn(128).bfloat16().float())
        q.weight.copy_((torch.randn(128) * 0.1).bfloat16().float())
        assert torch.equal(prologue.rms_norm(x, prologue.WEIGHT, g.weight.bfloat16(), 1e-6), g(x))
        assert torch.equal(prologue.rms_norm(x, prologue.ONE_PLUS, q.weight.bfloat16(), 1e-6), q(x))
        assert torch.equal(prologue.rms_norm(x, prologue.PLAIN, None, 1e-6), plain(x))


def test_prologue_rope_matches_apply_rotary_pos_emb():
    """Full and partial rotation equal transformers' apply_rotary_pos_emb (the function families/qwen/fused.py:47-48
    calls) evaluated in float32 and rounded once."""
    from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

    from oracle import prologue

    torch.manual_seed(22)
    x = torch.randn(50, 3, 128).bfloat16()
    for r in (128, 64, 32):
        angle = torch.randn(50, r // 2)
        cos = torch.cat((angle.cos(), angle.cos()), -1).bfloat16()
        sin = torch.cat((angle.sin(), angle.sin()), -1).bfloat16()
        xf = x.float()[None]  # (batch, rows, heads, D)
        want, _ = apply_rotary_pos_emb(xf, xf, cos.float()[None], sin.float()[None], unsqueeze_dim=2)
        assert torch.equal(prologue.rope(x, cos, sin), want[0].bfloat16()), r


def test_prologue_closed_forms():
    from oracle import prologue

    # a constant vector c normalises to c / sqrt(c^2 + eps) times the weight
    x = torch.full((1, 1, 64), 2.0)
    out = prologue.rms_norm(x, prologue.WEIGHT, torch.full((64,), 3.0), 0.0)
    assert torch.allclose(out, torch.full_like(out, 3.0))
    # without a weight the mean square of the output is 1
    y = prologue.rms_norm(torch.randn(10, 2, 128) * 7, prologue.PLAIN, None, 0.0)
    assert torch.allclose(y.pow(2).mean(-1), torch.ones(10, 2), atol=1e-5)
    # cos 1, sin 0: identity; cos 0, sin 1: the quarter turn (-x2, x1); twice: negation; tail untouched
    v = torch.randn(4, 2, 128)
    one, zero = torch.ones(4, 64), torch.zeros(4, 64)
    assert torch.equal(prologue.rope(v, one, zero), v)
    turn = prologue.rope(v, zero, one)
    assert torch.equal(turn[..., :32], -v[..., 32:64]) and torch.equal(turn[..., 32:64], v[..., :32])
    assert torch.equal(turn[..., 64:], v[..., 64:])
    assert torch.equal(prologue.rope(turn, zero, one)[..., :64], -v[..., :64])
    # a rotation keeps each (d, d + R/2) pair's norm
    a = torch.rand(4, 32) * 6
    c, s = torch.cat((a.cos(), a.cos()), -1), torch.cat((a.sin(), a.sin()), -1)
    w = prologue.rope(v, c, s)
    pair = lambda t: t[..., :32].pow(2) + t[..., 32:64].pow(2)  # noqa: E731
    assert torch.allclose(pair(w), pair(v), atol=1e-4)
    # the gate: sigmoid(0) halves, large gates pass or close
    o = torch.randn(3, 2, 64)
    assert torch.equal(prologue.gate(o, torch.zeros_like(o)), o * 0.5)
    assert torch.allclose(prologue.gate(o, torch.full_like(o, 40.0)), o)
    assert torch.equal(prologue.gate(o, torch.full_like(o, -200.0)), torch.zeros_like(o) * o)


# ---- the backward's oracle: log-sum-exp and gradients (oracle/attention.py packed_lse, packed_grads)

@pytest.mark.parametrize("layout", LAYOUTS)
def test_lse_reweights_the_values_into_the_output(layout):
    """exp(scale * q.k - lse) over the visible keys sums to 1 and averages v into the loop oracle's output; rows that
    see no key have lse = -inf (the identity the backward's P = exp(s - lse) rests on)."""
    q_lens, k_lens, left, right, local_spans = layout
    q, k, v, q_cu, k_cu = _pack(q_lens, k_lens, 4, 2, 8, seed=11 + len(q_lens))
    spans = [(q_cu[s] + a, q_cu[s] + b) for s, a, b in local_spans]
    lse = oa.packed_lse(q, k, q_cu, k_cu, 0.7, left, right, spans)
    want = brute.attention(q.numpy(), k.numpy(), v.numpy(), q_cu, k_cu, 0.7, left, right, spans)
    for n in range(len(q_lens)):
        qa, lq, ka, lk = q_cu[n], q_lens[n], k_cu[n], k_lens[n]
        for i in range(lq):
            row = qa + i
            q_span = brute._span_of(row, spans)
            for h in range(4):
                seen = [j for j in range(lk) if brute.sees(i, j, lq, lk, left, right, q_span,
                                                           brute._span_of(qa + j - (lk - lq), spans))]
                if not seen:
                    assert lse[h, row] == float("-inf")
                    continue
                w = np.array([math.exp(0.7 * float(q[row, h] @ k[ka + j, h // 2]) - float(lse[h, row]))
                              for j in seen])
                assert abs(w.sum() - 1.0) < 1e-12
                np.testing.assert_allclose(w @ v[[ka + j for j in seen], h // 2].numpy(), want[row, h], atol=1e-12)


def test_lse_of_zero_queries_counts_the_visible_keys():
    q, k, _, q_cu, k_cu = _pack([20], [20], 2, 1, 4, seed=12)
    lse = oa.packed_lse(torch.zeros_like(q), k, q_cu, k_cu, 1.0, 5, 0)
    want = torch.log(torch.minimum(torch.arange(1, 21), torch.tensor(6)).double())
    torch.testing.assert_close(lse, want[None].expand(2, 20), atol=1e-15, rtol=0)


def test_gradients_are_the_oracles_derivative():
    """torch autograd through the oracle against central differences (float64), with a window, a span, GQA and a
    branch (Lk > Lq)."""
    q, k, v, q_cu, k_cu = _pack([6, 5], [6, 8], 4, 2, 4, seed=13)
    spans = [(1, 4)]

    def f(q_, k_, v_):
        return oa.packed_attention(q_, k_, v_, q_cu, k_cu, 0.6, 3, 0, spans, dtype=torch.float64)

    xs = [t.clone().requires_grad_(True) for t in (q, k, v)]
    assert torch.autograd.gradcheck(f, xs, eps=1e-6, atol=1e-8, rtol=1e-6)


def test_value_gradient_of_zero_queries_is_a_causal_mean():
    """q = 0, causal: out_i = mean(v_0..v_i), so dv_j = sum over i >= j of grad_i / (i + 1); dk = scale dS^T q = 0;
    dq_i = scale * sum over j <= i of (dP_ij - rowsum(grad_i * out_i)) k_j / (i + 1) (a dS that drops the rowsum term
    or a transposed dP fails it)."""
    q, k, v, q_cu, k_cu = _pack([10], [10], 2, 1, 4, seed=14)
    g = torch.randn(10, 2, 4, generator=torch.Generator().manual_seed(15), dtype=torch.float64)
    out, dq, dk, dv = oa.packed_grads(torch.zeros_like(q), k, v, g, q_cu, k_cu, 1.0, -1, 0, dtype=torch.float64)
    weights = 1.0 / torch.arange(1, 11, dtype=torch.float64)
    want = torch.flip(torch.cumsum(torch.flip(g.sum(1) * weights[:, None], [0]), 0), [0])
    torch.testing.assert_close(dv[:, 0], want, atol=1e-12, rtol=0)
    # with q = 0, dk = scale * dS^T q = 0 exactly, whatever dS is
    torch.testing.assert_close(dk, torch.zeros_like(dk), atol=1e-15, rtol=0)
    # dq_i = scale * sum_j P_ij (dP_ij - D_i) k_j with P uniform over j <= i
    for i in range(10):
        for h in range(2):
            p = torch.full((i + 1,), 1.0 / (i + 1), dtype=torch.float64)
            dp = v[: i + 1, 0] @ g[i, h]
            d = (g[i, h] * out[i, h]).sum()
            torch.testing.assert_close(dq[i, h], (p * (dp - d)) @ k[: i + 1, 0], atol=1e-12, rtol=0)
