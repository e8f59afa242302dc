"""The reference's torch attention path for packed sequences, restated on the CPU. TEST INFRASTRUCTURE ONLY.

Follows, line by line in behaviour:
  * src/karpo_decision/families/gemma/packed.py:195-220 (``Packed._global``): one scaled_dot_product_attention per
    virtual sequence, ``is_causal`` when the sequence is plain causal with Lq == Lk, an explicit mask otherwise
    (``causal_lower_right`` at :215), ``enable_gqa`` when the head counts differ, empty sequences skipped;
  * tests/test_gemma_blocks.py:28-43 (``varlen_reference``): query i sees key j when
    i + (Lk - Lq) - left <= j <= i + (Lk - Lq) + right, -1 meaning unbounded (families/qwen/packed.py:31-33);
  * tests/test_gemma_images.py:127-131 and families/gemma/vision.py:198-210: image soft tokens additionally see their
    whole image (``rule_a(...) | same``);
  * families/gemma/global_attention.py:71-79 / tests/test_gemma_padded.py:23-33 (padded contract: each sequence
    attends within itself, causal from its first row: the Lq == Lk case of the rule above).
A query row that sees no key (possible only when Lq > Lk under a causal rule) is defined as 0.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch
import torch.nn.functional as F


def span_ids(qa: int, lq: int, lk: int, spans: Sequence[tuple[int, int]]) -> tuple[torch.Tensor, torch.Tensor]:
    """Per query (lq) and per key (lk) of the sequence starting at query row ``qa``: the index of the span it lies
    in, or -1. A span [s, e) of query rows covers the keys aligned with those rows, [s - qa + d, e - qa + d) with
    d = Lk - Lq."""
    q_id = torch.full((lq,), -1, dtype=torch.long)
    k_id = torch.full((lk,), -1, dtype=torch.long)
    delta = lk - lq
    for n, (s, e) in enumerate(spans):
        if e <= qa or s >= qa + lq:
            continue
        q_id[max(0, s - qa):min(lq, e - qa)] = n
        k_id[max(0, s - qa + delta):max(0, min(lk, e - qa + delta))] = n
    return q_id, k_id


def visible(lq: int, lk: int, left: int = -1, right: int = -1, q_span: torch.Tensor | None = None,
            k_span: torch.Tensor | None = None, rows: torch.Tensor | None = None) -> torch.Tensor:
    """(lq, lk) bool: which keys each query of one sequence sees (varlen_reference's rule, OR same span); with
    ``rows`` (local query indices) only those queries' rows, (len(rows), lk)."""
    local = torch.arange(lq) if rows is None else rows.long()
    i = local[:, None] + (lk - lq)
    j = torch.arange(lk)[None, :]
    ok = torch.ones(local.shape[0], lk, dtype=torch.bool)
    if right >= 0:
        ok &= j <= i + right
    if left >= 0:
        ok &= j >= i - left
    if q_span is not None and k_span is not None:
        qs = q_span[local]
        ok |= (qs[:, None] == k_span[None, :]) & (qs[:, None] >= 0)
    return ok


def packed_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, q_cu: Sequence[int],
                     k_cu: Sequence[int], scale: float, window_left: int = -1, window_right: int = -1,
                     spans: Sequence[tuple[int, int]] = (), dtype: torch.dtype = torch.float32,
                     rows: Sequence[int] | None = None, heads: Sequence[int] | None = None) -> torch.Tensor:
    """(Tq, H, D) attention of a pack in ``dtype`` on the CPU. ``rows``: only these query rows (pack indices, the
    result then has len(rows) rows in that order); ``heads``: only these query heads (with their KV heads)."""
    q_cu, k_cu = [int(x) for x in q_cu], [int(x) for x in k_cu]
    n_heads, n_kv = query.shape[1], key.shape[1]
    group = n_heads // n_kv
    head_list = list(range(n_heads)) if heads is None else [int(h) for h in heads]
    kv_list = sorted({h // group for h in head_list})
    head_sel = torch.tensor(head_list)
    q = query.index_select(1, head_sel).to("cpu", dtype)
    k = key.index_select(1, torch.tensor(kv_list)).to("cpu", dtype)
    v = value.index_select(1, torch.tensor(kv_list)).to("cpu", dtype)
    # the selected query heads over their own KV heads, each query head mapped to its KV head explicitly
    kv_index = torch.tensor([kv_list.index(h // group) for h in head_list])
    want = None if rows is None else np.asarray(rows, dtype=np.int64)
    out = torch.zeros(q.shape[0] if want is None else len(want), len(head_list), q.shape[2], dtype=dtype)
    for n, (qa, qb, ka, kb) in enumerate(zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:])):
        lq, lk = qb - qa, kb - ka
        if lq == 0:
            continue
        if want is None:
            local = np.arange(lq)
            dest = torch.arange(qa, qb)
        else:
            hit = np.nonzero((want >= qa) & (want < qb))[0]
            if hit.size == 0:
                continue
            local = want[hit] - qa
            dest = torch.from_numpy(hit)
        qs = q[qa + torch.from_numpy(local)].transpose(0, 1)[None]  # (1, h, m, D)
        ks = k[ka:kb].index_select(1, kv_index).transpose(0, 1)[None]
        vs = v[ka:kb].index_select(1, kv_index).transpose(0, 1)[None]
        q_id, k_id = span_ids(qa, lq, lk, spans)
        has_span = bool((q_id >= 0).any())
        # torch's CPU is_causal path is only used for positive scales (with a negative scale it returns NaN)
        plain_causal = (window_left < 0 and window_right == 0 and lq == lk and not has_span and want is None
                        and scale > 0)
        if lk == 0:
            continue
        if plain_causal:
            o = F.scaled_dot_product_attention(qs, ks, vs, scale=scale, is_causal=True)
        elif window_left < 0 and window_right < 0 and not has_span:
            o = F.scaled_dot_product_attention(qs, ks, vs, scale=scale)
        else:
            mask = visible(lq, lk, window_left, window_right, q_id, k_id, rows=torch.from_numpy(local))
            o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, scale=scale)
            o = torch.where(mask.any(-1)[None, None, :, None], o, torch.zeros((), dtype=o.dtype))
        out[dest] = o[0].transpose(0, 1)
    return out


def packed_lse(query: torch.Tensor, key: torch.Tensor, q_cu: Sequence[int], k_cu: Sequence[int], scale: float,
               window_left: int = -1, window_right: int = -1,
               spans: Sequence[tuple[int, int]] = ()) -> torch.Tensor:
    """(H, Tq) float64 log-sum-exp of each query row's scaled logits over its visible keys (the softmax normaliser
    of ``packed_attention``; the reference's ``return_lse``, families/gemma/sliding_attention.py:39-41), -inf for a
    row that sees no key."""
    q_cu, k_cu = [int(x) for x in q_cu], [int(x) for x in k_cu]
    group = query.shape[1] // key.shape[1]
    q = query.to("cpu", torch.float64)
    k = key.to("cpu", torch.float64).repeat_interleave(group, dim=1)
    out = torch.full((query.shape[1], query.shape[0]), float("-inf"), dtype=torch.float64)
    for qa, qb, ka, kb in zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:]):
        lq, lk = qb - qa, kb - ka
        if lq == 0 or lk == 0:
            continue
        s = torch.einsum("qhd,khd->hqk", q[qa:qb], k[ka:kb]) * scale
        q_id, k_id = span_ids(qa, lq, lk, spans)
        mask = visible(lq, lk, window_left, window_right, q_id, k_id)
        out[:, qa:qb] = torch.logsumexp(s.masked_fill(~mask[None], float("-inf")), dim=-1)
    return out


def packed_grads(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, grad: torch.Tensor,
                 q_cu: Sequence[int], k_cu: Sequence[int], scale: float, window_left: int = -1,
                 window_right: int = -1, spans: Sequence[tuple[int, int]] = (),
                 dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, ...]:
    """(out, dq, dk, dv) in ``dtype`` on the CPU: ``packed_attention`` and torch autograd's gradients of
    sum(out * grad) (the backward the reference's attention ops compute, families/gemma/sliding_attention.py:50-61)."""
    xs = [t.detach().to("cpu", dtype).requires_grad_(True) for t in (query, key, value)]
    out = packed_attention(*xs, q_cu, k_cu, scale, window_left, window_right, spans, dtype=dtype)
    out.backward(grad.to("cpu", dtype))
    return (out.detach(), *(x.grad for x in xs))
