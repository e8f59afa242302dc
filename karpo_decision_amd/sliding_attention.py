"""Gemma's sliding-window layers on MI355X: causal by position, a query sees itself and the ``window`` keys before
it, over a pack's virtual sequences with separate query and key bounds (a branch's keys are the shared block's tail,
then its own rows; causal aligned at each sequence's end).

Mirror of src/karpo_decision/families/gemma/sliding_attention.py:85-93 (``attend``); the image soft tokens'
bidirectional spans that the reference recomputes afterwards with ``vision.see_whole`` (families/gemma/vision.py:
198-210) are folded into the same launch through ``spans``.
"""

from __future__ import annotations

import torch

from . import ops


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, q_cu: torch.Tensor, k_cu: torch.Tensor,
           max_q: int, max_k: int, scale: float, window: int, *, spans: torch.Tensor | None = None,
           plan: ops.Plan | None = None, rows: torch.Tensor | None = None) -> torch.Tensor:
    """(T, heads, D) queries over (Tk, kv heads, D) keys and values (``q_cu`` / ``k_cu``: int32 boundaries), each
    query seeing at most ``window`` keys before its own position; ``rows``: the block plan's ``s_rows`` gather read
    in place (key row r is row rows[r] of ``key`` / ``value``); (T, heads, D).

    Differentiable like the reference's FA4 operator pair (sliding_attention.py:36-66): when autograd needs
    gradients the forward also keeps its log-sum-exp and the backward runs ``karpo_attn_bwd`` (keys and values as
    tensors, not through ``rows``)."""
    if window < 0:
        raise ValueError(f"a sliding window needs a non-negative left size, not {window}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        if rows is not None:
            raise ValueError("gradients need the gathered keys and values as tensors (index_select first), not rows")
        return ops.attention(query, key, value, q_cu, k_cu, max_q, scale, window, 0, spans)
    return ops.run(query, key, value, q_cu, k_cu, max_q, scale, window_left=window, window_right=0, spans=spans,
                   plan=plan, key_rows=rows)
