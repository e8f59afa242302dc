"""Gemma's sliding-window attention on MI355X: each query sees its own position and the ``window`` positions before
it, within its virtual sequence of the pack. Queries and keys carry separate bounds, so a branch sequence reads the
shared prefix it extends followed by its own rows; positions line up at the sequences' last rows.

Mirror of src/karpo_decision/families/gemma/sliding_attention.py:85-93 (``attend``). The bidirectional image spans
that the reference applies in a second pass (``vision.see_whole``, families/gemma/vision.py:198-210) are part of the
same launch here (``spans``).
"""

from __future__ import annotations

import torch

from . import ops


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, q_cu: torch.Tensor, k_cu: torch.Tensor,
           max_q: int, max_k: int, scale: float, window: int, *, spans: torch.Tensor | None = None,
           plan: ops.Plan | None = None, rows: torch.Tensor | None = None) -> torch.Tensor:
    """The (T, heads, D) output of (T, heads, D) queries over (Tk, kv heads, D) keys and values, the sequences
    bounded by the int32 device offsets ``q_cu`` / ``k_cu``; a query's visible keys are its own position and the
    ``window`` before it. ``rows`` takes key row r from row rows[r] of ``key`` / ``value`` (the block plan's
    ``s_rows``, without a gathered copy).

    Under autograd (grad enabled and an input that requires it) the call goes through ``ops.attention``, which keeps
    the forward's log-sum-exp and runs ``karpo_attn_bwd`` for the gradients, as the reference's FA4 operator pair
    (sliding_attention.py:36-66) does; keys and values must then be tensors rather than read through ``rows``."""
    if window < 0:
        raise ValueError(f"a sliding window needs a non-negative left size, not {window}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        if rows is not None:
            raise ValueError("gradients need the gathered keys and values as tensors (index_select first), not rows")
        return ops.attention(query, key, value, q_cu, k_cu, max_q, scale, window, 0, spans)
    return ops.run(query, key, value, q_cu, k_cu, max_q, scale, window_left=window, window_right=0, spans=spans,
                   plan=plan, key_rows=rows)
