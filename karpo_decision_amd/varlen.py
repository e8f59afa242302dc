"""The varlen attention entry point the Qwen3.5 family binds (src/karpo_decision/families/qwen/packed.py:36-44; called
at :123-124 for the full-attention layers and :136-137 for the markers-only last layer), with the keyword contract of
torch's ``varlen_attn`` as the reference uses it: ``scale``, ``window_size=(left, right)`` (-1 unbounded; (-1, 0)
causal, (-1, -1) bidirectional, ``WINDOWS`` at :31-33) and ``enable_gqa``."""

from __future__ import annotations

import math

import torch

from . import ops


def varlen_attn(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cu_seq_q: torch.Tensor,
                cu_seq_k: torch.Tensor, max_q: int, max_k: int, *, scale: float | None = None,
                window_size: tuple[int, int] = (-1, -1), enable_gqa: bool = False, is_causal: bool = False,
                plan: ops.Plan | None = None) -> torch.Tensor:
    """(T, H, D) over (Tk, Hkv, D), per sequence; query i sees key j when i' - left <= j <= i' + right with
    i' = i + Lk - Lq; ``is_causal`` sets right to 0. Forward only."""
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        raise RuntimeError("varlen_attn on MI355X runs the forward only (no backward kernel)")
    if key.shape[1] != query.shape[1] and not enable_gqa:
        raise ValueError(f"{query.shape[1]} query heads over {key.shape[1]} key/value heads needs enable_gqa=True")
    left, right = window_size
    if is_causal:
        right = 0
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    return ops.run(query, key, value, cu_seq_q, cu_seq_k, max_q, scale, window_left=left, window_right=right,
                   plan=plan)
