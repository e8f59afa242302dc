"""The padded-plan global attention for CUDA-graph replays on MI355X.

Mirror of ``padded`` (src/karpo_decision/families/gemma/global_attention.py:71-79): query (1, P, heads, D) over key
and value (1, P, kv heads, D), each sequence of ``cu`` (int32 on the device, read when the kernel runs, so a captured
graph sees the bounds written before each replay, serve/graphs.py:107-115) attending within itself, causal from its
first row. The reference repeats K and V to every query head first (:76-77); here GQA heads read the shared K/V
directly. The work list is planned on the device inside the same stream, so the call is capture-safe.
"""

from __future__ import annotations

import torch

from . import ops


def padded(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cu: torch.Tensor, size: int, causal: bool,
           scale: float) -> torch.Tensor:
    """(1, P, heads, D) bf16 of the padded pack's attention."""
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"padded attention takes (1, P, heads, D) queries, got {tuple(query.shape)}")
    out = ops.run(query[0], key[0], value[0], cu, cu, size, scale, window_left=-1, window_right=0 if causal else -1)
    return out[None]
