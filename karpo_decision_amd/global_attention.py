"""Gemma's global layers on MI355X, mirroring src/karpo_decision/families/gemma/global_attention.py:

* ``padded`` (:71-79): the padded plan for CUDA-graph replays. Query (1, P, heads, D) over key and value
  (1, P, kv heads, D), each sequence of ``cu`` (int32 on the device, read when the kernel runs, so a captured graph
  sees the bounds written before each replay, serve/graphs.py:107-115) attending within itself, causal from its
  first row. The reference repeats K and V to every query head first (:76-77); here GQA heads read the shared K/V
  directly. The work list is planned on the device inside the same stream, so the call is capture-safe.
* ``attend`` (:125-129), ``usable`` (:41-44), ``lengths`` (:61-68): one virtual sequence per call with its lengths
  on the device, differentiable (the reference's cuDNN forward / backward pair, :93-122): the training path of
  ``Packed._global`` (families/gemma/packed.py:195-208). No length buckets and nothing to compile ahead: the kernels
  take any length, causal aligned at the end (a branch's queries follow its shared keys).
"""

from __future__ import annotations

import torch

from . import ops

#: Head sizes the forward and the backward take (512: the 31B global layers).
HEADS = (64, 128, 256, 512)


def usable(query: torch.Tensor) -> bool:
    """True on an MI355X (gfx950) for bf16 queries of a supported head size."""
    return (query.is_cuda and query.dtype == torch.bfloat16 and query.shape[-1] in HEADS
            and ops._is_gfx950(query.device))


def lengths(q_bounds: list[int], k_bounds: list[int], device: torch.device) -> torch.Tensor:
    """(sequences, 2, 4) int32: [i, 0, 0] query rows, [i, 1, 0] key rows of sequence i (the reference's layout)."""
    t = torch.zeros(len(q_bounds) - 1, 2, 4, dtype=torch.int32)
    t[:, 0, 0] = torch.tensor(q_bounds).diff()
    t[:, 1, 0] = torch.tensor(k_bounds).diff()
    return t.to(device)


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, q_len: torch.Tensor, k_len: torch.Tensor,
           causal: bool, scale: float) -> torch.Tensor:
    """One virtual sequence: (Lq, heads, D) queries over (Lk, kv heads, D) keys and values, ``q_len`` / ``k_len``
    their lengths on the device (``lengths(...)[i, 0, :1]``, ``[i, 1, :1]``); (Lq, heads, D). Gradients flow to
    query, key and value."""
    zero = torch.zeros(1, dtype=torch.int32, device=query.device)
    q_cu = torch.cat([zero, q_len.reshape(-1)[:1].to(torch.int32)])
    k_cu = torch.cat([zero, k_len.reshape(-1)[:1].to(torch.int32)])
    right = 0 if causal else -1
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        return ops.attention(query, key, value, q_cu, k_cu, query.shape[0], scale, -1, right)
    return ops.run(query, key, value, q_cu, k_cu, query.shape[0], scale, window_left=-1, window_right=right)


def padded(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cu: torch.Tensor, size: int, causal: bool,
           scale: float) -> torch.Tensor:
    """(1, P, heads, D) bf16 of the padded pack's attention."""
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"padded attention takes (1, P, heads, D) queries, got {tuple(query.shape)}")
    out = ops.run(query[0], key[0], value[0], cu, cu, size, scale, window_left=-1, window_right=0 if causal else -1)
    return out[None]
