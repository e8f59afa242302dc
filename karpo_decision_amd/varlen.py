"""The varlen attention entry point the Qwen3.5 family binds (src/karpo_decision/families/qwen/packed.py:36-44; called
at :123-124 for the full-attention layers and :136-137 for the markers-only last layer), with the keyword contract of
torch's ``varlen_attn`` as the reference uses it: ``scale``, ``window_size=(left, right)`` (-1 unbounded; (-1, 0)
causal, (-1, -1) bidirectional, ``WINDOWS`` at :31-33) and ``enable_gqa``. The layer's query norm, rotation and
output gate (``_qkv`` :108-117, ``fused.rope`` :121, ``fused.sigmoid_mul`` :125) can ride along: ``q_norm`` (a
Qwen3_5RMSNorm module), ``cos`` / ``sin`` and ``gate`` fuse them into the kernel's query load and output store.

Like torch's operator, the call is differentiable: under autograd (grad enabled and an input that requires it) it runs
``ops.attention``, the registered forward / backward pair ``karpo_amd::packed_attention_lse`` /
``karpo_amd::packed_attention_backward`` (the op a selective-recompute policy keeps by name, as the reference keeps
``torch.ops.attn._varlen_attn.default``, model/packed.py:111-113)."""

from __future__ import annotations

import math

import torch

from . import ops


def varlen_attn(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, cu_seq_q: torch.Tensor,
                cu_seq_k: torch.Tensor, max_q: int, max_k: int, *, scale: float | None = None,
                window_size: tuple[int, int] = (-1, -1), enable_gqa: bool = False, is_causal: bool = False,
                plan: ops.Plan | None = None, q_norm=None, cos: torch.Tensor | None = None,
                sin: torch.Tensor | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
    """(T, H, D) over (Tk, Hkv, D), per sequence; query i sees key j when i' - left <= j <= i' + right with
    i' = i + Lk - Lq; ``is_causal`` sets right to 0. With ``q_norm`` (a Qwen3_5RMSNorm module or ``ops.Norm``),
    ``query`` is the projection's query half, normalised and (``cos`` / ``sin``: (T, R), partial rotation over the
    first R elements) rotated as the kernel loads it; ``gate`` (T, H, D) multiplies the output by its sigmoid.

    Under autograd gradients flow to query, key and value (``plan`` is then not used: the work list is planned on
    the device); the fused prologue and gate have no backward here (their gradients belong to the norm, rotation and
    gate ops around the attention), so asking for gradients with them is a RuntimeError."""
    if key.shape[1] != query.shape[1] and not enable_gqa:
        raise ValueError(f"{query.shape[1]} query heads over {key.shape[1]} key/value heads needs enable_gqa=True")
    left, right = window_size
    if is_causal:
        right = 0
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    if torch.is_grad_enabled() and any(t.requires_grad for t in (query, key, value)):
        if q_norm is not None or cos is not None or gate is not None:
            raise RuntimeError("varlen_attn's fused query norm, rotation and gate run forward only: apply them as "
                               "separate ops to train through them")
        return ops.attention(query, key, value, cu_seq_q, cu_seq_k, max_q, scale, left, right)
    norm = q_norm if q_norm is None or isinstance(q_norm, ops.Norm) else ops.qwen_norm(q_norm)
    rope = (cos, sin) if cos is not None else None
    return ops.run(query, key, value, cu_seq_q, cu_seq_k, max_q, scale, window_left=left, window_right=right,
                   plan=plan, q_norm=norm, rope=rope, gate=gate)
