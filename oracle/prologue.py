"""The fused query prologue and output gate, restated on the CPU. TEST INFRASTRUCTURE ONLY.

* ``rms_norm``: Gemma4RMSNorm as the reference applies it to queries, keys (with a weight) and values (without),
  families/gemma/fused.py:21-25 (``h * pow(mean(h^2) + eps, -0.5) * weight`` in float32, cast back), and
  Qwen3_5RMSNorm, families/qwen/fused.py:17-19 (``h * rsqrt(mean(h^2) + eps) * (1 + weight)``, cast back).
* ``rope``: rotation by halves, families/gemma/fused.py:41-45 (the whole head) and transformers'
  ``apply_rotary_pos_emb`` that families/qwen/fused.py:47-48 calls (the first ``cos.shape[-1]`` elements rotate, the
  rest pass through): ``x * cos + cat(-x2, x1) * sin`` over the rotated part, computed in float32 and rounded once to
  the input's dtype (what the reference's compiled kernels do with bf16 tensors).
* ``gate``: families/qwen/fused.py:38-39, ``x * sigmoid(gate)`` on the bf16 attention output, in float32.

Pinned in tests/test_oracle.py against the transformers modules the reference names (Gemma4RMSNorm, Qwen3_5RMSNorm,
Qwen3.5's ``apply_rotary_pos_emb``) and against closed forms (a constant vector, identity and quarter-turn rotations,
pair norms, sigmoid(0) = 1/2).
"""

from __future__ import annotations

import torch

WEIGHT, ONE_PLUS, PLAIN = 1, 2, 3  # the norm modes of karpo_attn.h (KARPO_NORM_*)


def rms_norm(x: torch.Tensor, mode: int, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """``x`` (..., D) normalised over its last dimension, in float32, returned in ``x``'s dtype."""
    h = x.float()
    ms = h.pow(2).mean(-1, keepdim=True) + eps
    out = h * (torch.rsqrt(ms) if mode == ONE_PLUS else torch.pow(ms, -0.5))
    if mode == WEIGHT:
        out = out * weight.float()
    elif mode == ONE_PLUS:
        out = out * (1.0 + weight.float())
    elif mode != PLAIN:
        raise ValueError(f"unknown norm mode {mode}")
    return out.to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x`` (rows, heads, D) rotated by halves over its first R = cos.shape[-1] elements; ``cos`` / ``sin``
    (rows, R) per row."""
    r = cos.shape[-1]
    h = x.float()
    rot, rest = h[..., :r], h[..., r:]
    c, s = cos.float()[:, None, :], sin.float()[:, None, :]
    turned = torch.cat((-rot[..., r // 2:], rot[..., : r // 2]), dim=-1)
    return torch.cat((rot * c + turned * s, rest), dim=-1).to(x.dtype)


def gate(out: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
    """The bf16 attention output times sigmoid of the gate, in float32, returned in ``out``'s dtype."""
    return (out.float() * torch.sigmoid(g.float())).to(out.dtype)
