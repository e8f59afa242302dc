"""Gemma's global-layer hook on MI355X: one HIP launch over every virtual sequence of a pack.

Mirror of src/karpo_decision/families/gemma/triton_attention.py (``supported`` :87-89, ``attend`` :92-110,
``enable`` :113-125) with the same positional signature, so ``Packed.global_attend`` and its call sites
(families/gemma/packed.py:242, :245-246, :276-277) take it unchanged. Differences, each a superset:

* causal models are served (the reference's kernel is bidirectional only and ``enable`` refuses causal models):
  ``attend`` takes keyword-only ``causal``, ``window`` and ``spans``, and ``enable`` installs a causal ``attend`` on a
  causal model;
* offsets are 64-bit everywhere, so there is no 131,071-token cap and no 32-bit-offset ValueError;
* GQA heads share one staged K/V tile instead of re-reading it per query head;
* ``rows`` reads a block plan's branch keys in place (``g_rows``, the gather ``Packed._gather`` makes with
  ``index_select``, families/gemma/packed.py:222-226, :245);
* ``q_norm`` / ``cos`` / ``sin`` fuse the query's ``Gemma4RMSNorm`` and rotation (``Packed._q``, packed.py:191-193,
  fused.norm_rope) into the kernel's query load; ``norm_rope`` / ``norm`` do the keys' and values' (``Packed._kv``,
  :183-189) in one pass each.
"""

from __future__ import annotations

import functools
from typing import Any

import torch

from . import _lib, ops


def supported(device: torch.device) -> bool:
    """A gfx950 (MI355X) GPU and a built library."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return False
    try:
        _lib.load()
    except RuntimeError:
        return False
    return ops._is_gfx950(device)


def attend(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, q_cu: torch.Tensor, k_cu: torch.Tensor,
           max_q: int, scale: float, *, causal: bool = False, window: int = -1, spans: torch.Tensor | None = None,
           plan: ops.Plan | None = None, rows: torch.Tensor | None = None, q_norm: Any = None,
           cos: torch.Tensor | None = None, sin: torch.Tensor | None = None) -> torch.Tensor:
    """One HIP launch over every virtual sequence of the pack; returns the (Lq, heads, D) bf16 output.

    ``query`` is (Lq, heads, D) bf16, ``key`` / ``value`` (Lk, kv heads, D) bf16, query head h reading key/value head
    h // (heads / kv heads). The int32 device offsets ``q_cu`` / ``k_cu`` (n + 1 each) give virtual sequence i the
    query rows [q_cu[i], q_cu[i + 1]) and the key rows [k_cu[i], k_cu[i + 1]); ``max_q`` bounds every sequence's
    query count and selects the tile shape. Visible keys: the whole sequence, or with ``causal`` those up to the
    query's own position (the last query lined up with the last key), narrowed by ``window`` (how many earlier keys
    stay visible; -1 for all) and widened by ``spans`` ((n, 2) int32 query-row ranges, each seen whole by its own
    rows). ``rows`` (int32 / int64 on the device) takes key row r from row rows[r] of ``key`` / ``value``, so a block
    plan's branch gather needs no copy. With ``q_norm`` (a Gemma4RMSNorm or an ``ops.Norm``) ``query`` is q_proj's
    raw output, which the kernel normalises while loading it, and also rotates when ``cos`` / ``sin`` are given
    ((Lq, R) or (1, Lq, R) tables, row i for query row i)."""
    if torch.is_grad_enabled():
        raise RuntimeError("hip_attention.attend has no backward: call it under torch.inference_mode() or "
                           "torch.no_grad(), or use ops.attention, which has one")
    norm = q_norm if q_norm is None or isinstance(q_norm, ops.Norm) else ops.gemma_norm(q_norm)
    rope = (cos, sin) if cos is not None else None
    return ops.run(query, key, value, q_cu, k_cu, max_q, scale, window_left=window, window_right=0 if causal else -1,
                   spans=spans, plan=plan, key_rows=rows, q_norm=norm, rope=rope)


def norm_rope(module: Any, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``fused.norm_rope(module, x, cos, sin)`` (families/gemma/fused.py:86-88) for (1, T, heads, D) keys and
    (1, T, D) cos / sin, in one pass on the GPU; (1, T, heads, D)."""
    return ops.norm_rope(x[0], ops.gemma_norm(module), (cos, sin))[None]


def norm(module: Any, x: torch.Tensor) -> torch.Tensor:
    """``fused.norm(module, x)`` (families/gemma/fused.py:81-83) for (1, T, heads, D) values; (1, T, heads, D)."""
    return ops.norm_rope(x[0], ops.gemma_norm(module))[None]


def enable(model: Any, max_length: int) -> None:
    """Point ``model.global_attend``, the hook a ``Packed`` model's global layers call, at ``attend`` (made causal when
    ``model.causal_global`` is set). ``max_length``, the longest sequence the caller will pack, only has to be
    positive: offsets are 64-bit. ValueError without a gfx950 GPU and a built library, or for max_length < 1."""
    if not supported(model.lm.embed_tokens.weight.device):
        raise ValueError("hip_attention needs an MI355X (gfx950) GPU and a built libkarpo_attn.so")
    if max_length < 1:
        raise ValueError(f"max_length must be positive, not {max_length}")
    model.global_attend = functools.partial(attend, causal=True) if model.causal_global else attend
