"""Host-side behaviour of the reference-shaped entry points, checked without a GPU: the global hook's ``attend``
refuses an autograd call with RuntimeError (as triton_attention.py:98-99 does), ``enable`` refuses a machine without
a gfx950 GPU with ValueError and leaves the model's hook alone (as :116-117), and the sliding ``attend`` refuses a
negative window."""

from __future__ import annotations

import types

import pytest
import torch

from karpo_decision_amd import hip_attention, sliding_attention


def _pack():
    q = torch.zeros(8, 2, 64, dtype=torch.bfloat16)
    kv = torch.zeros(8, 1, 64, dtype=torch.bfloat16)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    return q, kv, kv, cu


def test_global_attend_refuses_an_autograd_call():
    q, k, v, cu = _pack()
    with torch.enable_grad(), pytest.raises(RuntimeError, match="no backward"):
        hip_attention.attend(q, k, v, cu, cu, 8, 0.125)


def test_enable_refuses_a_machine_without_gfx950():
    weight = torch.zeros(1)  # the model's embedding lives on the CPU
    model = types.SimpleNamespace(lm=types.SimpleNamespace(embed_tokens=types.SimpleNamespace(weight=weight)),
                                  causal_global=False)
    with pytest.raises(ValueError, match="gfx950"):
        hip_attention.enable(model, 1024)
    assert not hasattr(model, "global_attend")


def test_sliding_attend_refuses_a_negative_window():
    q, k, v, cu = _pack()
    with torch.inference_mode(), pytest.raises(ValueError, match="window"):
        sliding_attention.attend(q, k, v, cu, cu, 8, 8, 0.125, -1)
