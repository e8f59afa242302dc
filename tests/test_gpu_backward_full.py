"""The backward (karpo_attn_bwd) at the sizes it is measured at, against the CPU oracle on an MI355X.

Four layers, each run whole through the C ABI (the forward's output and log-sum-exp from ``packed_attention_lse``,
then ``karpo_attn_bwd`` into NaN-filled dQ, dK and dV): the 32k-token global layer (32 / 16 heads, head_dim 128,
causal; its dK / dV in the two-group kernel), the 16k sliding layer (16 / 8 heads, head_dim 256, window 1023), the Qwen
8k pack (16 / 8 heads, head_dim 128, causal) and the 31B global layer (32 / 4 heads, head_dim 512, causal, the pair
kernels). Checks:

* every (row, head) of dQ, dK and dV is written and finite;
* the first and the last key/value head group (the key/value head and its query heads: their gradients depend on no
  other head) against torch autograd through the oracle restricted to those heads, in float32 on the same bf16
  inputs: relative Frobenius error below 1e-2 for out, dq, dk and dv, and below twice the error of the oracle's own
  bf16 run plus 2e-3 (the reference's criterion for its backward kernels, tests/gpu/test_packed_gemma.py:173-184).
"""

from __future__ import annotations

import ctypes
import functools

import pytest
import torch

from karpo_decision_amd import _lib, ops, workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu

REL_FRO = 1e-2
LAYERS = ("global32k", "sliding", "qwen", "global32k_d512")


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _backward_c_abi(w, do, out, lse, q_cu, k_cu, spans):
    """karpo_attn_bwd into NaN-filled gradient buffers (a row it skipped stays NaN)."""
    lib = _lib.load()
    q, k, v = w.query, w.key, w.value
    dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
    b = _lib.KarpoAttnBwdArgs()
    b.fwd = ops._args(q, k, v, out, q_cu, k_cu, q_cu.numel() - 1, w.max_q, w.scale, w.window_left, w.window_right,
                      spans, None)
    b.fwd.total_k = k.shape[0]
    b.d_o, b.d_o_stride_tok, b.d_o_stride_head = do.data_ptr(), do.stride(0), do.stride(1)
    b.lse = lse.data_ptr()
    b.d_q, b.d_q_stride_tok, b.d_q_stride_head = dq.data_ptr(), dq.stride(0), dq.stride(1)
    b.d_k, b.d_k_stride_tok, b.d_k_stride_head = dk.data_ptr(), dk.stride(0), dk.stride(1)
    b.d_v, b.d_v_stride_tok, b.d_v_stride_head = dv.data_ptr(), dv.stride(0), dv.stride(1)
    need = ctypes.c_size_t()
    _lib.check(lib.karpo_attn_bwd_workspace_bytes(ctypes.byref(b), ctypes.byref(need)), "workspace")
    ws = torch.full((need.value,), 0x7F, dtype=torch.uint8, device=q.device)  # garbage: nothing may rely on zeros
    b.fwd.workspace, b.fwd.workspace_bytes = ws.data_ptr(), need.value
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.karpo_attn_bwd(ctypes.byref(b), stream), "karpo_attn_bwd")
    torch.cuda.synchronize()
    return dq, dk, dv


@functools.lru_cache(maxsize=None)  # host copies of the compared heads only: the layer's GPU tensors are freed
def _layer(name: str):
    dev = torch.device("cuda", 0)
    w = workloads.named(name, dev, seed=0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    do = torch.randn(w.query.shape, generator=gen, device=dev).bfloat16()
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=dev)
    k_cu = torch.tensor(w.k_cu, dtype=torch.int32, device=dev)
    spans = torch.tensor(w.spans, dtype=torch.int32, device=dev) if w.spans else None
    print(f"layer {name}: forward with lse", flush=True)
    with torch.no_grad():
        out, lse = ops.packed_attention_lse(w.query, w.key, w.value, q_cu, k_cu, w.max_q, w.scale, w.window_left,
                                            w.window_right, spans)
    print(f"layer {name}: backward through the C ABI", flush=True)
    dq, dk, dv = _backward_c_abi(w, do, out, lse, q_cu, k_cu, spans)
    written = {n: bool(torch.isfinite(t).all()) for n, t in (("dq", dq), ("dk", dk), ("dv", dv))}
    group = w.heads // w.kv_heads
    keep = {}
    for g in (0, w.kv_heads - 1):
        h = slice(g * group, (g + 1) * group)
        keep[g] = {"inputs": tuple(t.cpu() for t in (w.query[:, h], w.key[:, g:g + 1], w.value[:, g:g + 1], do[:, h])),
                   "got": tuple(t.cpu() for t in (out[:, h], dq[:, h], dk[:, g:g + 1], dv[:, g:g + 1]))}
    return {"w": (w.q_cu, w.k_cu, w.scale, w.window_left, w.window_right, list(w.spans), w.kv_heads),
            "written": written, "groups": keep}


@pytest.mark.parametrize("name", LAYERS)
def test_every_gradient_row_is_written(gpu, name):
    """dQ, dK and dV of the whole layer (NaN-filled before the call): every (row, head) written and finite."""
    layer = _layer(name)
    assert all(layer["written"].values()), layer["written"]


@functools.lru_cache(maxsize=None)
def _oracle(name: str, g: int, dtype: torch.dtype):
    layer = _layer(name)
    q_cu, k_cu, scale, left, right, spans, _ = layer["w"]
    q, k, v, do = layer["groups"][g]["inputs"]
    print(f"layer {name}: oracle ({dtype}) for key/value head {g}", flush=True)
    return oa.packed_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans, dtype=dtype)


def _group(name: str, which: str) -> int:
    return 0 if which == "first" else _layer(name)["w"][-1] - 1


@pytest.mark.parametrize("which", ["first", "last"])
@pytest.mark.parametrize("name", LAYERS)
def test_head_group_gradients_match_the_oracle(gpu, name, which):
    """The first or last key/value head group's out, dq, dk, dv against autograd through the oracle in float32:
    relative Frobenius error below 1e-2."""
    g = _group(name, which)
    got = _layer(name)["groups"][g]["got"]
    want = _oracle(name, g, torch.float32)
    for label, x, w in zip(("out", "dq", "dk", "dv"), got, want):
        r = rel(x, w)
        print(name, g, label, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (label, r)


@pytest.mark.parametrize("which", ["first", "last"])
@pytest.mark.parametrize("name", LAYERS)
def test_head_group_gradients_within_twice_the_bf16_error(gpu, name, which):
    """The same gradients within twice the error of the oracle's own bf16 run plus 2e-3 (both against the float32
    oracle): the reference's criterion for its backward kernels."""
    g = _group(name, which)
    got = _layer(name)["groups"][g]["got"]
    want = _oracle(name, g, torch.float32)
    base = _oracle(name, g, torch.bfloat16)
    for label, x, w, b in zip(("out", "dq", "dk", "dv"), got, want, base):
        r, rb = rel(x, w), rel(b, w)
        print(name, g, label, f"rel {r:.2e} (oracle bf16 {rb:.2e})", flush=True)
        assert r < 2 * rb + 2e-3, (label, r, rb)
