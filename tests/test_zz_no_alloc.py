"""karpo_attn_fwd_noalloc (the forward with its scratch in the library's own device array) against karpo_attn_fwd
with a caller's workspace, through the C ABI: two calls in a row, the second on a smaller input, each bitwise equal to
the workspace call. The packs split tiles over their keys (the partials live in the scratch), plan on the device
and from a host plan, and read keys through a row table. Under HIP graph capture (the callers it is for): the first
call on the device made inside a capture, in a process of its own (tests/noalloc_capture.py), replayed with rewritten
bounds."""

from __future__ import annotations

import ctypes
import json
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from karpo_decision_amd import _lib, ops
from oracle import attention as oa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _call(entry, q, k, v, q_cu, k_cu, max_q, scale, left, right, plan=None, rows=None):
    lib = _lib.load()
    o = torch.full_like(q, float("nan"))
    a = ops._args(q, k, v, o, q_cu, k_cu, q_cu.numel() - 1, max_q, scale, left, right, None,
                  plan.tensor if plan is not None else None, list(plan.header) if plan is not None else None, rows)
    keep = None
    if entry == "workspace":
        need = ctypes.c_size_t()
        _lib.check(lib.karpo_attn_workspace_bytes(ctypes.byref(a), ctypes.byref(need)), "workspace")
        keep = torch.empty(need.value, dtype=torch.uint8, device=q.device)
        a.workspace, a.workspace_bytes = keep.data_ptr(), need.value
        fn = lib.karpo_attn_fwd
    else:
        a.workspace, a.workspace_bytes = 0, 0  # ignored by the allocation-free entry point
        fn = lib.karpo_attn_fwd_noalloc
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(fn(ctypes.byref(a), stream), entry)
    torch.cuda.synchronize()
    return o


def _pack(lengths, heads, kv_heads, head, seed, device):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    g = torch.Generator(device="cpu").manual_seed(seed)
    q, k, v = (torch.randn(cu[-1], h, head, generator=g).to(torch.bfloat16).to(device)
               for h in (heads, kv_heads, kv_heads))
    return cu, q, k, v


@pytest.mark.parametrize("planned", [False, True])
def test_noalloc_matches_the_workspace_entry_point(gpu, planned):
    """Two calls in a row (the second smaller, reusing the scratch the first left behind), device plan or host plan:
    every output bitwise equal to karpo_attn_fwd with a fresh workspace, and the first against the oracle."""
    # the first in the wide tiles (max_q 8192): its longest tiles split; the second in the four-wave tiles
    first = _pack([2210, 1547, 1138, 861, 680, 666, 526, 351, 213], 16, 8, 128, 1, gpu)
    second = _pack([900, 300, 40], 16, 8, 128, 2, gpu)
    for n, (cu, q, k, v) in enumerate((first, second)):
        cu_t = torch.tensor(cu, dtype=torch.int32, device=gpu)
        max_q = 8192 if n == 0 else max(b - a for a, b in zip(cu[:-1], cu[1:]))
        plan = ops.make_plan(cu, cu, 16, 8, 128, -1, 0, gpu, max_q=max_q) if planned else None
        if n == 0:
            assert plan is None or plan.split_tiles > 0
        want = _call("workspace", q, k, v, cu_t, cu_t, max_q, 0.088, -1, 0, plan)
        got = _call("noalloc", q, k, v, cu_t, cu_t, max_q, 0.088, -1, 0, plan)
        assert not torch.isnan(got).any(), f"call {n}: rows left unwritten"
        assert torch.equal(got, want), f"call {n} (planned {planned})"
        if n == 0:
            ref = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), cu, cu, 0.088, -1, 0)
            diff = (got.float().cpu() - ref).abs()
            assert float(diff.max()) <= 2e-2 and float(diff.mean()) <= 2e-3


def test_noalloc_decode_shaped_and_row_table_calls(gpu):
    """One query per sequence over all of its keys (split across the GPU, merged from the scratch's partials), then a
    smaller pack read through a row table: bitwise equal to the workspace entry point."""
    heads, kv_heads, head = 32, 16, 128
    k_cu = [0, 20000, 26000, 30000]
    g = torch.Generator(device="cpu").manual_seed(3)
    k = torch.randn(k_cu[-1], kv_heads, head, generator=g).to(torch.bfloat16).to(gpu)
    v = torch.randn(k_cu[-1], kv_heads, head, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(3, heads, head, generator=g).to(torch.bfloat16).to(gpu)
    m_cu = torch.tensor([0, 1, 2, 3], dtype=torch.int32, device=gpu)
    kc = torch.tensor(k_cu, dtype=torch.int32, device=gpu)
    want = _call("workspace", q, k, v, m_cu, kc, 1, 0.088, -1, -1)
    got = _call("noalloc", q, k, v, m_cu, kc, 1, 0.088, -1, -1)
    assert torch.equal(got, want)
    rows = torch.arange(4000, 4600, dtype=torch.int32, device=gpu)
    q2 = torch.randn(600, heads, head, generator=g).to(torch.bfloat16).to(gpu)
    cu2 = torch.tensor([0, 600], dtype=torch.int32, device=gpu)
    want = _call("workspace", q2, k, v, cu2, cu2, 600, 0.088, -1, 0, rows=rows)
    got = _call("noalloc", q2, k, v, cu2, cu2, 600, 0.088, -1, 0, rows=rows)
    assert torch.equal(got, want)


def test_noalloc_first_call_inside_a_graph_capture(gpu):
    """The entry point's first call on the device made inside a capture (a fresh process, tests/noalloc_capture.py):
    the call succeeds, every replay with rewritten bounds equals the workspace entry point's eager call bit for bit
    and writes every row, and eager calls after the first leave the device's free memory unchanged."""
    child = Path(__file__).resolve().parent / "noalloc_capture.py"
    done = subprocess.run([sys.executable, "-u", str(child)], capture_output=True, text=True, timeout=180)
    print(done.stdout[-3000:], done.stderr[-3000:], flush=True)
    assert done.returncode == 0, done.stderr[-3000:]
    result = json.loads(done.stdout.strip().splitlines()[-1])
    assert result["status_in_capture"] == 0, result
    assert len(result["replays"]) == 5
    for r in result["replays"]:
        assert r["equal"] and not r["nan"], r
    assert result["eager_status"] == [0, 0, 0]
    assert len(set(result["free_bytes"])) == 1, result["free_bytes"]
