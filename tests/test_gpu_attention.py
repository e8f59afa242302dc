"""The HIP kernel against the CPU oracle on an MI355X, through the C ABI (the torch operator and the reference-shaped
entry points all call karpo_attn_fwd).

Tolerance, bf16 kernel against the fp32 oracle on the same bf16 inputs: max-abs <= 2e-2 and mean-abs <= 2e-3, and
relative Frobenius error < 1e-2 (tests/gpu/test_triton_attention.py:66). Workloads the oracle cannot finish in
seconds are compared on sampled query rows (first, last and seeded random rows of every sequence) and heads.
The edge cases follow the reference's kernel tests (tests/gpu/test_triton_attention.py): one sequence against fp32
math, a branched varlen pack with an empty virtual sequence, keys past 2^31 elements, bitwise-equal repeated calls,
large logits; plus every row written (NaN-filled output), device plan == host plan, and graph replays that read
rewritten bounds.
"""

from __future__ import annotations

import ctypes
import math
import os
import types

import numpy as np
import pytest
import torch

import golden_io
from karpo_decision_amd import _lib, global_attention, hip_attention, ops, sliding_attention, varlen, vision, workloads
from oracle import attention as oa

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS, REL_FRO = 2e-2, 2e-3, 1e-2


def assert_close(got: torch.Tensor, want: torch.Tensor, label: str = "") -> dict:
    got = got.detach().float().cpu()
    want = want.float().cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    assert torch.isfinite(got).all(), f"{label}: non-finite output"
    diff = (got - want).abs()
    stats = {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()),
             "rel_fro": float((got - want).norm() / want.norm().clamp_min(1e-30))}
    print(label, stats, flush=True)
    assert stats["max_abs"] <= MAX_ABS, (label, stats)
    assert stats["mean_abs"] <= MEAN_ABS, (label, stats)
    assert stats["rel_fro"] < REL_FRO, (label, stats)
    return stats


def sample_rows(q_cu: list[int], per_seq: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    rows = []
    for a, b in zip(q_cu[:-1], q_cu[1:]):
        n = b - a
        if n == 0:
            continue
        edge = list(range(a, min(b, a + 8))) + list(range(max(a, b - 8), b))
        extra = rng.integers(a, b, size=min(per_seq, n)).tolist()
        rows.extend(edge + extra)
    return sorted(set(rows))


def run_workload(w: workloads.Workload, plan: ops.Plan | None = None, spans_t=None) -> torch.Tensor:
    dev = w.query.device
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=dev)
    k_cu = torch.tensor(w.k_cu, dtype=torch.int32, device=dev)
    if spans_t is None and w.spans:
        spans_t = torch.tensor(w.spans, dtype=torch.int32, device=dev)
    rows = torch.tensor(w.key_rows, dtype=torch.int32, device=dev) if w.key_rows is not None else None
    fused = {}
    if w.q_norm is not None:
        fused["q_norm"] = ops.Norm(*w.q_norm)
    if w.rope is not None:
        fused["rope"] = w.rope
    if w.gate is not None:
        fused["gate"] = w.gate
    with torch.inference_mode():
        return ops.run(w.query, w.key, w.value, q_cu, k_cu, w.max_q, w.scale, w.window_left, w.window_right,
                       spans_t, plan, rows, **fused)


def check_workload(w: workloads.Workload, rows=None, groups=None, label=""):
    """Kernel vs oracle on ``rows`` (all when None) of the query heads of KV heads ``groups`` (all when None)."""
    from oracle import prologue

    got = run_workload(w)
    torch.cuda.synchronize()
    q, (k, v), gate = w.query.cpu(), w.gathered(), w.gate
    if w.q_norm is not None:  # the layer's query prologue on the CPU first
        q = prologue.rms_norm(q, w.q_norm[0], w.q_norm[1].cpu(), w.q_norm[2])
    if w.rope is not None:
        q = prologue.rope(q, *(t.cpu() for t in w.rope))
    if groups is not None:
        g = w.heads // w.kv_heads
        heads = [kv * g + i for kv in groups for i in range(g)]
        q, k, v = q[:, heads], k[:, groups], v[:, groups]
        got = got[:, heads]
        gate = gate[:, heads] if gate is not None else None
    want = oa.packed_attention(q, k.cpu(), v.cpu(), w.q_cu, w.k_cu, w.scale, w.window_left, w.window_right,
                               w.spans, dtype=torch.float32, rows=rows)
    if rows is not None:
        got = got[torch.tensor(rows, device=got.device)]
        gate = gate[torch.tensor(rows, device=gate.device)] if gate is not None else None
    if gate is not None:  # the output gate on the bf16 output, as the reference's sigmoid_mul
        want = prologue.gate(want.bfloat16(), gate.cpu())
    return assert_close(got, want, label or w.name)


@pytest.mark.parametrize("name", golden_io.names("random"))
def test_golden_vectors(gpu, name):
    c = golden_io.load(name)
    q, k, v = (c[t].to(gpu, torch.bfloat16) for t in ("q", "k", "v"))
    q_cu = torch.tensor(c["q_cu"], dtype=torch.int32, device=gpu)
    k_cu = torch.tensor(c["k_cu"], dtype=torch.int32, device=gpu)
    spans = torch.tensor(c["spans"], dtype=torch.int32, device=gpu) if c["spans"] else None
    max_q = max(b - a for a, b in zip(c["q_cu"][:-1], c["q_cu"][1:]))
    with torch.inference_mode():
        got = ops.run(q, k, v, q_cu, k_cu, max_q, c["scale"], c["left"], c["right"], spans)
    assert_close(got, c["want"], name)


def test_tiny_workload(gpu):
    check_workload(workloads.tiny(gpu))


def test_tiny_workload_fp32_is_refused(gpu):
    w = workloads.tiny(gpu, dtype=torch.float32)
    with pytest.raises(ValueError, match="bfloat16"):
        run_workload(w)


def test_qwen_full_attention_workload(gpu):
    w = workloads.qwen_full(gpu)
    check_workload(w)


def test_gemma_sliding_workload(gpu):
    w = workloads.gemma_sliding(gpu)
    check_workload(w, rows=sample_rows(w.q_cu, 64, 1), groups=[0, 7])


def test_gemma_sliding_workload_unit_scale(gpu):
    """Gemma's own scale is 1.0 (families/gemma/global_attention.py:130-131): logits in the tens."""
    w = workloads.gemma_sliding(gpu, scale=1.0)
    check_workload(w, rows=sample_rows(w.q_cu, 32, 2), groups=[1, 6])


@pytest.mark.parametrize("length", [32768, 131072])
def test_gemma_global_workload(gpu, length):
    w = workloads.gemma_global(length, gpu)
    check_workload(w, rows=sample_rows(w.q_cu, 384, 3), groups=[0, 15])


def test_global_layer_with_fused_query_prologue(gpu):
    w = workloads.with_prologue(workloads.gemma_global(32768, gpu), "gemma")
    check_workload(w, rows=sample_rows(w.q_cu, 256, seed=7), groups=[3])


def test_qwen_layer_with_fused_prologue_and_gate(gpu):
    w = workloads.with_prologue(workloads.qwen_full(gpu), "qwen")
    check_workload(w, rows=sample_rows(w.q_cu, 96, seed=8), groups=[0, 7])


def test_branched_workload(gpu):
    w = workloads.branched(gpu)
    check_workload(w, rows=sample_rows(w.q_cu, 48, seed=6), groups=[0, 15])


def test_mixed_multimodal_workload(gpu):
    w = workloads.mixed_multimodal(gpu)
    span_rows = [r for s, e in w.spans[:4] for r in (s, s + 1, (s + e) // 2, e - 2, e - 1, e)]
    rows = sorted(set(sample_rows(w.q_cu, 24, 4) + span_rows))
    check_workload(w, rows=rows, groups=[0, 2, 15])


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 4, 128), (4, 1, 64), (16, 8, 256), (32, 4, 512)])
def test_one_sequence_matches_float32_math(gpu, heads, kv_heads, head):
    torch.manual_seed(0)
    q = (torch.randn(300, heads, head, device=gpu) / 8).bfloat16()
    k = (torch.randn(300, kv_heads, head, device=gpu) / 8).bfloat16()
    v = torch.randn(300, kv_heads, head, device=gpu).bfloat16()
    cu = torch.tensor([0, 300], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, cu, cu, 300, 1.0)
    rep = heads // kv_heads
    qf, kf, vf = (t.float().transpose(0, 1) for t in (q, k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)))
    want = (torch.softmax(qf @ kf.transpose(1, 2), -1) @ vf).transpose(0, 1)
    assert_close(got, want.cpu(), f"one-sequence {heads}/{kv_heads}/{head}")


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 4, 128), (4, 1, 64), (32, 4, 512)])
@pytest.mark.parametrize("causal", [False, True])
def test_branched_varlen_with_an_empty_sequence(gpu, heads, kv_heads, head, causal):
    """A shared block of 1,000 rows and branches of 37 and 120 rows (each over the shared keys, then its own), and
    an empty virtual sequence between them (tests/gpu/test_triton_attention.py:69-84)."""
    torch.manual_seed(1)
    shared, b1, b2 = 1000, 37, 120
    n = shared + b1 + b2
    q = (torch.randn(n, heads, head, device=gpu) / 8).bfloat16()
    kk = (torch.randn(n, kv_heads, head, device=gpu) / 8).bfloat16()
    vv = torch.randn(n, kv_heads, head, device=gpu).bfloat16()
    rows = torch.cat([torch.arange(shared), torch.arange(shared), torch.arange(shared, shared + b1),
                      torch.arange(shared), torch.arange(shared + b1, n)]).to(gpu)
    k, v = kk.index_select(0, rows), vv.index_select(0, rows)
    q_cu = [0, shared, shared + b1, shared + b1, n]
    k_cu = [0, shared, 2 * shared + b1, 2 * shared + b1, 3 * shared + b1 + b2]
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, torch.tensor(q_cu, dtype=torch.int32, device=gpu),
                                   torch.tensor(k_cu, dtype=torch.int32, device=gpu), shared, 1.0, causal=causal)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, k_cu, 1.0, -1, 0 if causal else -1)
    assert_close(got, want, f"branched causal={causal}")


@pytest.mark.parametrize("heads,kv_heads,head,shapes", [(32, 16, 128, {1400: 2, 5000: 4, 70000: 3}),
                                                       (12, 4, 128, {1400: 2, 5000: 0, 70000: 3}),
                                                       (10, 2, 128, {1400: 2, 5000: 4, 70000: 3}),
                                                       (16, 8, 256, {1400: 2, 9000: 0})])
@pytest.mark.parametrize("left", [-1, 200])
def test_every_tile_shape_matches_the_oracle(gpu, heads, kv_heads, head, shapes, left):
    """max_q is an upper bound of the query runs that selects the tile shape (small, dual-block, wide, long; the
    narrow shape has its own tests; a GQA group of 3 takes the twelve-wave wide tile at head size 128, one of 5 the
    dual-block tile with one head per item): one pack run under each shape its max_q values select, each against
    the oracle."""
    torch.manual_seed(5)
    lengths = [1400, 513, 1, 700]
    cu = _lengths_cu(lengths)
    n = cu[-1]
    q = (torch.randn(n, heads, head, device=gpu) / 4).bfloat16()
    k = (torch.randn(n, kv_heads, head, device=gpu) / 4).bfloat16()
    v = torch.randn(n, kv_heads, head, device=gpu).bfloat16()
    cu_t = torch.tensor(cu, dtype=torch.int32, device=gpu)
    scale = 1 / math.sqrt(head)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), cu, cu, scale, left, 0)
    for max_q, shape in shapes.items():
        assert _lib.kernel_shape(heads, kv_heads, head, max_q) == shape
        with torch.inference_mode():
            got = ops.run(q, k, v, cu_t, cu_t, max_q, scale, window_left=left, window_right=0)
        assert_close(got, want, f"shape {shape} (max_q {max_q}, D={head}, left={left})")


def test_keys_past_32_bit_offsets(gpu):
    """Key rows of 16 heads x 128 = 2,048 elements: row 2^20 starts at element 2^31. A first sequence holds 2^20
    keys and no queries, a second 64 queries over the 300 keys after them (tests/gpu/test_triton_attention.py:93-104)."""
    torch.manual_seed(2)
    start, rows, keys = 1 << 20, 64, 300
    q = (torch.randn(rows, 32, 128, device=gpu) / 8).bfloat16()
    k = torch.zeros(start + keys, 16, 128, device=gpu, dtype=torch.bfloat16)
    v = torch.zeros(start + keys, 16, 128, device=gpu, dtype=torch.bfloat16)
    k[start:] = (torch.randn(keys, 16, 128, device=gpu) / 8).bfloat16()
    v[start:] = torch.randn(keys, 16, 128, device=gpu).bfloat16()
    q_cu = torch.tensor([0, 0, rows], dtype=torch.int32, device=gpu)
    k_cu = torch.tensor([0, start, start + keys], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, q_cu, k_cu, rows, 1.0)
    want = oa.packed_attention(q.cpu(), k[start:].cpu(), v[start:].cpu(), [0, rows], [0, keys], 1.0)
    assert_close(got, want, "keys past 2^31 elements")


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 16, 128), (4, 1, 64), (16, 8, 256), (32, 4, 512)])
def test_repeated_calls_are_bitwise_equal(gpu, heads, kv_heads, head):
    torch.manual_seed(3)
    q = torch.randn(500, heads, head, device=gpu).bfloat16()
    k = torch.randn(700, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(700, kv_heads, head, device=gpu).bfloat16()
    q_cu = torch.tensor([0, 200, 500], dtype=torch.int32, device=gpu)
    k_cu = torch.tensor([0, 300, 700], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        a = hip_attention.attend(q, k, v, q_cu, k_cu, 300, 0.1, causal=True)
        b = hip_attention.attend(q, k, v, q_cu, k_cu, 300, 0.1, causal=True)
    assert torch.equal(a, b)


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 4, 128), (4, 1, 64), (32, 4, 512)])
def test_large_logits_match_float32_math(gpu, heads, kv_heads, head):
    """Queries and keys without the usual 1/8, at scale 8: logits reach the hundreds, past float32's exp unless the
    kernel subtracts a running maximum (tests/gpu/test_triton_attention.py:116-128)."""
    torch.manual_seed(4)
    q = torch.randn(300, heads, head, device=gpu).bfloat16()
    k = torch.randn(300, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(300, kv_heads, head, device=gpu).bfloat16()
    cu = torch.tensor([0, 300], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, cu, cu, 300, 8.0)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), [0, 300], [0, 300], 8.0)
    assert_close(got, want, "large logits")


@pytest.mark.parametrize("heads,kv_heads,head", [(12, 4, 128), (10, 2, 128), (6, 2, 256), (12, 4, 64), (5, 5, 128)])
def test_gqa_groups_that_do_and_do_not_divide_a_tile(gpu, heads, kv_heads, head):
    """A group of 3 divides a 384-vector tile (its heads share one K/V stream), a group of 5 does not (one query head
    per work item); both must read K/V head h // G."""
    torch.manual_seed(10)
    q_cu = [0, 333, 1000, 1001]
    q = torch.randn(1001, heads, head, device=gpu).bfloat16()
    k = torch.randn(1001, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(1001, kv_heads, head, device=gpu).bfloat16()
    cu = torch.tensor(q_cu, dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        got = ops.run(q, k, v, cu, cu, 667, 1 / math.sqrt(head), -1, 0)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, q_cu, 1 / math.sqrt(head), -1, 0)
    assert_close(got, want, f"gqa {heads}/{kv_heads}/{head}")


def test_negative_and_zero_scale(gpu):
    torch.manual_seed(5)
    q = torch.randn(200, 8, 64, device=gpu).bfloat16()
    k = torch.randn(200, 2, 64, device=gpu).bfloat16()
    v = torch.randn(200, 2, 64, device=gpu).bfloat16()
    cu = torch.tensor([0, 80, 200], dtype=torch.int32, device=gpu)
    for scale in (-0.2, 0.0):
        with torch.inference_mode():
            got = ops.run(q, k, v, cu, cu, 120, scale, -1, 0)
        want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), [0, 80, 200], [0, 80, 200], scale, -1, 0)
        assert_close(got, want, f"scale {scale}")


def test_windows_and_spans_on_both_sides(gpu):
    torch.manual_seed(6)
    q_cu = [0, 700, 1500, 1510, 2600]
    q = torch.randn(2600, 16, 128, device=gpu).bfloat16()
    k = torch.randn(2600, 8, 128, device=gpu).bfloat16()
    v = torch.randn(2600, 8, 128, device=gpu).bfloat16()
    spans = [(100, 300), (1000, 1090), (1600, 2160)]
    st = torch.tensor(spans, dtype=torch.int32, device=gpu)
    cu = torch.tensor(q_cu, dtype=torch.int32, device=gpu)
    for left, right in ((200, 0), (-1, 0), (63, 64), (300, -1), (0, 0)):
        with torch.inference_mode():
            got = ops.run(q, k, v, cu, cu, 1090, 0.09, left, right, st)
        want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, q_cu, 0.09, left, right, spans)
        assert_close(got, want, f"window ({left}, {right}) with spans")


@pytest.mark.parametrize("seed", range(int(os.environ.get("KARPO_RANDOM_PACKS", "16"))))
def test_random_packs_under_every_shape(gpu, seed):
    """Seeded random packs: sequence lengths (some empty, Lq < Lk for branches), head geometry, head size, window
    sides, image spans, and a max_q that selects each tile shape the head size has (its runs' longest, or bounds
    above the small shape's and the wide shape's limits), each call against the oracle."""
    rng = np.random.default_rng(100 + seed)
    head = int(rng.choice([64, 128, 256, 512]))
    kv = int(rng.choice([1, 2, 4]))
    heads = kv * int(rng.choice([1, 2, 3, 8]))
    n_seq = int(rng.integers(1, 5))
    q_lens = [int(x) for x in rng.integers(0, 700, size=n_seq)]
    k_lens = [ql + (int(rng.integers(0, 300)) if rng.random() < 0.4 else 0) for ql in q_lens]
    q_cu, k_cu = _lengths_cu(q_lens), _lengths_cu(k_lens)
    left = int(rng.choice([-1, 0, 17, 200]))
    right = int(rng.choice([-1, 0, 0, 5]))
    spans = []
    if left >= 17 and right == 0 and q_lens[0] > 60:  # an image span inside the first sequence, within the window
        a = int(rng.integers(0, q_lens[0] - 40))
        spans = [(a, a + int(rng.integers(2, min(40, left + 2))))]
    torch.manual_seed(seed)
    q = (torch.randn(q_cu[-1], heads, head, device=gpu) / 3).bfloat16()
    k = (torch.randn(k_cu[-1], kv, head, device=gpu) / 3).bfloat16()
    v = torch.randn(k_cu[-1], kv, head, device=gpu).bfloat16()
    scale = 1 / math.sqrt(head)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, k_cu, scale, left, right, spans)
    cu_q = torch.tensor(q_cu, dtype=torch.int32, device=gpu)
    cu_k = torch.tensor(k_cu, dtype=torch.int32, device=gpu)
    st = torch.tensor(spans, dtype=torch.int32, device=gpu) if spans else None
    longest = max(q_lens)
    for max_q in sorted({longest, 9000, 70000}):
        with torch.inference_mode():
            got = ops.run(q, k, v, cu_q, cu_k, max_q, scale, left, right, st)
        shape = _lib.kernel_shape(heads, kv, head, max_q)
        assert_close(got, want, f"seed {seed}: lengths {q_lens}/{k_lens} H={heads}/{kv} D={head} window "
                                f"({left}, {right}) spans {spans} max_q {max_q} shape {shape}")


def _c_abi_call(q, k, v, o, q_cu, k_cu, max_q, scale, left, right, plan: ops.Plan | None = None, spans=None,
                status: list | None = None, gate=None, lse=None):
    """One karpo_attn_fwd through the C ABI into ``o`` (and ``lse``, (heads, total_q) fp32, if given); returns the
    workspace, which starts as 0x7f bytes (nothing in it may be read before the call writes it). With ``status`` (a
    list) the device planner's status word is appended to it (karpo_attn_device_status)."""
    lib = _lib.load()
    a = ops._args(q, k, v, o, q_cu, k_cu, q_cu.numel() - 1, max_q, scale, left, right, spans,
                  plan.tensor if plan is not None else None, list(plan.header) if plan is not None else None,
                  gate=gate)
    if lse is not None:
        a.lse = lse.data_ptr()
    need = ctypes.c_size_t()
    _lib.check(lib.karpo_attn_workspace_bytes(ctypes.byref(a), ctypes.byref(need)), "workspace")
    ws = torch.full((need.value,), 0x7F, dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), need.value
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.check(lib.karpo_attn_fwd(ctypes.byref(a), stream), "fwd")
    if status is not None:
        word = ctypes.c_int32(-1)
        _lib.check(lib.karpo_attn_device_status(ctypes.byref(a), stream, ctypes.byref(word)), "status")
        status.append(word.value)
    torch.cuda.synchronize()
    return ws


def _plan_parts(plan: torch.Tensor) -> tuple[list[int], list[tuple], list[tuple]]:
    """(header, merges, items) of a plan in the layout of karpo_attn.h."""
    plan = plan.cpu()
    h = _lib.PLAN_HEADER
    header = plan[:h].tolist()
    merges = [tuple(x) for x in plan[h: h + 4 * header[4]].view(-1, 4).tolist()]
    items = [tuple(x) for x in plan[header[6]: header[6] + 4 * header[0]].view(-1, 4).tolist()]
    return header, merges, items


def test_every_row_is_written_and_device_plan_matches_host_plan(gpu):
    """Through the C ABI: an output pre-filled with NaN has no NaN left; the device planner's work list is the host
    planner's (same header and split tiles, the same items as a multiset, ordered by non-increasing cost); running
    from the host plan gives the same bits. The Qwen-class pack in the dual-block tile shape (max_q 8192: above the
    small shape's runs) is small enough that its longest tiles split."""
    w = workloads.qwen_full(gpu, seed=7)
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=gpu)
    max_q = 8192
    o = torch.full_like(w.query, float("nan"))
    ws = _c_abi_call(w.query, w.key, w.value, o, q_cu, q_cu, max_q, w.scale, -1, 0)
    assert not torch.isnan(o).any()
    plan = ops.make_plan(w.q_cu, w.k_cu, w.heads, w.kv_heads, w.head_dim, -1, 0, device=gpu, max_q=max_q)
    assert plan.header[5] == 8 and plan.header[10] == 4  # eight waves of two query blocks
    host_header, host_merges, host_items = _plan_parts(plan.tensor)
    dev_header, dev_merges, dev_items = _plan_parts(ws.view(torch.int32)[: plan.tensor.numel()])
    assert host_header[4] > 0, "expected split tiles in this pack"
    assert dev_header == host_header
    assert dev_merges == host_merges
    assert sorted(dev_items) == sorted(host_items)
    # non-increasing cost along the device list (causal self-attention: steps 0 .. the tile's last row)
    rows, bn = host_header[1], host_header[2]
    costs = []
    for seg, t, pp, _ in dev_items:
        lq = w.q_cu[seg + 1] - w.q_cu[seg]
        steps = -(-min(lq, (t + 1) * rows) // bn)
        parts = pp >> 16
        costs.append(-(-steps // parts) + 1)
    assert all(a >= b for a, b in zip(costs, costs[1:]))
    o2 = torch.empty_like(w.query)
    _c_abi_call(w.query, w.key, w.value, o2, q_cu, q_cu, max_q, w.scale, -1, 0, plan=plan)
    assert torch.equal(o, o2)


@pytest.mark.parametrize("heads,kv_heads,head,max_q,decode,shape", [
    (8, 2, 128, 6000, False, 4), (12, 4, 128, 6000, False, 0), (8, 2, 128, 4096, False, 2),
    (8, 2, 128, 70000, False, 3), (8, 2, 128, 1, True, 1),
    (8, 2, 64, 6000, False, 0), (8, 2, 64, 1, True, 1), (8, 2, 256, 9000, False, 0), (8, 2, 256, 4096, False, 2),
    (8, 2, 256, 1, True, 1), (8, 2, 512, 6000, False, 0), (8, 2, 512, 1, True, 1)])
def test_split_tiles_device_plan_matches_host_plan(gpu, heads, kv_heads, head, max_q, decode, shape):
    """Split tiles in every tile shape that stores partials: the device planner's work list (planned into a workspace
    that starts as garbage) is the host planner's, so the output with its LSE, and the gated output (the C ABI takes
    no LSE with a gate), are the same bits either way, with every row written. Causal packs with one long sequence
    (its last tiles split), or decode-shaped ones (one query per sequence over many keys: the key steps split)."""
    if decode:
        q_lens, k_lens, left, right = [1] * 6, [24000, 9000, 3000, 700, 40, 0], -1, -1
    else:
        q_lens = [min(max_q, 2000), 300, 40, 0, 7]
        k_lens, left, right = q_lens, -1, 0
    cu_q, cu_k = _lengths_cu(q_lens), _lengths_cu(k_lens)
    assert _lib.kernel_shape(heads, kv_heads, head, max_q) == shape
    g = torch.Generator(device="cpu").manual_seed(head + max_q)
    q = torch.randn(cu_q[-1], heads, head, generator=g).to(torch.bfloat16).to(gpu)
    k, v = (torch.randn(cu_k[-1], kv_heads, head, generator=g).to(torch.bfloat16).to(gpu) for _ in range(2))
    gate = torch.randn(cu_q[-1], heads, head, generator=g).to(torch.bfloat16).to(gpu)
    q_cu = torch.tensor(cu_q, dtype=torch.int32, device=gpu)
    k_cu = torch.tensor(cu_k, dtype=torch.int32, device=gpu)
    plan = ops.make_plan(cu_q, cu_k, heads, kv_heads, head, left, right, device=gpu, max_q=max_q)
    assert plan.header[4] > 0, "expected split tiles in this pack"
    outs = []
    for use_plan in (None, plan):
        for use_gate in (None, gate):
            o = torch.full_like(q, float("nan"))
            lse = torch.full((heads, cu_q[-1]), float("nan") if use_gate is None else 0.0, dtype=torch.float32,
                             device=gpu)
            ws = _c_abi_call(q, k, v, o, q_cu, k_cu, max_q, head ** -0.5, left, right, plan=use_plan, gate=use_gate,
                             lse=lse if use_gate is None else None)
            if use_plan is None:
                dev_header, dev_merges, _ = _plan_parts(ws.view(torch.int32)[: plan.tensor.numel()])
                assert dev_header == list(plan.header) and dev_merges == _plan_parts(plan.tensor)[1]
            assert not torch.isnan(o).any() and not torch.isnan(lse).any()
            outs.append((o, lse))
    for (o_dev, lse_dev), (o_host, lse_host) in zip(outs[:2], outs[2:]):
        assert torch.equal(o_dev, o_host) and torch.equal(lse_dev, lse_host)
    assert not torch.equal(outs[0][0], outs[1][0])  # the gate applied
    # the longest sequence against the oracle (its tiles are the split ones)
    a, b = cu_q[1] - cu_q[0], cu_k[1] - cu_k[0]
    if not decode:
        want = oa.packed_attention(q[:a].cpu(), k[:b].cpu(), v[:b].cpu(), [0, a], [0, b], head ** -0.5, left, right)
        assert_close(outs[0][0][:a], want, f"split tiles: D={head} max_q {max_q} shape {shape}")


@pytest.mark.parametrize("n_seq", [1024, 1025, 6000])
def test_device_plan_of_many_sequences(gpu, n_seq):
    """Packs of a thousand sequences and more, empty ones among them (the device planner's workgroup scans 1,024
    sequences per pass): the device work list is the host planner's, and the output matches the oracle on a sample
    of the sequences."""
    rng = np.random.default_rng(n_seq)
    lengths = rng.integers(0, 24, n_seq)
    lengths[rng.integers(0, n_seq, 3)] = [3000, 1500, 700]
    cu = _lengths_cu(lengths.tolist())
    heads, kv_heads, head = 4, 2, 64
    g = torch.Generator(device="cpu").manual_seed(n_seq)
    q, k, v = (torch.randn(cu[-1], h, head, generator=g).to(torch.bfloat16).to(gpu) for h in (heads, kv_heads, kv_heads))
    q_cu = torch.tensor(cu, dtype=torch.int32, device=gpu)
    max_q = int(lengths.max())
    o = torch.full_like(q, float("nan"))
    ws = _c_abi_call(q, k, v, o, q_cu, q_cu, max_q, 0.125, -1, 0)
    assert not torch.isnan(o).any()
    plan = ops.make_plan(cu, cu, heads, kv_heads, head, -1, 0, device=gpu, max_q=max_q)
    host_header, host_merges, host_items = _plan_parts(plan.tensor)
    dev_header, dev_merges, dev_items = _plan_parts(ws.view(torch.int32)[: plan.tensor.numel()])
    assert dev_header == host_header
    assert dev_merges == host_merges
    assert sorted(dev_items) == sorted(host_items)
    for s in sorted(set(rng.integers(0, n_seq, 6).tolist()) | {int(np.argmax(lengths))}):
        a, b = cu[s], cu[s + 1]
        if a == b:
            continue
        want = oa.packed_attention(q[a:b].cpu(), k[a:b].cpu(), v[a:b].cpu(), [0, b - a], [0, b - a], 0.125, -1, 0)
        assert_close(o[a:b], want, f"{n_seq} sequences: sequence {s} of length {b - a}")


def _lengths_cu(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 16, 128), (32, 4, 256), (16, 8, 256), (8, 2, 64), (10, 2, 128), (32, 4, 512)])
def test_markers_only_layer(gpu, heads, kv_heads, head):
    """The markers-only global layer (families/gemma/packed.py:267-281): one query per virtual sequence over all of
    its keys, bidirectional, max_q = 1, through the reference-shaped hook. One-wave tiles, key steps split across
    the GPU and merged; compared with the oracle on every row, and every row written (NaN-filled, C ABI)."""
    torch.manual_seed(10 + head)
    k_lens = [32768, 7000, 1, 0, 300, 4097]
    k_cu = _lengths_cu(k_lens)
    m_cu = _lengths_cu([1 if n else 0 for n in k_lens])
    q = torch.randn(m_cu[-1], heads, head, device=gpu).bfloat16()
    k = torch.randn(k_cu[-1], kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(k_cu[-1], kv_heads, head, device=gpu).bfloat16()
    mc, kc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (m_cu, k_cu))
    scale = head ** -0.5
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, mc, kc, 1, scale)
    want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), m_cu, k_cu, scale, -1, -1)
    assert_close(got, want, f"markers {heads}/{kv_heads}/{head}")
    o = torch.full_like(q, float("nan"))
    _c_abi_call(q, k, v, o, mc, kc, 1, scale, -1, -1)
    assert torch.equal(o, got)


@pytest.mark.parametrize("left", [-1, 1023])
@pytest.mark.parametrize("heads,kv_heads,head", [(32, 16, 128), (16, 8, 256)])
def test_decode_shaped_causal_pack(gpu, heads, kv_heads, head, left):
    """Few queries per sequence over long key runs with the bottom-right alignment (branches, chunked prefill):
    causal and windowed, one-wave tiles when every sequence's queries fit one wave, wide tiles otherwise."""
    torch.manual_seed(11)
    k_lens = [9000, 40, 3000, 1, 17000]
    for q_lens in ([1, 1, 1, 1, 1], [7, 3, 16, 1, 12], [40, 17, 33, 1, 5]):
        q_cu, k_cu = _lengths_cu(q_lens), _lengths_cu(k_lens)
        q = torch.randn(q_cu[-1], heads, head, device=gpu).bfloat16()
        k = torch.randn(k_cu[-1], kv_heads, head, device=gpu).bfloat16()
        v = torch.randn(k_cu[-1], kv_heads, head, device=gpu).bfloat16()
        qc, kc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, k_cu))
        with torch.inference_mode():
            got = ops.run(q, k, v, qc, kc, max(q_lens), 0.08, left, 0)
        want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, k_cu, 0.08, left, 0)
        assert_close(got, want, f"decode {heads}/{kv_heads}/{head} left {left} q {q_lens}")


def test_reference_shaped_entry_points(gpu):
    """sliding_attention.attend, varlen.varlen_attn and global_attention.padded against the oracle."""
    torch.manual_seed(8)
    q = torch.randn(900, 16, 256, device=gpu).bfloat16()
    k = torch.randn(1100, 8, 256, device=gpu).bfloat16()
    v = torch.randn(1100, 8, 256, device=gpu).bfloat16()
    q_cu, k_cu = [0, 400, 900], [0, 500, 1100]
    qc, kc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, k_cu))
    with torch.inference_mode():
        got = sliding_attention.attend(q, k, v, qc, kc, 500, 600, 0.0625, 255)
    assert_close(got, oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), q_cu, k_cu, 0.0625, 255, 0), "sliding")

    q2, k2, v2 = q[:, :, :128].contiguous(), k[:, :, :128].contiguous(), v[:, :, :128].contiguous()
    with torch.inference_mode():
        got = varlen.varlen_attn(q2, k2, v2, qc, kc, 500, 600, window_size=(-1, 0), enable_gqa=True)
    want = oa.packed_attention(q2.cpu(), k2.cpu(), v2.cpu(), q_cu, k_cu, 1 / math.sqrt(128), -1, 0)
    assert_close(got, want, "varlen causal")
    with pytest.raises(ValueError, match="enable_gqa"):
        varlen.varlen_attn(q2, k2, v2, qc, kc, 500, 600)

    cu = torch.tensor([0, 700, 900], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        got = global_attention.padded(q2[None], k2[:900][None], v2[:900][None], cu, 900, True, 0.1)
    want = oa.packed_attention(q2.cpu(), k2[:900].cpu(), v2[:900].cpu(), [0, 700, 900], [0, 700, 900], 0.1, -1, 0)
    assert got.shape == (1, 900, 16, 128)
    assert_close(got[0], want, "padded")


def test_graph_replays_read_rewritten_bounds(gpu):
    """A captured call reads the bounds from device memory at replay time (serve/graphs.py:107-115): rewriting
    cu in place between replays changes the split, and each replay equals the eager call with those bounds."""
    torch.manual_seed(9)
    q = torch.randn(256, 8, 64, device=gpu).bfloat16()
    k = torch.randn(256, 2, 64, device=gpu).bfloat16()
    v = torch.randn(256, 2, 64, device=gpu).bfloat16()
    cu = torch.tensor([0, 100, 256], dtype=torch.int32, device=gpu)
    with torch.inference_mode():
        hip_attention.attend(q, k, v, cu, cu, 256, 0.125, causal=True)  # warm: library loaded, allocator primed
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = hip_attention.attend(q, k, v, cu, cu, 256, 0.125, causal=True)
        for split in (13, 64, 65, 200, 13):
            cu[1] = split
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            eager = hip_attention.attend(q, k, v, cu.clone(), cu.clone(), 256, 0.125, causal=True)
            torch.cuda.synchronize()
            assert torch.equal(out, eager), split
            want = oa.packed_attention(q.cpu(), k.cpu(), v.cpu(), [0, split, 256], [0, split, 256], 0.125, -1, 0)
            assert_close(out, want, f"graph split {split}")


def test_enable_installs_the_hook(gpu):
    import types

    def stub(causal):
        weight = torch.zeros(1, device=gpu)
        return types.SimpleNamespace(lm=types.SimpleNamespace(embed_tokens=types.SimpleNamespace(weight=weight)),
                                     causal_global=causal, global_attend=None)

    m = stub(False)
    hip_attention.enable(m, 131_072)
    assert m.global_attend is hip_attention.attend
    m = stub(True)
    hip_attention.enable(m, 32_768)
    assert m.global_attend.keywords == {"causal": True}


def _block_pack(prompts, window):
    """Bounds and gather tables of a block plan (families/gemma/packed.py:103-151): per prompt a shared block (its own
    virtual sequence) and branches whose keys are the shared rows (global) or the shared tail of window - 1 rows
    (sliding) followed by the branch's own rows. ``prompts``: [(shared, [branch lengths])]. Returns the pack's row
    count, q_cu, g_cu, s_cu, g_rows, s_rows (int64 lists), and m_cu (one marker per virtual sequence, its last row)."""
    q_cu, g_cu, s_cu, g_rows, s_rows, markers = [0], [0], [0], [], [], []
    at = 0
    for shared, branches in prompts:
        own = list(range(at, at + shared))
        q_cu.append(at + shared)
        g_rows += own
        s_rows += own
        g_cu.append(g_cu[-1] + shared)
        s_cu.append(s_cu[-1] + shared)
        markers.append(at + shared - 1)
        tail = own[max(0, shared - (window - 1)):]
        at += shared
        for n in branches:
            rows = list(range(at, at + n))
            q_cu.append(at + n)
            g_rows += own + rows
            s_rows += tail + rows
            g_cu.append(g_cu[-1] + shared + n)
            s_cu.append(s_cu[-1] + len(tail) + n)
            if n:
                markers.append(at + n - 1)
            at += n
    m_cu = [0]
    for a, b in zip(q_cu[:-1], q_cu[1:]):
        m_cu.append(m_cu[-1] + (1 if b > a else 0))
    return at, q_cu, g_cu, s_cu, g_rows, s_rows, m_cu, markers


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 16, 128), (16, 8, 256), (8, 2, 64), (32, 4, 512)])
def test_branch_keys_read_through_row_tables(gpu, heads, kv_heads, head):
    """The fused branch gather (families/gemma/packed.py:222-226): global, sliding and markers-only calls over the
    pack's own K/V with g_rows / s_rows equal, bit for bit, the calls on index_select copies, and match the oracle."""
    torch.manual_seed(12 + head)
    window = 300
    prompts = [(1000, [37, 120, 0]), (5, [400]), (700, []), (2, [3, 1])]
    total, q_cu, g_cu, s_cu, g_rows, s_rows, m_cu, markers = _block_pack(prompts, window)
    q = torch.randn(total, heads, head, device=gpu).bfloat16()
    k = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    qc, gc, sc, mc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, g_cu, s_cu, m_cu))
    gr, sr = (torch.tensor(x, dtype=torch.int64, device=gpu) for x in (g_rows, s_rows))
    max_q = max(b - a for a, b in zip(q_cu[:-1], q_cu[1:]))
    max_s = max(b - a for a, b in zip(s_cu[:-1], s_cu[1:]))
    scale = head ** -0.5
    with torch.inference_mode():
        fused = hip_attention.attend(q, k, v, qc, gc, max_q, scale, causal=True, rows=gr)
        copied = hip_attention.attend(q, k[gr], v[gr], qc, gc, max_q, scale, causal=True)
        assert torch.equal(fused, copied)
        want = oa.packed_attention(q.cpu(), k[gr].cpu(), v[gr].cpu(), q_cu, g_cu, scale, -1, 0)
        assert_close(fused, want, f"global gather {heads}/{kv_heads}/{head}")

        fused = sliding_attention.attend(q, k, v, qc, sc, max_q, max_s, scale, window - 1, rows=sr)
        copied = sliding_attention.attend(q, k[sr], v[sr], qc, sc, max_q, max_s, scale, window - 1)
        assert torch.equal(fused, copied)
        want = oa.packed_attention(q.cpu(), k[sr].cpu(), v[sr].cpu(), q_cu, s_cu, scale, window - 1, 0)
        assert_close(fused, want, f"sliding gather {heads}/{kv_heads}/{head}")

        qm = q[torch.tensor(markers, device=gpu)]
        fused = hip_attention.attend(qm, k, v, mc, gc, 1, scale, rows=gr)
        copied = hip_attention.attend(qm, k[gr], v[gr], mc, gc, 1, scale)
        assert torch.equal(fused, copied)
        want = oa.packed_attention(qm.cpu(), k[gr].cpu(), v[gr].cpu(), m_cu, g_cu, scale, -1, -1)
        assert_close(fused, want, f"markers gather {heads}/{kv_heads}/{head}")


def test_row_table_entries_outside_the_tensor_read_as_zero_keys(gpu):
    """Row-table entries outside [0, total_k) read as zero keys and values (logit 0, value 0), never out of bounds."""
    torch.manual_seed(13)
    q = torch.randn(64, 4, 128, device=gpu).bfloat16()
    k = torch.randn(100, 2, 128, device=gpu).bfloat16()
    v = torch.randn(100, 2, 128, device=gpu).bfloat16()
    rows = torch.arange(0, 100, device=gpu)
    rows[[3, 50, 77]] = torch.tensor([-1, 100, 1 << 30], device=gpu)
    cu = torch.tensor([0, 64], dtype=torch.int32, device=gpu)
    kc = torch.tensor([0, 100], dtype=torch.int32, device=gpu)
    kz, vz = k.clone(), v.clone()
    kz[[3, 50, 77]] = 0
    vz[[3, 50, 77]] = 0
    with torch.inference_mode():
        got = hip_attention.attend(q, k, v, cu, kc, 64, 0.1, causal=True, rows=rows)
    want = oa.packed_attention(q.cpu(), kz.cpu(), vz.cpu(), [0, 64], [0, 100], 0.1, -1, 0)
    assert_close(got, want, "out-of-range rows")


# ---- fused query prologue (norm, rotation) and output gate; keys' and values' norm_rope pass

def _angles(rows: int, r: int, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    a = torch.rand(rows, r // 2, generator=g) * 20
    return torch.cat((a.cos(), a.cos()), -1).bfloat16(), torch.cat((a.sin(), a.sin()), -1).bfloat16()


def assert_prologue_close(got: torch.Tensor, want: torch.Tensor, label: str) -> None:
    """The kernel's bf16 query after the prologue against oracle/prologue.py's: equal but on a small fraction of
    elements (below 1e-4), each within two bf16 ulps at its magnitude, or at unit magnitude (the normalised vector's
    scale) where the rotation cancels. The sum of squares adds in another order than torch's CPU reduction, which
    moves rsqrt by an fp32 ulp and, rarely, a normalised element across a bf16 rounding boundary; the rotation
    x cos - x' sin carries such one-ulp steps of both operands into its own rounding."""
    g, w = got.detach().float().cpu(), want.float()
    diff = (g - w).abs()
    tol = torch.clamp(w.abs(), min=1.0) * 2.0 ** -6
    frac = float((diff > 0).float().mean())
    worst = float((diff / tol).max())
    print(label, {"differing": frac, "worst_in_ulps": worst, "max_abs": float(diff.max())}, flush=True)
    assert worst <= 1.0 and frac < 1e-4, (label, worst, frac)


@pytest.mark.parametrize("heads,kv_heads,head", [(32, 16, 128), (16, 8, 256)])
def test_fused_gemma_query_norm_and_rotation(gpu, heads, kv_heads, head):
    """The query's Gemma4RMSNorm and rotation (Packed._q, families/gemma/packed.py:191-193; fused.py:21-26, :40-50) in
    the kernel's query load, on global and sliding layers at the reference's scale and at Gemma's own 1.0: the
    query the kernel used (query_out) is oracle/prologue.py's within two bf16 ulps at its magnitude (on fewer than
    1e-4 of the elements; equal elsewhere), and the attention on it matches
    the oracle with all three criteria at every scale (at 1.0 the running maximum is kept exact, p.tau = 0); against
    the oracle's own query all three hold at the reference's scale, the relative ones at 1.0."""
    from oracle import prologue

    torch.manual_seed(14)
    q_cu = [0, 700, 1500, 1501, 2600]
    raw = (torch.randn(q_cu[-1], heads, head) * 4).bfloat16()
    k = torch.randn(q_cu[-1], kv_heads, head).bfloat16()
    v = torch.randn(q_cu[-1], kv_heads, head).bfloat16()
    w = (torch.randn(head) * 0.5 + 1).bfloat16()
    cos, sin = _angles(q_cu[-1], head, 1)
    q_want = prologue.rope(prologue.rms_norm(raw, prologue.WEIGHT, w, 1e-6), cos, sin)
    cu = torch.tensor(q_cu, dtype=torch.int32, device=gpu)
    norm = ops.Norm(ops.NORM_WEIGHT, w.to(gpu), 1e-6)
    checks = []
    for left, causal, scale in ((-1, True, head ** -0.5), (511, True, head ** -0.5), (-1, False, head ** -0.5),
                                (-1, True, 1.0), (511, True, 1.0)):
        label = f"gemma prologue {heads}/{kv_heads}/{head} left {left} causal {causal} scale {scale:.3f}"
        used = torch.empty(raw.shape, dtype=torch.bfloat16, device=gpu)
        with torch.inference_mode():
            got = ops.run(raw.to(gpu), k.to(gpu), v.to(gpu), cu, cu, 1100, scale, left, 0 if causal else -1,
                          q_norm=norm, rope=(cos.to(gpu), sin.to(gpu)), query_out=used)
            # the same kernel on the query it used, without the prologue: the same bits
            again = ops.run(used, k.to(gpu), v.to(gpu), cu, cu, 1100, scale, left, 0 if causal else -1)
        assert torch.equal(got, again), label
        assert_prologue_close(used, q_want, label)
        right = 0 if causal else -1
        checks.append((got, oa.packed_attention(used.cpu(), k, v, q_cu, q_cu, scale, left, right),
                       label + " (its own query)", True))
        # against the oracle's own query: at scale 1.0 a one-ulp difference of a normalised element (the sum of
        # squares' order) moves a peaked row's output by up to ~1e-2 on top of the bf16 output grid (half an ulp is
        # 0.0156 at |o| >= 4), so there the relative criteria hold and max-abs is reported
        checks.append((got, oa.packed_attention(q_want, k, v, q_cu, q_cu, scale, left, right), label, scale < 1.0))
    failed = []
    for got, want, label, all_three in checks:  # every configuration's figures first, then the verdict
        try:
            if all_three:
                assert_close(got, want, label)
            else:
                diff = (got.float().cpu() - want.float()).abs()
                rel = float((got.float().cpu() - want.float()).norm() / want.float().norm())
                print(label, {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()), "rel_fro": rel}, flush=True)
                assert rel < REL_FRO and float(diff.mean()) <= MEAN_ABS, label
        except AssertionError as e:
            failed.append(str(e))
    assert not failed, failed


@pytest.mark.parametrize("max_q_of", ["pack", "markers"])
def test_fused_qwen_query_norm_rotation_and_gate(gpu, max_q_of):
    """Qwen3.5's full-attention layer (families/qwen/packed.py:108-125): the query half of q_proj's output with a
    Qwen3_5RMSNorm (1 + weight), partial rotation of the first 32 of 128 elements, and sigmoid(gate) on the output,
    all fused; the pack splits tiles (gate applied by the merge) and the markers-only form runs one-wave tiles."""
    from oracle import prologue

    torch.manual_seed(15)
    heads, kv_heads, head = 16, 8, 128
    lens = [2210, 1547, 1138, 861, 680]
    cu = _lengths_cu(lens)
    proj = (torch.randn(cu[-1], heads, 2 * head) * 3).bfloat16()  # q_proj output: (query, gate) halves per head
    raw, g = proj[..., :head], proj[..., head:]
    k = torch.randn(cu[-1], kv_heads, head).bfloat16()
    v = torch.randn(cu[-1], kv_heads, head).bfloat16()
    w = (torch.randn(head) * 0.2).bfloat16()
    cos, sin = _angles(cu[-1], 32, 2)
    if max_q_of == "markers":
        rows = [b - 1 for b in cu[1:]]
        raw, g, cos, sin = raw[rows], g[rows], cos[rows], sin[rows]
        q_cu, window = _lengths_cu([1] * len(lens)), (-1, -1)
    else:
        q_cu, window = cu, (-1, 0)
    q_want = prologue.rope(prologue.rms_norm(raw, prologue.ONE_PLUS, w, 1e-6), cos, sin)
    want = prologue.gate(oa.packed_attention(q_want, k, v, q_cu, cu, 1 / math.sqrt(head), *window).bfloat16(), g)
    proj_d = proj.to(gpu) if max_q_of == "pack" else torch.cat((raw, g), -1).to(gpu)
    qc, kc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, cu))
    module = types.SimpleNamespace(weight=w.to(gpu), variance_epsilon=1e-6)
    with torch.inference_mode():
        got = varlen.varlen_attn(proj_d[..., :head], k.to(gpu), v.to(gpu), qc, kc, max(b - a for a, b in zip(
            q_cu[:-1], q_cu[1:])), max(lens), scale=1 / math.sqrt(head), window_size=window, enable_gqa=True,
            q_norm=module, cos=cos.to(gpu), sin=sin.to(gpu), gate=proj_d[..., head:])
    assert_close(got, want, f"qwen prologue + gate ({max_q_of})")


@pytest.mark.parametrize("head", [64, 128, 256, 512])
def test_norm_rope_pass_for_keys_and_values(gpu, head):
    """karpo_attn_norm_rope (the keys' norm and rotation and the values' norm, Packed._kv) against
    oracle/prologue.py: bf16 results equal but for rare last-bit differences of the reciprocal square root."""
    from oracle import prologue

    torch.manual_seed(16)
    x = (torch.randn(333, 4, head) * 5).bfloat16()
    w = (torch.randn(head) * 0.5 + 1).bfloat16()
    cases = [(ops.NORM_WEIGHT, w, head), (ops.NORM_ONE_PLUS, w, 32), (ops.NORM_PLAIN, None, None),
             (ops.NORM_NONE, None, head)]
    for mode, weight, r in cases:
        cos, sin = _angles(333, r, 3) if r else (None, None)
        want = prologue.rms_norm(x, mode, weight, 1e-6) if mode != ops.NORM_NONE else x
        if r:
            want = prologue.rope(want, cos, sin)
        xd = x.to(gpu)
        norm = ops.Norm(mode, weight.to(gpu) if weight is not None else None, 1e-6)
        rope = (cos.to(gpu), sin.to(gpu)) if r else None
        with torch.inference_mode():
            got = ops.norm_rope(xd, norm, rope).cpu()
            inplace = ops.norm_rope(xd, norm, rope, out=xd).cpu()
        assert torch.equal(got, inplace)
        diff = (got.float() - want.float()).abs()
        ulp = want.float().abs().clamp_min(1e-30) * 2 ** -7
        assert (diff <= ulp).all(), (head, mode, float(diff.max()))
        assert (diff > 0).float().mean() < 1e-2, (head, mode, float((diff > 0).float().mean()))


# ---- every row of the full-size layers; row tables under long runs; the device planner's contract check

def check_every_row(w: workloads.Workload, per_group: int, seed: int):
    """The layer through the C ABI with its host plan (as bench.py runs it) into a NaN-filled output: every row of
    every head is written and finite; then ``per_group`` seeded rows of every KV group against the oracle."""
    dev = w.query.device
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=dev)
    k_cu = torch.tensor(w.k_cu, dtype=torch.int32, device=dev)
    spans = torch.tensor(w.spans, dtype=torch.int32, device=dev) if w.spans else None
    plan = ops.make_plan(w.q_cu, w.k_cu, w.heads, w.kv_heads, w.head_dim, w.window_left, w.window_right, dev)
    o = torch.full_like(w.query, float("nan"))
    _c_abi_call(w.query, w.key, w.value, o, q_cu, k_cu, w.max_q, w.scale, w.window_left, w.window_right, plan=plan,
                spans=spans)
    finite = torch.isfinite(o).all(dim=2)  # (rows, heads)
    bad = (~finite).nonzero()
    assert bad.numel() == 0, f"{w.name}: {bad.shape[0]} (row, head) vectors unwritten or not finite, e.g. {bad[:4]}"
    rng = np.random.default_rng(seed)
    rows = sorted(set(rng.integers(0, w.q_cu[-1], per_group * w.kv_heads).tolist()))
    want = oa.packed_attention(w.query.cpu(), w.key.cpu(), w.value.cpu(), w.q_cu, w.k_cu, w.scale, w.window_left,
                               w.window_right, w.spans, dtype=torch.float32, rows=rows)
    got = o[torch.tensor(rows, device=dev)]
    for kv in range(w.kv_heads):  # every head of every KV group on the sampled rows
        g = w.heads // w.kv_heads
        assert_close(got[:, kv * g:(kv + 1) * g], want[:, kv * g:(kv + 1) * g], f"{w.name} KV group {kv}")


@pytest.mark.parametrize("name", ["global32k", "global131k", "sliding", "multimodal"])
def test_full_size_layers_write_every_row_of_every_head(gpu, name):
    """The metric's layer at 32k and 131k, the sliding layer and the multimodal pack: no (row, head) output is left
    unwritten or non-finite, and every head matches the oracle on 16 seeded rows per KV group."""
    w = workloads.named(name, gpu, 0)
    check_every_row(w, 16, seed=len(name))


@pytest.mark.parametrize("heads,kv_heads,head,max_q", [(32, 16, 128, 5000), (32, 16, 128, 70000),
                                                        (16, 8, 256, 9000)])
def test_row_tables_with_long_runs_take_the_four_wave_tiles(gpu, heads, kv_heads, head, max_q):
    """Calls through a row table whose max_q selects the wide or long tiles without one (head size 128 above 4,096
    and 65,536 queries, 256 above 8,192) run the four-wave tiles instead: global and sliding layers of a block plan
    against the oracle."""
    assert _lib.kernel_shape(heads, kv_heads, head, max_q, gather=True) == 2
    torch.manual_seed(29 + head)
    window = 300
    prompts = [(1000, [37, 120, 0]), (5, [400]), (700, []), (2, [3, 1])]
    total, q_cu, g_cu, s_cu, g_rows, s_rows, m_cu, markers = _block_pack(prompts, window)
    q = torch.randn(total, heads, head, device=gpu).bfloat16()
    k = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    qc, gc, sc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, g_cu, s_cu))
    gr, sr = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (g_rows, s_rows))
    scale = head ** -0.5
    with torch.inference_mode():
        got = ops.run(q, k, v, qc, gc, max_q, scale, -1, 0, None, None, gr)
        want = oa.packed_attention(q.cpu(), k[gr].cpu(), v[gr].cpu(), q_cu, g_cu, scale, -1, 0)
        assert_close(got, want, f"global rows {heads}/{kv_heads}/{head} max_q {max_q}")
        plan = ops.make_plan(q_cu, g_cu, heads, kv_heads, head, -1, 0, gpu, max_q=max_q, gather=True)
        planned = ops.run(q, k, v, qc, gc, max_q, scale, -1, 0, None, plan, gr)
        assert torch.equal(planned, got)
        got = ops.run(q, k, v, qc, sc, max_q, scale, window - 1, 0, None, None, sr)
        want = oa.packed_attention(q.cpu(), k[sr].cpu(), v[sr].cpu(), q_cu, s_cu, scale, window - 1, 0)
        assert_close(got, want, f"sliding rows {heads}/{kv_heads}/{head} max_q {max_q}")


def test_device_planner_refuses_bounds_that_break_the_contract(gpu):
    """Device bounds the host cannot see: a query run longer than max_q, or rows past total_q. The device planner
    plans nothing (no row is read or written: a sentinel output stays as it was) and leaves KARPO_ATTN_ERR_BOUNDS in
    the workspace's status word; valid bounds leave KARPO_ATTN_OK. The 200-row query and output of the second case
    are views of 300-row buffers (total_q 200): were the guard to fail, the kernel's reads and writes of rows
    200-259 would stay inside the allocations and show as changed sentinel rows, never as an access past them."""
    torch.manual_seed(31)
    q = torch.randn(300, 4, 64, device=gpu).bfloat16()
    k = torch.randn(300, 2, 64, device=gpu).bfloat16()
    cases = [([0, 100, 300], 150), ([0, 100, 260], 300)]  # a run of 200 over max_q 150; rows past a 200-row query
    for cu, max_q in cases:
        rows = 300 if cu == cases[0][0] else 200
        cu_t = torch.tensor(cu, dtype=torch.int32, device=gpu)
        sentinel = torch.full_like(q, 7.0)  # 300 rows whatever the call's total_q
        status = []
        _c_abi_call(q[:rows], k, k, sentinel[:rows], cu_t, cu_t, max_q, 0.125, -1, 0, status=status)
        assert status == [_lib.ERR_BOUNDS], (cu, max_q, status)
        assert bool((sentinel == 7.0).all()), "a refused plan wrote output rows"
    # key rows past the key tensor (key_bound 250: a view of the 300-row keys, so a failed guard stays in bounds)
    q_cu_t = torch.tensor([0, 100, 200], dtype=torch.int32, device=gpu)
    k_cu_t = torch.tensor([0, 100, 280], dtype=torch.int32, device=gpu)
    sentinel = torch.full_like(q, 7.0)
    status = []
    _c_abi_call(q[:200], k[:250], k[:250], sentinel[:200], q_cu_t, k_cu_t, 200, 0.125, -1, 0, status=status)
    assert status == [_lib.ERR_BOUNDS], status
    assert bool((sentinel == 7.0).all()), "a refused plan wrote output rows"
    cu_t = torch.tensor([0, 100, 300], dtype=torch.int32, device=gpu)
    o = torch.full_like(q, float("nan"))
    status = []
    _c_abi_call(q, k, k, o, cu_t, cu_t, 200, 0.125, -1, 0, status=status)
    assert status == [_lib.OK] and not torch.isnan(o).any()


def test_branched_sliding_pack_with_row_tables_and_image_spans(gpu):
    """A sliding layer of a block plan with images in the shared blocks and in branches (the reference's image
    layouts), its branch keys read through the plan's s_rows table and the images' spans folded into the same
    launch: against the oracle on the gathered keys with the spans (the spans' semantics against rule_a | same-image
    are pinned on the CPU, tests/test_vision.py)."""
    from test_vision import LAYOUTS, SOFT, WINDOW, pack, sliding_plan

    seqs = (LAYOUTS["images-in-the-shared-block-and-two-branches"]() + LAYOUTS["image-in-a-branch"]()
            + LAYOUTS["branch-image-within-a-window-of-the-shared-block"]())
    ids, seg, _, bounds, spans = pack(seqs)
    found = vision.soft_token_spans(ids, SOFT, WINDOW, bounds)
    assert found == spans
    q_cu, s_cu, s_rows = sliding_plan(seg, bounds, WINDOW)
    heads, kv_heads, head = 16, 8, 256
    torch.manual_seed(33)
    total = len(ids)
    q = torch.randn(total, heads, head, device=gpu).bfloat16()
    k = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    v = torch.randn(total, kv_heads, head, device=gpu).bfloat16()
    qc, sc = (torch.tensor(x, dtype=torch.int32, device=gpu) for x in (q_cu, s_cu))
    sr = torch.tensor(s_rows, dtype=torch.int32, device=gpu)
    span_t = vision.span_tensor(found, gpu)
    max_q = max(b - a for a, b in zip(q_cu[:-1], q_cu[1:]))
    max_s = max(b - a for a, b in zip(s_cu[:-1], s_cu[1:]))
    for scale in (head ** -0.5, 1.0):
        with torch.inference_mode():
            got = sliding_attention.attend(q, k, v, qc, sc, max_q, max_s, scale, WINDOW - 1, spans=span_t, rows=sr)
        gathered = torch.tensor(s_rows)
        want = oa.packed_attention(q.cpu(), k.cpu()[gathered], v.cpu()[gathered], q_cu, s_cu, scale, WINDOW - 1, 0,
                                   found)
        assert_close(got, want, f"branched sliding pack with spans and s_rows, scale {scale}")
