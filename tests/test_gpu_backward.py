"""The backward kernels (karpo_attn_bwd) and the forward's log-sum-exp against the CPU oracle on an MI355X.

Gradients of sum(out * grad) for bf16 inputs, against torch autograd through the oracle in float32 on the same
inputs (oracle/attention.py packed_grads): relative Frobenius error < 1e-2 for out, dq, dk and dv, and within twice
the error of the oracle's own bf16 run plus 2e-3 (the reference's criterion for its backward kernels,
tests/gpu/test_packed_gemma.py:173-184). The log-sum-exp within 1e-2 absolute of the oracle's float64 value (P sums
are bf16-rounded in the kernel), -inf exactly for rows that see no key. Layouts: causal GQA with an empty and a
one-row sequence, branches (Lk > Lq), more queries than keys, sliding and two-sided windows, image spans,
bidirectional packs, a group size that does not divide a tile, negative and zero scales (at zero the oracle's dq and
dk are exact zeros, and so must the kernels' be); bitwise-equal repeated calls.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from karpo_decision_amd import ops
from oracle import attention as oa

pytestmark = pytest.mark.gpu

REL_FRO = 1e-2


def rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def make_pack(q_lens, k_lens, heads, kv_heads, d, seed, spans_local=()):
    g = torch.Generator().manual_seed(seed)
    q_cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(int).tolist()
    k_cu = np.concatenate([[0], np.cumsum(k_lens)]).astype(int).tolist()
    q = torch.randn(q_cu[-1], heads, d, generator=g).bfloat16()
    k = torch.randn(k_cu[-1], kv_heads, d, generator=g).bfloat16()
    v = torch.randn(k_cu[-1], kv_heads, d, generator=g).bfloat16()
    do = torch.randn(q_cu[-1], heads, d, generator=g).bfloat16()
    spans = [(q_cu[s] + a, q_cu[s] + b) for s, a, b in spans_local]
    return q, k, v, do, q_cu, k_cu, spans


def kernel_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans):
    dev = torch.device("cuda")
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
    qc = torch.tensor(q_cu, dtype=torch.int32, device=dev)
    kc = torch.tensor(k_cu, dtype=torch.int32, device=dev)
    sp = torch.tensor(spans, dtype=torch.int32, device=dev) if spans else None
    max_q = max(b - a for a, b in zip(q_cu[:-1], q_cu[1:]))
    out = ops.attention(*xs, qc, kc, max_q, scale, left, right, sp)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    return [out.detach()] + [x.grad for x in xs]


LAYOUTS = [
    # (q lengths, k lengths, heads, kv heads, head_dim, left, right, spans (sequence, start, end), scale)
    ([300, 1, 0, 130], [300, 1, 0, 130], 8, 2, 128, -1, 0, [], None),
    ([64, 100], [200, 100], 8, 4, 128, -1, 0, [], None),                 # branches: Lk > Lq
    ([40, 70], [20, 70], 4, 2, 64, -1, 0, [], None),                     # Lq > Lk: leading rows see nothing
    ([257, 190], [257, 190], 4, 2, 256, 63, 0, [], None),               # sliding window
    ([150, 90], [150, 90], 4, 1, 64, -1, -1, [(0, 10, 50)], None),      # bidirectional with a span
    ([200], [200], 8, 8, 128, -1, 0, [(0, 30, 90), (0, 120, 121)], None),  # image spans under causal
    ([160, 33], [160, 33], 4, 2, 128, 5, 7, [(0, 40, 72)], None),       # two-sided window and a span
    ([129, 77], [129, 77], 6, 2, 128, -1, 0, [], None),                  # group 3 does not divide a tile
    ([700, 333], [700, 333], 16, 2, 128, -1, 0, [], None),               # group 8: steps cross head boundaries
    ([500, 47], [500, 47], 16, 4, 128, 100, 0, [], None),                # group 4 under a window
    ([100], [130], 4, 2, 128, 31, 0, [], -0.09),                         # negative scale, window, branch
    ([90, 33], [90, 33], 4, 2, 128, -1, 0, [], 0.0),                     # zero scale: P uniform, dQ = dK = 0
    ([70, 51], [90, 51], 4, 2, 256, 40, 0, [], 0.0),                     # zero scale at 256 under a window
    ([96, 64], [96, 64], 4, 2, 256, -1, 0, [(1, 8, 40)], None),
    ([300, 1, 0, 130], [300, 1, 0, 130], 8, 1, 512, -1, 0, [], None),   # head size 512: wave pairs
    ([64, 100], [200, 100], 8, 2, 512, -1, 0, [(1, 10, 40)], None),      # branches and a span at 512
    ([40, 70], [20, 70], 4, 4, 512, 31, 0, [], -0.05),                  # Lq > Lk, window, negative scale at 512
]


@pytest.mark.parametrize("layout", LAYOUTS, ids=[f"L{i}" for i in range(len(LAYOUTS))])
def test_gradients_match_float32(gpu, layout):
    q_lens, k_lens, heads, kv_heads, d, left, right, spans_local, scale = layout
    q, k, v, do, q_cu, k_cu, spans = make_pack(q_lens, k_lens, heads, kv_heads, d, seed=len(q_lens) + d + heads,
                                               spans_local=spans_local)
    scale = d ** -0.5 if scale is None else scale
    print("case", q_lens, k_lens, heads, kv_heads, d, left, right, spans, scale, flush=True)
    got = kernel_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans)
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans, dtype=torch.float32)
    base = oa.packed_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans, dtype=torch.bfloat16)
    for name, x, w, b in zip(("out", "dq", "dk", "dv"), got, want, base):
        assert torch.isfinite(x).all(), name
        r, rb = rel(x, w), rel(b, w)
        print(name, f"rel {r:.2e} (oracle bf16 {rb:.2e})", flush=True)
        assert r < REL_FRO, (name, r)
        assert r < 2 * rb + 2e-3, (name, r, rb)


@pytest.mark.parametrize("seed", range(int(os.environ.get("KARPO_RANDOM_TRAIN_PACKS", "10"))))
def test_random_packs_train(gpu, seed):
    """Seeded random packs through the differentiable operator: lengths (empty sequences, Lk > Lq branches), head
    geometry, head sizes 64-512, window sides, an image span; out, dq, dk, dv against autograd through the oracle,
    to the layouts' criterion."""
    rng = np.random.default_rng(700 + seed)
    d = int(rng.choice([64, 128, 256, 512]))
    kv = int(rng.choice([1, 2, 4]))
    heads = kv * int(rng.choice([1, 2, 3]))
    n = int(rng.integers(1, 4))
    q_lens = [int(x) for x in rng.integers(0, 260, size=n)]
    k_lens = [ql + (int(rng.integers(0, 120)) if rng.random() < 0.4 else 0) for ql in q_lens]
    left = int(rng.choice([-1, 0, 17, 90]))
    right = int(rng.choice([-1, 0, 0, 3]))
    spans_local = []
    if left >= 17 and right == 0 and q_lens[0] > 50:
        a = int(rng.integers(0, q_lens[0] - 30))
        spans_local = [(0, a, a + int(rng.integers(2, min(30, left + 2))))]
    q, k, v, do, q_cu, k_cu, spans = make_pack(q_lens, k_lens, heads, kv, d, seed=seed, spans_local=spans_local)
    scale = d ** -0.5
    print("case", seed, q_lens, k_lens, heads, kv, d, left, right, spans, flush=True)
    if max(q_lens) == 0:
        pytest.skip("an empty pack has no gradients to compare")
    got = kernel_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans)
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans, dtype=torch.float32)
    base = oa.packed_grads(q, k, v, do, q_cu, k_cu, scale, left, right, spans, dtype=torch.bfloat16)
    for name, x, w, b in zip(("out", "dq", "dk", "dv"), got, want, base):
        assert torch.isfinite(x).all(), name
        if float(w.float().abs().max()) < 1e-3:
            # the gradient vanishes in exact arithmetic (window (0, 0): every row sees one key, O = that V row, so
            # dS = P (dP - D) = 0 and dq, dk are rounding noise in both): the kernel's must be as small
            print(name, f"vanishing: max-abs {float(x.float().abs().max()):.1e} (oracle {float(w.float().abs().max()):.1e})")
            assert float(x.float().abs().max()) < 1e-3, name
            continue
        r, rb = rel(x, w), rel(b, w)
        print(name, f"rel {r:.2e} (oracle bf16 {rb:.2e})", flush=True)
        assert r < REL_FRO, (name, r)
        assert r < 2 * rb + 2e-3, (name, r, rb)


@pytest.mark.parametrize("heads,kv_heads,d", [(8, 2, 128), (4, 2, 64), (4, 2, 256)])
def test_lse_matches_the_oracle(gpu, heads, kv_heads, d):
    q, k, v, _, q_cu, k_cu, spans = make_pack([300, 40, 0, 77], [300, 20, 0, 90], heads, kv_heads, d, seed=3,
                                              spans_local=[(0, 50, 80)])
    dev = torch.device("cuda")
    qc = torch.tensor(q_cu, dtype=torch.int32, device=dev)
    kc = torch.tensor(k_cu, dtype=torch.int32, device=dev)
    sp = torch.tensor(spans, dtype=torch.int32, device=dev)
    scale = d ** -0.5
    out, lse = ops.packed_attention_lse(q.to(dev), k.to(dev), v.to(dev), qc, kc, 300, scale, -1, 0, sp)
    want = oa.packed_lse(q, k, q_cu, k_cu, scale, -1, 0, spans)
    got = lse.cpu().double()
    none = torch.isinf(want)
    assert none.any()  # sequence 1 has 40 queries over 20 keys: its first 20 rows see none
    assert torch.equal(torch.isinf(got), none) and (got[none] < 0).all()
    assert float((got[~none] - want[~none]).abs().max()) < 1e-2
    plain = ops.run(q.to(dev), k.to(dev), v.to(dev), qc, kc, 300, scale, -1, 0, sp)
    assert torch.equal(out, plain)  # asking for the lse leaves the output as it is


def test_larger_pack_matches_float32(gpu):
    """Four thousand rows, several tiles per sequence in both kernels, GQA 4."""
    q, k, v, do, q_cu, k_cu, spans = make_pack([2100, 1500, 400], [2100, 1500, 400], 8, 2, 128, seed=21)
    got = kernel_grads(q, k, v, do, q_cu, k_cu, 128 ** -0.5, -1, 0, spans)
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, 128 ** -0.5, -1, 0, spans, dtype=torch.float32)
    for name, x, w in zip(("out", "dq", "dk", "dv"), got, want):
        r = rel(x, w)
        print(name, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (name, r)


def test_backward_is_deterministic(gpu):
    """No atomics: GQA key/value gradients sum in a fixed order, so repeated calls agree bit for bit."""
    q, k, v, do, q_cu, k_cu, spans = make_pack([500, 260], [500, 300], 16, 4, 128, seed=5)
    a = kernel_grads(q, k, v, do, q_cu, k_cu, 0.1, -1, 0, spans)
    b = kernel_grads(q, k, v, do, q_cu, k_cu, 0.1, -1, 0, spans)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


@pytest.mark.parametrize("q_lens", [[2000, 100, 37], [3000] + [1] * 260],
                         ids=["mixed-lengths", "many-short-sequences"])
def test_long_key_tiles_split_over_their_query_steps(gpu, monkeypatch, q_lens):
    """One long causal sequence among short ones: the device planner splits its first key tiles over their query
    steps (each part of the dK / dV kernel stores fp32 partials, bwd_merge_kernel sums them in part order). The key
    tiles' plan in the workspace (which starts as garbage) lists split tiles; the gradients match the oracle and
    repeated calls are bitwise equal. With 260 one-token sequences beside it the key tiles number 2,296 workgroups of
    capacity (8 key/value heads); each part's two row-step groups add their sums before the part stores them."""
    seen = []
    real = ops._workspace

    def capture(lib, fn, args, device):
        ws = real(lib, fn, args, device)
        if fn.__name__ == "karpo_attn_bwd_workspace_bytes":
            ws.fill_(0x7F)
            seen.append(ws)
        return ws

    monkeypatch.setattr(ops, "_workspace", capture)
    heads, kv_heads, d = (8, 2, 128) if len(q_lens) < 10 else (16, 8, 128)
    q, k, v, do, q_cu, k_cu, spans = make_pack(q_lens, q_lens, heads, kv_heads, d, seed=41)
    got = kernel_grads(q, k, v, do, q_cu, k_cu, d ** -0.5, -1, 0, spans)
    # the workspace: per-row stats ([heads][2][total_q] fp32, 256-byte aligned), the query tiles' plan (header, then
    # 4 ints per tile of the capacity: 128 vectors per tile, 128 / group rows), then the key tiles' plan
    ws = seen[-1].view(torch.int32).cpu()
    total_q, n_seq, group = sum(q_lens), len(q_lens), heads // kv_heads
    rows = 128 // (group if 128 % group == 0 else 1)
    tiles_q = min(-(-total_q // rows) + n_seq, n_seq * -(-max(q_lens) // rows))
    plan_k = -(-(heads * 2 * total_q * 4) // 256) * 256 // 4 + 12 + 4 * tiles_q
    header = ws[plan_k: plan_k + 12].tolist()
    assert header[1] == 128 and header[2] == 32 and header[5] == 4, header  # keys per tile, rows per step, waves
    assert header[4] > 0, "expected split key tiles"
    merges = ws[plan_k + 12: plan_k + 12 + 4 * header[4]].view(-1, 4).tolist()
    assert all(seg == 0 and parts >= 2 for seg, _, parts, _ in merges)  # the long sequence's tiles
    tiles_k = -(-sum(q_lens) // 128) + n_seq
    assert (tiles_k * kv_heads >= 2048) == (len(q_lens) > 10)  # the two-launch path's threshold
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, d ** -0.5, -1, 0, spans, dtype=torch.float32)
    for name, x, w in zip(("out", "dq", "dk", "dv"), got, want):
        r = rel(x, w)
        print(name, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (name, r)
    again = kernel_grads(q, k, v, do, q_cu, k_cu, d ** -0.5, -1, 0, spans)
    for x, y in zip(got, again):
        assert torch.equal(x, y)


def test_backward_refuses_what_it_does_not_take(gpu):
    dev = torch.device("cuda")
    cu = torch.tensor([0, 8], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        ops.attention(*(torch.randn(8, 2, 96, device=dev).bfloat16(),) * 3, cu, cu, 8, 0.1)
    q = torch.randn(8, 2, 64, device=dev).bfloat16()
    out, lse = ops.packed_attention_lse(q, q, q, cu, cu, 8, 0.1, -1, 0, None)
    with pytest.raises(ValueError):
        ops.packed_attention_backward(out, q, q, q, out, lse[:, :4], cu, cu, 8, 0.1, -1, 0, None)


def test_many_key_tiles(gpu):
    """Head size 128 with 32 key/value heads over 8,192 keys (2,048 key-tile workgroups, eight GPU-fulls), against
    the oracle like the smaller packs above."""
    q, k, v, do, q_cu, k_cu, spans = make_pack([6000, 2192], [6000, 2192], 32, 32, 128, seed=31)
    got = kernel_grads(q, k, v, do, q_cu, k_cu, 128 ** -0.5, -1, 0, spans)
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, 128 ** -0.5, -1, 0, spans, dtype=torch.float32)
    for name, x, w in zip(("out", "dq", "dk", "dv"), got, want):
        r = rel(x, w)
        print(name, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (name, r)


def test_sliding_attend_trains(gpu):
    """sliding_attention.attend under autograd (the reference's FA4 operator pair): gradients of a windowed pack with
    an image span against the oracle; a row table with gradients is refused."""
    from karpo_decision_amd import sliding_attention

    q, k, v, do, q_cu, k_cu, spans = make_pack([300, 150], [340, 150], 8, 4, 256, seed=41, spans_local=[(0, 20, 60)])
    dev = torch.device("cuda")
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
    qc, kc = (torch.tensor(x, dtype=torch.int32, device=dev) for x in (q_cu, k_cu))
    sp = torch.tensor(spans, dtype=torch.int32, device=dev)
    out = sliding_attention.attend(*xs, qc, kc, 300, 340, 0.0625, 63, spans=sp)
    out.backward(do.to(dev))
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, 0.0625, 63, 0, spans, dtype=torch.float32)
    for name, x, w in zip(("out", "dq", "dk", "dv"), [out.detach()] + [x.grad for x in xs], want):
        r = rel(x, w)
        print("sliding", name, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (name, r)
    with pytest.raises(ValueError, match="rows"):
        sliding_attention.attend(*xs, qc, kc, 300, 340, 0.0625, 63, rows=torch.arange(490, device=dev))


@pytest.mark.parametrize("causal", [True, False])
def test_global_attend_one_sequence_trains(gpu, causal):
    """global_attention.attend (one virtual sequence, lengths on the device, the reference's cuDNN pair): a branch's
    queries over its shared keys plus its own, forward without grad and gradients with it, against the oracle."""
    from karpo_decision_amd import global_attention

    q, k, v, do, q_cu, k_cu, _ = make_pack([200], [520], 8, 2, 128, seed=43)
    dev = torch.device("cuda")
    lens = global_attention.lengths(q_cu, k_cu, dev)
    right = 0 if causal else -1
    with torch.no_grad():
        plain = global_attention.attend(q.to(dev), k.to(dev), v.to(dev), lens[0, 0, :1], lens[0, 1, :1], causal,
                                        0.1)
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
    out = global_attention.attend(*xs, lens[0, 0, :1], lens[0, 1, :1], causal, 0.1)
    out.backward(do.to(dev))
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, 0.1, -1, right, dtype=torch.float32)
    assert rel(plain, want[0]) < REL_FRO
    for name, x, w in zip(("out", "dq", "dk", "dv"), [out.detach()] + [x.grad for x in xs], want):
        r = rel(x, w)
        print("global", causal, name, f"rel {r:.2e}", flush=True)
        assert r < REL_FRO, (name, r)


@pytest.mark.parametrize("causal", [True, False])
def test_head_512_one_sequence_cases_of_the_reference(gpu, causal):
    """The reference's cuDNN backward cases (tests/gpu/test_packed_gemma.py:145-184: (Lq, Lk) pairs at head size 512,
    causal and bidirectional) through global_attention.attend, at 8 / 4 heads (the kernel's work per head is the
    reference's 32 / 16), against the oracle's float32 gradients."""
    from karpo_decision_amd import global_attention

    dev = torch.device("cuda")
    for n, (lq, lk) in enumerate([(700, 1900), (1500, 1500), (333, 2047), (37, 4100), (4097, 4097), (900, 9000),
                                  (256, 256)]):
        q, k, v, do, q_cu, k_cu, _ = make_pack([lq], [lk], 8, 4, 512, seed=50 + n)
        lens = global_attention.lengths(q_cu, k_cu, dev)
        xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
        out = global_attention.attend(*xs, lens[0, 0, :1], lens[0, 1, :1], causal, 1.0 / 16)
        out.backward(do.to(dev))
        torch.cuda.synchronize()
        want = oa.packed_grads(q, k, v, do, q_cu, k_cu, 1.0 / 16, -1, 0 if causal else -1, dtype=torch.float32)
        for name, x, w in zip(("out", "dq", "dk", "dv"), [out.detach()] + [x.grad for x in xs], want):
            r = rel(x, w)
            print((lq, lk), causal, name, f"rel {r:.2e}", flush=True)
            assert r < REL_FRO, ((lq, lk), name, r)


def test_sliding_case_of_the_reference(gpu):
    """The reference's FA4 sliding test (tests/gpu/test_packed_gemma.py:70-104): head size 256, 32 / 16 heads, window
    1023, queries and keys with their own bounds (three branches after a shared tail), loss sum(out * linspace(-1, 1));
    output and gradients within the reference's floor (relative 5e-3) of float32."""
    from karpo_decision_amd import sliding_attention

    q_len = [1500, 120, 300, 1023, 1024, 1025, 40, 2500, 7]
    k_len = [1500, 1143, 1323, 1023, 1024, 1025, 40, 2500, 1030]
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(sum(n), h, 256, generator=g).bfloat16() for n, h in ((q_len, 32), (k_len, 16), (k_len, 16)))
    q_cu = np.concatenate([[0], np.cumsum(q_len)]).astype(int).tolist()
    k_cu = np.concatenate([[0], np.cumsum(k_len)]).astype(int).tolist()
    dev = torch.device("cuda")
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
    qc, kc = (torch.tensor(x, dtype=torch.int32, device=dev) for x in (q_cu, k_cu))
    out = sliding_attention.attend(*xs, qc, kc, max(q_len), max(k_len), 256 ** -0.5, 1023)
    weight = torch.linspace(-1, 1, out.numel(), device=dev).view_as(out)
    (out.float() * weight).sum().backward()
    torch.cuda.synchronize()
    want = oa.packed_grads(q, k, v, weight.cpu(), q_cu, k_cu, 256 ** -0.5, 1023, 0, dtype=torch.float32)
    for name, x, w in zip(("out", "dq", "dk", "dv"), [out.detach()] + [x.grad for x in xs], want):
        r = rel(x, w)
        print("reference sliding case", name, f"rel {r:.2e}", flush=True)
        assert r < 5e-3, (name, r)


@pytest.mark.parametrize("form", ["full", "markers"])
def test_varlen_attn_trains_the_qwen_layer(gpu, form):
    """varlen.varlen_attn under autograd, as torch's varlen_attn that the Qwen family binds (families/qwen/packed.py:
    36-44) is differentiable: the Qwen full-attention layer's 8,192-token pack (16 / 8 heads, head_dim 128, causal,
    enable_gqa, :123-124), or its markers-only form (the last query of every sequence over the sequence's keys,
    bidirectional, :136-137). out, dq, dk, dv against autograd through the oracle by the layouts' criterion; the
    fused prologue under autograd is refused."""
    from karpo_decision_amd import varlen, workloads

    dev = torch.device("cuda")
    w = workloads.qwen_full(dev, seed=3)
    q_cu, k_cu = w.q_cu, w.k_cu
    q, k, v = w.query.cpu(), w.key.cpu(), w.value.cpu()
    if form == "markers":
        q = torch.stack([q[b - 1] for b in q_cu[1:]])  # one marker query per sequence
        q_cu = list(range(len(k_cu)))
        window, max_q = (-1, -1), 1
    else:
        window, max_q = (-1, 0), w.max_q
    g = torch.Generator().manual_seed(17)
    do = torch.randn(q.shape, generator=g).bfloat16()
    xs = [t.to(dev).requires_grad_(True) for t in (q, k, v)]
    qc = torch.tensor(q_cu, dtype=torch.int32, device=dev)
    kc = torch.tensor(k_cu, dtype=torch.int32, device=dev)
    print("varlen", form, len(k_cu) - 1, "sequences", flush=True)
    out = varlen.varlen_attn(*xs, qc, kc, max_q, w.max_q, scale=w.scale, window_size=window, enable_gqa=True)
    out.backward(do.to(dev))
    torch.cuda.synchronize()
    got = [out.detach()] + [x.grad for x in xs]
    want = oa.packed_grads(q, k, v, do, q_cu, k_cu, w.scale, window[0], window[1], dtype=torch.float32)
    base = oa.packed_grads(q, k, v, do, q_cu, k_cu, w.scale, window[0], window[1], dtype=torch.bfloat16)
    for name, x, ww, b in zip(("out", "dq", "dk", "dv"), got, want, base):
        assert torch.isfinite(x).all(), name
        r, rb = rel(x, ww), rel(b, ww)
        print("varlen", form, name, f"rel {r:.2e} (oracle bf16 {rb:.2e})", flush=True)
        assert r < REL_FRO, (name, r)
        assert r < 2 * rb + 2e-3, (name, r, rb)
    with pytest.raises(RuntimeError, match="forward only"):
        varlen.varlen_attn(*xs, qc, kc, max_q, w.max_q, scale=w.scale, window_size=window, enable_gqa=True,
                           q_norm=ops.Norm(ops.NORM_PLAIN, None, 1e-6))
