"""The C ABI on the CPU: the library loads and exports every function include/karpo_attn.h declares; the host planner
(karpo_attn_plan) lists exactly the tiles the brute-force scheduler finds, with the same key-step costs, longest
first; arguments the kernel cannot take are refused with their status code before anything reaches the GPU; the
algorithmic pair counts used for FLOPs match pair-by-pair enumeration."""

import ctypes
import re
from pathlib import Path

import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from karpo_decision_amd import _lib, ops, workloads
from oracle import schedule

HEADER = Path(__file__).resolve().parents[1] / "include" / "karpo_attn.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(karpo_attn_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert names, "no declarations parsed"
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.karpo_attn_version() == 1


def host_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right):
    lib = _lib.load()
    a = _lib.KarpoAttnArgs()
    a.heads, a.kv_heads, a.head_dim, a.window_left, a.window_right = heads, kv_heads, head_dim, left, right
    cap = 4 + 2 * 4096
    buf = (ctypes.c_int32 * cap)()
    n = len(q_cu) - 1
    st_ = lib.karpo_attn_plan(ctypes.byref(a), (ctypes.c_int32 * len(q_cu))(*q_cu),
                              (ctypes.c_int32 * len(k_cu))(*k_cu), n, buf, cap)
    _lib.check(st_, "plan")
    tiles = buf[0]
    return list(buf[:4]), [(buf[4 + 2 * i], buf[5 + 2 * i]) for i in range(tiles)]


GEOMETRIES = [(8, 2, 64), (16, 8, 128), (32, 16, 128), (16, 8, 256), (12, 4, 128), (10, 2, 128), (4, 4, 64)]


@settings(max_examples=60, deadline=None)
@given(q_lens=st.lists(st.integers(0, 700), min_size=1, max_size=5),
       extra=st.lists(st.integers(-200, 300), min_size=5, max_size=5),
       geom=st.sampled_from(GEOMETRIES), left=st.sampled_from([-1, 0, 5, 64, 300]),
       right=st.sampled_from([-1, 0, 3]))
def test_host_plan_matches_brute_force(q_lens, extra, geom, left, right):
    k_lens = [max(0, q + e) for q, e in zip(q_lens, extra)]
    q_cu = [0]
    k_cu = [0]
    for a, b in zip(q_lens, k_lens):
        q_cu.append(q_cu[-1] + a)
        k_cu.append(k_cu[-1] + b)
    heads, kv_heads, head_dim = geom
    rows, bn, per = _lib.tile_shape(heads, kv_heads, head_dim)
    header, items = host_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right)
    assert header == [len(items), rows, bn, per]
    want = schedule.work_list(q_cu, k_cu, rows, bn, left, right)
    assert items == [(seg, t) for _, seg, t in want]


def test_tile_geometry():
    # a tile holds 32 query vectors per wave (12 waves at head_dim 128, 8 at 256, 4 at 64); the GQA group's heads
    # share it when they divide it
    assert _lib.tile_shape(32, 16, 128) == (192, 64, 2)
    assert _lib.tile_shape(8, 2, 64) == (32, 64, 4)
    assert _lib.tile_shape(16, 8, 256) == (128, 32, 2)
    assert _lib.tile_shape(12, 4, 128) == (128, 64, 3)  # a group of 3 divides 384 vectors
    assert _lib.tile_shape(10, 2, 128) == (384, 64, 1)  # a group of 5 does not: one head per item


def test_plan_refuses_bad_bounds_and_small_buffers():
    lib = _lib.load()
    a = _lib.KarpoAttnArgs()
    a.heads, a.kv_heads, a.head_dim, a.window_left, a.window_right = 4, 2, 64, -1, 0
    buf = (ctypes.c_int32 * 8)()
    dec = (ctypes.c_int32 * 3)(0, 10, 5)
    inc = (ctypes.c_int32 * 3)(0, 300, 600)
    assert lib.karpo_attn_plan(ctypes.byref(a), dec, dec, 2, buf, 8) == _lib.ERR_BOUNDS
    assert lib.karpo_attn_plan(ctypes.byref(a), inc, inc, 2, buf, 8) == 10  # capacity


def _args(**kw):
    a = _lib.KarpoAttnArgs()
    a.q = a.k = a.v = a.o = 1 << 20  # never dereferenced: every case below is refused before a launch
    a.q_cu = a.k_cu = 1 << 21
    a.q_stride_tok, a.q_stride_head = 256, 64
    a.k_stride_tok, a.k_stride_head = 128, 64
    a.v_stride_tok, a.v_stride_head = 128, 64
    a.o_stride_tok, a.o_stride_head = 256, 64
    a.n_seq, a.heads, a.kv_heads, a.head_dim = 1, 4, 2, 64
    a.total_q, a.max_q, a.scale = 100, 100, 0.125
    a.window_left, a.window_right = -1, 0
    for name, value in kw.items():
        setattr(a, name, value)
    return a


@pytest.mark.parametrize("change,status", [
    (dict(head_dim=96), _lib.ERR_HEAD_DIM),
    (dict(heads=6, kv_heads=4), _lib.ERR_HEADS),
    (dict(kv_heads=0), _lib.ERR_HEADS),
    (dict(window_left=-2), _lib.ERR_WINDOW),
    (dict(window_right=-5), _lib.ERR_WINDOW),
    (dict(n_spans=2), _lib.ERR_SPANS),
    (dict(n_seq=-1), _lib.ERR_ARG),
    (dict(q=(1 << 20) + 2), _lib.ERR_LAYOUT),
    (dict(k_stride_tok=130), _lib.ERR_LAYOUT),
    (dict(q=0), 1),
    (dict(), 5),  # no workspace and no plan
])
def test_fwd_refuses_before_launch(change, status):
    lib = _lib.load()
    a = _args(**change)
    assert lib.karpo_attn_fwd(ctypes.byref(a), None) == status
    assert _lib.message(status)


def test_empty_pack_is_a_no_op():
    lib = _lib.load()
    assert lib.karpo_attn_fwd(ctypes.byref(_args(total_q=0)), None) == 0
    assert lib.karpo_attn_fwd(ctypes.byref(_args(n_seq=0)), None) == 0


def test_workspace_and_capacity():
    lib = _lib.load()
    a = _args(n_seq=3, total_q=1000, max_q=600)
    entries, size = ctypes.c_int64(), ctypes.c_size_t()
    assert lib.karpo_attn_plan_capacity(ctypes.byref(a), ctypes.byref(entries)) == 0
    rows, _, _ = _lib.tile_shape(4, 2, 64)
    tiles = min(-(-1000 // rows) + 3, 3 * -(-600 // rows))
    assert entries.value == 4 + 2 * tiles
    assert lib.karpo_attn_workspace_bytes(ctypes.byref(a), ctypes.byref(size)) == 0
    assert size.value >= 4 * (entries.value + 4) and size.value % 256 == 0


def test_python_plan_object():
    plan = ops.make_plan([0, 100, 400], [0, 100, 400], 32, 16, 128, -1, 0, device="cpu")
    assert plan.tiles == 1 + 2 and plan.rows_per_tile == 192
    assert plan.tensor.dtype.is_signed and plan.tensor.numel() == 4 + 2 * plan.tiles


@pytest.mark.parametrize("q_cu,k_cu,left,right,spans", [
    ([0, 7, 7, 20], [0, 7, 7, 20], -1, 0, []),
    ([0, 5, 14], [0, 11, 20], -1, 0, []),
    ([0, 13], [0, 13], 3, 0, [(4, 8)]),
    ([0, 10, 16], [0, 10, 16], 2, 2, [(1, 3), (11, 15)]),
    ([0, 9, 13], [0, 9, 11], -1, -1, []),
])
def test_pair_counts_match_enumeration(q_cu, k_cu, left, right, spans):
    assert workloads.allowed_pairs(q_cu, k_cu, left, right, spans) == schedule.pairs(q_cu, k_cu, left, right, spans)


def test_closed_form_pair_counts():
    # causal L(L+1)/2; window W (left W-1): W(W+1)/2 + (L-W)W; a causal span of n rows adds n(n-1)/2
    assert workloads.allowed_pairs([0, 32768], [0, 32768], -1, 0) == 32768 * 32769 // 2
    assert workloads.allowed_pairs([0, 5000], [0, 5000], 1023, 0) == 1024 * 1025 // 2 + (5000 - 1024) * 1024
    assert workloads.allowed_pairs([0, 2000], [0, 2000], -1, 0, [(100, 660)]) == 2000 * 2001 // 2 + 560 * 559 // 2


def test_tiny_workload_flops():
    w = workloads.tiny("cpu")
    assert w.pairs() == 184_925
    assert w.flops() == 378_726_400
