"""The C ABI on the CPU: the library loads and exports every function include/karpo_attn.h declares; the host planner
(karpo_attn_plan) lists exactly the tiles the brute-force scheduler finds, with the same key-step costs, longest
first; arguments the kernel cannot take are refused with their status code before anything reaches the GPU; the
algorithmic pair counts used for FLOPs match pair-by-pair enumeration."""

import ctypes
import re
from pathlib import Path

import pytest
import torch
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
    assert lib.karpo_attn_version() == 4


def host_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right, max_q=_lib.LONG):
    """(header, merges, items) of karpo_attn_plan's output: merges (segment, tile, parts, slot); items
    (segment, tile, part, parts) with the item's slot checked against its tile's merge entry."""
    lib = _lib.load()
    a = _lib.KarpoAttnArgs()
    a.heads, a.kv_heads, a.head_dim, a.window_left, a.window_right = heads, kv_heads, head_dim, left, right
    a.n_seq, a.total_q, a.max_q = len(q_cu) - 1, q_cu[-1], max_q
    entries = ctypes.c_int64()
    _lib.check(lib.karpo_attn_plan_capacity(ctypes.byref(a), ctypes.byref(entries)), "capacity")
    cap = entries.value
    buf = (ctypes.c_int32 * cap)()
    n = len(q_cu) - 1
    st_ = lib.karpo_attn_plan(ctypes.byref(a), (ctypes.c_int32 * len(q_cu))(*q_cu),
                              (ctypes.c_int32 * len(k_cu))(*k_cu), n, buf, cap)
    _lib.check(st_, "plan")
    header = list(buf[:_lib.PLAN_HEADER])
    h = _lib.PLAN_HEADER
    merges = [tuple(buf[h + 4 * i: h + 4 + 4 * i]) for i in range(header[4])]
    slot_of = {(m[0], m[1]): m[3] for m in merges}
    items = []
    for i in range(header[0]):
        seg, tile, pp, slot = buf[header[6] + 4 * i: header[6] + 4 * i + 4]
        part, parts = pp & 0xFFFF, pp >> 16
        assert slot == (slot_of[(seg, tile)] if parts > 1 else -1)
        items.append((seg, tile, part, parts))
    return header, merges, items


#: Workgroups per CU the split policy plans for, per (head_dim, one-wave tiles): the register and LDS budgets of the
#: kernels (small tiles, 4 waves at head_dim 128 / 256, are planned one per CU like the wide ones; one-wave tiles at
#: 64 / 128 two per CU, their ring of four K/V buffers).
TILES_PER_CU = {(64, False): 4, (128, False): 1, (256, False): 1, (512, False): 1, (64, True): 2, (128, True): 2,
                (256, True): 2, (512, True): 1}
GEOMETRIES = [(8, 2, 64), (16, 8, 128), (32, 16, 128), (16, 8, 256), (12, 4, 128), (10, 2, 128), (4, 4, 64),
              (32, 4, 512), (6, 2, 512)]


def waves_of(rows, per, head_dim, shape=0):
    """Waves of a tile: 32 query vectors per wave (64 in the dual-block tiles, shape 4), per pair of waves at
    head_dim 512."""
    return rows * per // (64 if shape == 4 else 32) * (2 if head_dim == 512 else 1)


def expected_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right, max_q):
    rows, bn, per = _lib.tile_shape(heads, kv_heads, head_dim, max_q)
    narrow = rows * per == 32
    conc = 256 * TILES_PER_CU[(head_dim, narrow)]
    merges, items = schedule.split_plan(q_cu, k_cu, rows, bn, left, right, heads // per, conc)
    return rows, bn, per, narrow, merges, items


@settings(max_examples=80, deadline=None)
@given(q_lens=st.lists(st.integers(0, 700), min_size=1, max_size=5),
       extra=st.lists(st.integers(-200, 300), min_size=5, max_size=5),
       geom=st.sampled_from(GEOMETRIES), left=st.sampled_from([-1, 0, 5, 64, 300]),
       right=st.sampled_from([-1, 0, 3]), short=st.booleans())
def test_host_plan_matches_brute_force(q_lens, extra, geom, left, right, short):
    if short:  # decode-shaped: a few queries per sequence over longer key runs
        q_lens = [q % 5 for q in q_lens]
    k_lens = [max(0, q + e) for q, e in zip(q_lens, extra)]
    q_cu = [0]
    k_cu = [0]
    for a, b in zip(q_lens, k_lens):
        q_cu.append(q_cu[-1] + a)
        k_cu.append(k_cu[-1] + b)
    heads, kv_heads, head_dim = geom
    max_q = max(q_lens)
    rows, bn, per, narrow, merges, items = expected_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right, max_q)
    header, got_merges, got_items = host_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right, max_q)
    shape = _lib.kernel_shape(heads, kv_heads, head_dim, max_q)
    assert header[:7] == [len(items), rows, bn, per, len(merges), waves_of(rows, per, head_dim, shape),
                          _lib.PLAN_HEADER + 4 * len(merges)]
    assert header[7] == sum(m[2] for m in merges)
    assert header[8:] == [len(q_cu) - 1, 0, _lib.kernel_shape(heads, kv_heads, head_dim, max_q), 0]
    assert got_merges == merges
    assert got_items == items
    # every part of a split tile is listed once; the slots of split tiles do not overlap
    for seg, tile, parts, slot in merges:
        assert sorted(q for s_, t, q, n in items if (s_, t) == (seg, tile)) == list(range(parts))
    assert header[7] <= 2 * 256 * TILES_PER_CU[(head_dim, narrow)] // (heads // per)


def test_split_bound_is_tight_enough():
    # one long causal segment in a pack of 16 KV heads: the parts of split tiles stay within the fixed slot budget
    for lens in ([2210, 1547, 1138, 861, 680, 666, 526, 351, 213], [8192], [1] * 64, [3000, 5]):
        q_cu = [0]
        for n in lens:
            q_cu.append(q_cu[-1] + n)
        for heads, kv, d in ((16, 8, 128), (32, 16, 128), (16, 8, 256), (8, 2, 64), (32, 4, 512)):
            header, merges, items = host_plan(q_cu, q_cu, heads, kv, d, -1, 0, max(lens))
            rows, bn, per = _lib.tile_shape(heads, kv, d, max(lens))
            narrow = rows * per == 32
            assert header[7] <= 2 * 256 * TILES_PER_CU[(d, narrow)] // (heads // per)


def test_markers_plan_splits_keys():
    # markers-only shape: one query per sequence over all of its keys (bidirectional) takes one-wave tiles whose
    # key steps are split across the GPU
    k_cu = [0, 32768, 40000]
    q_cu = [0, 1, 2]
    header, merges, items = host_plan(q_cu, k_cu, 32, 16, 128, -1, -1, 1)
    assert header[1:4] == [16, 32, 2] and header[5] == 1
    # 1024 + 226 steps of 32 keys x 16 head groups over 2 x 256 one-wave workgroups: parts of at most 40 steps
    assert merges == [(0, 0, 26, 0), (1, 0, 6, 26)]
    assert len(items) == 32 and header[7] == 32


def test_tile_geometry():
    # a tile holds 32 query vectors per wave (12 waves at head_dim 128, 8 at 256, 4 at 64); the GQA group's heads
    # share it when they divide it. Head size 128: 32-key steps, 64 for runs above 65,536 queries
    # head size 128 prefill: dual-block tiles of 512 vectors (eight waves of two 32-vector blocks), 32-key steps
    assert _lib.tile_shape(32, 16, 128, 32768) == (256, 32, 2)
    assert _lib.tile_shape(32, 16, 128, 65536) == (256, 32, 2)
    assert _lib.tile_shape(32, 16, 128, 65537) == (192, 64, 2)
    assert _lib.tile_shape(32, 16, 128) == (192, 64, 2)
    assert _lib.tile_shape(8, 2, 64) == (32, 64, 4)
    assert _lib.tile_shape(16, 8, 256) == (128, 32, 2)
    assert _lib.tile_shape(12, 4, 128) == (128, 64, 3)  # a group of 3 divides 384 vectors
    assert _lib.tile_shape(12, 4, 128, 5000) == (128, 32, 3)  # and not 512: the twelve-wave tile shares K/V
    assert _lib.tile_shape(10, 2, 128) == (384, 64, 1)  # a group of 5 does not: one head per item
    assert _lib.tile_shape(10, 2, 128, 5000) == (512, 32, 1)
    # small tiles (4 waves) for runs up to 4,096 queries at head size 128 and 8,192 at 256
    assert _lib.tile_shape(32, 16, 128, 4096) == (64, 32, 2)
    assert _lib.tile_shape(32, 16, 128, 4097) == (256, 32, 2)
    assert _lib.tile_shape(16, 8, 256, 8192) == (64, 32, 2)
    assert _lib.tile_shape(16, 8, 256, 8193) == (128, 32, 2)
    assert _lib.tile_shape(12, 4, 128, 1000) == (128, 32, 1)  # a group of 3 does not divide 128 vectors
    assert _lib.tile_shape(8, 2, 64, 1000) == (32, 64, 4)  # head size 64: the wide tile is already 4 waves
    # one-wave tiles when every sequence's queries fit 32 vectors
    assert _lib.tile_shape(32, 16, 128, 1) == (16, 32, 2)
    assert _lib.tile_shape(32, 16, 128, 16) == (16, 32, 2)
    assert _lib.tile_shape(32, 16, 128, 17) == (64, 32, 2)
    assert _lib.tile_shape(32, 4, 256, 4) == (4, 32, 8)
    assert _lib.tile_shape(8, 2, 64, 8) == (8, 64, 4)
    assert _lib.tile_shape(10, 2, 128, 32) == (32, 32, 1)
    # head_dim 512: a pair of waves per 32 vectors, 8 waves (128 vectors) wide, one pair narrow
    assert _lib.tile_shape(32, 4, 512) == (16, 32, 8)
    assert _lib.tile_shape(32, 4, 512, 4) == (4, 32, 8)
    assert _lib.tile_shape(6, 2, 512) == (128, 32, 1)  # a group of 3 does not divide 128 vectors
    # the kernels' shape numbering (wide 0, narrow 1, small 2, long 3), as bench.py labels the launch
    assert [_lib.kernel_shape(32, 16, 128, n) for n in (32768, 16, 4096, 65537)] == [4, 1, 2, 3]
    assert _lib.kernel_shape(12, 4, 128, 32768) == 0  # the twelve-wave tile for a group of 3
    assert [_lib.kernel_shape(16, 8, 256, n) for n in (16384, 8192)] == [0, 2]
    assert [_lib.kernel_shape(32, 4, 512, n) for n in (32768, 4)] == [0, 1]


def test_plan_refuses_bad_bounds_and_small_buffers():
    lib = _lib.load()
    a = _lib.KarpoAttnArgs()
    a.heads, a.kv_heads, a.head_dim, a.window_left, a.window_right, a.max_q = 4, 2, 64, -1, 0, 1000
    h = _lib.PLAN_HEADER
    buf = (ctypes.c_int32 * h)()
    dec = (ctypes.c_int32 * 3)(0, 10, 5)
    inc = (ctypes.c_int32 * 3)(0, 300, 600)
    assert lib.karpo_attn_plan(ctypes.byref(a), dec, dec, 2, buf, h) == _lib.ERR_BOUNDS
    assert lib.karpo_attn_plan(ctypes.byref(a), inc, inc, 2, buf, h) == 10  # capacity
    assert lib.karpo_attn_plan(ctypes.byref(a), inc, inc, 2, buf, h - 1) == 10  # not even the header
    a.max_q = 299  # max_q must bound every query run (it sizes the tiles and the launch)
    assert lib.karpo_attn_plan(ctypes.byref(a), inc, inc, 2, buf, h) == _lib.ERR_BOUNDS


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
    (dict(plan=1 << 22), _lib.ERR_PLAN),  # a host plan without its header copy
])
def test_fwd_refuses_before_launch(change, status):
    lib = _lib.load()
    a = _args(**change)
    assert lib.karpo_attn_fwd(ctypes.byref(a), None) == status
    assert _lib.message(status)


def _header(*values):
    return (ctypes.c_int32 * _lib.PLAN_HEADER)(*values)


def _call_header(a, gather=False):
    """The header karpo_attn_plan writes for the call ``a``'s geometry (one sequence of max_q rows)."""
    lib = _lib.load()
    b = _args(n_seq=a.n_seq, total_q=a.total_q, max_q=a.max_q)
    marker = ctypes.c_int32()
    if gather:
        b.k_rows = ctypes.addressof(marker)
    cu = (ctypes.c_int32 * 2)(0, a.max_q)
    entries = ctypes.c_int64()
    assert lib.karpo_attn_plan_capacity(ctypes.byref(b), ctypes.byref(entries)) == 0
    buf = (ctypes.c_int32 * entries.value)()
    assert lib.karpo_attn_plan(ctypes.byref(b), cu, cu, 1, buf, entries.value) == 0
    return list(buf[:_lib.PLAN_HEADER])


@pytest.mark.parametrize("field,value", [
    (1, 7), (2, 16), (3, 1), (5, 8),  # another tile geometry (rows, keys per step, heads per item, waves)
    (8, 2),  # another sequence count: the kernel would read bounds past the call's
    (9, 1),  # made for a row table
    (10, 2),  # another shape
    (0, 10 ** 6),  # more items than the launch covers
    (4, 10 ** 6),  # more split tiles than the merge launch covers
    (7, 10 ** 6),  # more partial slots than the workspace holds
    (6, 9),  # items not right after the split tiles
])
def test_fwd_refuses_a_plan_made_for_another_call(field, value):
    """karpo_attn_fwd checks a host plan's header against the call before launching anything: a plan for another
    geometry, row-table use, sequence count or beyond the launch's capacities would leave rows unwritten."""
    lib = _lib.load()
    a = _args(workspace=1 << 24, workspace_bytes=1 << 30)
    good = _call_header(a)
    assert good[8:11] == [1, 0, 0]
    bad = list(good)
    bad[field] = value
    a.plan, a.plan_header = 1 << 22, _header(*bad)
    assert lib.karpo_attn_fwd(ctypes.byref(a), None) == _lib.ERR_PLAN
    # a call through a row table refuses the plan made without one, and the other way round
    rows = _args(workspace=1 << 24, workspace_bytes=1 << 30, k_rows=1 << 22, total_k=100, plan=1 << 22)
    rows.plan_header = _header(*good)
    assert lib.karpo_attn_fwd(ctypes.byref(rows), None) == _lib.ERR_PLAN
    a.plan_header = _header(*_call_header(a, gather=True))
    assert lib.karpo_attn_fwd(ctypes.byref(a), None) == _lib.ERR_PLAN


def test_row_table_calls_take_the_four_wave_tiles():
    """At head sizes 128 and 256 a call through a row table takes the four-wave tiles whatever its longest run (the
    wide and long tiles are not built with a row table); head sizes 64 and 512 keep their shapes."""
    for max_q in (4097, 32768, 70000):
        assert _lib.kernel_shape(32, 16, 128, max_q, gather=True) == 2
    assert _lib.kernel_shape(16, 8, 256, 9000, gather=True) == 2
    assert _lib.kernel_shape(32, 16, 128, 16, gather=True) == 1  # one-wave tiles stay
    assert _lib.kernel_shape(8, 2, 64, 5000, gather=True) == 0
    assert _lib.kernel_shape(32, 4, 512, 5000, gather=True) == 0
    plan = ops.make_plan([0, 5000], [0, 5000], 32, 16, 128, -1, 0, device="cpu", gather=True)
    assert plan.gather and plan.header[9] == 1 and plan.header[10] == 2 and plan.rows_per_tile == 64


def _bwd_args(fwd=None, **kw):
    b = _lib.KarpoAttnBwdArgs()
    b.fwd = fwd if fwd is not None else _args(total_k=100)
    b.d_o = b.d_q = b.d_k = b.d_v = 1 << 20  # never dereferenced: every case below is refused before a launch
    b.lse = 1 << 23
    b.d_o_stride_tok, b.d_o_stride_head = 256, 64
    b.d_q_stride_tok, b.d_q_stride_head = 256, 64
    b.d_k_stride_tok, b.d_k_stride_head = 128, 64
    b.d_v_stride_tok, b.d_v_stride_head = 128, 64
    for name, value in kw.items():
        setattr(b, name, value)
    return b


@pytest.mark.parametrize("change,fwd_change,status", [
    ({}, dict(head_dim=96), _lib.ERR_HEAD_DIM),
    ({}, dict(plan=1 << 22), _lib.ERR_ARG),  # the backward plans on the device
    ({}, dict(k_rows=1 << 22), _lib.ERR_ARG),  # no gathered keys
    ({}, dict(q_norm=1), _lib.ERR_ARG),  # no prologue
    ({}, dict(gate=1 << 22), _lib.ERR_ARG),
    ({}, dict(total_k=0), _lib.ERR_ARG),
    (dict(lse=0), {}, 1),
    (dict(d_k=0), {}, 1),
    (dict(d_o=(1 << 20) + 8), {}, _lib.ERR_LAYOUT),
    (dict(lse=(1 << 23) + 2), {}, _lib.ERR_LAYOUT),
    (dict(d_v_stride_tok=130), {}, _lib.ERR_LAYOUT),
    ({}, {}, 5),  # no workspace
])
def test_bwd_refuses_before_launch(change, fwd_change, status):
    lib = _lib.load()
    b = _bwd_args(_args(**{"total_k": 100, **fwd_change}), **change)
    assert lib.karpo_attn_bwd(ctypes.byref(b), None) == status
    assert _lib.message(status)


def test_bwd_workspace_holds_stats_and_both_plans():
    lib = _lib.load()
    b = _bwd_args(_args(n_seq=3, total_q=1000, max_q=600, total_k=1500))
    size = ctypes.c_size_t()
    assert lib.karpo_attn_bwd_workspace_bytes(ctypes.byref(b), ctypes.byref(size)) == 0
    stats = 4 * 2 * 1000 * 4  # [heads][2][total_q] fp32
    tiles_q = min(-(-1000 // 64) + 3, 3 * -(-600 // 64))  # 128 vectors of 2 heads: 64 rows per query tile
    tiles_k = -(-1500 // 128) + 3
    # key tiles split over their query steps: parts in at most 2 x 256 / kv_heads slots per key/value head, each
    # holding fp32 dK and dV of 128 keys
    slots = 2 * 256 // 2
    items_k, merges_k = tiles_k + slots, min(tiles_k, slots // 2)
    partials = slots * 2 * 128 * 2 * 64 * 4
    # both plans (the key tiles' with their split tiles), and a tile-base array of n_seq + 1 ints per plan (the two
    # are built by one launch, side by side), then the partials
    ints = 12 + 4 * tiles_q + 12 + 4 * merges_k + 4 * items_k + 2 * 4
    assert size.value >= stats + 4 * ints + partials and size.value % 256 == 0
    assert lib.karpo_attn_bwd(ctypes.byref(_bwd_args(_args(total_q=0, total_k=100))), None) == 0  # nothing to do


def test_empty_pack_is_a_no_op():
    lib = _lib.load()
    assert lib.karpo_attn_fwd(ctypes.byref(_args(total_q=0)), None) == 0
    assert lib.karpo_attn_fwd(ctypes.byref(_args(n_seq=0)), None) == 0


def test_workspace_and_capacity():
    lib = _lib.load()
    a = _args(n_seq=3, total_q=1000, max_q=600)
    entries, size = ctypes.c_int64(), ctypes.c_size_t()
    assert lib.karpo_attn_plan_capacity(ctypes.byref(a), ctypes.byref(entries)) == 0
    rows, _, per = _lib.tile_shape(4, 2, 64)
    tiles = min(-(-1000 // rows) + 3, 3 * -(-600 // rows))
    slots = 2 * 256 * TILES_PER_CU[(64, False)] // (4 // per)
    assert entries.value == _lib.PLAN_HEADER + 4 * min(tiles, slots // 2) + 4 * (tiles + slots)
    assert lib.karpo_attn_workspace_bytes(ctypes.byref(a), ctypes.byref(size)) == 0
    partial = slots * (4 // per) * 128 * (64 + 2) * 4
    # the plan, the planner's tile bases (n_seq + 1) and its status word, then the partials
    assert size.value >= 4 * (entries.value + 4 + 1) + partial and size.value % 256 == 0


def test_python_plan_object():
    # max_q above 65,536: the 12-wave tiles with 64-key steps
    plan = ops.make_plan([0, 100, 400], [0, 100, 400], 32, 16, 128, -1, 0, device="cpu", max_q=70000)
    # tiles of 2, 3 and 5 key steps, none longer than the shortest split (8 steps)
    assert plan.items == 3 and plan.rows_per_tile == 192 and plan.split_tiles == 0
    assert plan.tensor.dtype.is_signed and plan.tensor.numel() == _lib.PLAN_HEADER + 4 * plan.items
    assert plan.header == (3, 192, 64, 2, 0, 12, 12, 0, 2, 0, 3, 0)
    assert plan.n_seq == 2 and not plan.gather
    # the default max_q (the longest run, 300): small tiles of 64 rows, 32-key steps, 4 waves; tiles of 2, 4 and 2, 4,
    # 6, 8, 10 steps: the 10-step tile is longer than the shortest split and takes two parts
    small = ops.make_plan([0, 100, 400], [0, 100, 400], 32, 16, 128, -1, 0, device="cpu")
    assert small.header[1:6] == (64, 32, 2, 1, 4) and small.items == 2 + 5 + 1
    long = ops.make_plan([0, 3000], [0, 3000], 32, 16, 128, -1, 0, device="cpu", max_q=70000)
    # 16 tiles of 3, 6, .., 45 and 47 steps: 407 x 16 = 6512 workgroup-steps over 256, parts of at most 26 steps
    assert long.split_tiles == 8 and long.items == 16 + 8
    with pytest.raises(ValueError):
        ops.make_plan([0, 100, 400], [0, 100, 400], 32, 16, 128, -1, 0, device="cpu", max_q=10)


def test_planned_call_refuses_bounds_past_the_tensors():
    """A plan knows its host bounds: a call whose bounds index rows past the query, the keys or the row table is
    refused before anything runs (the kernel would read past the allocations)."""
    plan = ops.make_plan([0, 100, 400], [0, 300, 900], 4, 2, 64, -1, 0, device="cpu")
    assert (plan.query_end, plan.key_end) == (400, 900)
    q = torch.zeros(400, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(500, 2, 64, dtype=torch.bfloat16)
    cu = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(ValueError, match="900 key rows"):
        ops.run(q, k, k, cu, cu, 300, 0.1, -1, 0, None, plan)
    gathered = ops.make_plan([0, 100, 400], [0, 300, 900], 4, 2, 64, -1, 0, device="cpu", gather=True)
    with pytest.raises(ValueError, match="the row table has 800"):
        ops.run(q, k, k, cu, cu, 300, 0.1, -1, 0, None, gathered, key_rows=torch.zeros(800, dtype=torch.int32))
    with pytest.raises(ValueError, match="query rows"):
        ops.run(q[:399], k, k, cu, cu, 300, 0.1, -1, 0, None, gathered,
                key_rows=torch.zeros(900, dtype=torch.int32))


def test_planned_call_refuses_another_pack_or_row_table_use():
    """A plan is for its own sequence count, row-table use and max_q: calls that differ are refused on the host."""
    plan = ops.make_plan([0, 100, 400], [0, 300, 900], 4, 2, 64, -1, 0, device="cpu")
    q = torch.zeros(400, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(900, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="2 sequences, the call has 3"):
        ops.run(q, k, k, torch.zeros(4, dtype=torch.int32), torch.zeros(4, dtype=torch.int32), 300, 0.1, -1, 0, None,
                plan)
    cu = torch.zeros(3, dtype=torch.int32)
    with pytest.raises(ValueError, match="without a row table"):
        ops.run(q, k, k, cu, cu, 300, 0.1, -1, 0, None, plan, key_rows=torch.zeros(900, dtype=torch.int32))
    with pytest.raises(ValueError, match="below the plan's 300"):
        ops.run(q, k, k, cu, cu, 299, 0.1, -1, 0, None, plan)


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


def test_registered_operators_have_fake_kernels():
    """The operators torch.compile and selective recompute (KEPT_OPS) see: their fake kernels give the real outputs'
    shapes and dtypes without running anything (eager calls through ops.run skip the dispatcher)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(10, 4, 64, dtype=torch.bfloat16, device="cuda")
        k = torch.empty(12, 2, 64, dtype=torch.bfloat16, device="cuda")
        cu = torch.empty(3, dtype=torch.int32, device="cuda")
        o = torch.ops.karpo_amd.packed_attention(q, k, k, cu, cu, 8, 0.1, -1, 0, None, None)
        assert (o.shape, o.dtype) == (q.shape, torch.bfloat16)
        o, lse = torch.ops.karpo_amd.packed_attention_lse(q, k, k, cu, cu, 8, 0.1, -1, 0, None)
        assert (lse.shape, lse.dtype) == ((4, 10), torch.float32)
        dq, dk, dv = torch.ops.karpo_amd.packed_attention_backward(o, q, k, k, o, lse, cu, cu, 8, 0.1, -1, 0, None)
        assert (dq.shape, dk.shape, dv.shape) == (q.shape, k.shape, k.shape)


def test_norm_rope_refuses_tables_that_do_not_fit():
    """karpo_attn_norm_rope reads weight[d] and cos / sin rows up to x's rows: tables that do not cover them are
    refused before any launch (shapes only: fake tensors on the GPU device)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty(10, 2, 128, dtype=torch.bfloat16, device="cuda")
        bf = dict(dtype=torch.bfloat16, device="cuda")
        with pytest.raises(ValueError, match="weight"):
            ops.norm_rope(x, ops.Norm(ops.NORM_WEIGHT, torch.empty(64, **bf), 1e-6))
        with pytest.raises(ValueError, match="weight"):
            ops.norm_rope(x, ops.Norm(ops.NORM_ONE_PLUS, None, 1e-6))
        norm = ops.Norm(ops.NORM_WEIGHT, torch.empty(128, **bf), 1e-6)
        for cos, sin in ((torch.empty(9, 128, **bf), torch.empty(9, 128, **bf)),  # fewer rows than x
                         (torch.empty(10, 128, **bf), torch.empty(10, 64, **bf)),  # two shapes
                         (torch.empty(10, 256, **bf), torch.empty(10, 256, **bf)),  # wider than the head
                         (torch.empty(10, 2, 128, **bf), torch.empty(10, 2, 128, **bf))):  # not a table
            with pytest.raises(ValueError, match="rope tables"):
                ops.norm_rope(x, norm, (cos, sin))
        with pytest.raises(ValueError, match="out must"):
            ops.norm_rope(x, norm, out=torch.empty(10, 2, 64, **bf))


def test_query_out_must_not_alias_the_query():
    """The parts of a split tile read the query when they start, possibly after part 0 has written the prologue's
    query to q_out: a q_out that shares a byte with q is refused (KARPO_ATTN_ERR_PROLOGUE) before any launch, by the
    C ABI and by ops.run; a q_out of its own passes those checks."""
    lib = _lib.load()
    base = 1 << 24
    weight = 1 << 23
    # q spans (100 - 1) * 256 + 3 * 64 + 64 elements = 25,600 elements = 51,200 bytes from base
    for q_out, refused in ((base, True), (base + 51_200 - 16, True), (base - 512, True), (base + 51_200, False),
                           (base - 51_200, False)):
        a = _args(q=base, q_norm=1, q_norm_weight=weight, q_norm_eps=1e-6, q_out=q_out)
        a.q_out_stride_tok, a.q_out_stride_head = 256, 64
        status = lib.karpo_attn_fwd(ctypes.byref(a), None)
        assert status == (_lib.ERR_PROLOGUE if refused else 5), (q_out - base, status)  # 5: no workspace, next check
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        bf = dict(dtype=torch.bfloat16, device="cuda")
        q = torch.empty(10, 4, 64, **bf)
        k = torch.empty(12, 2, 64, **bf)
        cu = torch.empty(3, dtype=torch.int32, device="cuda")
        norm = ops.Norm(ops.NORM_WEIGHT, torch.empty(64, **bf), 1e-6)
        for q_out in (q, q[:], q.view(10, 4, 64)):
            with pytest.raises(ValueError, match="must not share storage"):
                ops.run(q, k, k, cu, cu, 8, 0.1, -1, 0, q_norm=norm, query_out=q_out)


def test_noalloc_entry_point_refuses_calls_beyond_its_scratch():
    """karpo_attn_fwd_noalloc takes its scratch from a 144 MiB device array: a call whose workspace is larger (a plan
    of millions of work items) is refused with its status before any HIP call; argument errors keep their codes."""
    lib = _lib.load()
    a = _args(n_seq=5_000_000, total_q=500_000_000, max_q=100, heads=32, kv_heads=16, head_dim=128)
    a.q_stride_tok, a.o_stride_tok = 32 * 128, 32 * 128
    a.k_stride_tok = a.v_stride_tok = 16 * 128
    a.q_stride_head = a.k_stride_head = a.v_stride_head = a.o_stride_head = 128
    need = ctypes.c_size_t()
    assert lib.karpo_attn_workspace_bytes(ctypes.byref(a), ctypes.byref(need)) == 0
    assert need.value > 144 << 20
    assert lib.karpo_attn_fwd_noalloc(ctypes.byref(a), None) == _lib.ERR_SCRATCH
    assert "144 MiB" in _lib.message(_lib.ERR_SCRATCH)
    assert lib.karpo_attn_fwd_noalloc(ctypes.byref(_args(head_dim=96)), None) == _lib.ERR_HEAD_DIM
    assert lib.karpo_attn_fwd_noalloc(None, None) == 1
