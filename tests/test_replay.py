"""Host replay of the forward kernel's memory accesses (tests/replay/fwd_replay.cpp, built here with g++): for a call
and its host plan, every workgroup, wave, lane and key step of the launch computes its addresses with the kernel's
own functions (csrc/tile_addr.h, csrc/plan_common.h); each must stay inside its allocation, and every (query row,
head) of every sequence must be written exactly once.

The row-table workloads are the ones behind the one GPU memory fault this build has seen (a block plan's branched
pack read through its row table by the twelve-wave, 64-key tile at head size 128): their replay under that tile, and
under every shape a call can take now, finds every access in bounds."""

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from karpo_decision_amd import _lib, ops, workloads

ROOT = Path(__file__).resolve().parents[1]
SOURCE = ROOT / "tests" / "replay" / "fwd_replay.cpp"
WIDE, NARROW, SMALL, LONG, DUAL = 0, 1, 2, 3, 4


@pytest.fixture(scope="module")
def replay(tmp_path_factory):
    compiler = shutil.which("g++")
    if compiler is None:
        pytest.skip("no host C++ compiler")
    out = tmp_path_factory.mktemp("replay") / "libfwd_replay.so"
    subprocess.run([compiler, "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{ROOT / 'include'}",
                    f"-I{ROOT / 'karpo_decision_amd' / 'csrc'}", str(SOURCE), "-o", str(out)], check=True)
    lib = ctypes.CDLL(str(out))
    P = ctypes.POINTER
    lib.karpo_replay_fwd.argtypes = [P(_lib.KarpoAttnArgs), P(ctypes.c_int32), P(ctypes.c_int32), P(ctypes.c_int32),
                                     ctypes.c_int64, P(ctypes.c_int32), P(ctypes.c_int32), ctypes.c_int64,
                                     ctypes.c_int, P(ctypes.c_int64), ctypes.c_char_p, ctypes.c_int]
    lib.karpo_replay_fwd.restype = ctypes.c_int64
    lib.karpo_replay_pair_blocks.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.c_int64] * 4
    lib.karpo_replay_pair_blocks.restype = ctypes.c_int64
    return lib


def _i32(values) -> ctypes.Array:
    arr = np.ascontiguousarray(np.asarray(values, dtype=np.int32).reshape(-1))
    return (ctypes.c_int32 * max(1, arr.size))(*arr.tolist())


def run_replay(lib, q_cu, k_cu, heads, kv_heads, head_dim, left, right, *, rows=None, spans=(), max_q=None,
               total_k=None, plan_max_q=None, plan_gather=None, force_shape=-1, strides=None):
    """(violations, counts, first message) of one call's replay; the plan is karpo_attn_plan's, made with
    ``plan_max_q`` / ``plan_gather`` (default: the call's)."""
    longest = max(b - a for a, b in zip(q_cu[:-1], q_cu[1:]))
    max_q = longest if max_q is None else max_q
    gather = rows is not None
    plan = ops.make_plan(q_cu, k_cu, heads, kv_heads, head_dim, left, right, device="cpu",
                         max_q=max_q if plan_max_q is None else plan_max_q,
                         gather=gather if plan_gather is None else plan_gather)
    total_q = q_cu[-1]
    if total_k is None:
        total_k = max(k_cu[-1], max(rows) + 1 if rows else 0)
    a = _lib.KarpoAttnArgs()
    q_t, q_h = strides[0] if strides else (heads * head_dim, head_dim)
    k_t, k_h = strides[1] if strides else (kv_heads * head_dim, head_dim)
    a.q_stride_tok, a.q_stride_head = q_t, q_h
    a.k_stride_tok, a.k_stride_head = k_t, k_h
    a.v_stride_tok, a.v_stride_head = k_t, k_h
    a.o_stride_tok, a.o_stride_head = heads * head_dim, head_dim
    a.n_seq, a.heads, a.kv_heads, a.head_dim = len(q_cu) - 1, heads, kv_heads, head_dim
    a.total_q, a.max_q, a.window_left, a.window_right = total_q, max_q, left, right
    a.n_spans = len(spans)
    a.total_k = total_k
    table = _i32(rows if rows else [0])
    if gather:
        a.k_rows = ctypes.addressof(table)
    plan_host = plan.tensor.numpy()
    counts = (ctypes.c_int64 * 6)()
    first = ctypes.create_string_buffer(512)
    bad = lib.karpo_replay_fwd(ctypes.byref(a), _i32(q_cu), _i32(k_cu), table, len(rows) if rows else 0,
                               _i32(spans if spans else [0, 0]), _i32(plan_host), plan_host.size, force_shape,
                               counts, first, 512)
    return bad, list(counts), first.value.decode()


def _branched(prompts=4, shared=4096, branches=4, branch=512):
    w = workloads.branched("cpu", 0, prompts, shared, branches, branch)
    return w.q_cu, w.k_cu, w.key_rows


def test_branched_pack_under_the_tile_that_faulted(replay):
    """The twelve-wave, 64-key tile at head size 128 (the wide tile of the build that faulted, the long tile now) read
    through the block plan's row table: every row-table read, DMA chunk, LDS write and output row in bounds, and no
    chunk ever read past its resource (every step of that pack is whole)."""
    q_cu, k_cu, rows = _branched()
    bad, counts, first = run_replay(replay, q_cu, k_cu, 32, 16, 128, -1, 0, rows=rows, plan_max_q=70000,
                                    plan_gather=False, force_shape=LONG, total_k=q_cu[-1])
    assert bad == 0, first
    checks, blocks, copies, fetches, bad_rows, past = counts
    assert blocks > 1000 and copies > 0 and fetches > 0 and bad_rows == 0
    assert past == 0


@pytest.mark.parametrize("shape,max_q", [(DUAL, 5000), (LONG, 70000), (SMALL, 4096)])
def test_branched_row_tables_under_every_head_128_shape(replay, shape, max_q):
    """Branches of uneven lengths (partial key steps, so table rows past a sequence read at the resource's end)
    under the dual-block, long and four-wave tiles at head size 128."""
    q_cu, k_cu, rows = _branched(prompts=2, shared=1000, branches=3, branch=37)
    bad, counts, first = run_replay(replay, q_cu, k_cu, 32, 16, 128, -1, 0, rows=rows, max_q=max_q,
                                    plan_max_q=max_q, plan_gather=shape == SMALL, force_shape=shape,
                                    total_k=q_cu[-1])
    assert bad == 0, first
    assert counts[4] == 0 and counts[5] > 0  # every row written once; some chunks read past the resource


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(32, 16, 128), (16, 8, 256), (8, 2, 64), (32, 4, 512)])
@pytest.mark.parametrize("left,right", [(-1, 0), (299, 0), (-1, -1)])
def test_row_table_calls_as_the_library_plans_them(replay, heads, kv_heads, head_dim, left, right):
    """A call through a row table as karpo_attn_fwd launches it (the tile shape the library picks for it), with rows
    outside the tensor in the table (they read at the resource's end)."""
    q_cu, k_cu, rows = _branched(prompts=2, shared=700, branches=3, branch=45)
    rows = list(rows)
    rows[5] = -1
    rows[77] = 10 ** 6
    bad, counts, first = run_replay(replay, q_cu, k_cu, heads, kv_heads, head_dim, left, right, rows=rows,
                                    max_q=5000, total_k=q_cu[-1])
    assert bad == 0, first
    assert counts[4] == 0


@pytest.mark.parametrize("name", ["qwen", "sliding", "multimodal", "markers", "tiny"])
def test_workloads_without_a_row_table(replay, name):
    """The configs' packs (split tiles, windows, spans, decode-shaped tiles) as bench.py and the tests launch them."""
    w = workloads.named(name, "cpu", 0) if name != "tiny" else workloads.tiny("cpu")
    bad, counts, first = run_replay(replay, w.q_cu, w.k_cu, w.heads, w.kv_heads, w.head_dim, w.window_left,
                                    w.window_right, spans=w.spans or (), max_q=w.max_q)
    assert bad == 0, first
    assert counts[4] == 0


def test_long_layer_with_split_tiles(replay):
    """One long causal sequence whose longest tiles split (the merge kernel writes their rows)."""
    q_cu = [0, 3000]
    bad, counts, first = run_replay(replay, q_cu, q_cu, 32, 16, 128, -1, 0, max_q=70000)
    assert bad == 0, first
    assert counts[4] == 0


def test_the_replay_finds_planted_mistakes(replay):
    """A plan made for another tile shape, or a row table shorter than its bounds, is reported."""
    q_cu, k_cu, rows = _branched(prompts=1, shared=300, branches=2, branch=40)
    bad, _, first = run_replay(replay, q_cu, k_cu, 32, 16, 128, -1, 0, rows=rows, max_q=5000, plan_gather=False)
    assert bad > 0 and "tile shape" in first
    bad, _, first = run_replay(replay, q_cu, k_cu, 32, 16, 128, -1, 0, rows=rows[:-50], max_q=5000,
                               total_k=q_cu[-1])
    assert bad > 0 and "row-table read" in first
    # keys past the tensor's rows: the copies read outside the K allocation
    bad, _, first = run_replay(replay, [0, 200], [0, 200], 8, 2, 64, -1, 0, total_k=150)
    assert bad > 0 and "chunk" in first


@pytest.mark.parametrize("k_stride,v_stride", [(512, 512), (2048, 2048), (4104, 1032)])
def test_pair_ping_pong_copy_blocks(replay, k_stride, v_stride):
    """The head-size-512 ping-pong kernel copies a wave's four blocks of a K (V) tile from one offset register plus 64
    (256) bytes per block: the same sources as k_dma_source / v_dma_source per block, whatever the row strides (head
    strides of GQA layouts, padded rows); a wrong per-block step is reported."""
    assert replay.karpo_replay_pair_blocks(8, 4, k_stride, v_stride, 64, 256) == 0
    assert replay.karpo_replay_pair_blocks(8, 4, k_stride, v_stride, 32, 256) > 0
    assert replay.karpo_replay_pair_blocks(8, 4, k_stride, v_stride, 64, 128) > 0
