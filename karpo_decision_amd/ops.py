"""The packed attention forward as a torch operator (``karpo_amd::packed_attention``) over ``libkarpo_attn.so``.

The operator follows the reference's own pattern for attention kernels (``karpo::fa4_sliding``,
src/karpo_decision/families/gemma/sliding_attention.py:36-47): a ``torch.library.custom_op`` with no mutated
arguments and a fake implementation that returns ``query.new_empty(query.shape)``, so it traces and captures like any
aten op. The callee allocates the output (as triton_attention.py:103 does); inputs are never written; the bounds are
read on the device when the kernel runs; the launch goes on the current stream of the query's device; nothing syncs.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib

NAMESPACE = "karpo_amd"

#: Norm modes of the fused prologue (KARPO_NORM_* in karpo_attn.h).
NORM_NONE, NORM_WEIGHT, NORM_ONE_PLUS, NORM_PLAIN = 0, 1, 2, 3


@dataclass(frozen=True)
class Norm:
    """An RMSNorm the kernel applies as it loads query vectors (or ``norm_rope`` applies to keys and values):
    ``mode`` NORM_*, ``weight`` (head_dim,) for NORM_WEIGHT / NORM_ONE_PLUS, ``eps``."""

    mode: int
    weight: Tensor | None
    eps: float


def gemma_norm(module) -> Norm:
    """The fused-prologue form of a ``Gemma4RMSNorm`` (``weight`` times the normalised vector, or no weight when the
    module has no scale: the value norm), families/gemma/fused.py:21-25, :81-88."""
    if getattr(module, "with_scale", True):
        return Norm(NORM_WEIGHT, module.weight, float(module.eps))
    return Norm(NORM_PLAIN, None, float(module.eps))


def qwen_norm(module) -> Norm:
    """The fused-prologue form of a ``Qwen3_5RMSNorm`` (``1 + weight``), families/qwen/fused.py:17-19."""
    return Norm(NORM_ONE_PLUS, module.weight, float(getattr(module, "eps", getattr(module, "variance_epsilon", 1e-6))))


def _bf16_table(t: Tensor, device: torch.device) -> Tensor:
    """A (rows, n) bf16 table with contiguous rows (norm weights, rope cos / sin), converted once if needed."""
    if t.dim() == 3 and t.shape[0] == 1:
        t = t[0]
    if t.device != device:
        raise ValueError(f"a prologue table is on {t.device}, the tensors on {device}")
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    if t.stride(-1) != 1 or (t.dim() == 2 and t.stride(0) % 8) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def _is_gfx950(device: torch.device) -> bool:
    props = torch.cuda.get_device_properties(device)
    return getattr(props, "gcnArchName", "").split(":")[0] == "gfx950"


# The current stream's handle: torch's raw-stream accessor (what its compiled kernels call on every launch), a few
# microseconds cheaper per call than building a Stream object.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(index: int) -> int:
    return _raw_stream(index) if _raw_stream is not None else torch.cuda.current_stream(index).cuda_stream


class _Noop:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_NOOP = _Noop()


def _on_device(index: int):
    """torch.cuda.device(index) only when another device is current (entering it costs microseconds per call)."""
    return _NOOP if torch.cuda.current_device() == index else torch.cuda.device(index)


def check_inputs(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor) -> None:
    """ValueError for anything the kernel does not take (before any launch)."""
    if query.dim() != 3 or key.dim() != 3 or value.dim() != 3:
        raise ValueError(f"packed attention takes (rows, heads, head_dim) tensors, got {tuple(query.shape)}, "
                         f"{tuple(key.shape)}, {tuple(value.shape)}")
    if key.shape != value.shape:
        raise ValueError(f"key {tuple(key.shape)} and value {tuple(value.shape)} differ")
    if query.shape[2] != key.shape[2]:
        raise ValueError(f"query head_dim {query.shape[2]} != key head_dim {key.shape[2]}")
    if query.shape[2] not in (64, 128, 256, 512):
        raise ValueError(f"head_dim must be 64, 128, 256 or 512, not {query.shape[2]}")
    if key.shape[1] < 1 or query.shape[1] % key.shape[1] != 0:
        raise ValueError(f"{query.shape[1]} query heads are not a multiple of {key.shape[1]} key/value heads")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, not {t.dtype} (the kernel computes bf16 MFMA products)")
        st = t.stride()
        if st[2] != 1 or st[0] % 8 or st[1] % 8:
            raise ValueError(f"{name} needs a contiguous head_dim and row/head strides that are multiples of 8 "
                             f"(strides {st})")
    for name, t in (("q_cu", q_cu), ("k_cu", k_cu)):
        if t.dtype != torch.int32 or t.dim() != 1:
            raise ValueError(f"{name} must be a 1-D int32 tensor, got {t.dtype} {tuple(t.shape)}")
        if t.device != query.device:
            raise ValueError(f"{name} is on {t.device}, the query on {query.device}")
    if q_cu.numel() != k_cu.numel() or q_cu.numel() < 1:
        raise ValueError(f"q_cu ({q_cu.numel()}) and k_cu ({k_cu.numel()}) must hold the same number of bounds")
    if key.device != query.device or value.device != query.device:
        raise ValueError("query, key and value must be on one device")


def _args(query: Tensor, key: Tensor, value: Tensor, out: Tensor | None, q_cu: Tensor | None, k_cu: Tensor | None,
          n_seq: int, max_q: int, scale: float, window_left: int, window_right: int, spans: Tensor | None,
          plan: Tensor | None, plan_header: list[int] | None = None, key_rows: Tensor | None = None, q_norm: int = 0,
          q_norm_eps: float = 0.0, q_norm_weight: Tensor | None = None, rope_cos: Tensor | None = None,
          rope_sin: Tensor | None = None, gate: Tensor | None = None) -> _lib.KarpoAttnArgs:
    a = _lib.KarpoAttnArgs()
    a.q, a.k, a.v = query.data_ptr(), key.data_ptr(), value.data_ptr()
    a.o = out.data_ptr() if out is not None else 0
    a.q_stride_tok, a.q_stride_head = query.stride(0), query.stride(1)
    a.k_stride_tok, a.k_stride_head = key.stride(0), key.stride(1)
    a.v_stride_tok, a.v_stride_head = value.stride(0), value.stride(1)
    if out is not None:
        a.o_stride_tok, a.o_stride_head = out.stride(0), out.stride(1)
    a.q_cu = q_cu.data_ptr() if q_cu is not None else 0
    a.k_cu = k_cu.data_ptr() if k_cu is not None else 0
    a.n_seq = n_seq
    a.heads, a.kv_heads, a.head_dim = query.shape[1], key.shape[1], query.shape[2]
    a.total_q, a.max_q = query.shape[0], max_q
    a.scale = scale
    a.window_left, a.window_right = window_left, window_right
    if spans is not None and spans.numel():
        a.spans, a.n_spans = spans.data_ptr(), spans.shape[0]
    a.plan = plan.data_ptr() if plan is not None else 0
    if plan_header is not None:  # the struct keeps the array alive (ctypes holds assigned objects)
        a.plan_header = (ctypes.c_int32 * len(plan_header))(*plan_header)
    if key_rows is not None:
        a.k_rows, a.total_k = key_rows.data_ptr(), key.shape[0]
    # the rows the key bounds index (the device planner refuses bounds past them)
    a.key_bound = key_rows.shape[0] if key_rows is not None else key.shape[0]
    a.q_norm, a.q_norm_eps = q_norm, q_norm_eps
    if q_norm_weight is not None:
        a.q_norm_weight = q_norm_weight.data_ptr()
    if rope_cos is not None:
        a.rope_cos, a.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
        a.rope_stride, a.rope_dim = rope_cos.stride(0), rope_cos.shape[-1]
    if gate is not None:
        a.gate, a.gate_stride_tok, a.gate_stride_head = gate.data_ptr(), gate.stride(0), gate.stride(1)
    return a


def _packed_attention(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor, max_q: int,
                     scale: float, window_left: int, window_right: int, spans: Tensor | None,
                     plan: Tensor | None, plan_header: list[int] | None = None, key_rows: Tensor | None = None,
                     q_norm: int = 0, q_norm_eps: float = 0.0, q_norm_weight: Tensor | None = None,
                     rope_cos: Tensor | None = None, rope_sin: Tensor | None = None,
                     gate: Tensor | None = None) -> Tensor:
    return _attention_impl(query, key, value, q_cu, k_cu, max_q, scale, window_left, window_right, spans, plan,
                           plan_header, key_rows, q_norm, q_norm_eps, q_norm_weight, rope_cos, rope_sin, gate)


def _attention_impl(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor, max_q: int,
                    scale: float, window_left: int, window_right: int, spans: Tensor | None,
                    plan: Tensor | None, plan_header: list[int] | None = None, key_rows: Tensor | None = None,
                    q_norm: int = 0, q_norm_eps: float = 0.0, q_norm_weight: Tensor | None = None,
                    rope_cos: Tensor | None = None, rope_sin: Tensor | None = None,
                    gate: Tensor | None = None, query_out: Tensor | None = None) -> Tensor:
    """(Tq, heads, D) bf16: sequence i's query rows q_cu[i]:q_cu[i+1] over its key rows k_cu[i]:k_cu[i+1] (bounds
    int32 on the device), query i at key coordinate i + Lk - Lq, seeing keys j with i' - left <= j <= i' + right
    (-1: unbounded), or in its own span (``spans`` (n, 2) int32 query-row ranges); ``plan`` a device work list from
    ``make_plan`` or None (planned on the device), ``plan_header`` its host header (required with ``plan``);
    ``key_rows`` (int32 on the device) maps key row r to row key_rows[r] of ``key`` / ``value`` (a gather read in
    place, as ``key.index_select(0, key_rows)`` would give). Fused prologue: ``query`` is the projection's output,
    normalised (``q_norm`` NORM_*, ``q_norm_weight`` bf16 (D,), ``q_norm_eps``) and rotated by halves over the first
    ``rope_cos.shape[-1]`` elements (``rope_cos`` / ``rope_sin`` bf16 (Tq, R), row i for query row i) as the kernel
    loads it; fused epilogue: the output times sigmoid(``gate``) (bf16, the output's shape). ``query_out`` (bf16, the
    query's shape; eager calls only) receives the query after the prologue, the attention's actual query."""
    check_inputs(query, key, value, q_cu, k_cu)
    if query.device.type != "cuda":
        raise ValueError(f"packed attention runs on an MI355X GPU, not on {query.device}")
    if spans is not None and (spans.dtype != torch.int32 or spans.dim() != 2 or spans.shape[1] != 2
                              or spans.device != query.device or not spans.is_contiguous()):
        raise ValueError("spans must be a contiguous (n, 2) int32 tensor on the query's device")
    if max_q < 0:
        raise ValueError(f"max_q must be non-negative, not {max_q}")
    if key_rows is not None and (key_rows.dtype != torch.int32 or key_rows.dim() != 1
                                 or key_rows.device != query.device or not key_rows.is_contiguous()):
        raise ValueError("key_rows must be a contiguous 1-D int32 tensor on the query's device")
    for name, t, shape in (("q_norm_weight", q_norm_weight, (query.shape[2],)),
                           ("rope_cos", rope_cos, None), ("rope_sin", rope_sin, None),
                           ("gate", gate, tuple(query.shape))):
        if t is None:
            continue
        if t.dtype != torch.bfloat16 or t.device != query.device:
            raise ValueError(f"{name} must be bf16 on the query's device")
        if shape is not None and tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, not {shape}")
    if rope_cos is not None and (rope_sin is None or rope_cos.shape != rope_sin.shape or rope_cos.dim() != 2
                                 or rope_cos.shape[0] < query.shape[0]):
        raise ValueError("rope_cos and rope_sin must be (query rows, rotated elements) tables of one shape")
    if query_out is not None and (query_out.shape != query.shape or query_out.dtype != torch.bfloat16
                                  or query_out.device != query.device or query_out.stride(2) != 1
                                  or (q_norm == NORM_NONE and rope_cos is None)):
        raise ValueError("query_out must be a bf16 tensor of the query's shape, with a fused prologue")
    if query_out is not None and torch._C._is_alias_of(query_out, query):
        # split tiles read the query after their first part may have written query_out: never the same memory
        raise ValueError("query_out must not share storage with query (the kernel reads the query after writing it)")
    lib = _lib.load()
    out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if query.shape[0] == 0:
        return out
    q_cu, k_cu = q_cu.contiguous(), k_cu.contiguous()
    index = query.device.index
    with _on_device(index):
        args = _args(query, key, value, out, q_cu, k_cu, q_cu.numel() - 1, max_q, scale, window_left, window_right,
                     spans, plan, plan_header, key_rows, q_norm, q_norm_eps, q_norm_weight, rope_cos, rope_sin,
                     gate)
        if query_out is not None:
            args.q_out = query_out.data_ptr()
            args.q_out_stride_tok, args.q_out_stride_head = query_out.stride(0), query_out.stride(1)
        workspace = None
        if plan is None or plan_header is None or plan_header[4] != 0:  # a plan that splits nothing needs none
            need = ctypes.c_size_t()
            _lib.check(lib.karpo_attn_workspace_bytes(ctypes.byref(args), ctypes.byref(need)), "packed attention")
            # the device plan and the fp32 partials of split tiles, from the caching allocator (stream-ordered reuse)
            workspace = torch.empty(need.value, dtype=torch.uint8, device=query.device)
            args.workspace, args.workspace_bytes = workspace.data_ptr(), need.value
        _lib.check(lib.karpo_attn_fwd(ctypes.byref(args), ctypes.c_void_p(_current_stream(index))),
                   "packed attention")
    return out


# the registered operator (torch.compile, fake tensors, KEPT_OPS); ``run`` calls the implementation directly in eager
# mode, which saves the dispatcher's ~10 us per call on launch-bound packs
packed_attention = torch.library.custom_op(f"{NAMESPACE}::packed_attention", mutates_args=())(_packed_attention)


@packed_attention.register_fake
def _(query, key, value, q_cu, k_cu, max_q, scale, window_left, window_right, spans, plan, plan_header=None,
      key_rows=None, q_norm=0, q_norm_eps=0.0, q_norm_weight=None, rope_cos=None, rope_sin=None, gate=None):
    return query.new_empty(query.shape)


@dataclass(frozen=True)
class Plan:
    """A pack's work list on the device, built once on the host (like ``block_plan``'s bounds,
    families/gemma/packed.py:103-151) and reused by every layer of the same head geometry, window, tile shape and
    row-table use; ``header`` is its host copy of the plan's header (the C ABI checks it against each call)."""

    tensor: Tensor
    header: tuple[int, ...]
    heads: int
    kv_heads: int
    head_dim: int
    window_left: int
    window_right: int
    max_q: int
    n_seq: int
    gather: bool
    query_end: int = 0  # q_cu[-1] and k_cu[-1]: the rows the bounds index (checked against the tensors in ``run``)
    key_end: int = 0

    @property
    def items(self) -> int:
        return self.header[0]

    @property
    def rows_per_tile(self) -> int:
        return self.header[1]

    @property
    def split_tiles(self) -> int:
        return self.header[4]


def make_plan(q_cu: list[int] | Tensor, k_cu: list[int] | Tensor, heads: int, kv_heads: int, head_dim: int,
              window_left: int = -1, window_right: int = -1, device: torch.device | str = "cuda",
              max_q: int | None = None, gather: bool = False) -> Plan:
    """The longest-first work list for host bounds ``q_cu`` / ``k_cu`` (lists or CPU tensors), on ``device``.
    ``max_q`` (default: the longest query run) must be the value the calls pass: it selects the tile shape;
    ``gather``: the calls read their keys through a row table (``key_rows``), which selects the tile shape too."""
    qc = [int(x) for x in (q_cu.tolist() if isinstance(q_cu, Tensor) else q_cu)]
    kc = [int(x) for x in (k_cu.tolist() if isinstance(k_cu, Tensor) else k_cu)]
    if len(qc) != len(kc) or not qc:
        raise ValueError("q_cu and k_cu must hold the same, non-zero number of bounds")
    n = len(qc) - 1
    longest = max((qc[i + 1] - qc[i] for i in range(n)), default=0)
    if max_q is None:
        max_q = longest
    if max_q < longest:
        raise ValueError(f"max_q {max_q} is below the longest query run {longest}")
    lib = _lib.load()
    a = _lib.KarpoAttnArgs()
    a.heads, a.kv_heads, a.head_dim = heads, kv_heads, head_dim
    a.window_left, a.window_right = window_left, window_right
    a.n_seq, a.total_q, a.max_q = n, qc[-1] - qc[0], max_q
    marker = ctypes.c_int32()  # karpo_attn_plan reads only whether k_rows is set
    if gather:
        a.k_rows = ctypes.addressof(marker)
    entries = ctypes.c_int64()
    _lib.check(lib.karpo_attn_plan_capacity(ctypes.byref(a), ctypes.byref(entries)), "karpo_attn_plan_capacity")
    qa = (ctypes.c_int32 * len(qc))(*qc)
    ka = (ctypes.c_int32 * len(kc))(*kc)
    buf = (ctypes.c_int32 * entries.value)()
    _lib.check(lib.karpo_attn_plan(ctypes.byref(a), qa, ka, n, buf, entries.value), "karpo_attn_plan")
    used = buf[6] + 4 * buf[0]
    host = torch.tensor(list(buf[:used]), dtype=torch.int32)
    return Plan(host.to(device), tuple(buf[:_lib.PLAN_HEADER]), heads, kv_heads, head_dim, window_left, window_right,
                max_q, n, bool(gather), qc[-1], kc[-1])


def key_rows_of(rows: Tensor | None) -> Tensor | None:
    """A gather table (``block_plan``'s int64 ``g_rows`` / ``s_rows``) as the int32 rows the kernel reads."""
    if rows is None or (rows.dtype == torch.int32 and rows.is_contiguous()):
        return rows
    return rows.to(torch.int32).contiguous()


def run(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor, max_q: int, scale: float,
        window_left: int = -1, window_right: int = -1, spans: Tensor | None = None,
        plan: Plan | None = None, key_rows: Tensor | None = None, q_norm: Norm | None = None,
        rope: tuple[Tensor, Tensor] | None = None, gate: Tensor | None = None,
        query_out: Tensor | None = None) -> Tensor:
    """``packed_attention`` with a ``Plan`` checked against the call's geometry; ``key_rows`` (int32 or int64) reads
    the keys and values through a row table instead of a gathered copy; ``q_norm`` / ``rope`` ((cos, sin), (rows, R)
    or (1, rows, R)) the fused query prologue, ``gate`` the fused sigmoid gate on the output; ``query_out`` receives
    the query after the prologue (eager calls only: torch.compile sees an operator without it)."""
    tensor, header = None, None
    if plan is not None:
        if (plan.heads, plan.kv_heads, plan.head_dim, plan.window_left, plan.window_right) != (
                query.shape[1], key.shape[1], query.shape[2], window_left, window_right):
            raise ValueError("the plan was made for another head geometry or window")
        if plan.n_seq != q_cu.numel() - 1:
            raise ValueError(f"the plan was made for {plan.n_seq} sequences, the call has {q_cu.numel() - 1}")
        if plan.gather != (key_rows is not None):
            raise ValueError("the plan was made " + ("with" if plan.gather else "without") + " a row table, the call "
                             + ("has none" if plan.gather else "reads its keys through one"))
        if int(max_q) < plan.max_q:
            raise ValueError(f"max_q {max_q} is below the plan's {plan.max_q}: it must bound every query run")
        if _lib.tile_shape(plan.heads, plan.kv_heads, plan.head_dim, plan.max_q, plan.gather) != _lib.tile_shape(
                plan.heads, plan.kv_heads, plan.head_dim, int(max_q), plan.gather):
            raise ValueError(f"the plan was made for max_q {plan.max_q}, another tile shape than max_q {max_q}")
        # the plan's host bounds: rows past the tensors would be read out of their allocations
        if plan.query_end > query.shape[0]:
            raise ValueError(f"the bounds index {plan.query_end} query rows, the query has {query.shape[0]}")
        key_rows_len = key.shape[0] if key_rows is None else key_rows.shape[0]
        if plan.key_end > key_rows_len:
            raise ValueError(f"the bounds index {plan.key_end} key rows, the {'key' if key_rows is None else 'row table'}"
                             f" has {key_rows_len}")
        tensor, header = plan.tensor, list(plan.header)
    mode, eps, weight = NORM_NONE, 0.0, None
    if q_norm is not None:
        mode, eps = int(q_norm.mode), float(q_norm.eps)
        weight = _bf16_table(q_norm.weight, query.device) if q_norm.weight is not None else None
    cos = sin = None
    if rope is not None:
        cos, sin = (_bf16_table(t, query.device) for t in rope)
    # the registered operator while dynamo traces or autograd records (it has no gradient: an input that requires
    # one is torch's error, not a silently detached output); the implementation itself otherwise
    traced = torch.compiler.is_compiling() or (torch.is_grad_enabled() and (
        query.requires_grad or key.requires_grad or value.requires_grad))
    call = (query, key, value, q_cu, k_cu, int(max_q), float(scale), int(window_left), int(window_right), spans,
            tensor, header, key_rows_of(key_rows), mode, eps, weight, cos, sin, gate)
    if query_out is not None:
        if traced:
            raise RuntimeError("query_out is written by eager calls only (the registered operator has no such output)")
        return _attention_impl(*call, query_out=query_out)
    return (packed_attention if traced else _packed_attention)(*call)


def norm_rope(x: Tensor, norm: Norm | None, rope: tuple[Tensor, Tensor] | None = None,
              out: Tensor | None = None) -> Tensor:
    """``x`` (rows, heads, D) bf16 normalised and rotated in one pass over HBM (``karpo_attn_norm_rope``): keys
    (norm and rotation) and values (norm) for the attention, which stages each key for many query tiles. ``out``
    may be ``x`` (in place); a new tensor otherwise."""
    if x.dim() != 3 or x.dtype != torch.bfloat16 or x.device.type != "cuda":
        raise ValueError("norm_rope takes a (rows, heads, head_dim) bf16 tensor on the GPU")
    if x.shape[2] not in (64, 128, 256, 512) or x.stride(2) != 1:
        raise ValueError(f"norm_rope takes head_dim 64, 128, 256 or 512 with a contiguous head, not {tuple(x.shape)}")
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    elif out.shape != x.shape or out.dtype != x.dtype or out.device != x.device or out.stride(2) != 1:
        raise ValueError("out must have x's shape, dtype and device, with a contiguous head")
    if norm is not None and norm.mode in (NORM_WEIGHT, NORM_ONE_PLUS) and (
            norm.weight is None or tuple(norm.weight.shape) != (x.shape[2],)):
        raise ValueError(f"the norm's weight must have shape ({x.shape[2]},)")
    if rope is not None:
        cos, sin = rope
        cos, sin = (t[0] if t.dim() == 3 and t.shape[0] == 1 else t for t in (cos, sin))
        if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[0] < x.shape[0] or cos.shape[1] > x.shape[2]:
            raise ValueError(f"rope tables must be two (rows >= {x.shape[0]}, rotated <= {x.shape[2]}) tables of one "
                             f"shape, not {tuple(cos.shape)} / {tuple(sin.shape)}")
    lib = _lib.load()
    a = _lib.KarpoNormRopeArgs()
    a.x, a.y = x.data_ptr(), out.data_ptr()
    a.x_stride_tok, a.x_stride_head = x.stride(0), x.stride(1)
    a.y_stride_tok, a.y_stride_head = out.stride(0), out.stride(1)
    a.rows, a.heads, a.head_dim = x.shape[0], x.shape[1], x.shape[2]
    keep = []
    if norm is not None:
        a.norm, a.eps = int(norm.mode), float(norm.eps)
        if norm.weight is not None:
            w = _bf16_table(norm.weight, x.device)
            keep.append(w)
            a.weight = w.data_ptr()
    if rope is not None:
        cos, sin = (_bf16_table(t, x.device) for t in rope)
        keep += [cos, sin]
        a.rope_cos, a.rope_sin, a.rope_stride, a.rope_dim = cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[-1]
    with _on_device(x.device.index):
        stream = _current_stream(x.device.index)
        _lib.check(lib.karpo_attn_norm_rope(ctypes.byref(a), ctypes.c_void_p(stream)), "norm_rope")
    # converted tables in `keep` go back to the stream-ordered caching allocator after the launch: safe to reuse
    return out


# ---- training: the forward with its log-sum-exp and the backward, as a differentiable operator pair (the pattern of
# karpo::fa4_sliding / karpo::fa4_sliding_backward, families/gemma/sliding_attention.py:36-66)

def _workspace(lib, fn, args, device: torch.device) -> Tensor:
    need = ctypes.c_size_t()
    _lib.check(fn(ctypes.byref(args), ctypes.byref(need)), "packed attention")
    return torch.empty(need.value, dtype=torch.uint8, device=device)


@torch.library.custom_op(f"{NAMESPACE}::packed_attention_lse", mutates_args=())
def packed_attention_lse(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor, max_q: int,
                         scale: float, window_left: int, window_right: int,
                         spans: Tensor | None) -> tuple[Tensor, Tensor]:
    """``packed_attention`` and its log-sum-exp: (Tq, heads, D) bf16 and (heads, Tq) fp32,
    lse[h, i] = ln(sum over row i's visible keys of exp(scale * q.k)), -inf for a row that sees no key (the
    reference's ``return_lse``, families/gemma/sliding_attention.py:39-41)."""
    check_inputs(query, key, value, q_cu, k_cu)
    if query.device.type != "cuda":
        raise ValueError(f"packed attention runs on an MI355X GPU, not on {query.device}")
    lib = _lib.load()
    out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    lse = torch.empty((query.shape[1], query.shape[0]), dtype=torch.float32, device=query.device)
    if query.shape[0] == 0:
        return out, lse
    q_cu, k_cu = q_cu.contiguous(), k_cu.contiguous()
    with _on_device(query.device.index):
        args = _args(query, key, value, out, q_cu, k_cu, q_cu.numel() - 1, max_q, scale, window_left, window_right,
                     spans, None)
        args.lse = lse.data_ptr()
        workspace = _workspace(lib, lib.karpo_attn_workspace_bytes, args, query.device)
        args.workspace, args.workspace_bytes = workspace.data_ptr(), workspace.numel()
        stream = _current_stream(query.device.index)
        _lib.check(lib.karpo_attn_fwd(ctypes.byref(args), ctypes.c_void_p(stream)), "packed attention")
    return out, lse


@packed_attention_lse.register_fake
def _(query, key, value, q_cu, k_cu, max_q, scale, window_left, window_right, spans):
    return query.new_empty(query.shape), query.new_empty((query.shape[1], query.shape[0]), dtype=torch.float32)


@torch.library.custom_op(f"{NAMESPACE}::packed_attention_backward", mutates_args=())
def packed_attention_backward(grad: Tensor, query: Tensor, key: Tensor, value: Tensor, out: Tensor, lse: Tensor,
                              q_cu: Tensor, k_cu: Tensor, max_q: int, scale: float, window_left: int,
                              window_right: int, spans: Tensor | None) -> tuple[Tensor, Tensor, Tensor]:
    """Gradients of ``packed_attention_lse``'s output (dq, dk, dv, bf16, the shapes of query, key and value) from
    the output gradient ``grad``, the forward's output and lse (``karpo_attn_bwd``). Rows outside the sequences'
    bounds are not written."""
    check_inputs(query, key, value, q_cu, k_cu)
    for name, t in (("grad", grad), ("out", out)):
        if t.shape != query.shape or t.dtype != torch.bfloat16 or t.device != query.device:
            raise ValueError(f"{name} must be bf16 of the query's shape on its device")
    if lse.shape != (query.shape[1], query.shape[0]) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("lse must be the forward's contiguous (heads, rows) fp32 tensor")
    lib = _lib.load()
    grad = grad if grad.stride(-1) == 1 and grad.stride(0) % 8 == 0 and grad.stride(1) % 8 == 0 else grad.contiguous()
    dq = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    dk = torch.empty(key.shape, dtype=key.dtype, device=key.device)
    dv = torch.empty(value.shape, dtype=value.dtype, device=value.device)
    if query.shape[0] == 0:
        return dq, dk.zero_(), dv.zero_()
    q_cu, k_cu = q_cu.contiguous(), k_cu.contiguous()
    with _on_device(query.device.index):
        b = _lib.KarpoAttnBwdArgs()
        b.fwd = _args(query, key, value, out, q_cu, k_cu, q_cu.numel() - 1, max_q, scale, window_left, window_right,
                      spans, None)
        b.fwd.total_k = key.shape[0]
        b.d_o, b.d_o_stride_tok, b.d_o_stride_head = grad.data_ptr(), grad.stride(0), grad.stride(1)
        b.lse = lse.data_ptr()
        b.d_q, b.d_q_stride_tok, b.d_q_stride_head = dq.data_ptr(), dq.stride(0), dq.stride(1)
        b.d_k, b.d_k_stride_tok, b.d_k_stride_head = dk.data_ptr(), dk.stride(0), dk.stride(1)
        b.d_v, b.d_v_stride_tok, b.d_v_stride_head = dv.data_ptr(), dv.stride(0), dv.stride(1)
        workspace = _workspace(lib, lib.karpo_attn_bwd_workspace_bytes, b, query.device)
        b.fwd.workspace, b.fwd.workspace_bytes = workspace.data_ptr(), workspace.numel()
        stream = _current_stream(query.device.index)
        _lib.check(lib.karpo_attn_bwd(ctypes.byref(b), ctypes.c_void_p(stream)), "packed attention backward")
    return dq, dk, dv


@packed_attention_backward.register_fake
def _(grad, query, key, value, out, lse, q_cu, k_cu, max_q, scale, window_left, window_right, spans):
    return torch.empty_like(query), torch.empty_like(key), torch.empty_like(value)


def _setup(ctx, inputs, output):
    query, key, value, q_cu, k_cu, ctx.max_q, ctx.scale, ctx.window_left, ctx.window_right, spans = inputs
    ctx.save_for_backward(query, key, value, *output, q_cu, k_cu, spans)


def _gradient(ctx, grad, _lse_grad):
    query, key, value, out, lse, q_cu, k_cu, spans = ctx.saved_tensors
    dq, dk, dv = packed_attention_backward(grad.contiguous(), query, key, value, out, lse, q_cu, k_cu, ctx.max_q,
                                           ctx.scale, ctx.window_left, ctx.window_right, spans)
    return dq, dk, dv, None, None, None, None, None, None, None


packed_attention_lse.register_autograd(_gradient, setup_context=_setup)


def attention(query: Tensor, key: Tensor, value: Tensor, q_cu: Tensor, k_cu: Tensor, max_q: int, scale: float,
              window_left: int = -1, window_right: int = -1, spans: Tensor | None = None) -> Tensor:
    """The differentiable packed attention: (Tq, heads, D) bf16; gradients flow to query, key and value through
    ``karpo_attn_bwd``."""
    return packed_attention_lse(query, key, value, q_cu, k_cu, int(max_q), float(scale), int(window_left),
                                int(window_right), spans)[0]
