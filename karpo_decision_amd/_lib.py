"""ctypes binding of ``libkarpo_attn.so`` (``include/karpo_attn.h``, version 4). The library is the only compute path: if it is
missing this module raises, it never falls back to another implementation."""

from __future__ import annotations

import ctypes
import functools
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libkarpo_attn.so"

#: Every symbol ``include/karpo_attn.h`` declares.
EXPORTS = ("karpo_attn_fwd", "karpo_attn_plan", "karpo_attn_plan_capacity", "karpo_attn_workspace_bytes",
           "karpo_attn_tile_shape", "karpo_attn_strerror", "karpo_attn_version", "karpo_attn_norm_rope",
           "karpo_attn_bwd_workspace_bytes", "karpo_attn_bwd", "karpo_attn_device_status",
           "karpo_attn_fwd_noalloc")

OK = 0
ERR_HEAD_DIM, ERR_HEADS, ERR_LAYOUT, ERR_WINDOW, ERR_SPANS, ERR_ARG, ERR_BOUNDS = 2, 3, 4, 6, 7, 9, 11
ERR_PROLOGUE, ERR_PLAN, ERR_SCRATCH = 12, 13, 14
#: Int32 entries of a plan's header (KARPO_ATTN_PLAN_HEADER).
PLAN_HEADER = 12
#: Status codes that mean "these arguments are not supported" (ValueError), the rest are runtime failures.
VALUE_ERRORS = {1, ERR_HEAD_DIM, ERR_HEADS, ERR_LAYOUT, 5, ERR_WINDOW, ERR_SPANS, ERR_ARG, 10, ERR_BOUNDS,
                ERR_PROLOGUE, ERR_PLAN, ERR_SCRATCH}


class KarpoAttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("o", ctypes.c_void_p),
        ("q_stride_tok", ctypes.c_int64), ("q_stride_head", ctypes.c_int64),
        ("k_stride_tok", ctypes.c_int64), ("k_stride_head", ctypes.c_int64),
        ("v_stride_tok", ctypes.c_int64), ("v_stride_head", ctypes.c_int64),
        ("o_stride_tok", ctypes.c_int64), ("o_stride_head", ctypes.c_int64),
        ("q_cu", ctypes.c_void_p), ("k_cu", ctypes.c_void_p),
        ("n_seq", ctypes.c_int32), ("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("total_q", ctypes.c_int64), ("max_q", ctypes.c_int32), ("scale", ctypes.c_float),
        ("window_left", ctypes.c_int32), ("window_right", ctypes.c_int32),
        ("spans", ctypes.c_void_p), ("n_spans", ctypes.c_int32),
        ("plan", ctypes.c_void_p), ("plan_header", ctypes.POINTER(ctypes.c_int32)),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("k_rows", ctypes.c_void_p), ("total_k", ctypes.c_int64),
        ("q_norm", ctypes.c_int32), ("q_norm_eps", ctypes.c_float), ("q_norm_weight", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p), ("rope_stride", ctypes.c_int64),
        ("rope_dim", ctypes.c_int32), ("gate", ctypes.c_void_p), ("gate_stride_tok", ctypes.c_int64),
        ("gate_stride_head", ctypes.c_int64), ("lse", ctypes.c_void_p),
        ("q_out", ctypes.c_void_p), ("q_out_stride_tok", ctypes.c_int64), ("q_out_stride_head", ctypes.c_int64),
        ("key_bound", ctypes.c_int64),
    ]


class KarpoNormRopeArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p), ("y", ctypes.c_void_p),
        ("x_stride_tok", ctypes.c_int64), ("x_stride_head", ctypes.c_int64),
        ("y_stride_tok", ctypes.c_int64), ("y_stride_head", ctypes.c_int64),
        ("rows", ctypes.c_int64), ("heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("norm", ctypes.c_int32), ("eps", ctypes.c_float), ("weight", ctypes.c_void_p),
        ("rope_cos", ctypes.c_void_p), ("rope_sin", ctypes.c_void_p), ("rope_stride", ctypes.c_int64),
        ("rope_dim", ctypes.c_int32),
    ]


class KarpoAttnBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", KarpoAttnArgs),
        ("d_o", ctypes.c_void_p), ("d_o_stride_tok", ctypes.c_int64), ("d_o_stride_head", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("d_q", ctypes.c_void_p), ("d_q_stride_tok", ctypes.c_int64), ("d_q_stride_head", ctypes.c_int64),
        ("d_k", ctypes.c_void_p), ("d_k_stride_tok", ctypes.c_int64), ("d_k_stride_head", ctypes.c_int64),
        ("d_v", ctypes.c_void_p), ("d_v_stride_tok", ctypes.c_int64), ("d_v_stride_head", ctypes.c_int64),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """The loaded library (loaded once). RuntimeError when it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIBRARY.exists():
            raise RuntimeError(f"{LIBRARY} is missing: build it first (python -m karpo_decision_amd.build); there "
                               "is no fallback implementation")
        lib = ctypes.CDLL(str(LIBRARY))
        P = ctypes.POINTER
        lib.karpo_attn_fwd.argtypes = [P(KarpoAttnArgs), ctypes.c_void_p]
        lib.karpo_attn_fwd.restype = ctypes.c_int
        lib.karpo_attn_plan.argtypes = [P(KarpoAttnArgs), P(ctypes.c_int32), P(ctypes.c_int32), ctypes.c_int32,
                                        P(ctypes.c_int32), ctypes.c_int64]
        lib.karpo_attn_plan.restype = ctypes.c_int
        lib.karpo_attn_plan_capacity.argtypes = [P(KarpoAttnArgs), P(ctypes.c_int64)]
        lib.karpo_attn_plan_capacity.restype = ctypes.c_int
        lib.karpo_attn_workspace_bytes.argtypes = [P(KarpoAttnArgs), P(ctypes.c_size_t)]
        lib.karpo_attn_workspace_bytes.restype = ctypes.c_int
        lib.karpo_attn_tile_shape.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                              ctypes.c_int32, P(ctypes.c_int32), P(ctypes.c_int32),
                                              P(ctypes.c_int32), P(ctypes.c_int32)]
        lib.karpo_attn_tile_shape.restype = ctypes.c_int
        lib.karpo_attn_strerror.argtypes = [ctypes.c_int]
        lib.karpo_attn_strerror.restype = ctypes.c_char_p
        lib.karpo_attn_version.argtypes = []
        lib.karpo_attn_version.restype = ctypes.c_int
        lib.karpo_attn_norm_rope.argtypes = [P(KarpoNormRopeArgs), ctypes.c_void_p]
        lib.karpo_attn_norm_rope.restype = ctypes.c_int
        lib.karpo_attn_bwd_workspace_bytes.argtypes = [P(KarpoAttnBwdArgs), P(ctypes.c_size_t)]
        lib.karpo_attn_bwd_workspace_bytes.restype = ctypes.c_int
        lib.karpo_attn_bwd.argtypes = [P(KarpoAttnBwdArgs), ctypes.c_void_p]
        lib.karpo_attn_bwd.restype = ctypes.c_int
        lib.karpo_attn_device_status.argtypes = [P(KarpoAttnArgs), ctypes.c_void_p, P(ctypes.c_int32)]
        lib.karpo_attn_device_status.restype = ctypes.c_int
        lib.karpo_attn_fwd_noalloc.argtypes = [P(KarpoAttnArgs), ctypes.c_void_p]
        lib.karpo_attn_fwd_noalloc.restype = ctypes.c_int
        _lib = lib
        return lib


def message(status: int) -> str:
    return load().karpo_attn_strerror(status).decode()


def check(status: int, what: str) -> None:
    """Raises for a non-zero status: ValueError for refused arguments, RuntimeError otherwise."""
    if status == OK:
        return
    text = f"{what}: {message(status)} (status {status})"
    raise (ValueError if status in VALUE_ERRORS else RuntimeError)(text)


#: ``max_q`` of a prefill-sized pack (wide tiles whatever the head geometry).
LONG = 1 << 30


@functools.lru_cache(maxsize=1024)
def kernel_shape(heads: int, kv_heads: int, head_dim: int, max_q: int = LONG, gather: bool = False) -> int:
    """The forward kernel's tile-shape template argument for these heads, longest query run and row-table use (0
    wide, 1 narrow: one wave, or one pair at head_dim 512; 2 small: four waves at head_dim 128 / 256; 3 long: 64-key
    steps at 128; 4 dual-block: two query blocks per wave at 128)."""
    shape = ctypes.c_int32()
    check(load().karpo_attn_tile_shape(heads, kv_heads, head_dim, max_q, int(bool(gather)), None, None, None,
                                       ctypes.byref(shape)), "karpo_attn_tile_shape")
    return shape.value


@functools.lru_cache(maxsize=1024)
def tile_shape(heads: int, kv_heads: int, head_dim: int, max_q: int = LONG,
               gather: bool = False) -> tuple[int, int, int]:
    """(query rows per tile, keys per step, query heads per work item) for packs whose longest query run is
    ``max_q`` (one-wave tiles when every run fits one), read through a row table when ``gather`` (memoised: a pure
    function of its arguments, asked on every planned call)."""
    rows, keys, per = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    check(load().karpo_attn_tile_shape(heads, kv_heads, head_dim, max_q, int(bool(gather)), ctypes.byref(rows),
                                       ctypes.byref(keys), ctypes.byref(per), None), "karpo_attn_tile_shape")
    return rows.value, keys.value, per.value
