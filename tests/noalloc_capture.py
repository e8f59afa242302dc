"""Run by tests/test_zz_no_alloc.py in a process of its own (so the allocation-free entry point has not yet run on the
device): karpo_attn_fwd_noalloc's first call on the device is made inside a HIP graph capture (torch.cuda.graph,
global capture mode, on a side stream); the graph is then replayed with the bounds rewritten in place between
replays, each replay's output compared bitwise with the workspace entry point's eager call on the same bounds, and
device free memory read around eager calls after the first. Prints one JSON line."""

from __future__ import annotations

import ctypes
import json
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import torch  # noqa: E402

from karpo_decision_amd import _lib, ops  # noqa: E402

BOUNDS = ([0, 1200, 2900, 3000], [0, 3000, 3000, 3000], [0, 10, 20, 3000], [0, 1500, 1501, 3000])


def main() -> None:
    dev = torch.device("cuda", 0)
    torch.manual_seed(5)
    heads, kv_heads, head, rows, max_q, scale = 16, 8, 128, 3000, 3000, 0.088
    q = torch.randn(rows, heads, head, device=dev).bfloat16()
    k = torch.randn(rows, kv_heads, head, device=dev).bfloat16()
    v = torch.randn(rows, kv_heads, head, device=dev).bfloat16()
    cu = torch.tensor(BOUNDS[0], dtype=torch.int32, device=dev)
    o = torch.full_like(q, float("nan"))
    lib = _lib.load()
    a = ops._args(q, k, v, o, cu, cu, len(BOUNDS[0]) - 1, max_q, scale, -1, 0, None, None)
    a.workspace, a.workspace_bytes = 0, 0
    torch.cuda.synchronize()
    print("capture: first call of karpo_attn_fwd_noalloc on the device", flush=True)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        status = lib.karpo_attn_fwd_noalloc(ctypes.byref(a), ctypes.c_void_p(side.cuda_stream))
    result = {"status_in_capture": status, "replays": []}
    if status == 0:
        for bounds in BOUNDS + BOUNDS[:1]:
            cu.copy_(torch.tensor(bounds, dtype=torch.int32))
            o.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            want = ops.run(q, k, v, cu, cu, max_q, scale, -1, 0)  # the workspace entry point, device plan
            torch.cuda.synchronize()
            result["replays"].append({"bounds": bounds, "equal": bool(torch.equal(o, want)),
                                      "nan": bool(torch.isnan(o).any())})
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        free = []
        for _ in range(3):  # eager calls after the first: device memory unchanged
            free.append(torch.cuda.mem_get_info()[0])
            result.setdefault("eager_status", []).append(lib.karpo_attn_fwd_noalloc(ctypes.byref(a), stream))
            torch.cuda.synchronize()
        free.append(torch.cuda.mem_get_info()[0])
        result["free_bytes"] = free
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
