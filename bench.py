"""Packed causal attention throughput on one MI355X.

A step is one forward pass of the packed attention over one synthetic pack. The default workload is the
Gemma-31B-class global layer at 32,768 tokens (one causal segment, 32 query / 16 KV heads, head_dim 128, bf16): the
configuration the metric is quoted on. Inputs are resident in HBM before the timed region; the pack's work list is
built once (as the reference plans a pack once for all layers), so each timed step launches the attention kernel
and the merge kernel for tiles split over their keys (a no-op launch when none is), on the current stream, timed
with HIP events.

Prints one JSON line: value = TFLOP/s counting only unmasked (query, key) pairs (4 * D * H per pair), with the
roofline of the attention kernel (dense bf16 MFMA peak; HBM bandwidth for decode-shaped workloads such as the
markers-only layer) and the CPU baseline (the reference's torch SDPA path, restated in oracle/attention.py, timed on
this host's cores on a bounded sample of the same workload).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
METRIC = "packed causal attention TFLOP/s + % bf16 MFMA peak @32k tokens, 1 GPU"
#: MI355X dense bf16 MFMA peak: 256 CUs x 2.4 GHz x 4096 FLOP/clk/CU (AMD's published 2.5 PFLOP/s).
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0
TRAFFIC = ROOT / "profiles" / "traffic.json"


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="global32k",
                   help="global32k (default), global131k, global32k_d512, qwen, sliding, multimodal, markers, "
                        "branched, global32k_prologue, qwen_gated, tiny; keys_norm_rope times karpo_attn_norm_rope "
                        "over the 32k layer's keys instead")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-repeats", type=int, default=3)
    p.add_argument("--materialize-gather", action="store_true",
                   help="for workloads with a gather table: time index_select copies of K/V plus the attention on "
                        "them (the reference's Packed._gather path) instead of reading through the table")
    p.add_argument("--backward", action="store_true",
                   help="time the backward (karpo_attn_bwd: dq, dk, dv from the output gradient, the forward's "
                        "output and log-sum-exp) instead of the forward; head sizes 64, 128 and 256, no gather or "
                        "fused prologue")
    p.add_argument("--copy-bytes", type=int, default=0,
                   help="after the timed steps, copy this many bytes device to device once (a calibration kernel of "
                        "known traffic for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return p.parse_args()


def cpu_baseline(w, repeats: int) -> dict:
    """The oracle (the reference's per-sequence torch SDPA path) on the host cores, on one KV-head group of the pack
    (the query heads of the first four KV heads over every sequence; 8 of 32 heads at the 32k layer, about 10-30 s of
    CPU work in all), median of ``repeats`` runs after one warm-up, for bf16 and fp32 inputs;
    the faster is reported. TFLOP/s counts the same unmasked pairs as the GPU figure; the whole layer's CPU time is
    extrapolated from the sample (heads are independent: the sample's time times heads / group), and labelled so."""
    import torch

    from oracle import attention as oracle_attention

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    kv = min(4, w.kv_heads)  # the first KV heads and their query heads: seconds of CPU work per run at 32k
    group = w.heads // w.kv_heads * kv
    from oracle import prologue as oracle_prologue

    key, value = w.gathered()
    q = w.query[:, :group].cpu()
    k = key[:, :kv].cpu()
    v = value[:, :kv].cpu()
    weight = w.q_norm[1].cpu() if w.q_norm is not None else None
    rope = tuple(t.cpu() for t in w.rope) if w.rope is not None else None
    gate = w.gate[:, :group].cpu() if w.gate is not None else None
    sample_flops = w.flops() * group / w.heads
    best = None
    times_by_dtype = {}
    for dtype in (torch.bfloat16, torch.float32):
        times = []
        for n in range(repeats + 1):
            t0 = time.perf_counter()
            qe = q
            if w.q_norm is not None:  # the reference's fused.norm_rope / norm on the CPU, then the attention
                qe = oracle_prologue.rms_norm(q, w.q_norm[0], weight, w.q_norm[2])
            if rope is not None:
                qe = oracle_prologue.rope(qe, *rope)
            out = oracle_attention.packed_attention(qe, k, v, w.q_cu, w.k_cu, w.scale, w.window_left, w.window_right,
                                                    w.spans, dtype=dtype)
            if gate is not None:
                oracle_prologue.gate(out.to(torch.bfloat16), gate)
            if n:
                times.append(time.perf_counter() - t0)
        med = statistics.median(times)
        times_by_dtype[str(dtype).split(".")[-1]] = med
        if best is None or med < best[1]:
            best = (dtype, med)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    dtype, sec = best
    scale = w.heads / group  # the sample is one KV head's query heads: the whole layer's CPU time is this times it
    return {
        "value": round(sample_flops / sec / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
        "kind": "port", "extrapolated": True, "sample_fraction": round(1 / scale, 6),
        "full_layer_seconds_estimate": round(sec * scale, 3),
        "sample": (f"{w.name}: query heads 0-{group - 1} (KV heads 0-{kv - 1}) of {w.heads}, "
                   f"all {w.tokens} tokens; "
                   f"torch {torch.__version__} CPU SDPA per sequence; median of {repeats} after 1 warm-up; "
                   f"seconds bf16 {times_by_dtype['bfloat16']:.3f}, fp32 {times_by_dtype['float32']:.3f}; "
                   f"reported {str(dtype).split('.')[-1]}; os.cpu_count()={os.cpu_count()}; {cpu_model}"),
    }


def keys_norm_rope(args, device) -> int:
    """karpo_attn_norm_rope over the keys of the 32k global layer (32,768 rows x 16 heads x 128, Gemma4RMSNorm with
    a weight, rotation of the whole head), in place: HBM-bound (read and write every key once, plus the tables)."""
    import torch

    from karpo_decision_amd import ops, workloads

    w = workloads.gemma_global(32768, device, args.seed)
    keys = w.key.clone()
    weight = torch.ones(w.head_dim, dtype=torch.bfloat16, device=device)
    rope = workloads.rope_tables(keys.shape[0], w.head_dim, args.seed, device)
    norm = ops.Norm(ops.NORM_WEIGHT, weight, 1e-6)
    for _ in range(args.warmup):
        ops.norm_rope(keys, norm, rope, out=keys)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in marks:
        a.record(stream)
        ops.norm_rope(keys, norm, rope, out=keys)
        b.record(stream)
    torch.cuda.synchronize()
    ms = statistics.median(a.elapsed_time(b) for a, b in marks)
    nbytes = 2 * keys.numel() * 2 + 2 * rope[0].numel() * 2 + weight.numel() * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "karpo_attn_norm_rope over the 32k layer's keys (HBM bytes / s)", "value": round(gbs, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "keys-norm-rope-32768", "rows": keys.shape[0], "heads": keys.shape[1],
                   "head_dim": keys.shape[2], "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "norm_rope_kernel<128>",
                     "avg_launch_ms": round(ms, 4)}}), flush=True)
    return 0


def copy_once(nbytes: int, device) -> None:
    """One device-to-device copy of ``nbytes`` (a kernel of known traffic to calibrate FETCH_SIZE / WRITE_SIZE)."""
    import torch

    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def cpu_backward_baseline(w) -> dict:
    """The oracle's gradients (torch autograd through the per-sequence CPU SDPA path) on one KV-head group of the
    pack, float32, one run (the backward at 32k tokens takes seconds per group)."""
    import torch

    from oracle import attention as oracle_attention

    torch.set_num_threads(int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    group = w.heads // w.kv_heads
    q, k, v = w.query[:, :group].cpu(), w.key[:, :1].cpu(), w.value[:, :1].cpu()
    grad = torch.randn(q.shape, generator=torch.Generator().manual_seed(1)).to(q.dtype)
    t0 = time.perf_counter()
    oracle_attention.packed_grads(q, k, v, grad, w.q_cu, w.k_cu, w.scale, w.window_left, w.window_right, w.spans,
                                  dtype=torch.float32)
    sec = time.perf_counter() - t0
    sample_flops = 2.5 * w.flops() * group / w.heads
    scale = w.heads / group
    return {"value": round(sample_flops / sec / 1e12, 4), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "extrapolated": True, "sample_fraction": round(1 / scale, 6),
            "full_layer_seconds_estimate": round(sec * scale, 3),
            "sample": (f"{w.name} backward: query heads 0-{group - 1} (KV head 0) of {w.heads}, all {w.tokens} "
                       f"tokens; torch {torch.__version__} CPU SDPA per sequence + autograd, float32, one run "
                       f"{sec:.3f} s; os.cpu_count()={os.cpu_count()}")}


def backward(args, device, w) -> int:
    """One step = karpo_attn_bwd over the pack (the planner launch for both work lists, the dq kernel, which also
    writes the per-row statistics, and the dk/dv kernels; at head size 512 a statistics pass first and the wave-pair
    kernels) from a resident output gradient, output and log-sum-exp. TFLOP/s counts the algorithmic
    backward: 2.5x the forward's FLOPs (five products per visible pair: S, dP, dV, dQ, dK)."""
    import torch

    from karpo_decision_amd import ops

    if w.key_rows is not None or w.q_norm is not None or w.rope is not None or w.gate is not None:
        raise SystemExit(f"--backward takes workloads without gather tables or fused prologues, not {w.name}")
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=device)
    k_cu = torch.tensor(w.k_cu, dtype=torch.int32, device=device)
    spans = torch.tensor(w.spans, dtype=torch.int32, device=device) if w.spans else None
    out, lse = ops.packed_attention_lse(w.query, w.key, w.value, q_cu, k_cu, w.max_q, w.scale, w.window_left,
                                        w.window_right, spans)
    gen = torch.Generator(device=device).manual_seed(args.seed + 1)
    grad = torch.randn(out.shape, generator=gen, device=device).to(out.dtype)

    def step():
        return ops.packed_attention_backward(grad, w.query, w.key, w.value, out, lse, q_cu, k_cu, w.max_q, w.scale,
                                             w.window_left, w.window_right, spans)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    begin.record(stream)
    for a, b in marks:
        a.record(stream)
        step()
        b.record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    if args.copy_bytes:
        copy_once(args.copy_bytes, device)
    ms_per_step = begin.elapsed_time(end) / args.steps
    launch_ms = statistics.mean(a.elapsed_time(b) for a, b in marks)
    flops = 2.5 * w.flops()
    value = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (launch_ms * 1e-3) / 1e12
    result = {
        "metric": "packed causal attention backward TFLOP/s + % bf16 MFMA peak, 1 GPU", "value": round(value, 2),
        "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {**w.describe(), "pass": "backward", "pct_of_bf16_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
                   "flops_per_step": flops, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "kernel": (f"karpo_attn_bwd (bwd_stats_kernel, bwd_dq_pair_kernel<512>, bwd_dkdv_pair_kernel<512>)"
                                if w.head_dim == 512 else
                                f"karpo_attn_bwd (bwd_dq_kernel<{w.head_dim}>, "
                                f"bwd_dkdv_kernel<{w.head_dim}, *>)"),
                     "avg_launch_ms": round(launch_ms, 4)},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_backward_baseline(w)
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: the benchmark measures one GPU; the attention kernel "
                                   "runs on one GPU's share: (sequence, key/value head) work items are "
                                   "independent, so a pack shards by heads or by sequences without exchange"}))
        return 2
    import torch

    from karpo_decision_amd import _lib, ops, workloads

    device = torch.device("cuda", 0)
    if args.workload == "keys_norm_rope":
        return keys_norm_rope(args, device)
    w = workloads.named(args.workload, device, args.seed)
    if args.backward:
        return backward(args, device, w)
    q_cu = torch.tensor(w.q_cu, dtype=torch.int32, device=device)
    k_cu = torch.tensor(w.k_cu, dtype=torch.int32, device=device)
    spans = torch.tensor(w.spans, dtype=torch.int32, device=device) if w.spans else None
    rows = (torch.tensor(w.key_rows, dtype=torch.int32, device=device) if w.key_rows is not None else None)
    gather = rows is not None and not args.materialize_gather
    plan = ops.make_plan(w.q_cu, w.k_cu, w.heads, w.kv_heads, w.head_dim, w.window_left, w.window_right, device,
                         gather=gather)

    fused = {}
    if w.q_norm is not None:
        fused["q_norm"] = ops.Norm(*w.q_norm)
    if w.rope is not None:
        fused["rope"] = w.rope
    if w.gate is not None:
        fused["gate"] = w.gate

    def step():
        if rows is not None and args.materialize_gather:
            key, value = w.key.index_select(0, rows), w.value.index_select(0, rows)
            return ops.run(w.query, key, value, q_cu, k_cu, w.max_q, w.scale, w.window_left, w.window_right, spans,
                           plan, **fused)
        return ops.run(w.query, w.key, w.value, q_cu, k_cu, w.max_q, w.scale, w.window_left, w.window_right, spans,
                       plan, rows, **fused)

    with torch.inference_mode():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(device)
        marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(args.steps)]
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        begin.record(stream)
        for a, b in marks:
            a.record(stream)
            step()
            b.record(stream)
        end.record(stream)
        torch.cuda.synchronize()
    if args.copy_bytes:
        copy_once(args.copy_bytes, device)
    total_ms = begin.elapsed_time(end)
    launch_ms = statistics.mean(a.elapsed_time(b) for a, b in marks)
    ms_per_step = total_ms / args.steps
    flops = w.flops()
    value = flops / (ms_per_step * 1e-3) / 1e12
    achieved = flops / (launch_ms * 1e-3) / 1e12

    shape = _lib.kernel_shape(w.heads, w.kv_heads, w.head_dim, w.max_q, gather)
    # the head-size-512 prefill tile without a row table runs as the pair ping-pong kernel
    kernel = ("attn_fwd_pair_pp_kernel" if (w.head_dim, shape, gather) == (512, 0, False)
              else f"attn_fwd_kernel<{w.head_dim}, {shape}, {str(gather).lower()}>")
    # HBM traffic per launch is not counted in this run (it needs rocprofv3 counter passes, see profiles/): it is the
    # recorded figure for this workload's kernel, with where and when it was recorded, or null when none matches
    traffic, traffic_source = None, None
    if TRAFFIC.exists():
        entry = json.loads(TRAFFIC.read_text()).get(w.name)
        if entry and entry.get("kernel") == kernel:
            traffic = entry.get("bytes_per_launch")
            traffic_source = (f"not measured in this run: {TRAFFIC.relative_to(ROOT)}, rocprofv3 FETCH_SIZE x "
                              f"{entry.get('fetch_factor')} + WRITE_SIZE x {entry.get('write_factor')} per dispatch of "
                              f"{entry.get('kernel')} ({entry.get('summary')}, recorded {entry.get('recorded', '?')})")
    if w.bound(PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)) == "mfma":
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4)}
    else:
        gbs = w.bytes() / (launch_ms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4)}
    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {**w.describe(), **({"gather": "index_select copies" if args.materialize_gather else "fused"}
                                      if rows is not None else {}),
                   "pct_of_bf16_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
                   "tokens_per_s": round(w.tokens / (ms_per_step * 1e-3)), "flops_per_step": flops,
                   "min_hbm_bytes_per_step": w.bytes(), "parallelism": "single GPU"},
        "roofline": {**roof, "traffic": traffic, "traffic_source": traffic_source, "kernel": kernel,
                     "avg_launch_ms": round(launch_ms, 4)},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_repeats)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
