"""Synthetic packs of the five measured attention workloads, and their algorithmic FLOP counts.

Inputs: one seeded generator per workload (on the target device, so 131k-token packs are made where they live).
"RMS-normalised N(0,1)" is ``x / sqrt(mean(x^2) + 1e-6)`` per head vector; V is N(0,1). Segment lengths are
log-normal with mu = ln(median) and sigma = 1.0, clipped to the workload's range, drawn until the pack is full, the
last one truncated so the total is exact.

Algorithmic FLOPs = 4 * D * H * (allowed (query, key) pairs): 2 for Q.K and 2 for P.V per pair, excluding masked
pairs, softmax and any padded or skipped work.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

SIGMA = 1.0


@dataclass
class Workload:
    name: str
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    q_cu: list[int]
    k_cu: list[int]
    scale: float
    window_left: int = -1
    window_right: int = 0
    spans: list[tuple[int, int]] = field(default_factory=list)
    seed: int = 0
    key_rows: list[int] | None = None  # key row r of the pack is row key_rows[r] of key / value (a block plan's gather)
    # fused query prologue and gate: (mode, weight, eps) of the norm (oracle/prologue.py modes), (cos, sin) rows per
    # query row, and the gate; the query is then the projection's raw output
    q_norm: tuple[int, torch.Tensor, float] | None = None
    rope: tuple[torch.Tensor, torch.Tensor] | None = None
    gate: torch.Tensor | None = None

    @property
    def heads(self) -> int:
        return self.query.shape[1]

    @property
    def kv_heads(self) -> int:
        return self.key.shape[1]

    @property
    def head_dim(self) -> int:
        return self.query.shape[2]

    @property
    def max_q(self) -> int:
        return max((b - a for a, b in zip(self.q_cu[:-1], self.q_cu[1:])), default=0)

    @property
    def tokens(self) -> int:
        return self.q_cu[-1]

    def pairs(self) -> int:
        return allowed_pairs(self.q_cu, self.k_cu, self.window_left, self.window_right, self.spans)

    def flops(self) -> float:
        return 4.0 * self.head_dim * self.heads * self.pairs()

    def bytes(self) -> int:
        """HBM bytes the op must move at least: read Q, K, V once, write O (bf16)."""
        return 2 * (2 * self.query.numel() + self.key.numel() + self.value.numel())

    def gathered(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(key, value) with the gather applied (the copies ``index_select`` makes), or the tensors themselves."""
        if self.key_rows is None:
            return self.key, self.value
        rows = torch.tensor(self.key_rows, dtype=torch.int64, device=self.key.device)
        return self.key.index_select(0, rows), self.value.index_select(0, rows)

    def bound(self, ridge: float) -> str:
        """"mfma" when the algorithmic FLOPs per byte exceed the roofline's ridge point, else "hbm"."""
        return "mfma" if self.flops() / self.bytes() > ridge else "hbm"

    def describe(self) -> dict:
        return {"workload": self.name, "tokens": self.tokens, "segments": len(self.q_cu) - 1, "heads": self.heads,
                "kv_heads": self.kv_heads, "head_dim": self.head_dim, "window_left": self.window_left,
                "window_right": self.window_right, "spans": len(self.spans), "seed": self.seed,
                "sigma": SIGMA, "pairs": self.pairs()}


def _segment_pairs(lq: int, lk: int, left: int, right: int) -> int:
    i = np.arange(lq, dtype=np.int64) + (lk - lq)
    lo = np.zeros_like(i) if left < 0 else np.maximum(0, i - left)
    hi = np.full_like(i, lk) if right < 0 else np.minimum(lk, i + right + 1)
    return int(np.maximum(0, hi - lo).sum())


def allowed_pairs(q_cu: list[int], k_cu: list[int], left: int, right: int,
                  spans: list[tuple[int, int]] = ()) -> int:
    """Allowed (query, key) pairs of a pack: the window rule per sequence, plus each span's pairs the rule does not
    already allow (for a causal span of n rows no longer than the window: n(n-1)/2)."""
    total = 0
    for qa, qb, ka, kb in zip(q_cu[:-1], q_cu[1:], k_cu[:-1], k_cu[1:]):
        total += _segment_pairs(qb - qa, kb - ka, left, right)
    for s, e in spans:
        seg = int(np.searchsorted(np.asarray(q_cu), s, side="right")) - 1
        qa, qb, ka, kb = q_cu[seg], q_cu[seg + 1], k_cu[seg], k_cu[seg + 1]
        delta = (kb - ka) - (qb - qa)
        i = np.arange(s - qa, e - qa, dtype=np.int64)[:, None] + delta
        j = np.arange(max(0, s - qa + delta), min(kb - ka, e - qa + delta), dtype=np.int64)[None, :]
        base = np.ones((i.shape[0], j.shape[1]), dtype=bool)
        if right >= 0:
            base &= j <= i + right
        if left >= 0:
            base &= j >= i - left
        total += int((~base).sum())
    return total


def lognormal_lengths(total: int, median: float, lo: int, hi: int, seed: int) -> list[int]:
    rng = np.random.default_rng(seed)
    out, run = [], 0
    while run < total:
        n = int(np.clip(round(math.exp(rng.normal(math.log(median), SIGMA))), lo, hi))
        n = min(n, total - run)
        out.append(n)
        run += n
    return out


def bounds(lengths: list[int]) -> list[int]:
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


def _normal(shape, gen, device, rms: bool) -> torch.Tensor:
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if rms:
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6)
    return x


def make_tensors(tokens: int, heads: int, kv_heads: int, head_dim: int, seed: int, device, dtype=torch.bfloat16,
                 rms: bool = True):
    """(q, k, v): q and k RMS-normalised N(0,1) per head vector (plain N(0,1) if not ``rms``), v N(0,1)."""
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    q = _normal((tokens, heads, head_dim), gen, device, rms).to(dtype)
    k = _normal((tokens, kv_heads, head_dim), gen, device, rms).to(dtype)
    v = _normal((tokens, kv_heads, head_dim), gen, device, False).to(dtype)
    return q, k, v


def tiny(device="cpu", dtype=torch.bfloat16, seed: int = 0) -> Workload:
    """4 segments {37, 128, 300, 511} (976 tokens), 8 query / 2 KV heads, head_dim 64, N(0,1), causal, scale 1/8."""
    cu = [0, 37, 165, 465, 976]
    q, k, v = make_tensors(976, 8, 2, 64, seed, device, dtype, rms=False)
    return Workload("tiny-causal-gqa-976", q, k, v, cu, cu, 1 / 8, -1, 0, seed=seed)


def qwen_full(device="cuda", seed: int = 0, tokens: int = 8192) -> Workload:
    """Qwen3.5-0.8B-class full-attention layer: 16 / 8 heads, D 128, log-normal lengths (median 600, [16, 4096])."""
    cu = bounds(lognormal_lengths(tokens, 600, 16, 4096, seed))
    q, k, v = make_tensors(tokens, 16, 8, 128, seed, device)
    return Workload(f"qwen-full-{tokens}", q, k, v, cu, cu, 1 / math.sqrt(128), -1, 0, seed=seed)


def gemma_sliding(device="cuda", seed: int = 0, tokens: int = 16384, scale: float | None = None) -> Workload:
    """Gemma-12B-class sliding layer: 16 / 8 heads, D 256, window 1024 (left 1023), lengths median 1500 in
    [32, 8192]."""
    cu = bounds(lognormal_lengths(tokens, 1500, 32, 8192, seed))
    q, k, v = make_tensors(tokens, 16, 8, 256, seed, device)
    return Workload(f"gemma-sliding-{tokens}", q, k, v, cu, cu, scale if scale is not None else 1 / 16, 1023, 0,
                    seed=seed)


def gemma_global(length: int = 32768, device="cuda", seed: int = 0) -> Workload:
    """Gemma-31B-class global layer: one causal segment, 32 / 16 heads, D 128, scale 1/sqrt(128)."""
    q, k, v = make_tensors(length, 32, 16, 128, seed, device)
    return Workload(f"gemma-global-causal-{length}", q, k, v, [0, length], [0, length], 1 / math.sqrt(128), -1, 0,
                    seed=seed)


def rope_tables(rows: int, rotated: int, seed: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 (rows, rotated) cos / sin tables of rotation-by-halves form (each angle twice), seeded angles."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed + 7)
    angle = torch.rand(rows, rotated // 2, generator=gen, device=device) * 30
    return (torch.cat((angle.cos(), angle.cos()), -1).bfloat16(), torch.cat((angle.sin(), angle.sin()), -1).bfloat16())


def with_prologue(w: Workload, family: str) -> Workload:
    """``w`` with its layer's query prologue fused: Gemma (RMSNorm times a weight, rotation of the whole head) or
    Qwen (RMSNorm times 1 + weight, rotation of the first quarter, sigmoid gate on the output); the query becomes an
    un-normalised projection output (N(0, 3^2))."""
    gen = torch.Generator(device=w.query.device)
    gen.manual_seed(w.seed + 11)
    d = w.head_dim
    raw = (torch.randn(w.query.shape, generator=gen, device=w.query.device) * 3).bfloat16()
    weight = (torch.randn(d, generator=gen, device=w.query.device) * 0.2 + (1.0 if family == "gemma" else 0.0))
    weight = weight.bfloat16()
    if family == "gemma":
        return Workload(w.name + "-prologue", raw, w.key, w.value, w.q_cu, w.k_cu, w.scale, w.window_left,
                        w.window_right, w.spans, w.seed, w.key_rows, (1, weight, 1e-6),
                        rope_tables(raw.shape[0], d, w.seed, raw.device))
    gate = (torch.randn(w.query.shape, generator=gen, device=w.query.device) * 2).bfloat16()
    return Workload(w.name + "-gated", raw, w.key, w.value, w.q_cu, w.k_cu, w.scale, w.window_left, w.window_right,
                    w.spans, w.seed, w.key_rows, (2, weight, 1e-6), rope_tables(raw.shape[0], d // 4, w.seed,
                                                                                raw.device), gate)


def gemma_global_512(length: int = 32768, device="cuda", seed: int = 0) -> Workload:
    """Gemma 4 31B's global layer shape: one causal segment, 32 query / 4 KV heads, head_dim 512
    (families/gemma/packed.py:1-2; tests/gpu/test_triton_attention.py:32), scale 1/sqrt(512)."""
    q, k, v = make_tensors(length, 32, 4, 512, seed, device)
    return Workload(f"gemma-global-d512-causal-{length}", q, k, v, [0, length], [0, length], 1 / math.sqrt(512), -1,
                    0, seed=seed)


def branched(device="cuda", seed: int = 0, prompts: int = 4, shared: int = 4096, branches: int = 4,
             branch: int = 512) -> Workload:
    """A block plan's global layer (families/gemma/packed.py:103-151): ``prompts`` prompts, each a ``shared``-token
    block (its own virtual sequence) and ``branches`` branches of ``branch`` tokens whose keys are the shared rows
    followed by their own, read through the gather table ``g_rows`` (``key_rows``) from the pack's K/V; causal,
    32 / 16 heads, D 128."""
    q_cu, k_cu, rows = [0], [0], []
    at = 0
    for _ in range(prompts):
        own = list(range(at, at + shared))
        q_cu.append(at + shared)
        rows += own
        k_cu.append(k_cu[-1] + shared)
        at += shared
        for _ in range(branches):
            q_cu.append(at + branch)
            rows += own + list(range(at, at + branch))
            k_cu.append(k_cu[-1] + shared + branch)
            at += branch
    q, k, v = make_tensors(at, 32, 16, 128, seed, device)
    return Workload(f"branched-{prompts}x{shared}+{branches}x{branch}", q, k, v, q_cu, k_cu, 1 / math.sqrt(128), -1, 0,
                    seed=seed, key_rows=rows)


def _multimodal_lengths(rng: np.random.Generator, tokens: int, segments: int) -> np.ndarray:
    raw = np.exp(rng.normal(math.log(900), SIGMA, size=segments))
    lengths = np.maximum(16, np.floor(raw / raw.sum() * tokens)).astype(np.int64)
    lengths[np.argmax(lengths)] += tokens - int(lengths.sum())
    return lengths


def markers_only(device="cuda", seed: int = 0, tokens: int = 65536, segments: int = 48) -> Workload:
    """The markers-only last global layer (families/gemma/packed.py:267-281) of the mixed 65,536-token pack: one
    query per virtual sequence over all of its keys, bidirectional, 32 / 16 heads, D 128. Decode-shaped: every key is
    read once and used by the group's two query heads, so the bound is HBM bandwidth."""
    lengths = _multimodal_lengths(np.random.default_rng(seed), tokens, segments)
    k_cu = bounds([int(x) for x in lengths])
    m_cu = bounds([1] * segments)
    q, _, _ = make_tensors(segments, 32, 16, 128, seed + 1, device)
    _, k, v = make_tensors(tokens, 32, 16, 128, seed, device)
    return Workload(f"markers-only-{tokens}", q, k, v, m_cu, k_cu, 1 / math.sqrt(128), -1, -1, seed=seed)


def mixed_multimodal(device="cuda", seed: int = 0, tokens: int = 65536, segments: int = 48,
                     image_segments: int = 12, span: int = 560) -> Workload:
    """65,536 tokens in 48 log-normal segments (median 900, scaled to sum exactly); 12 segments carry one or two
    560-row image spans at seeded non-overlapping offsets; causal plus bidirectional within each span; 32 / 16
    heads, D 128."""
    rng = np.random.default_rng(seed)
    lengths = _multimodal_lengths(rng, tokens, segments)
    cu = bounds([int(x) for x in lengths])
    eligible = [i for i in range(segments) if lengths[i] >= span]
    chosen = sorted(rng.choice(eligible, size=min(image_segments, len(eligible)), replace=False).tolist())
    spans = []
    for i in chosen:
        n = int(lengths[i])
        count = 2 if (n >= 2 * span and rng.random() < 0.5) else 1
        # non-overlapping offsets: split the free rows into count + 1 gaps
        free = n - count * span
        cuts = np.sort(rng.integers(0, free + 1, size=count))
        at = cu[i]
        for c in range(count):
            start = at + int(cuts[c]) + c * span
            spans.append((start, start + span))
    q, k, v = make_tensors(tokens, 32, 16, 128, seed, device)
    return Workload(f"mixed-multimodal-{tokens}", q, k, v, cu, cu, 1 / math.sqrt(128), -1, 0, sorted(spans),
                    seed=seed)


def named(name: str, device="cuda", seed: int = 0) -> Workload:
    table = {
        "tiny": lambda: tiny(device, seed=seed),
        "qwen": lambda: qwen_full(device, seed),
        "sliding": lambda: gemma_sliding(device, seed),
        "global32k": lambda: gemma_global(32768, device, seed),
        "global131k": lambda: gemma_global(131072, device, seed),
        "global32k_d512": lambda: gemma_global_512(32768, device, seed),
        "multimodal": lambda: mixed_multimodal(device, seed),
        "markers": lambda: markers_only(device, seed),
        "branched": lambda: branched(device, seed),
        "global32k_prologue": lambda: with_prologue(gemma_global(32768, device, seed), "gemma"),
        "qwen_gated": lambda: with_prologue(qwen_full(device, seed), "qwen"),
    }
    if name not in table:
        raise ValueError(f"unknown workload {name!r}; one of {sorted(table)}")
    return table[name]()
