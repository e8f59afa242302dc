"""Image soft-token spans for the attention call.

The reference finds each image's contiguous soft-token rows (``plan_images``, src/karpo_decision/families/gemma/
vision.py:168-195) and, after the sliding layers' varlen call, recomputes those rows so they see their whole image
(``see_whole``, :198-210; the test contract is ``rule_a(...) | same``, tests/test_gemma_images.py:127-131). Here the
spans go into the attention launch itself: a query row inside span [s, e) also sees the keys aligned with rows
[s, e) of its own sequence, so no row is computed twice and no per-image launch or ``index_copy`` is needed. For an
image in a branch the alignment is the block plan's: a branch's sliding keys are the shared block's last window - 1
rows, then the branch's own rows, aligned at the end, so the span's rows map onto the branch's own keys.
"""

from __future__ import annotations

import bisect
from collections.abc import Iterable, Sequence

import torch


def soft_token_spans(input_ids: torch.Tensor, soft: int, window: int | None = None,
                     bounds: Sequence[int] | None = None) -> list[tuple[int, int]]:
    """The half-open row ranges [s, e) of ``input_ids`` (1-D, any device) holding runs of the soft token ``soft``:
    each image's soft tokens, in row order. The runs are read off the edges of the soft-token indicator: +1 where a
    run starts, -1 one past where it ends. ValueError for a run longer than ``window`` (an image must fit the sliding
    window, as vision.py:182-183 requires) or, with the pack's sequence ``bounds``, a run that crosses a sequence
    boundary (a span must lie inside one sequence)."""
    flag = (input_ids.reshape(-1) == soft).to(torch.int8).cpu()
    edges = torch.diff(torch.nn.functional.pad(flag, (1, 1)))
    starts = (edges == 1).nonzero().flatten().tolist()
    ends = (edges == -1).nonzero().flatten().tolist()
    spans = list(zip(starts, ends))
    for s, e in spans:
        if window is not None and e - s > window:
            raise ValueError(f"an image of {e - s} soft tokens (rows {s}..{e}) is longer than the sliding window "
                             f"({window})")
        if bounds is not None:
            inside = bisect.bisect_right(bounds, s) - 1
            if inside < 0 or inside + 1 >= len(bounds) or e > bounds[inside + 1]:
                raise ValueError(f"image rows {s}..{e} do not lie inside one sequence of the pack")
    return spans


def span_tensor(spans: Iterable[tuple[int, int]], device: torch.device | str) -> torch.Tensor | None:
    """(n, 2) int32 spans sorted by start on ``device`` (None for no spans); ValueError for empty or overlapping
    ranges."""
    items = sorted((int(s), int(e)) for s, e in spans)
    if not items:
        return None
    for n, (s, e) in enumerate(items):
        if e <= s:
            raise ValueError(f"span ({s}, {e}) is empty")
        if n + 1 < len(items) and items[n + 1][0] < e:
            raise ValueError(f"spans ({s}, {e}) and {items[n + 1]} overlap")
    return torch.tensor(items, dtype=torch.int32).to(device)
