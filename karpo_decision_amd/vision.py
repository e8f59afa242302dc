"""Image soft-token spans for the attention call.

The reference finds each image's contiguous soft-token rows (``plan_images``, src/karpo_decision/families/gemma/
vision.py:168-195) and, after the sliding layers' varlen call, recomputes those rows so they see their whole image
(``see_whole``, :198-210; the test contract is ``rule_a(...) | same``, tests/test_gemma_images.py:127-131). Here the
spans go into the attention launch itself: a query row inside span [s, e) also sees the keys aligned with rows
[s, e) of its own sequence, so no row is computed twice and no per-image launch or ``index_copy`` is needed.
"""

from __future__ import annotations

from collections.abc import Iterable

import torch


def soft_token_spans(input_ids: torch.Tensor, soft: int, window: int | None = None) -> list[tuple[int, int]]:
    """The (s, e) row ranges of contiguous runs of the soft token ``soft`` in ``input_ids`` (CPU), as
    ``plan_images`` finds them (vision.py:175-181); ValueError for a run longer than ``window`` (vision.py:182-183)."""
    rows = (input_ids == soft).nonzero().flatten()
    if rows.numel() == 0:
        return []
    breaks = ((rows[1:] != rows[:-1] + 1).nonzero().flatten() + 1).tolist()
    out = []
    for a, b in zip([0, *breaks], [*breaks, len(rows)], strict=True):
        s, e = int(rows[a]), int(rows[b - 1]) + 1
        if window is not None and e - s > window:
            raise ValueError(f"an image of {e - s} soft tokens is longer than the sliding window ({window})")
        out.append((s, e))
    return out


def span_tensor(spans: Iterable[tuple[int, int]], device: torch.device | str) -> torch.Tensor | None:
    """(n, 2) int32 spans sorted by start on ``device`` (None for no spans); ValueError for empty or overlapping
    ranges."""
    items = sorted((int(s), int(e)) for s, e in spans)
    for (s, e), nxt in zip(items, [*items[1:], None], strict=True):
        if e <= s:
            raise ValueError(f"span ({s}, {e}) is empty")
        if nxt is not None and nxt[0] < e:
            raise ValueError(f"spans ({s}, {e}) and {nxt} overlap")
    if not items:
        return None
    return torch.tensor(items, dtype=torch.int32).to(device)
