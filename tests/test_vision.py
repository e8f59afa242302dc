"""Image soft-token spans (karpo_decision_amd/vision.py) on the reference's image layouts
(tests/test_gemma_images.py:136-155): one block and branches, two images, text longer than the window before an
image, several sequences with images and a text-only one in one pack, an image at a sequence's start, images in the
shared block and in branches, a branch image within and past a window of the shared block.

Each layout is built here token by token, recording where each image's soft tokens go, so the expected spans are
known answers, not a second run of the finder. Then the spans folded into the sliding layer's launch are checked
against the reference's contract for those layers: a query sees ``rule_a(segments, positions, window) | same image``
(tests/test_gemma_blocks.py:86-94, tests/test_gemma_images.py:127-131), over the block plan's sliding virtual
sequences (``block_plan``: a branch's keys are the shared block's last window - 1 rows, then its own rows,
families/gemma/packed.py:103-134)."""

from __future__ import annotations

import pytest
import torch

from karpo_decision_amd import vision
from oracle import attention as oa

BEGIN, SOFT, END = 1, 2, 3
WINDOW = 96  # longer than every image below, as in the reference's image tests


class Builder:
    """One sequence of a pack: a shared block and branches, text tokens and images (begin, soft x n, end, text)."""

    def __init__(self, seed: int):
        self.gen = torch.Generator().manual_seed(seed)
        self.ids: list[int] = []
        self.seg: list[int] = []
        self.pos: list[int] = []
        self.spans: list[tuple[int, int]] = []  # soft rows of each image, relative to the sequence's first row
        self.shared = 0

    def _emit(self, parts, segment: int, first_pos: int) -> None:
        p = first_pos
        for part in parts:
            tokens = []
            if isinstance(part, int):
                tokens = torch.randint(4, 280, (part,), generator=self.gen).tolist()
            else:  # ("img", n): an image of n soft tokens
                s = len(self.ids) + 1
                self.spans.append((s, s + part[1]))
                tokens = [BEGIN, *[SOFT] * part[1], END, int(torch.randint(4, 280, (1,), generator=self.gen))]
            self.ids += tokens
            self.seg += [segment] * len(tokens)
            self.pos += range(p, p + len(tokens))
            p += len(tokens)

    def block(self, shared, branches=()):
        self._emit(shared, 0, 0)
        self.shared = len(self.ids)
        for k, parts in enumerate(branches, start=1):  # branches restart at the shared block's end position
            self._emit(parts, k, self.shared)
        return self


def img(n: int):
    return ("img", n)


def one(shared, branches=(), seed=0):
    return Builder(seed).block(shared, branches)


LAYOUTS = {
    "one-block": lambda: [one([12, img(70), 9])],
    "branches": lambda: [one([7, img(70), 5], [[6], [9], [4]])],
    "two-images": lambda: [one([5, img(70), img(48), 8], [[5]])],
    "text-past-the-window": lambda: [one([WINDOW + 30, img(64), 4])],
    "two-parts-and-text": lambda: [one([6, img(70), 3], [[5]], 1), one([8, img(70), 2], [[7]], 2), one([15], seed=3)],
    "image-at-a-sequence-start": lambda: [one([9, img(48), 2], [[4], [3]], 4), one([img(70), 6], seed=5)],
    "image-in-a-branch": lambda: [one([6], [[3, img(70), 4], [5]])],
    "images-in-the-shared-block-and-two-branches": lambda: [
        one([5, img(70), 3], [[2, img(70), 2], [4, img(48), 3]])],
    "branch-image-within-a-window-of-the-shared-block": lambda: [one([WINDOW + 10], [[7], [20, img(70), 5]])],
    "branch-image-past-a-window-of-the-shared-block": lambda: [one([12], [[9], [WINDOW + 5, img(70), 2]])],
    "one-block-text-then-an-image": lambda: [one([7, img(70), 6])],
    "branch-images-and-text-in-one-pack": lambda: [one([4], [[img(70), 3]], 6), one([12], seed=7),
                                                   one([3, img(70)], [[2], [img(70), 2]], 8)],
}


def pack(seqs):
    """(ids, segments, positions, sequence bounds, absolute spans) of the sequences packed one after another."""
    ids, seg, pos, bounds, spans = [], [], [], [0], []
    for s in seqs:
        spans += [(a + bounds[-1], b + bounds[-1]) for a, b in s.spans]
        ids += s.ids
        seg += s.seg
        pos += s.pos
        bounds.append(len(ids))
    return torch.tensor(ids), torch.tensor(seg), torch.tensor(pos), bounds, spans


@pytest.mark.parametrize("name", list(LAYOUTS))
def test_spans_are_each_images_soft_tokens(name):
    ids, _, _, bounds, spans = pack(LAYOUTS[name]())
    assert vision.soft_token_spans(ids, SOFT, WINDOW, bounds) == spans
    assert vision.soft_token_spans(ids, SOFT) == spans  # no window, no bounds: the same runs


def test_an_image_longer_than_the_window_is_refused():
    ids, *_ = pack([one([3, img(70), 3])])
    with pytest.raises(ValueError, match="longer than the sliding window"):
        vision.soft_token_spans(ids, SOFT, window=16)
    assert vision.soft_token_spans(ids, SOFT, window=70) == [(4, 74)]  # an image as long as the window fits


def test_runs_at_the_edges_and_none():
    assert vision.soft_token_spans(torch.tensor([2, 2, 5, 2]), SOFT) == [(0, 2), (3, 4)]
    assert vision.soft_token_spans(torch.tensor([5, 6]), SOFT) == []
    assert vision.soft_token_spans(torch.tensor([], dtype=torch.long), SOFT) == []
    with pytest.raises(ValueError, match="inside one sequence"):  # a run across a sequence boundary
        vision.soft_token_spans(torch.tensor([5, 2, 2, 5]), SOFT, bounds=[0, 2, 4])


def test_span_tensor_sorts_and_refuses_empty_or_overlapping_spans():
    t = vision.span_tensor([(10, 20), (3, 5)], "cpu")
    assert t.dtype == torch.int32 and t.tolist() == [[3, 5], [10, 20]]
    assert vision.span_tensor([], "cpu") is None
    assert vision.span_tensor([(5, 9), (9, 12)], "cpu").tolist() == [[5, 9], [9, 12]]  # touching is fine
    with pytest.raises(ValueError, match="empty"):
        vision.span_tensor([(4, 4)], "cpu")
    with pytest.raises(ValueError, match="empty"):
        vision.span_tensor([(6, 2)], "cpu")
    with pytest.raises(ValueError, match="overlap"):
        vision.span_tensor([(0, 10), (9, 12)], "cpu")


def sliding_plan(seg, bounds, window):
    """The block plan's sliding virtual sequences (families/gemma/packed.py:112-134, restated): per sequence its shared
    block over its own rows, then each branch over the shared block's last window - 1 rows and its own rows.
    Returns (q_cu, s_cu, s_rows) with rows in pack coordinates."""
    q_cu, s_cu, s_rows = [0], [0], []
    for a, b in zip(bounds[:-1], bounds[1:]):
        labels = seg[a:b].tolist()
        shared = labels.count(0)
        own = list(range(a, a + shared))
        tail = own[max(0, shared - (window - 1)):]
        q_cu.append(a + shared)
        s_rows += own
        s_cu.append(s_cu[-1] + shared)
        k = 1
        while a + shared < b and k in labels:
            rows = [a + i for i, x in enumerate(labels) if x == k]
            q_cu.append(rows[-1] + 1)
            s_rows += tail + rows
            s_cu.append(s_cu[-1] + len(tail) + len(rows))
            k += 1
    return q_cu, s_cu, s_rows


@pytest.mark.parametrize("name", list(LAYOUTS))
def test_spans_in_the_sliding_launch_give_the_references_image_masks(name):
    """For every query row: the pack rows it sees through the sliding launch (the window rule over its virtual
    sequence's keys, OR its span) are exactly those rule_a(window) | same-image gives on the unpacked sequence."""
    ids, seg, pos, bounds, spans = pack(LAYOUTS[name]())
    found = vision.soft_token_spans(ids, SOFT, WINDOW, bounds)
    q_cu, s_cu, s_rows = sliding_plan(seg, bounds, WINDOW)
    image = torch.full((len(ids),), -1)
    for n, (s, e) in enumerate(spans):
        image[s:e] = n
    for qa, qb, ka, kb in zip(q_cu[:-1], q_cu[1:], s_cu[:-1], s_cu[1:]):
        lq, lk = qb - qa, kb - ka
        if lq == 0:
            continue
        q_span, k_span = oa.span_ids(qa, lq, lk, found)
        seen = oa.visible(lq, lk, WINDOW - 1, 0, q_span, k_span)
        keys = torch.tensor(s_rows[ka:kb])
        start = max(b for b in bounds if b <= qa)
        end = min(b for b in bounds if b > qa)
        for i in range(lq):
            r = qa + i
            got = set(keys[seen[i]].tolist())
            cand = torch.arange(start, end)
            rule = ((seg[cand] == 0) | (seg[cand] == seg[r])) & (pos[cand] <= pos[r]) & (pos[r] - pos[cand] < WINDOW)
            rule |= (image[cand] == image[r]) & (image[r] >= 0)
            want = set(cand[rule].tolist())
            assert got == want, (name, r, sorted(got ^ want)[:8])
