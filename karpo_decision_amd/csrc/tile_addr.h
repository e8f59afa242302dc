// Per-lane addressing of the forward kernel (attn_fwd.hip), as host-and-device functions: where each lane's copy
// instructions read (the DMA sources), which keys a query lane sees, which key steps a part of a tile visits, and the
// byte offset of a row read through a row table. The kernel computes every address from these functions; a host
// replay (tests/replay/fwd_replay.cpp) walks every work item of a plan with the same functions and checks each access
// against the allocations.
#pragma once
#include <stdint.h>

#include "plan_common.h"

namespace karpo {

// Where lane `lane` of DMA instruction `blk` (1 KiB of the K tile each) reads: the key row inside the step and the
// element column. The inverse of k_offset (mfma_common.h) for byte offset blk * 1024 + lane * 16.
template <int D>
KA_HD inline void k_dma_source(int blk, int lane, int* key, int* col) {
  const int b = blk * 4 + (lane >> 4);  // 256-byte block: (key block, chunk)
  *key = (b / (D / 8)) * 16 + (lane & 15);
  *col = (b % (D / 8)) * 8;
}
// The same for the V tile (the inverse of v_offset).
template <int D>
KA_HD inline void v_dma_source(int blk, int lane, int* key, int* col) {
  const int b = blk * 8 + (lane >> 3);  // 128-byte block: (key group, d block)
  const int piece = lane & 7;
  *key = (b / (D / 16)) * 4 + (piece >> 1);
  *col = (b % (D / 16)) * 16 + (piece & 1) * 8;
}

// The tile vector that lane column `col` (0-31) of wave `wave` holds in its query block `block`: a wave's blocks (a
// pair's, at head_dim 512, where both waves hold the same vectors) are consecutive 32-vector runs of the tile.
KA_HD inline int lane_vector(int wave, int block, int col, bool pair, int blocks) {
  return ((pair ? wave >> 1 : wave) * blocks + block) * 32 + col;
}

// The keys query `pos` of a sequence sees (qa: the sequence's first query row in the pack, lq / lk: its query and key
// rows, query i at key coordinate i + lk - lq): [lo, hi) from the (left, right) window (-1: unbounded), and [sl, sh)
// from the image span holding its row (spans: sorted, non-overlapping half-open query-row ranges), empty when none.
// A query past the sequence (pos >= lq) sees nothing.
struct LaneKeys {
  int lo, hi, sl, sh;
};
KA_HD inline LaneKeys lane_keys(int pos, int qa, int lq, int lk, int left, int right, const int32_t* spans,
                                int n_spans) {
  LaneKeys r = {0, 0, 0, 0};
  if (pos >= lq) return r;
  const int ip = pos + (lk - lq);  // aligned key coordinate
  const int a = left < 0 ? 0 : (ip - left > 0 ? ip - left : 0);
  int b = right < 0 ? lk : (int)ka_min((int64_t)lk, (int64_t)ip + right + 1);
  if (b < a) b = a;
  r.lo = a;
  r.hi = b;
  if (n_spans > 0) {  // the last span starting at or before this query row
    const int row = qa + pos;
    int l0 = 0, l1 = n_spans;
    while (l1 - l0 > 1) {
      const int mid = (l0 + l1) >> 1;
      if (spans[2 * mid] <= row) l0 = mid; else l1 = mid;
    }
    const int s0 = spans[2 * l0], s1 = spans[2 * l0 + 1];
    if (s0 <= row && row < s1) {
      const int x = s0 - qa + (lk - lq), y = s1 - qa + (lk - lq);
      const int xc = x > 0 ? x : 0, yc = y < lk ? y : lk;
      if (xc < yc) {
        r.sl = xc;
        r.sh = yc;
      }
    }
  }
  return r;
}

// The key steps a part of a tile visits: the tile's envelope of visible keys [klo, khi) in steps of bn aligned to the
// sequence's first key, and part `part` of `parts` of those steps (all of them when parts <= 1).
KA_HD inline void part_steps(int klo, int khi, int bn, int part, int parts, int* j_first, int* n_steps) {
  int j = klo < khi ? (klo / bn) * bn : 0;
  int n = klo < khi ? (khi - j + bn - 1) / bn : 0;
  if (parts > 1) {
    const int s0 = (int)((int64_t)part * n / parts), s1 = (int)((int64_t)(part + 1) * n / parts);
    j += s0 * bn;
    n = s1 - s0;
  }
  *j_first = j;
  *n_steps = n;
}

// Byte offset, from a key/value head's first element, of the 16-byte chunk at byte column `colb` of row `row` read
// through a row table; a row outside [0, total) reads at `past`, the buffer's size in bytes, where every dword of
// the 16-byte access is past the buffer's bounds (the copy returns zeros; `past` + 16 stays below 2^32, so no
// dword offset wraps around into the buffer).
KA_HD inline uint32_t gather_offset(int row, int total, uint32_t row_bytes, uint32_t colb, uint32_t past) {
  return (unsigned)row < (unsigned)total ? (uint32_t)row * row_bytes + colb : past;
}

// Floats from the partial buffer's start to part `part` of the split tile whose parts start at slot `slot`, head
// group `hg`: per slot and head group O [vectors][D], then m [vectors], then l [vectors].
KA_HD inline int64_t partial_base(int slot, int part, int n_hg, int hg, int vectors, int head_dim) {
  return ((int64_t)(slot + part) * n_hg + hg) * (int64_t)vectors * (head_dim + 2);
}

}  // namespace karpo
