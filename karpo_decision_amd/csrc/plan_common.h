// Tile geometry and the per-tile cost shared by the host planner (plan.cpp) and the device planner (attn_fwd.hip).
//
// A work item is one query tile of one segment for one group of query heads. A tile holds 128 query vectors (32 per
// wave of a 4-wave workgroup); a vector is one (position, head) pair. When the GQA
// group size G divides `vectors`, a tile covers vectors / G positions of all G heads of one key/value head, so one
// staged K/V tile serves every head of the group; otherwise a tile covers `vectors` positions of one query head.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define KA_HD __host__ __device__
#else
#define KA_HD
#endif

namespace karpo {

#ifndef KA_W128
#define KA_W128 12
#endif
#ifndef KA_W256
#define KA_W256 8
#endif
#ifndef KA_BN128
#define KA_BN128 64
#endif
// Waves per workgroup (each holds 32 query vectors of the tile) and keys per step, per head size.
KA_HD constexpr int tile_waves(int head_dim) { return head_dim == 128 ? KA_W128 : head_dim == 256 ? KA_W256 : 4; }
KA_HD constexpr int tile_keys(int head_dim) { return head_dim == 128 ? KA_BN128 : head_dim == 256 ? 32 : 64; }
constexpr int kPlanHeader = 4;       // int32 header of a plan: tiles, rows per tile, keys per step, heads per item
constexpr int kCostBuckets = 2048;   // device planner's cost histogram (costs clamp to the last bucket)

struct Geometry {
  int vectors;   // query vectors per tile
  int bn;        // keys per step
  int ng;        // query heads per work item
  int rows;      // query positions per tile
  int n_hg;      // work items per tile (head groups)
};

KA_HD inline bool head_dim_supported(int d) { return d == 64 || d == 128 || d == 256; }

KA_HD inline Geometry geometry(int heads, int kv_heads, int head_dim) {
  Geometry g;
  g.vectors = 32 * tile_waves(head_dim);
  g.bn = tile_keys(head_dim);
  int group = heads / kv_heads;
  g.ng = (g.vectors % group == 0) ? group : 1;
  g.rows = g.vectors / g.ng;
  g.n_hg = heads / g.ng;
  return g;
}

KA_HD inline int64_t ka_min(int64_t a, int64_t b) { return a < b ? a : b; }
KA_HD inline int64_t ka_max(int64_t a, int64_t b) { return a > b ? a : b; }

// Key steps a tile visits: keys [lo, hi) any query of tile t can see under the (left, right) window with the
// bottom-right alignment (query i sits at key i + lk - lq), in steps of bn aligned to the segment's first key, plus one
// for the tile's own store. Spans are not counted (they only reorder equal work slightly).
KA_HD inline int tile_cost(int lq, int lk, int t, int rows, int bn, int left, int right) {
  const int64_t delta = (int64_t)lk - lq;
  int64_t p0 = (int64_t)t * rows;
  int64_t p1 = ka_min((int64_t)lq, p0 + rows) - 1;
  // queries that see at least one key: i' + right >= 0 and i' - left < lk (i' = p + delta)
  if (right >= 0) p0 = ka_max(p0, -(int64_t)right - delta);
  if (left >= 0) p1 = ka_min(p1, (int64_t)lk + left - 1 - delta);
  if (lk <= 0 || p1 < p0) return 1;
  const int64_t lo = left < 0 ? 0 : ka_max(0, p0 + delta - left);
  const int64_t hi = right < 0 ? (int64_t)lk : ka_min((int64_t)lk, p1 + delta + right + 1);
  if (hi <= lo) return 1;
  return (int)((hi + bn - 1) / bn - lo / bn) + 1;
}

KA_HD inline int64_t tiles_of(int64_t lq, int rows) { return lq <= 0 ? 0 : (lq + rows - 1) / rows; }

}  // namespace karpo
