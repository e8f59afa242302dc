// Host planner: the longest-first work list from host copies of the sequence bounds.
//
// The reference builds every device bound of a pack once on the host, before the first layer is queued
// (block_plan, families/gemma/packed.py:103-151), and reuses them in every layer. This is the same step for the
// kernel's work list: one pass over the sequences, one item per (sequence, query tile), sorted by the number of key
// steps the tile visits (ties: sequence, then tile order), so a workgroup that starts late takes short work. Fully
// masked key steps (outside the window, above the causal diagonal, across sequences) are never listed: a tile's
// steps are the window envelope of its queries only.
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "karpo_attn.h"
#include "plan_common.h"

using namespace karpo;

extern "C" int karpo_attn_plan(const KarpoAttnArgs* a, const int32_t* q_cu, const int32_t* k_cu, int32_t n_seq,
                               int32_t* plan, int64_t capacity) {
  if (a == nullptr || plan == nullptr || (n_seq > 0 && (q_cu == nullptr || k_cu == nullptr)))
    return KARPO_ATTN_ERR_NULL;
  if (a->heads < 1 || a->kv_heads < 1 || a->heads % a->kv_heads != 0) return KARPO_ATTN_ERR_HEADS;
  if (!head_dim_supported(a->head_dim)) return KARPO_ATTN_ERR_HEAD_DIM;
  if (a->window_left < -1 || a->window_right < -1) return KARPO_ATTN_ERR_WINDOW;
  if (n_seq < 0) return KARPO_ATTN_ERR_ARG;
  if (capacity < kPlanHeader) return KARPO_ATTN_ERR_CAPACITY;
  for (int32_t i = 0; i < n_seq; ++i)
    if (q_cu[i] < 0 || k_cu[i] < 0 || q_cu[i + 1] < q_cu[i] || k_cu[i + 1] < k_cu[i]) return KARPO_ATTN_ERR_BOUNDS;

  const Geometry g = geometry(a->heads, a->kv_heads, a->head_dim);
  struct Item {
    int32_t cost, seg, tile;
  };
  std::vector<Item> items;
  for (int32_t i = 0; i < n_seq; ++i) {
    const int32_t lq = q_cu[i + 1] - q_cu[i], lk = k_cu[i + 1] - k_cu[i];
    const int64_t nt = tiles_of(lq, g.rows);
    for (int64_t t = 0; t < nt; ++t) {
      int cost = tile_cost(lq, lk, (int)t, g.rows, g.bn, a->window_left, a->window_right);
      if (cost > kCostBuckets - 1) cost = kCostBuckets - 1;  // the device planner's histogram clamps the same way
      items.push_back({cost, i, (int32_t)t});
    }
  }
  if ((int64_t)kPlanHeader + 2 * (int64_t)items.size() > capacity) return KARPO_ATTN_ERR_CAPACITY;
  std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) { return x.cost > y.cost; });
  plan[0] = (int32_t)items.size();
  plan[1] = g.rows;
  plan[2] = g.bn;
  plan[3] = g.ng;
  for (size_t n = 0; n < items.size(); ++n) {
    plan[kPlanHeader + 2 * n] = items[n].seg;
    plan[kPlanHeader + 2 * n + 1] = items[n].tile;
  }
  return KARPO_ATTN_OK;
}
