// Host planner: the longest-first work list from host copies of the sequence bounds.
//
// The reference builds every device bound of a pack once on the host, before the first layer is queued
// (block_plan, families/gemma/packed.py:103-151), and reuses them in every layer. This is the same step for the
// kernel's work list: one pass over the sequences, one tile per (sequence, query tile), each visiting only the key
// steps its queries can see (steps outside the window, above the causal diagonal or in another sequence are never
// listed). Tiles longer than the pack's per-workgroup share are split into parts over their key steps (the policy in
// plan_common.h); the items are sorted by their steps, longest first (ties: sequence, tile, part order), so a
// workgroup that starts late takes short work.
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
  if (n_seq < 0 || a->max_q < 0) return KARPO_ATTN_ERR_ARG;
  if (capacity < kPlanHeader) return KARPO_ATTN_ERR_CAPACITY;
  for (int32_t i = 0; i < n_seq; ++i)
    if (q_cu[i] < 0 || k_cu[i] < 0 || q_cu[i + 1] < q_cu[i] || k_cu[i + 1] < k_cu[i]) return KARPO_ATTN_ERR_BOUNDS;
  for (int32_t i = 0; i < n_seq; ++i)  // max_q bounds every query run (it sizes the tiles and the launch)
    if (q_cu[i + 1] - q_cu[i] > a->max_q) return KARPO_ATTN_ERR_BOUNDS;

  const bool gather = a->k_rows != nullptr;  // calls through a row table take their own tile shape
  const Geometry g = geometry(a->heads, a->kv_heads, a->head_dim, a->max_q, gather);
  struct Tile {
    int32_t seg, tile;
    int64_t steps;
  };
  std::vector<Tile> tiles;
  int64_t total = 0;
  for (int32_t i = 0; i < n_seq; ++i) {
    const int32_t lq = q_cu[i + 1] - q_cu[i], lk = k_cu[i + 1] - k_cu[i];
    const int64_t nt = tiles_of(lq, g.rows);
    for (int64_t t = 0; t < nt; ++t) {
      const int64_t steps = tile_steps(lq, lk, t, g.rows, g.bn, a->window_left, a->window_right);
      tiles.push_back({i, (int32_t)t, steps});
      total += steps * g.n_hg;
    }
  }
  const int64_t tau = split_tau(total, g.conc);

  struct Item {
    int32_t cost, seg, tile, part_parts, slot;
  };
  std::vector<Item> items;
  std::vector<int32_t> merges;
  int32_t slots = 0;
  for (const Tile& t : tiles) {
    const int parts = split_parts(t.steps, tau);
    const int cost = part_cost(t.steps, parts);
    const int32_t slot = parts > 1 ? slots : -1;
    if (parts > 1) {
      merges.insert(merges.end(), {t.seg, t.tile, parts, slot});
      slots += parts;
    }
    for (int p = 0; p < parts; ++p) items.push_back({cost, t.seg, t.tile, p | (parts << 16), slot});
  }
  const int64_t n_merges = (int64_t)merges.size() / kMergeInts;
  const int64_t first = kPlanHeader + kMergeInts * n_merges;
  if (first + kItemInts * (int64_t)items.size() > capacity) return KARPO_ATTN_ERR_CAPACITY;
  std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) { return x.cost > y.cost; });
  plan[0] = (int32_t)items.size();
  plan[1] = g.rows;
  plan[2] = g.bn;
  plan[3] = g.ng;
  plan[4] = (int32_t)n_merges;
  plan[5] = g.waves;
  plan[6] = (int32_t)first;
  plan[7] = slots;
  plan[8] = n_seq;
  plan[9] = gather ? 1 : 0;
  plan[10] = g.shape;
  plan[11] = 0;
  std::copy(merges.begin(), merges.end(), plan + kPlanHeader);
  for (size_t n = 0; n < items.size(); ++n) {
    int32_t* e = plan + first + kItemInts * n;
    e[0] = items[n].seg;
    e[1] = items[n].tile;
    e[2] = items[n].part_parts;
    e[3] = items[n].slot;
  }
  return KARPO_ATTN_OK;
}
