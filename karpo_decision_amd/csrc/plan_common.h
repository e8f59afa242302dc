// Tile geometry, per-tile cost and the key-split policy shared by the host planner (plan.cpp) and the device
// planner (attn_fwd.hip).
//
// A work item is one query tile of one segment for one group of query heads, over all or one part of the key steps
// the tile visits. A tile holds 32 query vectors per wave of its workgroup; a vector is one (position, head) pair.
// When the GQA group size G divides the tile's vectors, a tile covers vectors / G positions of all G heads of one
// key/value head, so one staged K/V tile serves every head of the group; otherwise it covers `vectors` positions of
// one query head.
//
// Tile shapes, chosen per call from the longest query run (tile_shape):
//   * wide (prefill): several waves share one K/V stream (12 at head_dim 128, 8 at 256 and 512, 4 at 64), 32-key
//     steps (64 at head_dim 64);
//   * long (head_dim 128, runs above 65,536 queries): the wide tile with 64-key steps;
//   * small (head_dim 128 runs up to 4,096 queries, 256 up to 8,192): 4-wave workgroups, three (two) per CU, so a
//     pack of short sequences has three (two) times the work items to balance over the CUs;
//   * narrow (decode-shaped packs, every sequence's queries fit one wave's 32 vectors, e.g. the markers-only layer
//     with one query per sequence): one wave per workgroup (one pair at head_dim 512), several per CU.
// The thresholds are measured (one box, interleaved runs): 32-key wide steps against 64 are -5% at a 32k causal
// sequence and -7% on the 65k multimodal pack but +5% at 131k; small tiles are -17% on the Qwen pack (longest run
// 2,210) and -6% on the branched block plan (4,096), +12% at 131k.
// A tile whose key steps exceed the pack's per-workgroup share is split into parts over its key steps; each part
// writes an fp32 partial (O, running max, sum) and a merge kernel combines them. This bounds the critical path of
// small packs (few long tiles) and gives decode-shaped packs the parallelism of their keys.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define KA_HD __host__ __device__
#else
#define KA_HD
#endif

namespace karpo {

enum TileShape : int { kWide = 0, kNarrow = 1, kSmall = 2, kLong = 3, kDual = 4 };

// Head size 128 prefill in dual-block tiles (kDual): eight waves, two per SIMD, each holding two 32-vector query
// blocks, so every K / V operand read from LDS feeds two MFMAs and each wave has two independent softmaxes to
// interleave with its products (7.08 against 7.44 ms for the twelve-wave tile at the 32k layer, bitwise equal
// outputs). KA_DUAL 0 builds the twelve-wave tile for those runs instead (for A/B measurements).
#ifndef KA_DUAL
#define KA_DUAL 1
#endif

// Waves per workgroup (each holds 32 query vectors of the tile, a pair of waves at head_dim 512), keys per step and
// workgroups resident per CU (the register and LDS budget of the kernel), per head size and tile shape.
KA_HD constexpr int tile_waves(int head_dim, int shape) {
  return shape == kNarrow ? (head_dim == 512 ? 2 : 1)
         : shape == kSmall ? 4
         : shape == kDual ? 8
         : head_dim == 512 ? 8 : head_dim == 128 ? 12 : head_dim == 256 ? 8 : 4;
}
// 32-vector query blocks per wave (per pair of waves at head_dim 512): two in the dual-block tiles, else one.
KA_HD constexpr int tile_blocks(int head_dim, int shape) { return shape == kDual ? 2 : 1; }
// Query vectors per tile: 32 per block of a wave, or of a pair of waves at head_dim 512 (each wave of a pair holds
// half of every vector's elements: half of Q's operands and of O's accumulators).
KA_HD constexpr int tile_vectors(int head_dim, int shape) {
  return 32 * tile_waves(head_dim, shape) * tile_blocks(head_dim, shape) / (head_dim == 512 ? 2 : 1);
}
KA_HD constexpr int tile_keys(int head_dim, int shape) {
  return head_dim == 64 ? 64 : head_dim >= 256 ? 32 : shape == kLong ? 64 : 32;
}
// Workgroups per CU the split policy plans for (its concurrency): the resident ones (the K and V buffers of
// tile_keys x head_dim bf16 per workgroup in 160 KiB of LDS, and the registers), except small tiles, planned one per CU
// although two or three run there: splitting to the per-workgroup share made more split parts than their merge repays
// (Qwen pack 0.110 against 0.097 ms). One-wave tiles at head_dim 64 / 128 are two per CU (a ring of four K/V buffers;
// with the row table two buffers, five resident, planned two per CU all the same: the markers layer's merge halves).
KA_HD constexpr int tiles_per_cu(int head_dim, int shape) {
  return shape == kNarrow ? (head_dim == 512 ? 1 : 2) : head_dim == 64 ? 4 : 1;
}
constexpr int kComputeUnits = 256;   // MI355X
constexpr int kPlanHeader = 12;      // int32 header of a plan (see karpo_attn.h)
constexpr int kItemInts = 4;         // per work item: segment, tile, part | parts << 16, first partial slot or -1
constexpr int kMergeInts = 4;        // per split tile: segment, tile, parts, first partial slot
constexpr int kCostBuckets = 2048;   // device planner's cost histogram (costs clamp to the last bucket)
constexpr int kMinSplitSteps = 8;    // only tiles longer than this split (a merge costs a few steps' time)

struct Geometry {
  int shape;     // TileShape
  int waves;     // waves per workgroup
  int vectors;   // query vectors per tile
  int bn;        // keys per step
  int ng;        // query heads per work item
  int rows;      // query positions per tile
  int n_hg;      // work items per tile (head groups)
  int conc;      // workgroups the GPU runs at once
};

KA_HD inline bool head_dim_supported(int d) { return d == 64 || d == 128 || d == 256 || d == 512; }

KA_HD inline Geometry geometry_of(int heads, int kv_heads, int head_dim, int shape) {
  Geometry g;
  g.shape = shape;
  g.waves = tile_waves(head_dim, shape);
  g.vectors = tile_vectors(head_dim, shape);
  g.bn = tile_keys(head_dim, shape);
  const int group = heads / kv_heads;
  g.ng = (g.vectors % group == 0) ? group : 1;
  g.rows = g.vectors / g.ng;
  g.n_hg = heads / g.ng;
  g.conc = kComputeUnits * tiles_per_cu(head_dim, shape);
  return g;
}

// The tile shape for a pack whose longest query run is max_q: narrow when every sequence's queries fit one narrow
// tile; small for short runs at head_dim 128 and 256; long for very long runs at 128; else wide. Calls that read
// their keys through a row table (`gather`) take the small tiles at head_dim 128 and 256 whatever the run: the wide
// and long tiles are not built with a row table (their copies leave some waves without a copy instruction, a
// configuration whose only run through a row table ended in a GPU memory fault that no host replay of its
// addresses reproduces), and the small tiles are the faster shape on block plans' branched packs anyway.
KA_HD inline int tile_shape(int heads, int kv_heads, int head_dim, int64_t max_q, bool gather = false) {
  if (max_q <= geometry_of(heads, kv_heads, head_dim, kNarrow).rows) return kNarrow;
  if (head_dim == 128 || head_dim == 256) {
    if (gather || (head_dim == 128 && max_q <= 4096) || (head_dim == 256 && max_q <= 8192)) return kSmall;
  }
  if (head_dim == 128 && max_q > 65536) return kLong;
  // dual-block tiles (512 vectors) unless the GQA group divides the twelve-wave tile's 384 vectors but not 512 (3, 6,
  // 12, ...): the twelve-wave tile then stages one K/V stream for the whole group, the dual tile one per head
  const int group = heads / kv_heads;
  if (head_dim == 128 && KA_DUAL && !(384 % group == 0 && 512 % group != 0)) return kDual;
  return kWide;
}
KA_HD inline Geometry geometry(int heads, int kv_heads, int head_dim, int64_t max_q, bool gather = false) {
  return geometry_of(heads, kv_heads, head_dim, tile_shape(heads, kv_heads, head_dim, max_q, gather));
}

// K/V buffers of the forward kernel's ring (steps of copies in flight: buffers - 1). One-wave tiles that stream
// their keys without a row table (decode-shaped packs, HBM bound) keep three steps in flight at head_dim 64 and 128
// (four buffers); every other tile double-buffers.
KA_HD constexpr int kv_buffers(int head_dim, int shape, bool gather) {
  return shape == kNarrow && tile_waves(head_dim, shape) == 1 && !gather && head_dim <= 128 ? 4 : 2;
}

KA_HD inline int64_t ka_min(int64_t a, int64_t b) { return a < b ? a : b; }
KA_HD inline int64_t ka_max(int64_t a, int64_t b) { return a > b ? a : b; }

// Key steps a tile visits: keys [lo, hi) any query of tile t can see under the (left, right) window with the
// bottom-right alignment (query i sits at key i + lk - lq), in steps of bn aligned to the segment's first key; 0 when
// its queries see no key. Spans are not counted (they widen a few tiles' envelopes; the kernel finds the exact one).
KA_HD inline int64_t tile_steps(int lq, int lk, int64_t t, int rows, int bn, int left, int right) {
  const int64_t delta = (int64_t)lk - lq;
  int64_t p0 = t * rows;
  int64_t p1 = ka_min((int64_t)lq, p0 + rows) - 1;
  // queries that see at least one key: i' + right >= 0 and i' - left < lk (i' = p + delta)
  if (right >= 0) p0 = ka_max(p0, -(int64_t)right - delta);
  if (left >= 0) p1 = ka_min(p1, (int64_t)lk + left - 1 - delta);
  if (lk <= 0 || p1 < p0) return 0;
  const int64_t lo = left < 0 ? 0 : ka_max(0, p0 + delta - left);
  const int64_t hi = right < 0 ? (int64_t)lk : ka_min((int64_t)lk, p1 + delta + right + 1);
  if (hi <= lo) return 0;
  return (hi + bn - 1) / bn - lo / bn;
}

KA_HD inline int64_t tiles_of(int64_t lq, int rows) { return lq <= 0 ? 0 : (lq + rows - 1) / rows; }

// Split policy. With `total` = sum over tiles of steps x head groups (the pack's workgroup-steps), a part is at most
// tau = max(kMinSplitSteps, ceil(total / conc)) steps: no workgroup's work exceeds the GPU's average share, so the
// longest-first schedule ends within about two shares. Only tiles longer than tau split, so the parts of split tiles
// number below 2 * total / (tau * n_hg) <= 2 * conc / n_hg: the partial buffer has a size fixed by the geometry.
KA_HD inline int64_t split_tau(int64_t total, int conc) {
  const int64_t tau = (total + conc - 1) / conc;
  return tau < kMinSplitSteps ? kMinSplitSteps : tau;
}
KA_HD inline int split_parts(int64_t steps, int64_t tau) { return steps > tau ? (int)((steps + tau - 1) / tau) : 1; }
// Ordering cost of one part of a tile: its steps, plus one for the store (clamped to the histogram).
KA_HD inline int part_cost(int64_t steps, int parts) {
  const int64_t c = (steps + parts - 1) / parts + 1;
  return (int)ka_min(c, kCostBuckets - 1);
}
// Partial slots (per head group) the parts of split tiles can take, and the split tiles there can be.
KA_HD inline int64_t split_slots(const Geometry& g) { return 2 * (int64_t)g.conc / g.n_hg; }
KA_HD inline int64_t split_tiles(const Geometry& g) { return split_slots(g) / 2; }

// Tiles a forward launch covers at most: every sequence adds at most one partial tile, and none has more than max_q
// rows (rows: the query rows the bounds span, at most total_q).
KA_HD inline int64_t tile_capacity(int64_t total_q, int n_seq, int64_t max_q, const Geometry& g) {
  const int64_t by_rows = (total_q + g.rows - 1) / g.rows + n_seq;
  const int64_t by_max = (int64_t)n_seq * tiles_of(max_q, g.rows);
  return by_rows < by_max ? by_rows : by_max;
}

// Sizes of one forward call's plan and workspace. Items: every unsplit tile once plus the parts of split tiles (at
// most split_slots); split tiles: at most half the slots. (Bound: with `total` the pack's workgroup-steps and
// tau >= total / conc, a tile of s > tau steps splits into ceil(s / tau) < 2 s / tau parts, so the parts of all split
// tiles number below 2 total / (tau n_hg) <= 2 conc / n_hg, an integer bound of split_slots.) The workspace holds
// the device plan, the planner's tile bases (n_seq + 1), its status word, then the fp32 partials.
struct FwdSizes {
  int64_t tiles, items, merges, plan_entries, status_offset, partial_offset, bytes;
};
KA_HD inline FwdSizes fwd_sizes(int64_t total_q, int n_seq, int64_t max_q, int head_dim, const Geometry& g) {
  FwdSizes z;
  z.tiles = tile_capacity(total_q, n_seq, max_q, g);
  z.items = z.tiles + split_slots(g);
  z.merges = ka_min(z.tiles, split_tiles(g));
  z.plan_entries = kPlanHeader + kMergeInts * z.merges + kItemInts * z.items;
  z.status_offset = z.plan_entries + (int64_t)n_seq + 1;  // int offset: after the plan and the tile bases
  const int64_t ints = z.status_offset + 1;
  z.partial_offset = (ints * 4 + 255) / 256 * 256;
  const int64_t partial = split_slots(g) * g.n_hg * (int64_t)g.vectors * (head_dim + 2) * 4;
  z.bytes = z.partial_offset + (partial + 255) / 256 * 256;
  return z;
}

// Backward tiles (attn_bwd.hip). Query tiles never split (conc 1 makes the split length the whole pack); key tiles at
// head sizes 64 and 128 split like the forward's, planned one per CU (the dK / dV kernel's residency at one wave per
// SIMD), their parts' fp32 partials summed by bwd_merge_kernel (at 256 the kernel's one wave per SIMD has no
// registers left for the partials' store path):
//   * dkdv kernel: four waves of 32 keys, 32 query rows per step;
//   * dq kernel: four waves of 32 query vectors, 32 keys per step (eight waves with 64-key steps, which the kernel
//     also takes up to head size 128, measured no faster: the step's fixed costs are not what bounds it).
constexpr int kBwdWaves = 4;
constexpr int kBwdStep = 32;
#ifndef KA_BWD_WQ
#define KA_BWD_WQ 4
#endif
#ifndef KA_BWD_BNQ
#define KA_BWD_BNQ 32
#endif
KA_HD constexpr int bwd_q_waves(int head_dim) { return head_dim <= 128 ? KA_BWD_WQ : 4; }
KA_HD constexpr int bwd_q_step(int head_dim) { return head_dim <= 128 ? KA_BWD_BNQ : 32; }
// At head size 512 two waves share 32 query vectors or 32 keys (each holds half of D): 64 per four-wave tile.
KA_HD constexpr int bwd_tile_vectors(int head_dim, bool key_tiles) {
  return 32 * (key_tiles ? kBwdWaves : bwd_q_waves(head_dim)) / (head_dim == 512 ? 2 : 1);
}
// The dq kernel's query tiles (heads grouped as the forward groups them) and the dkdv kernel's key tiles (one
// key/value head per item; the planner sees keys as queries and query rows as keys).
KA_HD inline Geometry bwd_geometry(int heads, int kv_heads, int head_dim, bool key_tiles) {
  Geometry g;
  g.shape = kWide;
  g.waves = key_tiles ? kBwdWaves : bwd_q_waves(head_dim);
  g.vectors = bwd_tile_vectors(head_dim, key_tiles);
  g.bn = key_tiles ? kBwdStep : bwd_q_step(head_dim);
  const int group = heads / kv_heads;
  g.ng = key_tiles ? 1 : (g.vectors % group == 0 ? group : 1);
  g.rows = g.vectors / g.ng;
  g.n_hg = key_tiles ? kv_heads : heads / g.ng;
  g.conc = key_tiles && head_dim <= 128 ? kComputeUnits : 1;
  return g;
}

// Floats from the backward's partial buffer to part `part` of the split key tile whose parts start at slot `slot`,
// key/value head kvh: per slot and head dK [keys][head_dim] (before the logit scale), then dV [keys][head_dim].
KA_HD inline int64_t bwd_partial_base(int slot, int part, int n_hg, int kvh, int keys, int head_dim) {
  return ((int64_t)(slot + part) * n_hg + kvh) * (int64_t)keys * 2 * head_dim;
}

}  // namespace karpo
