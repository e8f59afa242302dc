// Host replay of the forward kernel's memory accesses (attn_fwd.hip: attn_fwd_kernel and merge_kernel) for one call
// and one plan. It walks every workgroup of the launch grid, every wave and lane, and every key step in the order the
// kernel issues them, computing each address with the kernel's own functions (tile_addr.h, plan_common.h), and
// checks it against the allocations: plan entries and bounds read inside their arrays, query rows and output rows
// inside the tensors, row-table reads inside the table, every DMA chunk either wholly inside its buffer resource
// (and that range inside the K / V allocation) or wholly past it without a 32-bit wrap, LDS writes inside the tile,
// partial writes inside the workspace. It also records which (query row, head) outputs the launch writes, so a
// plan that leaves a row of a sequence unwritten, or writes one twice, is reported.
//
// Test infrastructure only (built by tests/test_replay.py with the host compiler); it mirrors the kernel's control
// flow (which steps copy, which fetch table rows) by hand, and shares every address formula with it. At head size 512
// without a row table the library launches attn_fwd_pair_pp_kernel instead: the same plan items, tiles, bounds and
// copy sources, its copies of a step's tiles issued one iteration earlier; karpo_replay_pair_blocks checks the one
// address it forms differently (a block's source as block 0's plus a fixed step).
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "karpo_attn.h"
#include "plan_common.h"
#include "tile_addr.h"

using namespace karpo;

namespace {

struct Report {
  int64_t checks = 0, violations = 0, blocks = 0, copies = 0, fetches = 0, past_chunks = 0;
  char first[512] = {0};
  void fail(const char* what) {
    if (violations++ == 0) snprintf(first, sizeof(first), "%s", what);
  }
};

struct Call {
  const KarpoAttnArgs* a;
  const int32_t* q_cu;
  const int32_t* k_cu;
  const int32_t* k_rows;
  int64_t n_rows;
  const int32_t* spans;
  const int32_t* plan;
  int64_t plan_len;
  int force_shape;  // -1: the call's own tile shape
};

// Elements of a [rows][heads][head_dim] tensor addressed with these strides (the last element's index + 1).
int64_t extent(int64_t rows, int heads, int d, int64_t s_tok, int64_t s_head) {
  if (rows <= 0) return 0;
  return (rows - 1) * s_tok + (int64_t)(heads - 1) * s_head + d;
}

template <int D>
int replay(const Call& c, Report& r, std::vector<uint8_t>& written) {
  const KarpoAttnArgs* a = c.a;
  const bool gather = a->k_rows != nullptr;
  const Geometry g = c.force_shape >= 0 ? geometry_of(a->heads, a->kv_heads, D, c.force_shape)
                                         : geometry(a->heads, a->kv_heads, D, a->max_q, gather);
  const FwdSizes z = fwd_sizes(a->total_q, a->n_seq, a->max_q, D, g);
  const int W = g.waves, BN = g.bn, QB = tile_blocks(D, g.shape);
  const bool pair = D == 512;
  const int NB = kv_buffers(D, g.shape, gather);
  const int TILE = BN * D * 2, BLKS = TILE / 1024, INSTS = (BLKS + W - 1) / W;
  const int V = g.vectors;
  const int group = a->heads / a->kv_heads;
  const bool split_plan = c.plan[4] != 0;
  const int slots = split_plan ? (int)split_slots(g) : 0;
  const int64_t partial_floats = split_slots(g) * g.n_hg * (int64_t)V * (D + 2);
  const int64_t k_elems = extent(a->total_k, a->kv_heads, D, a->k_stride_tok, a->k_stride_head);
  const int64_t v_elems = extent(a->total_k, a->kv_heads, D, a->v_stride_tok, a->v_stride_head);
  char msg[512];
  auto plan_at = [&](int64_t i) -> int32_t {
    ++r.checks;
    if (i < 0 || i >= c.plan_len) {
      snprintf(msg, sizeof(msg), "plan read at %lld of %lld entries", (long long)i, (long long)c.plan_len);
      r.fail(msg);
      return 0;
    }
    return c.plan[i];
  };
  if (plan_at(2) != BN || plan_at(5) != W) {
    r.fail("the plan's tile shape differs from the call's: the kernel would write nothing");
    return 0;
  }
  const int n_items = plan_at(0);
  for (int64_t b = 0; b < z.items * g.n_hg; ++b) {
    const int item = (int)(b / g.n_hg), hg = (int)(b - (int64_t)item * g.n_hg);
    if (item >= n_items) continue;
    ++r.blocks;
    const int64_t e = plan_at(6) + kItemInts * (int64_t)item;
    const int seg = plan_at(e), tile = plan_at(e + 1), pp = plan_at(e + 2), slot = plan_at(e + 3);
    const int part = pp & 0xffff, parts = pp >> 16;
    if (parts > 1 && (slot < 0 || slot + part >= slots)) {
      snprintf(msg, sizeof(msg), "item %d: partial slot %d + %d outside the %d slots (nothing written)", item, slot,
               part, slots);
      r.fail(msg);
      continue;
    }
    ++r.checks;
    if (seg < 0 || seg >= a->n_seq) {
      snprintf(msg, sizeof(msg), "item %d: sequence %d outside the %d bounds", item, seg, a->n_seq);
      r.fail(msg);
      continue;
    }
    const int qa = c.q_cu[seg], lq = c.q_cu[seg + 1] - qa, ka = c.k_cu[seg], lk = c.k_cu[seg + 1] - ka;
    const int kvh = (hg * g.ng) / group;
    // the lanes' keys and the workgroup's envelope
    int klo = INT32_MAX, khi = INT32_MIN;
    for (int w = 0; w < W; ++w)
      for (int b = 0; b < QB; ++b)
      for (int col = 0; col < 32; ++col) {
        const int vec = lane_vector(w, b, col, pair, QB);
        const int off = vec / g.ng, pos = tile * g.rows + off, head = hg * g.ng + (vec - off * g.ng);
        if (pos >= lq) continue;
        const LaneKeys k = lane_keys(pos, qa, lq, lk, a->window_left, a->window_right, c.spans, a->n_spans);
        if (k.lo < k.hi) {
          klo = klo < k.lo ? klo : k.lo;
          khi = khi > k.hi ? khi : k.hi;
        }
        if (k.sl < k.sh) {
          klo = klo < k.sl ? klo : k.sl;
          khi = khi > k.sh ? khi : k.sh;
        }
        ++r.checks;  // the query row the lane loads (both halves of the wave: the same row)
        const int64_t row = (int64_t)qa + pos;
        if (row < 0 || row >= a->total_q || head >= a->heads) {
          snprintf(msg, sizeof(msg), "item %d: query row %lld head %d outside [%lld rows, %d heads]", item,
                   (long long)row, head, (long long)a->total_q, a->heads);
          r.fail(msg);
        }
      }
    int j_first, n_steps;
    part_steps(klo, khi, BN, part, parts, &j_first, &n_steps);
    // the copies and table reads of the kernel's prologue and steps, in issue order
    std::vector<int> k_row(W * INSTS * 64), v_row(W * INSTS * 64);
    auto fetch_rows = [&](int j0) {
      for (int w = 0; w < W; ++w)
        for (int ri = 0; ri < INSTS; ++ri)
          for (int lane = 0; lane < 64; ++lane) {
            int kk, vk, col;
            k_dma_source<D>(w * INSTS + ri, lane, &kk, &col);
            v_dma_source<D>(w * INSTS + ri, lane, &vk, &col);
            const int at = (w * INSTS + ri) * 64 + lane;
            for (int which = 0; which < 2; ++which) {
              const int key = which ? vk : kk;
              int row = -1;
              if (j0 + key < lk) {
                const int64_t idx = (int64_t)ka + j0 + key;
                ++r.checks;
                ++r.fetches;
                if (idx < 0 || idx >= c.n_rows) {
                  snprintf(msg, sizeof(msg), "item %d: row-table read at %lld of %lld", item, (long long)idx,
                           (long long)c.n_rows);
                  r.fail(msg);
                } else {
                  row = c.k_rows[idx];
                }
              }
              (which ? v_row : k_row)[at] = row;
            }
          }
    };
    auto copy = [&](int j0) {
      const int rows = lk - j0 < BN ? lk - j0 : BN;
      for (int which = 0; which < 2; ++which) {
        const int64_t s_tok = which ? a->v_stride_tok : a->k_stride_tok;
        const int64_t s_head = which ? a->v_stride_head : a->k_stride_head;
        const int64_t elems = which ? v_elems : k_elems;
        // the buffer resource: base element and size in bytes
        const int64_t base = (int64_t)kvh * s_head + (gather ? 0 : ((int64_t)ka + j0) * s_tok);
        const uint32_t past = (uint32_t)(((a->total_k - 1) * s_tok + D) * 2);
        const uint32_t bytes = gather ? past : (uint32_t)(rows * s_tok * 2);
        for (int w = 0; w < W; ++w)
          for (int ri = 0; ri < INSTS; ++ri) {
            if (!(BLKS % W == 0 || w * INSTS + ri < BLKS)) continue;
            ++r.copies;
            for (int lane = 0; lane < 64; ++lane) {
              int key, col;
              if (which) v_dma_source<D>(w * INSTS + ri, lane, &key, &col);
              else k_dma_source<D>(w * INSTS + ri, lane, &key, &col);
              uint32_t voff;
              if (gather) {
                const int row = (which ? v_row : k_row)[(w * INSTS + ri) * 64 + lane];
                voff = gather_offset(row, (int)a->total_k, (uint32_t)(s_tok * 2), (uint32_t)col * 2u, past);
              } else {
                voff = (uint32_t)(key * s_tok + col) * 2u;
              }
              r.checks += 2;
              const int lds = (w * INSTS + ri) * 1024 + lane * 16;
              if (lds < 0 || lds + 16 > TILE) {
                snprintf(msg, sizeof(msg), "item %d: LDS write at %d of a %d-byte tile", item, lds, TILE);
                r.fail(msg);
              }
              if (voff < bytes) {  // read: the whole chunk inside the resource and inside the allocation
                const int64_t first = base + voff / 2;
                if ((uint64_t)voff + 16 > bytes || first < 0 || first + 8 > elems) {
                  snprintf(msg, sizeof(msg),
                           "item %d step at key %d: %s chunk at byte %u of a %u-byte resource (elements %lld..%lld "
                           "of %lld)", item, j0, which ? "V" : "K", voff, bytes, (long long)first,
                           (long long)first + 8, (long long)elems);
                  r.fail(msg);
                }
              } else {
                ++r.past_chunks;
                if ((uint64_t)voff + 16 > 0xffffffffull) {  // a dword of the chunk would wrap into range
                  snprintf(msg, sizeof(msg), "item %d: %s offset %u wraps past 2^32", item, which ? "V" : "K", voff);
                  r.fail(msg);
                }
              }
            }
          }
      }
    };
    if (NB == 2) {
      if (n_steps > 0) {
        if (gather) fetch_rows(j_first);
        copy(j_first);
        if (gather && n_steps > 1) fetch_rows(j_first + BN);
      }
    } else {
      for (int i = 0; i < NB - 1; ++i)
        if (i < n_steps) copy(j_first + i * BN);
    }
    for (int s = 0; s < n_steps; ++s) {
      const int j0 = j_first + s * BN;
      if (s + NB - 1 < n_steps) copy(j0 + (NB - 1) * BN);
      if (gather && s + NB < n_steps) fetch_rows(j0 + NB * BN);
    }
    // the store: the tile's rows, or this part's partial
    for (int w = 0; w < W; ++w)
      for (int b = 0; b < QB; ++b)
      for (int lane = 0; lane < 64; ++lane) {
        const int col = lane & 31, half = lane >> 5;
        const int vec = lane_vector(w, b, col, pair, QB);
        const int off = vec / g.ng, pos = tile * g.rows + off, head = hg * g.ng + (vec - off * g.ng);
        const int dh = pair ? (w & 1) : 0;
        if (parts > 1) {
          const int64_t o = partial_base(slot, part, g.n_hg, hg, V, D) + (int64_t)vec * D + dh * (D / 2) + half * 4;
          r.checks += 2;
          const int ob = pair ? D / 64 : D / 32;
          if (o < 0 || o + (ob - 1) * 32 + 3 * 8 + 4 > partial_floats ||
              partial_base(slot, part, g.n_hg, hg, V, D) + (int64_t)V * D + V + vec >= partial_floats) {
            snprintf(msg, sizeof(msg), "item %d: partial write at float %lld of %lld", item, (long long)o,
                     (long long)partial_floats);
            r.fail(msg);
          }
          continue;
        }
        if (pos >= lq || half != 0 || dh != 0) continue;
        const int64_t row = (int64_t)qa + pos;
        if (row >= 0 && row < a->total_q && head < a->heads) ++written[row * a->heads + head];
      }
  }
  // the merge kernel: the parts of each split tile combine into its rows
  const int merges = plan_at(4);
  for (int m = 0; m < merges; ++m) {
    const int64_t e = kPlanHeader + kMergeInts * (int64_t)m;
    const int seg = plan_at(e), tile = plan_at(e + 1), parts = plan_at(e + 2), slot = plan_at(e + 3);
    ++r.checks;
    if (slot < 0 || parts < 2 || slot + parts > slots || seg < 0 || seg >= a->n_seq) {
      snprintf(msg, sizeof(msg), "merge %d: slots %d..%d of %d, sequence %d (rows left unwritten)", m, slot,
               slot + parts, slots, seg);
      r.fail(msg);
      continue;
    }
    const int qa = c.q_cu[seg], lq = c.q_cu[seg + 1] - qa;
    for (int hg = 0; hg < g.n_hg; ++hg)
      for (int vec = 0; vec < V; ++vec) {
        const int off = vec / g.ng, pos = tile * g.rows + off, head = hg * g.ng + (vec - off * g.ng);
        if (pos >= lq) continue;
        const int64_t row = (int64_t)qa + pos;
        if (row >= 0 && row < a->total_q) ++written[row * a->heads + head];
      }
  }
  return 0;
}

}  // namespace

extern "C" {

// Replays one karpo_attn_fwd call (a: its arguments; the pointers in it are not read) with host copies of its bounds,
// row table, spans and plan, under the call's tile shape or `force_shape` (>= 0: a TileShape). Returns the number of
// violations; `counts` receives (checks, blocks, copy instructions, table reads, rows written twice or never, DMA
// chunks read past their resource); `first` the first violation's description.
int64_t karpo_replay_fwd(const KarpoAttnArgs* a, const int32_t* q_cu, const int32_t* k_cu, const int32_t* k_rows,
                         int64_t n_rows, const int32_t* spans, const int32_t* plan, int64_t plan_len, int force_shape,
                         int64_t* counts, char* first, int first_len) {
  Call c = {a, q_cu, k_cu, k_rows, n_rows, spans, plan, plan_len, force_shape};
  Report r;
  std::vector<uint8_t> written((size_t)(a->total_q * a->heads), 0);
  switch (a->head_dim) {
    case 64: replay<64>(c, r, written); break;
    case 128: replay<128>(c, r, written); break;
    case 256: replay<256>(c, r, written); break;
    case 512: replay<512>(c, r, written); break;
    default: r.fail("head_dim"); break;
  }
  // every (row, head) inside a sequence written exactly once, none outside
  int64_t bad_rows = 0;
  std::vector<uint8_t> inside((size_t)a->total_q, 0);
  for (int i = 0; i < a->n_seq; ++i)
    for (int64_t row = q_cu[i]; row < q_cu[i + 1] && row < a->total_q; ++row) inside[row] = 1;
  for (int64_t row = 0; row < a->total_q; ++row)
    for (int h = 0; h < a->heads; ++h)
      if (written[row * a->heads + h] != (inside[row] ? 1 : 0)) {
        if (bad_rows++ == 0) {
          char msg[160];
          snprintf(msg, sizeof(msg), "row %lld head %d written %d times", (long long)row, h,
                   written[row * a->heads + h]);
          r.fail(msg);
        } else {
          ++r.violations;
        }
      }
  counts[0] = r.checks;
  counts[1] = r.blocks;
  counts[2] = r.copies;
  counts[3] = r.fetches;
  counts[4] = bad_rows;
  counts[5] = r.past_chunks;
  if (first_len > 0) {
    strncpy(first, r.first, (size_t)first_len - 1);
    first[first_len - 1] = 0;
  }
  return r.violations;
}

// The head-size-512 pair ping-pong (attn_fwd_pair_pp_kernel) addresses a wave's `insts` copy blocks of a K (V) tile
// from block wave * insts plus k_block (v_block) bytes per block: returns how many (wave, lane, block) sources, for
// these row strides (elements), differ from k_dma_source / v_dma_source of the block itself.
int64_t karpo_replay_pair_blocks(int waves, int insts, int64_t k_stride, int64_t v_stride, int64_t k_block,
                                 int64_t v_block) {
  int64_t bad = 0;
  for (int w = 0; w < waves; ++w)
    for (int lane = 0; lane < 64; ++lane) {
      int k0, c0, v0, d0;
      k_dma_source<512>(w * insts, lane, &k0, &c0);
      v_dma_source<512>(w * insts, lane, &v0, &d0);
      for (int r = 0; r < insts; ++r) {
        int k, c, v, d;
        k_dma_source<512>(w * insts + r, lane, &k, &c);
        v_dma_source<512>(w * insts + r, lane, &v, &d);
        bad += (k * k_stride + c) * 2 != (k0 * k_stride + c0) * 2 + k_block * r;
        bad += (v * v_stride + d) * 2 != (v0 * v_stride + d0) * 2 + v_block * r;
      }
    }
  return bad;
}
}
