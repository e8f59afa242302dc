// The C ABI: argument checks, workspace sizing and the two launches (device planner, attention kernel).
//
// Error behaviour follows the reference's host wrapper (families/gemma/triton_attention.py:98-102): unsupported
// shapes and layouts are refused before anything is launched; here as status codes, which the Python layer turns
// into ValueError / RuntimeError.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "internal.h"
#include "karpo_attn.h"
#include "plan_common.h"

using namespace karpo;

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_shape(const KarpoAttnArgs* a) {
  if (a == nullptr) return KARPO_ATTN_ERR_NULL;
  if (a->heads < 1 || a->kv_heads < 1 || a->heads % a->kv_heads != 0) return KARPO_ATTN_ERR_HEADS;
  if (!head_dim_supported(a->head_dim)) return KARPO_ATTN_ERR_HEAD_DIM;
  if (a->window_left < -1 || a->window_right < -1) return KARPO_ATTN_ERR_WINDOW;
  if (a->n_seq < 0 || a->total_q < 0 || a->max_q < 0 || a->key_bound < 0) return KARPO_ATTN_ERR_ARG;
  return KARPO_ATTN_OK;
}

int64_t tile_capacity(const KarpoAttnArgs* a, const Geometry& g) {
  return karpo::tile_capacity(a->total_q, a->n_seq, a->max_q, g);
}

// The forward's tile geometry for these arguments (a row table takes the four-wave tiles at head sizes 128 / 256).
Geometry fwd_geometry(const KarpoAttnArgs* a) {
  return geometry(a->heads, a->kv_heads, a->head_dim, a->max_q, a->k_rows != nullptr);
}

FwdSizes sizes_of(const KarpoAttnArgs* a, const Geometry& g) {
  return fwd_sizes(a->total_q, a->n_seq, a->max_q, a->head_dim, g);
}

// A host plan's header against the call: the same tile geometry, row-table use and sequence count, and counts
// within the launch's capacities (the items, split tiles and partial slots the grid, merge launch and workspace
// cover), with the items right after the split tiles. Anything else would leave rows unwritten.
bool plan_matches(const int32_t* h, const KarpoAttnArgs* a, const Geometry& g, const FwdSizes& z) {
  return h[1] == g.rows && h[2] == g.bn && h[3] == g.ng && h[5] == g.waves && h[8] == a->n_seq &&
         h[9] == (a->k_rows != nullptr ? 1 : 0) && h[10] == g.shape && h[0] >= 0 && h[0] <= z.items && h[4] >= 0 &&
         h[4] <= z.merges && h[6] == kPlanHeader + kMergeInts * h[4] && h[7] >= 0 && h[7] <= split_slots(g) &&
         (h[4] == 0) == (h[7] == 0);
}

int check_stride(int64_t s) { return s >= 0 && s % 8 == 0; }

// The running maximum m (log2 units) is raised only when a step's maximum exceeds it by more than this, so O is
// rescaled on few steps and P = 2^(x - m) stays below 2^8. The key that sets a row's maximum then carries a P above 1,
// rounded to bf16 like every other P: harmless where the softmax is flat, but where one key dominates its weight's
// rounding moves the output by up to ~2^-9 of its spread. A logit scale of order one (Gemma's unit scale on normed
// queries and keys: logits of standard deviation ~sqrt(D)) is that regime; there the maximum is kept exact (P of
// the dominant key exactly 1), at the cost of a rescale on every step whose maximum grows.
float rescale_threshold(float scale) { return fabsf(scale) >= 0.5f ? 0.f : 8.f; }

bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Bytes from the first to one past the last bf16 element of a [rows][heads][head_dim] tensor with these strides.
uintptr_t extent_bytes(int64_t rows, int32_t heads, int32_t head_dim, int64_t s_tok, int64_t s_head) {
  if (rows <= 0) return 0;
  return (uintptr_t)(((rows - 1) * s_tok + (int64_t)(heads - 1) * s_head + head_dim) * 2);
}

// Whether two byte ranges [a, a + na) and [b, b + nb) share a byte.
bool overlaps(const void* a, uintptr_t na, const void* b, uintptr_t nb) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return na > 0 && nb > 0 && x < y + nb && y < x + na;
}

// The fused prologue's norm, weight and rotation table (shared by karpo_attn_fwd and karpo_attn_norm_rope).
int check_norm_rope(int norm, const void* weight, const void* cos, const void* sin, int64_t stride, int rope_dim,
                    int head_dim) {
  if (norm < KARPO_NORM_NONE || norm > KARPO_NORM_PLAIN) return KARPO_ATTN_ERR_PROLOGUE;
  if ((norm == KARPO_NORM_WEIGHT || norm == KARPO_NORM_ONE_PLUS) && (weight == nullptr || !aligned16(weight)))
    return KARPO_ATTN_ERR_PROLOGUE;
  if ((cos == nullptr) != (sin == nullptr)) return KARPO_ATTN_ERR_PROLOGUE;
  if (cos != nullptr && (rope_dim <= 0 || rope_dim % 32 != 0 || rope_dim > head_dim || stride < rope_dim ||
                         stride % 8 != 0 || !aligned16(cos) || !aligned16(sin)))
    return KARPO_ATTN_ERR_PROLOGUE;
  return KARPO_ATTN_OK;
}

}  // namespace

extern "C" int karpo_attn_version(void) { return 4; }

extern "C" const char* karpo_attn_strerror(int status) {
  switch (status) {
    case KARPO_ATTN_OK: return "ok";
    case KARPO_ATTN_ERR_NULL: return "a required pointer is NULL";
    case KARPO_ATTN_ERR_HEAD_DIM: return "head_dim must be 64, 128, 256 or 512";
    case KARPO_ATTN_ERR_HEADS: return "heads must be a positive multiple of kv_heads";
    case KARPO_ATTN_ERR_LAYOUT:
      return "tensors need a contiguous head dimension, strides that are multiples of 8 elements and 16-byte aligned "
             "bases";
    case KARPO_ATTN_ERR_WORKSPACE: return "workspace missing or smaller than karpo_attn_workspace_bytes";
    case KARPO_ATTN_ERR_WINDOW: return "window sides must be -1 (unbounded) or non-negative";
    case KARPO_ATTN_ERR_SPANS: return "n_spans must be non-negative, with a spans pointer when positive";
    case KARPO_ATTN_ERR_LAUNCH: return "the HIP runtime refused a kernel launch";
    case KARPO_ATTN_ERR_ARG: return "sizes and the sequence count must be non-negative";
    case KARPO_ATTN_ERR_CAPACITY: return "the plan buffer is smaller than the plan";
    case KARPO_ATTN_ERR_BOUNDS:
      return "sequence bounds must be non-negative and non-decreasing, within the rows they index and max_q";
    case KARPO_ATTN_ERR_PROLOGUE:
      return "unsupported fused prologue / gate: norm mode 0-3 with a 16-byte aligned weight for modes 1-2, both rope "
             "tables 16-byte aligned with a row stride that is a multiple of 8, rope_dim a multiple of 32 up to "
             "head_dim, gate strides multiples of 4, q_out only with a prologue and not overlapping q";
    case KARPO_ATTN_ERR_SCRATCH:
      return "the call needs more scratch than karpo_attn_fwd_noalloc's 144 MiB (use karpo_attn_fwd with a workspace)";
    case KARPO_ATTN_ERR_PLAN:
      return "the plan was made for another call (tile geometry, row-table use, sequence count or sizes differ), or "
             "its host header copy is missing";
    default: return "unknown karpo_attn status";
  }
}

extern "C" int karpo_attn_tile_shape(int32_t heads, int32_t kv_heads, int32_t head_dim, int32_t max_q,
                                     int32_t gather, int32_t* rows_per_tile, int32_t* keys_per_step,
                                     int32_t* heads_per_item, int32_t* shape) {
  if (heads < 1 || kv_heads < 1 || heads % kv_heads != 0) return KARPO_ATTN_ERR_HEADS;
  if (!head_dim_supported(head_dim)) return KARPO_ATTN_ERR_HEAD_DIM;
  if (max_q < 0) return KARPO_ATTN_ERR_ARG;
  const Geometry g = geometry(heads, kv_heads, head_dim, max_q, gather != 0);
  if (rows_per_tile) *rows_per_tile = g.rows;
  if (keys_per_step) *keys_per_step = g.bn;
  if (heads_per_item) *heads_per_item = g.ng;
  if (shape) *shape = g.shape;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_plan_capacity(const KarpoAttnArgs* a, int64_t* entries) {
  const int st = check_shape(a);
  if (st != KARPO_ATTN_OK) return st;
  if (entries == nullptr) return KARPO_ATTN_ERR_NULL;
  *entries = sizes_of(a, fwd_geometry(a)).plan_entries;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_workspace_bytes(const KarpoAttnArgs* a, size_t* bytes) {
  const int st = check_shape(a);
  if (st != KARPO_ATTN_OK) return st;
  if (bytes == nullptr) return KARPO_ATTN_ERR_NULL;
  *bytes = (size_t)sizes_of(a, fwd_geometry(a)).bytes;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_fwd(const KarpoAttnArgs* a, void* stream) {
  int st = check_shape(a);
  if (st != KARPO_ATTN_OK) return st;
  if (a->n_spans < 0 || (a->n_spans > 0 && a->spans == nullptr)) return KARPO_ATTN_ERR_SPANS;
  if (a->total_q == 0 || a->n_seq == 0) return KARPO_ATTN_OK;  // no query rows: nothing to write
  if (!a->q || !a->k || !a->v || !a->o || !a->q_cu || !a->k_cu) return KARPO_ATTN_ERR_NULL;
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return KARPO_ATTN_ERR_LAYOUT;
  if (!check_stride(a->q_stride_tok) || !check_stride(a->q_stride_head) || !check_stride(a->k_stride_tok) ||
      !check_stride(a->k_stride_head) || !check_stride(a->v_stride_tok) || !check_stride(a->v_stride_head) ||
      !check_stride(a->o_stride_tok) || !check_stride(a->o_stride_head))
    return KARPO_ATTN_ERR_LAYOUT;

  st = check_norm_rope(a->q_norm, a->q_norm_weight, a->rope_cos, a->rope_sin, a->rope_stride, a->rope_dim,
                       a->head_dim);
  if (st != KARPO_ATTN_OK) return st;
  if (a->gate != nullptr && (!aligned8(a->gate) || a->gate_stride_tok < 0 || a->gate_stride_head < 0 ||
                             a->gate_stride_tok % 4 != 0 || a->gate_stride_head % 4 != 0))
    return KARPO_ATTN_ERR_PROLOGUE;
  if (a->lse != nullptr && (a->gate != nullptr || (reinterpret_cast<uintptr_t>(a->lse) & 3u) != 0))
    return KARPO_ATTN_ERR_ARG;
  if (a->q_out != nullptr && ((a->q_norm == KARPO_NORM_NONE && a->rope_cos == nullptr) || !aligned16(a->q_out) ||
                              !check_stride(a->q_out_stride_tok) || !check_stride(a->q_out_stride_head)))
    return KARPO_ATTN_ERR_PROLOGUE;
  // q_out must not share a byte with q: the parts of a split tile run in other workgroups and read q at their start,
  // after part 0 may have written q_out (a query normalised and rotated twice)
  if (a->q_out != nullptr &&
      overlaps(a->q, extent_bytes(a->total_q, a->heads, a->head_dim, a->q_stride_tok, a->q_stride_head), a->q_out,
               extent_bytes(a->total_q, a->heads, a->head_dim, a->q_out_stride_tok, a->q_out_stride_head)))
    return KARPO_ATTN_ERR_PROLOGUE;

  const Geometry g = fwd_geometry(a);
  // a step's key rows are addressed with 32-bit byte offsets
  if ((a->k_stride_tok + a->head_dim) * g.bn * 2 >= (int64_t)INT32_MAX ||
      (a->v_stride_tok + a->head_dim) * g.bn * 2 >= (int64_t)INT32_MAX)
    return KARPO_ATTN_ERR_LAYOUT;
  if (a->k_rows != nullptr) {  // gathered rows are addressed with 32-bit byte offsets from each head's first element
    if (a->total_k < 1 || a->total_k > INT32_MAX) return KARPO_ATTN_ERR_ARG;
    const int64_t kspan = (a->total_k - 1) * a->k_stride_tok + a->head_dim;
    const int64_t vspan = (a->total_k - 1) * a->v_stride_tok + a->head_dim;
    if (kspan * 2 >= (int64_t)UINT32_MAX - 16 || vspan * 2 >= (int64_t)UINT32_MAX - 16) return KARPO_ATTN_ERR_LAYOUT;
  }
  const FwdSizes z = sizes_of(a, g);
  if (z.plan_entries > (int64_t)INT32_MAX / 2 || z.items * g.n_hg > (int64_t)INT32_MAX) return KARPO_ATTN_ERR_ARG;
  if (a->plan != nullptr && (a->plan_header == nullptr || !plan_matches(a->plan_header, a, g, z)))
    return KARPO_ATTN_ERR_PLAN;
  // a host plan that splits no tile needs neither the planner's space nor partials
  const bool merge = split_slots(g) >= 2 && !(a->plan != nullptr && a->plan_header[4] == 0);
  if ((a->plan == nullptr || merge) &&
      (a->workspace == nullptr || a->workspace_bytes < (size_t)z.bytes || !aligned16(a->workspace)))
    return KARPO_ATTN_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(a->workspace);

  const int32_t* plan = a->plan;
  if (plan == nullptr) {
    int32_t* dplan = reinterpret_cast<int32_t*>(ws);
    const PlanJob job = {a->q_cu,        a->k_cu,       g,          a->window_left, a->window_right,
                         dplan,          (int)z.tiles,  (int)z.merges, (int)z.items, dplan + z.plan_entries,
                         dplan + z.status_offset, a->total_q, a->max_q, a->k_rows != nullptr, a->key_bound};
    if (launch_plan(&job, 1, a->n_seq, s) != hipSuccess) return KARPO_ATTN_ERR_LAUNCH;
    plan = dplan;
  }

  Params p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<uint16_t*>(a->o);
  p.sq_t = a->q_stride_tok;
  p.sq_h = a->q_stride_head;
  p.sk_t = a->k_stride_tok;
  p.sk_h = a->k_stride_head;
  p.sv_t = a->v_stride_tok;
  p.sv_h = a->v_stride_head;
  p.so_t = a->o_stride_tok;
  p.so_h = a->o_stride_head;
  p.q_cu = a->q_cu;
  p.k_cu = a->k_cu;
  p.spans = a->spans;
  p.n_spans = a->n_spans;
  p.plan = plan;
  p.k_rows = a->k_rows;
  if (a->k_rows != nullptr) {
    p.total_k = (int32_t)a->total_k;
    p.k_bytes = (uint32_t)(((a->total_k - 1) * a->k_stride_tok + a->head_dim) * 2);
    p.v_bytes = (uint32_t)(((a->total_k - 1) * a->v_stride_tok + a->head_dim) * 2);
  }
  p.partial = ws != nullptr ? reinterpret_cast<float*>(ws + z.partial_offset) : nullptr;
  p.slots = merge ? (int32_t)split_slots(g) : 0;  // 0: a split item (none in such a plan) would write nothing
  p.group = a->heads / a->kv_heads;
  p.ng = g.ng;
  p.n_hg = g.n_hg;
  p.left = a->window_left;
  p.right = a->window_right;
  // exp2-domain logit factor; a zero scale keeps a tiny positive factor so masked (-inf) logits stay -inf
  float c = fabsf(a->scale) * 1.4426950408889634f;
  p.c = c > 1e-30f ? c : 1e-30f;
  p.qsign = a->scale < 0.f ? 0x80008000u : 0u;
  p.tau = rescale_threshold(a->scale);
  p.q_norm = a->q_norm;
  p.q_eps = a->q_norm_eps;
  // without a weight the kernel still reads (and multiplies by zero) head_dim elements: q's first row stands in
  p.q_norm_w = a->q_norm_weight != nullptr ? static_cast<const uint16_t*>(a->q_norm_weight) : p.q;
  p.rope_cos = static_cast<const uint16_t*>(a->rope_cos);
  p.rope_sin = static_cast<const uint16_t*>(a->rope_sin);
  p.rope_stride = a->rope_stride;
  p.rope_dim = a->rope_dim;
  p.gate = static_cast<const uint16_t*>(a->gate);
  p.sg_t = a->gate_stride_tok;
  p.sg_h = a->gate_stride_head;
  p.lse = a->lse;
  p.lse_stride = a->total_q;
  p.q_out = static_cast<uint16_t*>(a->q_out);
  p.sqo_t = a->q_out_stride_tok;
  p.sqo_h = a->q_out_stride_head;
  if (launch_forward(p, a->head_dim, g, z.items, merge ? z.merges : 0, s) != hipSuccess)
    return KARPO_ATTN_ERR_LAUNCH;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_device_status(const KarpoAttnArgs* a, void* stream, int32_t* status) {
  const int st = check_shape(a);
  if (st != KARPO_ATTN_OK) return st;
  if (status == nullptr || a->workspace == nullptr) return KARPO_ATTN_ERR_NULL;
  const FwdSizes z = sizes_of(a, fwd_geometry(a));
  if (a->workspace_bytes < (size_t)z.bytes) return KARPO_ATTN_ERR_WORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t* word = static_cast<const int32_t*>(a->workspace) + z.status_offset;
  if (hipMemcpyAsync(status, word, sizeof(int32_t), hipMemcpyDeviceToHost, s) != hipSuccess ||
      hipStreamSynchronize(s) != hipSuccess)
    return KARPO_ATTN_ERR_LAUNCH;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_norm_rope(const KarpoNormRopeArgs* a, void* stream) {
  if (a == nullptr) return KARPO_ATTN_ERR_NULL;
  if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256 && a->head_dim != 512)
    return KARPO_ATTN_ERR_HEAD_DIM;
  if (a->heads < 1 || a->rows < 0) return KARPO_ATTN_ERR_ARG;
  const int st = check_norm_rope(a->norm, a->weight, a->rope_cos, a->rope_sin, a->rope_stride, a->rope_dim,
                                 a->head_dim);
  if (st != KARPO_ATTN_OK) return st;
  if (a->rows == 0) return KARPO_ATTN_OK;
  if (a->x == nullptr || a->y == nullptr) return KARPO_ATTN_ERR_NULL;
  if (!aligned16(a->x) || !aligned16(a->y) || !check_stride(a->x_stride_tok) || !check_stride(a->x_stride_head) ||
      !check_stride(a->y_stride_tok) || !check_stride(a->y_stride_head))
    return KARPO_ATTN_ERR_LAYOUT;
  NormRopeParams p;
  memset(&p, 0, sizeof(p));
  p.x = static_cast<const uint16_t*>(a->x);
  p.y = static_cast<uint16_t*>(a->y);
  p.w = static_cast<const uint16_t*>(a->weight);
  p.cos = static_cast<const uint16_t*>(a->rope_cos);
  p.sin = static_cast<const uint16_t*>(a->rope_sin);
  p.sx_t = a->x_stride_tok;
  p.sx_h = a->x_stride_head;
  p.sy_t = a->y_stride_tok;
  p.sy_h = a->y_stride_head;
  p.rope_stride = a->rope_stride;
  p.vectors = a->rows * a->heads;
  p.heads = a->heads;
  p.norm = a->norm;
  p.rope_dim = a->rope_dim;
  p.eps = a->eps;
  if (launch_norm_rope(p, a->head_dim, static_cast<hipStream_t>(stream)) != hipSuccess) return KARPO_ATTN_ERR_LAUNCH;
  return KARPO_ATTN_OK;
}

namespace {

// The backward's workspace: per-row stats, then the query-tile and key-tile plans (the key tiles' with their split
// tiles), then the planners' tile bases, then the split key tiles' fp32 partials.
struct BwdSizes {
  int64_t tiles_q, tiles_k, items_k, merges_k, stats_bytes, plan_q, plan_k, tile_bases, partial_offset, bytes;
  // plan_q / plan_k / tile_bases: int offsets from the stats end
};

BwdSizes bwd_sizes_of(const KarpoAttnBwdArgs* b) {
  const KarpoAttnArgs* a = &b->fwd;
  const Geometry gq = bwd_geometry(a->heads, a->kv_heads, a->head_dim, false);
  const Geometry gk = bwd_geometry(a->heads, a->kv_heads, a->head_dim, true);
  BwdSizes z;
  z.tiles_q = tile_capacity(a, gq);
  const int keys = bwd_tile_vectors(a->head_dim, true);
  z.tiles_k = (a->total_k + keys - 1) / keys + a->n_seq;
  z.items_k = z.tiles_k + split_slots(gk);
  z.merges_k = ka_min(z.tiles_k, split_tiles(gk));
  z.stats_bytes = ((int64_t)a->heads * 2 * a->total_q * 4 + 255) / 256 * 256;
  z.plan_q = 0;
  z.plan_k = kPlanHeader + kItemInts * z.tiles_q;
  z.tile_bases = z.plan_k + kPlanHeader + kMergeInts * z.merges_k + kItemInts * z.items_k;
  const int64_t ints = z.tile_bases + 2 * ((int64_t)a->n_seq + 1);  // 2 tile bases
  z.partial_offset = z.stats_bytes + (ints * 4 + 255) / 256 * 256;
  const int64_t partial = split_slots(gk) * gk.n_hg * (int64_t)keys * 2 * a->head_dim * 4;
  z.bytes = z.partial_offset + (partial + 255) / 256 * 256;
  return z;
}

int check_bwd(const KarpoAttnBwdArgs* b) {
  if (b == nullptr) return KARPO_ATTN_ERR_NULL;
  const KarpoAttnArgs* a = &b->fwd;
  const int st = check_shape(a);
  if (st != KARPO_ATTN_OK) return st;
  if (a->total_k < 0) return KARPO_ATTN_ERR_ARG;
  return KARPO_ATTN_OK;
}

}  // namespace

extern "C" int karpo_attn_bwd_workspace_bytes(const KarpoAttnBwdArgs* b, size_t* bytes) {
  const int st = check_bwd(b);
  if (st != KARPO_ATTN_OK) return st;
  if (bytes == nullptr) return KARPO_ATTN_ERR_NULL;
  *bytes = (size_t)bwd_sizes_of(b).bytes;
  return KARPO_ATTN_OK;
}

extern "C" int karpo_attn_bwd(const KarpoAttnBwdArgs* b, void* stream) {
  int st = check_bwd(b);
  if (st != KARPO_ATTN_OK) return st;
  const KarpoAttnArgs* a = &b->fwd;
  if (a->n_spans < 0 || (a->n_spans > 0 && a->spans == nullptr)) return KARPO_ATTN_ERR_SPANS;
  if (a->plan != nullptr || a->k_rows != nullptr || a->q_norm != KARPO_NORM_NONE || a->rope_cos != nullptr ||
      a->gate != nullptr)
    return KARPO_ATTN_ERR_ARG;
  if (a->total_q == 0 || a->n_seq == 0) return KARPO_ATTN_OK;
  if (!a->q || !a->k || !a->v || !a->o || !a->q_cu || !a->k_cu || !b->d_o || !b->lse || !b->d_q || !b->d_k ||
      !b->d_v)
    return KARPO_ATTN_ERR_NULL;
  if (a->total_k < 1) return KARPO_ATTN_ERR_ARG;
  if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o) || !aligned16(b->d_o) ||
      !aligned16(b->d_q) || !aligned16(b->d_k) || !aligned16(b->d_v) ||
      (reinterpret_cast<uintptr_t>(b->lse) & 3u) != 0)
    return KARPO_ATTN_ERR_LAYOUT;
  const int64_t strides[] = {a->q_stride_tok,    a->q_stride_head,    a->k_stride_tok,    a->k_stride_head,
                             a->v_stride_tok,    a->v_stride_head,    a->o_stride_tok,    a->o_stride_head,
                             b->d_o_stride_tok,  b->d_o_stride_head,  b->d_q_stride_tok,  b->d_q_stride_head,
                             b->d_k_stride_tok,  b->d_k_stride_head,  b->d_v_stride_tok,  b->d_v_stride_head};
  for (int64_t s : strides)
    if (!check_stride(s)) return KARPO_ATTN_ERR_LAYOUT;
  // a step's rows (32 keys, or 32 query rows) and a key tile's (the 128 keys the dK / dV kernel stages) are
  // addressed with 32-bit byte offsets
  const int64_t d = a->head_dim;
  const int64_t key_rows = 32 * kBwdWaves > bwd_q_step(a->head_dim) ? 32 * kBwdWaves : bwd_q_step(a->head_dim);
  if ((a->k_stride_tok + d) * key_rows * 2 >= (int64_t)INT32_MAX ||
      (a->v_stride_tok + d) * key_rows * 2 >= (int64_t)INT32_MAX ||
      (a->q_stride_tok + d) * kBwdStep * 2 >= (int64_t)INT32_MAX ||
      (b->d_o_stride_tok + d) * kBwdStep * 2 >= (int64_t)INT32_MAX || (a->total_q + kBwdStep) * 4 >= INT32_MAX)
    return KARPO_ATTN_ERR_LAYOUT;
  const BwdSizes z = bwd_sizes_of(b);
  const Geometry gq = bwd_geometry(a->heads, a->kv_heads, a->head_dim, false);
  const Geometry gk = bwd_geometry(a->heads, a->kv_heads, a->head_dim, true);
  if (z.tiles_q * gq.n_hg > (int64_t)INT32_MAX || z.items_k * gk.n_hg > (int64_t)INT32_MAX ||
      z.tile_bases > (int64_t)INT32_MAX)
    return KARPO_ATTN_ERR_ARG;
  if (a->workspace == nullptr || a->workspace_bytes < (size_t)z.bytes || !aligned16(a->workspace))
    return KARPO_ATTN_ERR_WORKSPACE;

  char* ws = static_cast<char*>(a->workspace);
  int32_t* ints = reinterpret_cast<int32_t*>(ws + z.stats_bytes);
  BwdParams p;
  memset(&p, 0, sizeof(p));
  p.q = static_cast<const uint16_t*>(a->q);
  p.k = static_cast<const uint16_t*>(a->k);
  p.v = static_cast<const uint16_t*>(a->v);
  p.o = static_cast<const uint16_t*>(a->o);
  p.dout = static_cast<const uint16_t*>(b->d_o);
  p.lse = b->lse;
  p.dq = static_cast<uint16_t*>(b->d_q);
  p.dk = static_cast<uint16_t*>(b->d_k);
  p.dv = static_cast<uint16_t*>(b->d_v);
  p.stats = reinterpret_cast<float*>(ws);
  p.sq_t = a->q_stride_tok;
  p.sq_h = a->q_stride_head;
  p.sk_t = a->k_stride_tok;
  p.sk_h = a->k_stride_head;
  p.sv_t = a->v_stride_tok;
  p.sv_h = a->v_stride_head;
  p.so_t = a->o_stride_tok;
  p.so_h = a->o_stride_head;
  p.sdo_t = b->d_o_stride_tok;
  p.sdo_h = b->d_o_stride_head;
  p.sdq_t = b->d_q_stride_tok;
  p.sdq_h = b->d_q_stride_head;
  p.sdk_t = b->d_k_stride_tok;
  p.sdk_h = b->d_k_stride_head;
  p.sdv_t = b->d_v_stride_tok;
  p.sdv_h = b->d_v_stride_head;
  p.q_cu = a->q_cu;
  p.k_cu = a->k_cu;
  p.spans = a->spans;
  p.total_q = a->total_q;
  p.n_spans = a->n_spans;
  p.heads = a->heads;
  p.group = a->heads / a->kv_heads;
  p.left = a->window_left;
  p.right = a->window_right;
  p.c = a->scale * 1.4426950408889634f;
  p.scale = a->scale;
  p.partial = reinterpret_cast<float*>(ws + z.partial_offset);
  p.slots = (int32_t)split_slots(gk);
  int32_t* const tile_base = ints + z.tile_bases;
  if (launch_bwd(p, a->head_dim, gq, gk, ints + z.plan_q, ints + z.plan_k, z.tiles_q, z.items_k, (int)z.tiles_q, 0,
                 (int)z.tiles_k, (int)z.merges_k, tile_base, tile_base + a->n_seq + 1, a->n_seq,
                 static_cast<hipStream_t>(stream)) != hipSuccess)
    return KARPO_ATTN_ERR_LAUNCH;
  return KARPO_ATTN_OK;
}
