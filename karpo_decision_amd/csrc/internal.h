// Declarations shared by the C ABI (capi.cpp) and the kernels (attn_fwd.hip).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "plan_common.h"

namespace karpo {

// Kernel arguments: strides in elements, bounds and plan in device memory.
struct Params {
  const uint16_t* __restrict__ q;
  const uint16_t* __restrict__ k;
  const uint16_t* __restrict__ v;
  uint16_t* __restrict__ o;
  int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, so_t, so_h;
  const int32_t* __restrict__ q_cu;
  const int32_t* __restrict__ k_cu;
  const int32_t* __restrict__ spans;
  const int32_t* __restrict__ plan;
  const int32_t* __restrict__ k_rows;  // gathered key rows, or null
  uint32_t k_bytes, v_bytes;           // with k_rows: bytes from a head's first element to past the last row
  int32_t total_k;                     // with k_rows: rows of k and v
  float* __restrict__ partial;  // per split part and head group: O [vectors][D], then m [vectors], l [vectors]
  int32_t slots;                // partial slots per head group the buffer holds
  int32_t n_spans;
  int32_t group;    // heads / kv_heads
  int32_t ng;       // query heads per work item
  int32_t n_hg;     // work items per tile
  int32_t left, right;
  float c;          // |scale| * log2(e)
  float tau;        // lazy-rescale threshold in log2 units (0: the running maximum is always exact)
  uint32_t qsign;   // 0x80008000 to negate Q (negative scale), else 0
  // fused query prologue (norm, rotation) and output gate; see KarpoAttnArgs
  const uint16_t* __restrict__ q_norm_w;
  const uint16_t* __restrict__ rope_cos;
  const uint16_t* __restrict__ rope_sin;
  const uint16_t* __restrict__ gate;
  int64_t rope_stride, sg_t, sg_h;
  int32_t q_norm;
  float q_eps;
  int32_t rope_dim;
  float* __restrict__ lse;  // [heads][lse_stride] natural-log sums, or null
  int64_t lse_stride;       // total_q
  uint16_t* __restrict__ q_out;  // the query after the fused prologue, or null
  int64_t sqo_t, sqo_h;
};

// The backward kernels' arguments (karpo_attn_bwd): the forward's tensors and bounds, the output gradient and the
// gradients to write; stats holds (log2-domain LSE, -rowsum(dO * O)) per (head, query row).
struct BwdParams {
  const uint16_t* __restrict__ q;
  const uint16_t* __restrict__ k;
  const uint16_t* __restrict__ v;
  const uint16_t* __restrict__ o;
  const uint16_t* __restrict__ dout;
  const float* __restrict__ lse;
  uint16_t* __restrict__ dq;
  uint16_t* __restrict__ dk;
  uint16_t* __restrict__ dv;
  float* __restrict__ stats;  // [heads][2][total_q]: each row's log2-domain LSE, then -rowsum(dout * o)
  int64_t sq_t, sq_h, sk_t, sk_h, sv_t, sv_h, so_t, so_h, sdo_t, sdo_h, sdq_t, sdq_h, sdk_t, sdk_h, sdv_t, sdv_h;
  const int32_t* __restrict__ q_cu;
  const int32_t* __restrict__ k_cu;
  const int32_t* __restrict__ spans;
  const int32_t* __restrict__ plan;  // dq kernel: query tiles; dkdv kernel: key tiles
  int64_t total_q;
  int32_t n_spans, heads, group, ng, n_hg;
  int32_t left, right;
  float c;      // scale * log2(e) (signed)
  float scale;  // the logit scale (signed): dq and dk carry it
  float* __restrict__ partial;  // split key tiles' fp32 dK / dV per part (bwd_partial_base)
  int32_t slots;                // partial slots per key/value head the buffer holds
};
// Head size 512: the dQ and dK / dV kernels of wave pairs (attn_bwd_pair.hip), after the statistics pass.
hipError_t launch_bwd_pair(const BwdParams& p, const Geometry& gq, const Geometry& gk, int32_t* plan_q,
                           int32_t* plan_k, int64_t items_q, int64_t items_k, hipStream_t stream);
// items_q / items_k: the work lists' item capacities (the grids), tiles_q / tiles_k their tile capacities, merges_k
// the key tiles' split capacity.
hipError_t launch_bwd(const BwdParams& p, int head_dim, const Geometry& gq, const Geometry& gk, int32_t* plan_q,
                      int32_t* plan_k, int64_t items_q, int64_t items_k, int tiles_q, int merges_q, int tiles_k,
                      int merges_k, int32_t* tile_base_q, int32_t* tile_base_k, int n_seq, hipStream_t stream);

// karpo_attn_norm_rope's kernel.
struct NormRopeParams {
  const uint16_t* __restrict__ x;
  uint16_t* y;
  const uint16_t* __restrict__ w;
  const uint16_t* __restrict__ cos;
  const uint16_t* __restrict__ sin;
  int64_t sx_t, sx_h, sy_t, sy_h, rope_stride, vectors;
  int32_t heads, norm, rope_dim;
  float eps;
};
hipError_t launch_norm_rope(const NormRopeParams& p, int head_dim, hipStream_t stream);

// The attention kernel over `items` x head groups workgroups, then (when `merges` > 0) the merge kernel over
// `merges` x head groups, on `stream`.
hipError_t launch_forward(const Params& p, int head_dim, const Geometry& g, int64_t items, int64_t merges,
                          hipStream_t stream);
// The head-size-128 wide and long tiles (attn_fwd_128.hip), which launch_forward hands on.
hipError_t launch_forward_128(const Params& p, int shape, int64_t items, int64_t merges, int n_hg,
                              hipStream_t stream);

// One work list for the device planner: from the bounds into `plan` (room for `merges` split tiles and `items`
// items; at most `tiles` tiles are planned), with `tile_base` (n_seq + 1 ints) as its scratch. With a `status` word
// the planner first checks the bounds against the call's contract (non-decreasing from 0, query rows within
// total_q, every query run at most max_q): bounds that break it get an empty plan and KARPO_ATTN_ERR_BOUNDS in
// `status` (else KARPO_ATTN_OK), so no kernel reads or writes a row through them.
struct PlanJob {
  const int32_t* q_cu;
  const int32_t* k_cu;
  Geometry g;
  int left, right;
  int32_t* plan;
  int tiles, merges, items;
  int32_t* tile_base;
  int32_t* status;   // or null: no bounds check (the backward's work lists)
  int64_t total_q;
  int32_t max_q;
  int32_t gather;    // the plan header's row-table flag
  int64_t key_bound; // key rows the bounds may index, or 0: not checked
};
// The device planner: one workgroup per job (one or two), one launch.
hipError_t launch_plan(const PlanJob* jobs, int n_jobs, int n_seq, hipStream_t stream);

}  // namespace karpo
