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
  uint32_t qsign;   // 0x80008000 to negate Q (negative scale), else 0
};

// The attention kernel over `items` x head groups workgroups, then (when `merges` > 0) the merge kernel over
// `merges` x head groups, on `stream`.
hipError_t launch_forward(const Params& p, int head_dim, const Geometry& g, int64_t items, int64_t merges,
                          hipStream_t stream);

// The device planner: writes the work list for the bounds into `plan` (room for `merges` split tiles and `items`
// items; at most `tiles` tiles are planned) using `tile_base` (n_seq + 1 ints) as scratch.
hipError_t launch_plan(const int32_t* q_cu, const int32_t* k_cu, int n_seq, const Geometry& g, int left, int right,
                       int32_t* plan, int tiles, int merges, int items, int32_t* tile_base, hipStream_t stream);

}  // namespace karpo
