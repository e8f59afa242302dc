// Packed varlen attention forward for gfx950 (MI355X): bf16 MFMA, fp32 online softmax, per-tile masks.
//
// Algorithm (the same arithmetic as the reference's Triton kernel, families/gemma/triton_attention.py:53-84, and the
// per-sequence SDPA path it replaces, families/gemma/packed.py:195-220): for each query, a running maximum m and sum l
// in the exp2 domain (logit * scale * log2 e), P = exp2(logit - m) rounded to bf16 for the P.V product, the output
// accumulated in fp32 and divided by l at the end. Masks (causal / window / image span, varlen alignment of
// tests/test_gemma_blocks.py:28-43) are evaluated per element only on key steps that cut through a wave's queries.
//
// Data flow of one workgroup (4 waves, one work item = one query tile x one head group):
//   * each wave holds 32*NB query vectors (position, head) of the tile in registers as MFMA B operands;
//   * per step, BN keys of K and V are staged in LDS (double buffered; V transposed to [d][key] on the way in);
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: a lane then owns one query column, so the row max and sum are
//     in-lane plus one v_permlane32_swap between the two half-waves;
//   * K rows are fed to the MFMA in the order that swaps bits 2 and 3 of the row index, which makes each lane's 8
//     consecutive S^T registers hold 8 consecutive keys: the P registers are directly the B operand of
//     O^T = V^T P^T, and V^T is read from LDS with one 16-byte read per MFMA;
//   * the running maximum is only raised when a step's maximum exceeds it by more than 2^8 (exact: the final
//     division by l cancels any common factor), so O is rescaled on few steps.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "karpo_attn.h"
#include "internal.h"
#include "plan_common.h"

namespace karpo {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Lazy-rescale threshold in log2 units: P values stay below 2^8.
constexpr float kTau = 8.0f;

__device__ __forceinline__ float half_swap_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float half_swap_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o));
  return x;
}

__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x = max(x, __shfl_xor(x, o));
  return x;
}

// Row of the 32-key block that MFMA A-row r reads: bits 2 and 3 of r swapped.
__device__ __forceinline__ int key_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

template <int D, int NB, int BN>
__global__ __launch_bounds__(kThreads, 1) void attn_fwd_kernel(Params p) {
  constexpr int DC = D / 16;       // 16-wide head-dim chunks of the QK^T contraction
  constexpr int DB = D / 32;       // 32-row head-dim blocks of O^T
  constexpr int KB = BN / 32;      // 32-key blocks of S^T
  constexpr int KC = BN / 16;      // 16-key chunks of the PV contraction
  constexpr int KROW = D + 8;      // LDS pitch of a K row (elements), padded against bank conflicts
  constexpr int VROW = BN + 8;     // LDS pitch of a V^T row
  constexpr int R = BN * D / (8 * kThreads);  // 16-byte chunks per thread per step, for K and for V
  constexpr int KQ = BN / R;       // threads along keys in the V^T staging
  static_assert(R == 2 || R == 4, "staging assumes 2 or 4 keys per thread");
  constexpr int VW = 32 * NB;      // query vectors per wave

  __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][BN * KROW];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][D * VROW];
  __shared__ int red[2][kWaves];

  const int n_tiles = p.plan[0];
  const int item = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item * p.n_hg;
  if (item >= n_tiles) return;
  const int seg = p.plan[kPlanHeader + 2 * item];
  const int tile = p.plan[kPlanHeader + 2 * item + 1];
  const int rows_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int delta = lk - lq;
  const int kvh = (hg * p.ng) / p.group;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 31, half = lane >> 5;

  // ---- this lane's query vectors: positions, heads, visible key ranges, Q operands
  int pos[NB], head[NB], lo[NB], hi[NB], sl[NB], sh[NB];
  bool valid[NB];
  int wlo = INT32_MAX, whi = INT32_MIN, wflo = INT32_MIN, wfhi = INT32_MAX;
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const int vec = wave * VW + cb * 32 + col;
    const int off = vec / p.ng;
    pos[cb] = tile * rows_per_tile + off;
    head[cb] = hg * p.ng + (vec - off * p.ng);
    valid[cb] = pos[cb] < lq;
    lo[cb] = hi[cb] = sl[cb] = sh[cb] = 0;
    if (valid[cb]) {
      const int ip = pos[cb] + delta;  // aligned key coordinate
      int a = p.left < 0 ? 0 : max(0, ip - p.left);
      int b = p.right < 0 ? lk : (int)min((int64_t)lk, (int64_t)ip + p.right + 1);
      if (b < a) b = a;
      lo[cb] = a;
      hi[cb] = b;
      wflo = max(wflo, a);
      wfhi = min(wfhi, b);
      if (a < b) {
        wlo = min(wlo, a);
        whi = max(whi, b);
      }
      if (p.n_spans > 0) {  // the last span starting at or before this query row
        const int row = qa + pos[cb];
        int l0 = 0, l1 = p.n_spans;
        while (l1 - l0 > 1) {
          const int mid = (l0 + l1) >> 1;
          if (p.spans[2 * mid] <= row) l0 = mid; else l1 = mid;
        }
        const int s0 = p.spans[2 * l0], s1 = p.spans[2 * l0 + 1];
        if (s0 <= row && row < s1) {
          const int x = max(0, s0 - qa + delta), y = min(lk, s1 - qa + delta);
          if (x < y) {
            sl[cb] = x;
            sh[cb] = y;
            wlo = min(wlo, x);
            whi = max(whi, y);
          }
        }
      }
    }
  }
  wlo = wave_min(wlo);
  whi = wave_max(whi);
  wflo = wave_max(wflo);
  wfhi = wave_min(wfhi);
  if (lane == 0) {
    red[0][wave] = wlo;
    red[1][wave] = whi;
  }

  bf16x8 qop[NB][DC];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const uint16_t* qp = p.q + (int64_t)(qa + pos[cb]) * p.sq_t + (int64_t)head[cb] * p.sq_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      u32x4 x = {0, 0, 0, 0};
      if (valid[cb]) x = *(const u32x4*)(qp + dc * 16);
      x ^= p.qsign;
      qop[cb][dc] = __builtin_bit_cast(bf16x8, x);
    }
  }
  __syncthreads();
  int klo = INT32_MAX, khi = INT32_MIN;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    klo = min(klo, red[0][w]);
    khi = max(khi, red[1][w]);
  }
  const int j_first = klo < khi ? (klo / BN) * BN : 0;
  const int n_steps = klo < khi ? (khi - j_first + BN - 1) / BN : 0;

  // ---- K/V staging: global -> registers (issued a step ahead) -> LDS
  const uint16_t* kbase = p.k + (int64_t)kvh * p.sk_h;
  const uint16_t* vbase = p.v + (int64_t)kvh * p.sv_h;
  u32x4 kreg[R], vreg[R];
  const int vkq = tid % KQ, vdq = tid / KQ;
  auto load_step = [&](int j0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ci = tid + r * kThreads;
      const int row = ci / (D / 8), dq = ci % (D / 8);
      const int key = min(j0 + row, lk - 1);
      kreg[r] = *(const u32x4*)(kbase + (int64_t)(ka + key) * p.sk_t + dq * 8);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int key = min(j0 + vkq * R + r, lk - 1);
      vreg[r] = *(const u32x4*)(vbase + (int64_t)(ka + key) * p.sv_t + vdq * 8);
    }
  };
  auto store_step = [&](int buf) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int ci = tid + r * kThreads;
      const int row = ci / (D / 8), dq = ci % (D / 8);
      *(u32x4*)&k_lds[buf][row * KROW + dq * 8] = kreg[r];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const unsigned sel = (e & 1) ? 0x07060302u : 0x05040100u;
      uint16_t* dst = &v_lds[buf][(vdq * 8 + e) * VROW + vkq * R];
      if constexpr (R == 4) {
        u32x2 w;
        w[0] = __builtin_amdgcn_perm(vreg[1][e >> 1], vreg[0][e >> 1], sel);
        w[1] = __builtin_amdgcn_perm(vreg[3][e >> 1], vreg[2][e >> 1], sel);
        *(u32x2*)dst = w;
      } else {
        *(unsigned*)dst = __builtin_amdgcn_perm(vreg[1][e >> 1], vreg[0][e >> 1], sel);
      }
    }
  };

  f32x16 acc[DB][NB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) acc[db][cb] = f32x16{};
  float m[NB], l[NB];
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    m[cb] = -INFINITY;
    l[cb] = 0.f;
  }
  const float c = p.c;

  if (n_steps > 0) {
    load_step(j_first);
    store_step(0);
  }
  __syncthreads();

  for (int s = 0; s < n_steps; ++s) {
    const int buf = s & 1;
    const int j0 = j_first + s * BN;
    if (s + 1 < n_steps) load_step(j0 + BN);
    if (j0 < whi && j0 + BN > wlo) {  // wave-uniform: some query of this wave sees a key of this step
      const uint16_t* kl = k_lds[buf];
      const uint16_t* vl = v_lds[buf];
      f32x16 st[KB][NB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) st[kb][cb] = f32x16{};
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const bf16x8 a = *(const bf16x8*)&kl[(kb * 32 + key_row(col)) * KROW + dc * 16 + half * 8];
#pragma unroll
          for (int cb = 0; cb < NB; ++cb)
            st[kb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[cb][dc], st[kb][cb], 0, 0, 0);
        }
      }
      if (!(j0 >= wflo && j0 + BN <= wfhi)) {  // some query of this wave does not see every key of the step
#pragma unroll
        for (int cb = 0; cb < NB; ++cb) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
              const int key = j0 + kb * 32 + (jj >> 3) * 16 + half * 8 + (jj & 7);
              const bool vis = (unsigned)(key - lo[cb]) < (unsigned)(hi[cb] - lo[cb]) ||
                               (unsigned)(key - sl[cb]) < (unsigned)(sh[cb] - sl[cb]);
              if (!vis) st[kb][cb][jj] = -INFINITY;
            }
          }
        }
      }
      float alpha[NB];
      bool raise = false;
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) mx = fmaxf(mx, st[kb][cb][jj]);
        const float mt = half_swap_max(mx) * c;
        const bool need = mt > m[cb] + kTau;
        const float mn = need ? mt : m[cb];
        alpha[cb] = need ? __builtin_amdgcn_exp2f(m[cb] - mn) : 1.f;
        raise |= need;
        m[cb] = mn;
        l[cb] *= alpha[cb];
        const float msub = mn == -INFINITY ? 0.f : mn;
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int jj = 0; jj < 16; ++jj) {
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kb][cb][jj], c, -msub));
            st[kb][cb][jj] = e;
            sum += e;
          }
        l[cb] += sum;
      }
      if (__builtin_amdgcn_ballot_w64(raise)) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int cb = 0; cb < NB; ++cb) acc[db][cb] *= alpha[cb];
      }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        bf16x8 pb[NB];
#pragma unroll
        for (int cb = 0; cb < NB; ++cb)
#pragma unroll
          for (int t = 0; t < 8; ++t) pb[cb][t] = (__bf16)st[kc >> 1][cb][(kc & 1) * 8 + t];
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 a = *(const bf16x8*)&vl[(db * 32 + col) * VROW + kc * 16 + half * 8];
#pragma unroll
          for (int cb = 0; cb < NB; ++cb)
            acc[db][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[cb], acc[db][cb], 0, 0, 0);
        }
      }
    }
    if (s + 1 < n_steps) store_step(buf ^ 1);
    __syncthreads();
  }

  // ---- normalise and store: lane (col, half) holds d = db*32 + (j/4)*8 + half*4 + j%4 of its query
#pragma unroll
  for (int cb = 0; cb < NB; ++cb) {
    const float lt = half_swap_sum(l[cb]);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (!valid[cb]) continue;
    uint16_t* op = p.o + (int64_t)(qa + pos[cb]) * p.so_t + (int64_t)head[cb] * p.so_h + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 w;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const __bf16 x0 = (__bf16)(acc[db][cb][g4 * 4 + 2 * t] * inv);
          const __bf16 x1 = (__bf16)(acc[db][cb][g4 * 4 + 2 * t + 1] * inv);
          w[t] = (unsigned)__builtin_bit_cast(uint16_t, x0) | ((unsigned)__builtin_bit_cast(uint16_t, x1) << 16);
        }
        *(u32x2*)(op + db * 32 + g4 * 8) = w;
      }
    }
  }
}

// ---- device planner: one workgroup turns the device bounds into the longest-first work list.

constexpr int kPlanThreads = 1024;

__device__ int block_exclusive_scan(int x, int* total, int* scratch /* >= kPlanThreads/64 + 1 */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kPlanThreads / 64; ++w) {
      const int t = scratch[w];
      scratch[w] = run;
      run += t;
    }
    scratch[kPlanThreads / 64] = run;
  }
  __syncthreads();
  const int ex = scratch[wave] + incl - x;
  *total = scratch[kPlanThreads / 64];
  __syncthreads();
  return ex;
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int32_t* __restrict__ q_cu,
                                                            const int32_t* __restrict__ k_cu, int n_seq, int rows,
                                                            int bn, int ng, int left, int right,
                                                            int32_t* __restrict__ plan, int capacity,
                                                            int32_t* __restrict__ tile_base) {
  __shared__ int hist[kCostBuckets];
  __shared__ int scratch[kPlanThreads / 64 + 1];
  const int tid = threadIdx.x;
  int carry = 0;
  for (int base = 0; base < n_seq; base += kPlanThreads) {
    const int i = base + tid;
    const int nt = i < n_seq ? (int)tiles_of(q_cu[i + 1] - q_cu[i], rows) : 0;
    int total;
    const int ex = block_exclusive_scan(nt, &total, scratch);
    if (i < n_seq) tile_base[i] = carry + ex;
    carry += total;
  }
  if (tid == 0) tile_base[n_seq] = carry;
  const int n_tiles = min(carry, capacity);
  for (int b = tid; b < kCostBuckets; b += kPlanThreads) hist[b] = 0;
  __syncthreads();

  auto locate = [&](int f, int* seg, int* cost) {
    int l0 = 0, l1 = n_seq;  // last segment whose first tile is at or before f
    while (l1 - l0 > 1) {
      const int mid = (l0 + l1) >> 1;
      if (tile_base[mid] <= f) l0 = mid; else l1 = mid;
    }
    const int t = f - tile_base[l0];
    const int lq = q_cu[l0 + 1] - q_cu[l0], lk = k_cu[l0 + 1] - k_cu[l0];
    *seg = l0;
    *cost = min(tile_cost(lq, lk, t, rows, bn, left, right), kCostBuckets - 1);
    return t;
  };
  for (int f = tid; f < n_tiles; f += kPlanThreads) {
    int seg, cost;
    locate(f, &seg, &cost);
    atomicAdd(&hist[cost], 1);
  }
  __syncthreads();
  // descending exclusive scan: bucket b starts after every item of higher cost
  {
    constexpr int per = kCostBuckets / kPlanThreads;
    int h[per], s = 0;
#pragma unroll
    for (int r = 0; r < per; ++r) {
      h[r] = hist[kCostBuckets - 1 - (tid * per + r)];
      s += h[r];
    }
    int total;
    int ex = block_exclusive_scan(s, &total, scratch);
#pragma unroll
    for (int r = 0; r < per; ++r) {
      hist[kCostBuckets - 1 - (tid * per + r)] = ex;
      ex += h[r];
    }
  }
  __syncthreads();
  for (int f = tid; f < n_tiles; f += kPlanThreads) {
    int seg, cost;
    const int t = locate(f, &seg, &cost);
    const int at = atomicAdd(&hist[cost], 1);
    plan[kPlanHeader + 2 * at] = seg;
    plan[kPlanHeader + 2 * at + 1] = t;
  }
  if (tid == 0) {
    plan[0] = n_tiles;
    plan[1] = rows;
    plan[2] = bn;
    plan[3] = ng;
  }
}

// ---- launch


template <int D, int NB, int BN>
static hipError_t launch_attn(const Params& p, int64_t grid, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<D, NB, BN>), dim3((unsigned)grid), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_forward(const Params& p, int head_dim, int64_t grid, hipStream_t stream) {
  if (grid <= 0) return hipSuccess;
  switch (head_dim) {
    case 64: return launch_attn<64, 2, 64>(p, grid, stream);
    case 128: return launch_attn<128, 2, 64>(p, grid, stream);
    case 256: return launch_attn<256, 1, 32>(p, grid, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_plan(const int32_t* q_cu, const int32_t* k_cu, int n_seq, const Geometry& g, int left, int right,
                       int32_t* plan, int capacity, int32_t* tile_base, hipStream_t stream) {
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, q_cu, k_cu, n_seq, g.rows, g.bn, g.ng, left,
                     right, plan, capacity, tile_base);
  return hipGetLastError();
}

}  // namespace karpo
