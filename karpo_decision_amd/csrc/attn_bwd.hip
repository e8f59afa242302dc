// Packed varlen attention backward for gfx950 (MI355X): bf16 MFMA, fp32 accumulation, the forward's masks.
//
// Arithmetic (the textbook flash-attention backward the reference's FA4 / cuDNN backward ops compute,
// families/gemma/sliding_attention.py:50-61, families/gemma/global_attention.py:107-118): with t = scale * q.k over a
// query row's visible keys, P = exp(t - lse) (the forward's log-sum-exp), D = rowsum(dO * O),
//   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - D),  dQ = scale * dS K,  dK = scale * dS^T Q.
// P and dS enter the MFMAs as bf16 (as P does in the forward), every product accumulates in fp32. The rows'
// statistics hold -D (negated once where D is formed): the dK / dV kernels start their dP accumulators from it, so
// dP - D comes out of the MFMAs and a step's softmax saves a subtraction per element.
//
// Two kernels after the planner (plan_kernel of attn_fwd.hip: both work lists in one launch; at head sizes 64 and 128
// the longest key tiles split over their query steps, their parts' fp32 dK / dV summed by bwd_merge_kernel):
//   * bwd_dq_kernel (query-stationary, the forward's tiles): per (head, query row) first the log2-domain LSE (+inf
//     for a row that sees no key, so its P are 0) and -D = -rowsum(dO * O), written for the dK / dV kernel (every
//     vector is in exactly one query tile); then Q and dO of 32 query vectors per wave as MFMA B operands
//     in registers, K and V streamed through LDS; S^T = K Q^T and dP^T = V dO^T with K and V read as row operands,
//     dQ^T += K^T dS^T with K read transposed from the same tile (the S layout of mfma_common.h serves both reads);
//   * bwd_dkdv_kernel (key-stationary, tiles of 128 keys, four waves of 32): K and V of the wave's keys in registers,
//     the query rows that see the tile streamed in steps of 32 rows of one head (every head of the GQA group in turn,
//     which sums the group's gradients): S = Q K^T and dP = dO V^T with Q and dO as row operands, dV^T += dO^T P and
//     dK^T += Q^T dS with Q and dO read transposed from the same tiles (S layout; a dV-only launch stages dO in the
//     transposed-read layout, whose copies read whole rows). One launch computes both (MODE 3; at head sizes 64 and
//     256 one wave per SIMD holds both accumulators in 256 AGPRs);
//   * bwd_dkdv2_kernel (head size 128): both gradients in one launch at two waves per SIMD, eight waves per key tile
//     in two groups that take alternate row steps, K and V in LDS instead of registers (30.7 -> 28.1 ms for the 32k
//     layer's backward against dV and dK as two launches, MODE 1 and MODE 2, each recomputing S: KA_BWD2 0).
// Both streams advance their copy addresses by pointer increments per step (no per-step address recomputation: the
// scalar unit is shared by the CU's waves and a step is short).
// Rows of a product's row operand are fed in the order that swaps bits 2 and 3 of the row index (key_row), so each
// lane's 8 consecutive result registers are 8 consecutive rows: P, dS (S^T layout) are directly the B operands of the
// next products, as in the forward.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"
#include "karpo_attn.h"
#include "mfma_common.h"
#include "plan_common.h"

namespace karpo {

constexpr float kLog2e = 1.4426950408889634f;

// Key-tile workgroups from which head size 128 runs dK and dV as two launches.
constexpr int64_t kSplitKeyTiles = 8 * kComputeUnits;
// Head size 128 computes dK and dV in bwd_dkdv2_kernel; KA_BWD2 0 restores the two launches (large packs) or the
// one-wave-per-SIMD MODE 3 launch (small packs), for A/B measurements.
#ifndef KA_BWD2
#define KA_BWD2 1
#endif

template <int D> struct BwdCfg {
  static constexpr int OCC_Q = D >= 256 ? 1 : 2;  // waves per SIMD the registers are budgeted for
  static constexpr int BLOCKS_Q = OCC_Q * 4 / bwd_q_waves(D) > 0 ? OCC_Q * 4 / bwd_q_waves(D) : 1;
  template <int MODE> static constexpr int occ_k() { return MODE == 3 ? 1 : MODE == 1 ? 3 : 2; }
};

// Row (within a 32-row step) of result register j of a lane in half `half` (row operands fed in key_row order).
__device__ __forceinline__ int result_row(int j, int half) { return (j >> 3) * 16 + half * 8 + (j & 7); }

// ---- stats: L = D / 8 lanes per (row, head) vector, 8 elements per lane; the log2 LSE and -D of each
template <int D>
__global__ __launch_bounds__(256) void bwd_stats_kernel(BwdParams p) {
  constexpr int L = D / 8, VPW = 64 / L;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / L, l = lane - sub * L;
  const int64_t vectors = p.total_q * p.heads;
  for (int64_t v0 = ((int64_t)blockIdx.x * 4 + wave) * VPW; v0 < vectors; v0 += (int64_t)gridDim.x * 4 * VPW) {
    const int64_t v = v0 + sub;
    const bool ok = v < vectors;
    const int64_t row = ok ? v / p.heads : 0;
    const int head = ok ? (int)(v - row * p.heads) : 0;
    u32x4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0};
    if (ok) {
      x = *(const u32x4*)(p.dout + row * p.sdo_t + (int64_t)head * p.sdo_h + l * 8);
      y = *(const u32x4*)(p.o + row * p.so_t + (int64_t)head * p.so_h + l * 8);
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) s = __builtin_fmaf(bf16_at(x, e), bf16_at(y, e), s);
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (ok && l == 0) {
      const float lse = p.lse[(int64_t)head * p.total_q + row];
      p.stats[((int64_t)head * 2) * p.total_q + row] = lse == -INFINITY ? INFINITY : lse * kLog2e;
      p.stats[((int64_t)head * 2 + 1) * p.total_q + row] = -s;
    }
  }
}

// ---- dQ: query tiles (plan items: segment, tile), 32 query vectors per wave, BN keys (KB blocks of 32) per step
template <int D>
__global__ __launch_bounds__(64 * bwd_q_waves(D), BwdCfg<D>::BLOCKS_Q) void bwd_dq_kernel(BwdParams p) {
  constexpr int W = bwd_q_waves(D), BN = bwd_q_step(D), KB = BN / 32;
  constexpr int DC = D / 16, DB = D / 32, KC = BN / 16;
  constexpr int TILE = BN * D * 2, BLKS = TILE / 1024, INSTS = (BLKS + W - 1) / W;
  __shared__ __attribute__((aligned(1024))) char kk0[TILE];  // K (S layout: read as rows and transposed)
  __shared__ __attribute__((aligned(1024))) char kk1[TILE];
  __shared__ __attribute__((aligned(1024))) char vk0[TILE];  // V (S layout, read as rows)
  __shared__ __attribute__((aligned(1024))) char vk1[TILE];
  __shared__ int red[2][W];

  if (p.plan[2] != BN || p.plan[5] != W) return;
  const int item = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item * p.n_hg;
  if (item >= p.plan[0]) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0], tile = entry[1];
  const int rows_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int delta = lk - lq;
  const int kvh = (hg * p.ng) / p.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;

  // this lane's query vector and the keys it sees (the forward's rule)
  const int vec = wave * 32 + col;
  const int off = vec / p.ng;
  const int pos = tile * rows_per_tile + off;
  const int head = hg * p.ng + (vec - off * p.ng);
  const bool valid = pos < lq;
  int lo = 0, hi = 0, sl = 0, sh = 0;
  int wlo = INT32_MAX, whi = INT32_MIN, wflo = INT32_MIN, wfhi = INT32_MAX;
  if (valid) {
    const int ip = pos + delta;
    int a = p.left < 0 ? 0 : max(0, ip - p.left);
    int b = p.right < 0 ? lk : (int)min((int64_t)lk, (int64_t)ip + p.right + 1);
    if (b < a) b = a;
    lo = a;
    hi = b;
    wflo = a;
    wfhi = b;
    if (a < b) {
      wlo = a;
      whi = b;
    }
    if (p.n_spans > 0) {
      const int row = qa + pos;
      int l0 = 0, l1 = p.n_spans;
      while (l1 - l0 > 1) {
        const int mid = (l0 + l1) >> 1;
        if (p.spans[2 * mid] <= row) l0 = mid; else l1 = mid;
      }
      const int s0 = p.spans[2 * l0], s1 = p.spans[2 * l0 + 1];
      if (s0 <= row && row < s1) {
        const int x = max(0, s0 - qa + delta), y = min(lk, s1 - qa + delta);
        if (x < y) {
          sl = x;
          sh = y;
          wlo = min(wlo, x);
          whi = max(whi, y);
        }
      }
    }
  }
  wlo = __builtin_amdgcn_readfirstlane(wave_min(wlo));
  whi = __builtin_amdgcn_readfirstlane(wave_max(whi));
  wflo = __builtin_amdgcn_readfirstlane(wave_max(wflo));
  wfhi = __builtin_amdgcn_readfirstlane(wave_min(wfhi));
  if (lane == 0) {
    red[0][wave] = wlo;
    red[1][wave] = whi;
  }
  // Q and dO as B operands (lane: its vector, elements dc*16 + half*8 .. +8); the row's log2 LSE and
  // D = rowsum(dO * O) (the two half-waves hold the two halves of the row), also written (LSE and -D) for the dK / dV
  // kernel, which runs after this one (every (row, head) vector is in exactly one query tile)
  bf16x8 qop[DC], dop[DC];
  float lse2 = INFINITY, dsum = 0.f;
  {
    const uint16_t* qp = p.q + (int64_t)(qa + pos) * p.sq_t + (int64_t)head * p.sq_h + half * 8;
    const uint16_t* dp = p.dout + (int64_t)(qa + pos) * p.sdo_t + (int64_t)head * p.sdo_h + half * 8;
    const uint16_t* opp = p.o + (int64_t)(qa + pos) * p.so_t + (int64_t)head * p.so_h + half * 8;
    float part = 0.f;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      u32x4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0}, z = {0, 0, 0, 0};
      if (valid) {
        x = *(const u32x4*)(qp + dc * 16);
        y = *(const u32x4*)(dp + dc * 16);
        z = *(const u32x4*)(opp + dc * 16);
      }
      qop[dc] = __builtin_bit_cast(bf16x8, x);
      dop[dc] = __builtin_bit_cast(bf16x8, y);
#pragma unroll
      for (int e = 0; e < 8; ++e) part = __builtin_fmaf(bf16_at(y, e), bf16_at(z, e), part);
    }
    dsum = half_swap_sum(part);
    if (valid) {
      const float lse = p.lse[(int64_t)head * p.total_q + qa + pos];
      lse2 = lse == -INFINITY ? INFINITY : lse * kLog2e;
      if (half == 0) {
        p.stats[((int64_t)head * 2) * p.total_q + qa + pos] = lse2;
        p.stats[((int64_t)head * 2 + 1) * p.total_q + qa + pos] = -dsum;
      }
    }
  }
  __syncthreads();
  int klo = INT32_MAX, khi = INT32_MIN;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    klo = min(klo, red[0][w]);
    khi = max(khi, red[1][w]);
  }
  klo = __builtin_amdgcn_readfirstlane(klo);
  khi = __builtin_amdgcn_readfirstlane(khi);
  const int j_first = klo < khi ? (klo / BN) * BN : 0;
  const int n_steps = klo < khi ? (khi - j_first + BN - 1) / BN : 0;

  // copies: K and V in the S layout (zeros past the sequence's last key)
  const uint16_t* kbase = p.k + (int64_t)kvh * p.sk_h + (int64_t)ka * p.sk_t;
  const uint16_t* vbase = p.v + (int64_t)kvh * p.sv_h + (int64_t)ka * p.sv_t;
  uint32_t kk_off[INSTS], vk_off[INSTS];
#pragma unroll
  for (int r = 0; r < INSTS; ++r) {
    int key, colm;
    s_dma_source<D>(wave * INSTS + r, lane, &key, &colm);
    kk_off[r] = (uint32_t)(key * p.sk_t + colm) * 2u;
    vk_off[r] = (uint32_t)(key * p.sv_t + colm) * 2u;
  }
  const uint16_t* c_k = kbase + (int64_t)j_first * p.sk_t;
  const uint16_t* c_v = vbase + (int64_t)j_first * p.sv_t;
  const int64_t k_step = (int64_t)BN * p.sk_t, v_step = (int64_t)BN * p.sv_t;
  auto copy_step = [&](int j0, KA_LDS char* tkk, KA_LDS char* tvk) {
    const int rows = min(lk - j0, BN);
    const uint16_t* ks = c_k;
    const uint16_t* vs = c_v;
    c_k += k_step;
    c_v += v_step;
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      if (BLKS % W == 0 || wave * INSTS + r < BLKS) {
        const int at = (wave * INSTS + r) * 1024;
        dma_16b(ks, rows * (int)p.sk_t * 2, tkk + at, kk_off[r]);
        dma_16b(vs, rows * (int)p.sv_t * 2, tvk + at, vk_off[r]);
      }
  };
  // row reads of chunk 2 dc + half: k_read[dc & 1] + (dc >> 1) * 1024; transposed reads: t_read[rr] + kc, db offsets
  const int k_read[2] = {s_offset<D>(key_row(col), half), s_offset<D>(key_row(col), 2 + half)};
  const int t_read[2] = {s_tr_base(lane, 0), s_tr_base(lane, 1)};
  f32x16 acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) acc[db] = f32x16{};
  const float c = p.c;

  KA_LDS char* const tkk0 = (KA_LDS char*)kk0;
  KA_LDS char* const tkk1 = (KA_LDS char*)kk1;
  KA_LDS char* const tvk0 = (KA_LDS char*)vk0;
  KA_LDS char* const tvk1 = (KA_LDS char*)vk1;
  if (n_steps > 0) copy_step(j_first, tkk0, tvk0);
  wait_vmcnt<0>();
  __syncthreads();

  auto step = [&](int s, const KA_LDS char* tkk, const KA_LDS char* tvk, KA_LDS char* nkk, KA_LDS char* nvk) {
    const int j0 = j_first + s * BN;
    if (s + 1 < n_steps) copy_step(j0 + BN, nkk, nvk);
    if (j0 < whi && j0 + BN > wlo) {
      f32x16 st[KB], dpt[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        st[kb] = f32x16{};
        dpt[kb] = f32x16{};
      }
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {  // key block kb: rows kb * 32 .. of the step
          const int at = k_read[dc & 1] + (dc >> 1) * 1024 + kb * (2 * (D / 8) * 256);
          const bf16x8 a = *(const KA_LDS bf16x8*)(tkk + at);
          st[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], st[kb], 0, 0, 0);
          const bf16x8 b = *(const KA_LDS bf16x8*)(tvk + at);
          dpt[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, dop[dc], dpt[kb], 0, 0, 0);
        }
      }
      // exponents of P^T (key kc * 16 + half * 8 + t of the step: register (kc & 1) * 8 + t of key block kc / 2);
      // on a step some lane's window or span cuts, -inf (exp2 gives 0) for the keys that lane does not see: one
      // uniform branch around the masking, none per element and no mask work on the other steps
      float x[KC][8];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t) x[kc][t] = __builtin_fmaf(st[kc >> 1][(kc & 1) * 8 + t], c, -lse2);
      if (!(j0 >= wflo && j0 + BN <= wfhi)) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int key = j0 + kc * 16 + half * 8 + t;
            const bool vis = ((unsigned)(key - lo) < (unsigned)(hi - lo)) | ((unsigned)(key - sl) < (unsigned)(sh - sl));
            x[kc][t] = vis ? x[kc][t] : -INFINITY;
          }
      }
      bf16x8 dsb[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t)
          dsb[kc][t] = (__bf16)(__builtin_amdgcn_exp2f(x[kc][t]) * (dpt[kc >> 1][(kc & 1) * 8 + t] - dsum));
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          bf16x4 pv[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            pv[rr] = __builtin_bit_cast(
                bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (KA_LDS s16x4*)(tkk + t_read[rr] + kc * (D / 8) * 256 + db * 1024)));
          const bf16x8 a = __builtin_shufflevector(pv[0], pv[1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, dsb[kc], acc[db], 0, 0, 0);
        }
      }
    }
    wait_vmcnt<0>();
    __syncthreads();
  };
  int s = 0;
  for (; s + 1 < n_steps; s += 2) {
    step(s, tkk0, tvk0, tkk1, tvk1);
    step(s + 1, tkk1, tvk1, tkk0, tvk0);
  }
  if (s < n_steps) step(s, tkk0, tvk0, tkk1, tvk1);

  if (valid) {  // dq = scale * acc: lane (col, half) holds d = db*32 + (j/4)*8 + half*4 + j%4
    uint16_t* dp = p.dq + (int64_t)(qa + pos) * p.sdq_t + (int64_t)head * p.sdq_h + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 w;
        w[0] = pack_bf16(acc[db][g4 * 4] * p.scale, acc[db][g4 * 4 + 1] * p.scale);
        w[1] = pack_bf16(acc[db][g4 * 4 + 2] * p.scale, acc[db][g4 * 4 + 3] * p.scale);
        *(u32x2*)(dp + db * 32 + g4 * 8) = w;
      }
  }
}

// The query rows that see key `key` of a sequence (qa: the sequence's first query row in the pack; lq, delta = lk -
// lq): rows [lo, hi) by the window (j - right <= i + delta <= j + left) and [sl, sh), the image span holding the
// key's aligned row, when it is in one; and over the wave, the envelope [wlo, whi) of the rows any lane's key is seen
// by and the range [wflo, wfhi) of rows that see every lane's key. A lane past the sequence (not valid) sees none.
struct KeyRows {
  int lo, hi, sl, sh;
  int wlo, whi, wflo, wfhi;
};
__device__ __forceinline__ KeyRows key_rows_seen(const BwdParams& p, int key, bool valid, int qa, int lq, int delta) {
  KeyRows r = {0, 0, 0, 0, INT32_MAX, INT32_MIN, INT32_MIN, INT32_MAX};
  if (valid) {
    int a = p.right < 0 ? 0 : max(0, key - p.right - delta);
    int b = p.left < 0 ? lq : (int)min((int64_t)lq, (int64_t)key + p.left - delta + 1);
    if (b < a) b = a;
    r.lo = a;
    r.hi = b;
    r.wflo = a;
    r.wfhi = b;
    if (a < b) {
      r.wlo = a;
      r.whi = b;
    }
    const int kq = key - delta;  // the key's position in query rows
    if (p.n_spans > 0 && kq >= 0 && kq < lq) {
      const int row = qa + kq;
      int l0 = 0, l1 = p.n_spans;
      while (l1 - l0 > 1) {
        const int mid = (l0 + l1) >> 1;
        if (p.spans[2 * mid] <= row) l0 = mid; else l1 = mid;
      }
      const int s0 = p.spans[2 * l0], s1 = p.spans[2 * l0 + 1];
      if (s0 <= row && row < s1) {
        const int x = max(0, s0 - qa), y = min(lq, s1 - qa);
        if (x < y) {
          r.sl = x;
          r.sh = y;
          r.wlo = min(r.wlo, x);
          r.whi = max(r.whi, y);
        }
      }
    }
  }
  r.wlo = __builtin_amdgcn_readfirstlane(wave_min(r.wlo));
  r.whi = __builtin_amdgcn_readfirstlane(wave_max(r.whi));
  r.wflo = __builtin_amdgcn_readfirstlane(wave_max(r.wflo));
  r.wfhi = __builtin_amdgcn_readfirstlane(wave_min(r.wfhi));
  return r;
}

// ---- dK, dV: key tiles of 128 (plan items of the bounds swapped: segment, key tile), 32 keys per wave. MODE bit 0:
// compute dV, bit 1: dK.
template <int D, int MODE>
__global__ __launch_bounds__(64 * kBwdWaves, BwdCfg<D>::template occ_k<MODE>()) void bwd_dkdv_kernel(BwdParams p) {
  constexpr bool DV = (MODE & 1) != 0, DK = (MODE & 2) != 0;
  constexpr int W = kBwdWaves, BQ = kBwdStep;
  constexpr int DC = D / 16, DB = D / 32, KC = BQ / 16;
  constexpr int TILE = BQ * D * 2, BLKS = TILE / 1024, INSTS = (BLKS + W - 1) / W;
  __shared__ __attribute__((aligned(1024))) char qk0[TILE];  // Q (S layout: rows for S, transposed for dK)
  __shared__ __attribute__((aligned(1024))) char qk1[TILE];
  __shared__ __attribute__((aligned(1024))) char ok0[TILE];  // dO (S layout: rows for dP, transposed for dV; dV alone: transposed-read layout)
  __shared__ __attribute__((aligned(1024))) char ok1[TILE];
  __shared__ __attribute__((aligned(256))) float sts0[2 * BQ];  // log2 LSE, then -D, of the step's rows
  __shared__ __attribute__((aligned(256))) float sts1[2 * BQ];
  __shared__ int red[2][W];

  if (p.plan[2] != BQ || p.plan[5] != W) return;
  const int item = blockIdx.x / p.n_hg;
  const int kvh = blockIdx.x - item * p.n_hg;
  if (item >= p.plan[0]) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0], ktile = entry[1];
  const int part = entry[2] & 0xffff, parts = entry[2] >> 16;
  const int slot = entry[3];
  if (parts > 1 && (slot < 0 || slot + part >= p.slots)) return;  // a partial slot outside the workspace
  const int keys_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int delta = lk - lq;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;

  // this lane's key and the query rows that see it
  const int key = ktile * keys_per_tile + wave * 32 + col;
  const bool valid = key < lk;
  const KeyRows seen = key_rows_seen(p, key, valid, qa, lq, delta);
  const int rlo = seen.lo, rhi = seen.hi, srl = seen.sl, srh = seen.sh;
  const int wlo = seen.wlo, whi = seen.whi, wflo = seen.wflo, wfhi = seen.wfhi;
  if (lane == 0) {
    red[0][wave] = wlo;
    red[1][wave] = whi;
  }
  // K and V of the lane's key as B operands (elements dc*16 + half*8 .. +8)
  bf16x8 kop[DC], vop[DC];
  {
    const uint16_t* kp = p.k + (int64_t)(ka + key) * p.sk_t + (int64_t)kvh * p.sk_h + half * 8;
    const uint16_t* vp = p.v + (int64_t)(ka + key) * p.sv_t + (int64_t)kvh * p.sv_h + half * 8;
#pragma unroll
    for (int dc = 0; dc < DC; ++dc) {
      u32x4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0};
      if (valid) {
        x = *(const u32x4*)(kp + dc * 16);
        if constexpr (DK) y = *(const u32x4*)(vp + dc * 16);
      }
      kop[dc] = __builtin_bit_cast(bf16x8, x);
      if constexpr (DK) vop[dc] = __builtin_bit_cast(bf16x8, y);
    }
  }
  __syncthreads();
  int qlo = INT32_MAX, qhi = INT32_MIN;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    qlo = min(qlo, red[0][w]);
    qhi = max(qhi, red[1][w]);
  }
  qlo = __builtin_amdgcn_readfirstlane(qlo);
  qhi = __builtin_amdgcn_readfirstlane(qhi);
  const int r_first = qlo < qhi ? (qlo / BQ) * BQ : 0;
  const int n_rsteps = qlo < qhi ? (qhi - r_first + BQ - 1) / BQ : 0;
  const int all_steps = n_rsteps * p.group;  // every head of the group in turn
  // a part of a split tile: steps [s_begin, s_begin + n_steps) of that sequence
  const int s_begin = parts > 1 ? (int)((int64_t)part * all_steps / parts) : 0;
  const int n_steps = parts > 1 ? (int)((int64_t)(part + 1) * all_steps / parts) - s_begin : all_steps;

  // dV alone reads dO only transposed: it keeps the transposed-read layout, whose copy reads whole rows (the S
  // layout's reads 64 bytes of each of 16 rows per instruction)
  constexpr bool OV = MODE == 1;
  uint32_t qk_off[INSTS], ok_off[INSTS];
#pragma unroll
  for (int r = 0; r < INSTS; ++r) {
    int row, colm;
    s_dma_source<D>(wave * INSTS + r, lane, &row, &colm);
    qk_off[r] = (uint32_t)(row * p.sq_t + colm) * 2u;
    if constexpr (OV) v_dma_source<D>(wave * INSTS + r, lane, &row, &colm);
    ok_off[r] = (uint32_t)(row * p.sdo_t + colm) * 2u;
  }
  // Steps visit the row steps of head kvh * group from the last (r_last) down to r_first, then the group's next
  // head's. Downwards: under a causal mask every key tile's rows end at the sequence's end, so the tiles that run at
  // once read the same Q / dO rows at about the same time (L2 hits) instead of rows a tile apart. The copy cursor
  // moves by pointer increments (no per-step address recomputation).
  const int r_last = r_first + (n_rsteps - 1) * BQ;
  const int h0 = kvh * p.group;
  const int64_t q_step = (int64_t)BQ * p.sq_t, o_step = (int64_t)BQ * p.sdo_t;
  const int64_t q_wrap = p.sq_h + n_rsteps * q_step, o_wrap = p.sdo_h + n_rsteps * o_step;
  const int64_t st_wrap = 2 * p.total_q + (int64_t)n_rsteps * BQ;
  const int h_begin = n_rsteps > 0 ? s_begin / n_rsteps : 0;   // the first step's head (of the group) and row
  const int r_begin = r_last - (s_begin - h_begin * n_rsteps) * BQ;
  int c_r0 = r_begin;
  const uint16_t* c_q = p.q + (int64_t)(qa + r_begin) * p.sq_t + (int64_t)(h0 + h_begin) * p.sq_h;
  const uint16_t* c_o = p.dout + (int64_t)(qa + r_begin) * p.sdo_t + (int64_t)(h0 + h_begin) * p.sdo_h;
  const float* c_st = p.stats + (int64_t)(h0 + h_begin) * 2 * p.total_q + qa + r_begin;
  auto copy_step = [&](KA_LDS char* tqk, KA_LDS char* tok, KA_LDS float* tst) {
    const int rows = min(lq - c_r0, BQ);
    const uint16_t* qs = c_q;
    const uint16_t* os = c_o;
    const float* src = c_st;
    c_r0 -= BQ;
    c_q -= q_step;
    c_o -= o_step;
    c_st -= BQ;
    if (c_r0 < r_first) {  // the group's next head
      c_r0 = r_last;
      c_q += q_wrap;
      c_o += o_wrap;
      c_st += st_wrap;
    }
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      if (BLKS % W == 0 || wave * INSTS + r < BLKS) {
        const int at = (wave * INSTS + r) * 1024;
        dma_16b(qs, rows * (int)p.sq_t * 2, tqk + at, qk_off[r]);
        dma_16b(os, rows * (int)p.sdo_t * 2, tok + at, ok_off[r]);
      }
    if (wave == W - 1) {  // 32 log2 LSE (lanes 0-31) then 32 -D (lanes 32-63), 4 B per lane; zeros past the stats
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (int)(p.total_q + rows) * 4, kBufferFlags);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (KA_LDS void*)tst, 4,
                                               (uint32_t)((lane >> 5) * p.total_q + (lane & 31)) * 4u, 0, 0, 0);
    }
  };
  // row reads of chunk 2 dc + half: q_read[dc & 1] + (dc >> 1) * 1024; transposed reads: t_read[rr] + kc, db offsets
  const int q_read[2] = {s_offset<D>(key_row(col), half), s_offset<D>(key_row(col), 2 + half)};
  const int t_read[2] = {s_tr_base(lane, 0), s_tr_base(lane, 1)};
  const int g = lane >> 4, jl = lane & 15;
  const int v_read = v_offset<D>(8 * (g >> 1) + (jl >> 2), 16 * (g & 1) + 4 * (jl & 3));
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  const float c = p.c;

  KA_LDS char* const tqk0 = (KA_LDS char*)qk0;
  KA_LDS char* const tqk1 = (KA_LDS char*)qk1;
  KA_LDS char* const tok0 = (KA_LDS char*)ok0;
  KA_LDS char* const tok1 = (KA_LDS char*)ok1;
  KA_LDS float* const tst0 = (KA_LDS float*)sts0;
  KA_LDS float* const tst1 = (KA_LDS float*)sts1;
  int r_cur = r_begin;
  if (n_steps > 0) copy_step(tqk0, tok0, tst0);
  wait_vmcnt<0>();
  __syncthreads();

  auto step = [&](int s, const KA_LDS char* tqk, const KA_LDS char* tok, const KA_LDS float* tst, KA_LDS char* nqk,
                  KA_LDS char* nok, KA_LDS float* nst) {
    if (s + 1 < n_steps) copy_step(nqk, nok, nst);
    const int r0 = r_cur;
    r_cur = r_cur == r_first ? r_last : r_cur - BQ;
    if (r0 < whi && r0 + BQ > wlo) {
      // dP starts from -D of this lane's result rows (half*8 .. and 16 + half*8 ..): the MFMAs leave dP - D
      f32x16 st = f32x16{}, dpt = f32x16{};
      if constexpr (DK) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f32x4 nd = *(const KA_LDS f32x4*)(tst + BQ + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) dpt[4 * u + e] = nd[e];
        }
      }
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        const bf16x8 a = *(const KA_LDS bf16x8*)(tqk + q_read[dc & 1] + (dc >> 1) * 1024);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kop[dc], st, 0, 0, 0);
        if constexpr (DK) {
          const bf16x8 b = *(const KA_LDS bf16x8*)(tok + q_read[dc & 1] + (dc >> 1) * 1024);
          dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, vop[dc], dpt, 0, 0, 0);
        }
      }
      // the step rows' log2 LSE for this lane's result registers
      f32x4 ls[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) ls[u] = *(const KA_LDS f32x4*)(tst + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
      // exponents of P; on a step some lane's window or span cuts, -inf for the rows that do not see the lane's key
      // (one uniform branch around the masking)
      float x[2 * KC * 4];
#pragma unroll
      for (int jj = 0; jj < 2 * KC * 4; ++jj) x[jj] = __builtin_fmaf(st[jj], c, -ls[jj >> 2][jj & 3]);
      if (!(r0 >= wflo && r0 + BQ <= wfhi)) {
#pragma unroll
        for (int jj = 0; jj < 2 * KC * 4; ++jj) {
          const int row = r0 + result_row(jj, half);
          const bool vis =
              ((unsigned)(row - rlo) < (unsigned)(rhi - rlo)) | ((unsigned)(row - srl) < (unsigned)(srh - srl));
          x[jj] = vis ? x[jj] : -INFINITY;
        }
      }
      bf16x8 pb[KC], dsb[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int jj = kc * 8 + t;
          const float pr = __builtin_amdgcn_exp2f(x[jj]);
          if constexpr (DV) pb[kc][t] = (__bf16)pr;
          if constexpr (DK) dsb[kc][t] = (__bf16)(pr * dpt[jj]);
        }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          bf16x4 ov[2], qv[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const int at = t_read[rr] + kc * (D / 8) * 256 + db * 1024;
            const int vt = OV ? v_read + (kc * 4 + rr) * (D / 16) * 128 + db * 256 : at;
            if constexpr (DV)
              ov[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(tok + vt)));
            if constexpr (DK)
              qv[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(tqk + at)));
          }
          if constexpr (DV) {
            const bf16x8 ao = __builtin_shufflevector(ov[0], ov[1], 0, 1, 2, 3, 4, 5, 6, 7);
            dv[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao, pb[kc], dv[db], 0, 0, 0);
          }
          if constexpr (DK) {
            const bf16x8 aq = __builtin_shufflevector(qv[0], qv[1], 0, 1, 2, 3, 4, 5, 6, 7);
            dk[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, dsb[kc], dk[db], 0, 0, 0);
          }
        }
      }
    }
    wait_vmcnt<0>();
    __syncthreads();
  };
  int s = 0;
  for (; s + 1 < n_steps; s += 2) {
    step(s, tqk0, tok0, tst0, tqk1, tok1, tst1);
    step(s + 1, tqk1, tok1, tst1, tqk0, tok0, tst0);
  }
  if (s < n_steps) step(s, tqk0, tok0, tst0, tqk1, tok1, tst1);

  if (D <= 128 && parts > 1) {  // one part of a split tile: fp32 dK (before the scale) and dV for bwd_merge_kernel
    constexpr int KT = 32 * W;
    float* base = p.partial + bwd_partial_base(slot, part, p.n_hg, kvh, KT, D) + (wave * 32 + col) * D + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        if constexpr (DK)
          *(float4*)(base + db * 32 + g4 * 8) = float4{dk[db][g4 * 4], dk[db][g4 * 4 + 1], dk[db][g4 * 4 + 2],
                                                       dk[db][g4 * 4 + 3]};
        if constexpr (DV)
          *(float4*)(base + KT * D + db * 32 + g4 * 8) = float4{dv[db][g4 * 4], dv[db][g4 * 4 + 1],
                                                                dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3]};
      }
    return;
  }
  if (valid) {  // lane (col, half) holds d = db*32 + (j/4)*8 + half*4 + j%4 of its key
    uint16_t* kq = p.dk + (int64_t)(ka + key) * p.sdk_t + (int64_t)kvh * p.sdk_h + half * 4;
    uint16_t* vq = p.dv + (int64_t)(ka + key) * p.sdv_t + (int64_t)kvh * p.sdv_h + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        if constexpr (DK) {
          u32x2 a;
          a[0] = pack_bf16(dk[db][g4 * 4] * p.scale, dk[db][g4 * 4 + 1] * p.scale);
          a[1] = pack_bf16(dk[db][g4 * 4 + 2] * p.scale, dk[db][g4 * 4 + 3] * p.scale);
          *(u32x2*)(kq + db * 32 + g4 * 8) = a;
        }
        if constexpr (DV) {
          u32x2 b;
          b[0] = pack_bf16(dv[db][g4 * 4], dv[db][g4 * 4 + 1]);
          b[1] = pack_bf16(dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3]);
          *(u32x2*)(vq + db * 32 + g4 * 8) = b;
        }
      }
  }
}

// ---- dK and dV in one launch with two waves per SIMD (head size 128): eight waves per key tile of 128 keys, as two
// groups of four (group rs = wave / 4, each wave of a group holding 32 keys) that take alternate query-row steps of
// the tile's rows (group 0 steps 0, 2, .., group 1 steps 1, 3, ..). K and V of the tile sit in LDS (the S layout,
// read as the B operands of S = Q K^T and dP = dO V^T) instead of registers, which leaves room for both fp32
// accumulators at 256 registers; at the end group 1's sums are added to group 0's through LDS in a fixed order
// (repeated calls stay bitwise equal). Four products per step instead of the five of the dV and dK launches.
template <int D>
__global__ __launch_bounds__(64 * 2 * kBwdWaves, 2) void bwd_dkdv2_kernel(BwdParams p) {
  constexpr int KW = kBwdWaves, W = 2 * KW, BQ = kBwdStep;
  constexpr int KT = 32 * KW;  // keys per tile
  constexpr int DC = D / 16, DB = D / 32, KC = BQ / 16;
  constexpr int TILE = BQ * D * 2, BLKS = TILE / 1024, INSTS = BLKS / KW;  // a step's copies per wave of a group
  constexpr int KTILE = KT * D * 2, KINSTS = KTILE / 1024 / W;              // the K (and V) tile's per wave
  static_assert(BLKS % KW == 0 && (KTILE / 1024) % W == 0, "every wave issues the same copies");
  static_assert(2 * KTILE >= KW * 32 * D * 4, "the K and V tiles hold group 1's fp32 dK (or dV) at the end");
  __shared__ __attribute__((aligned(1024))) char kt_lds[KTILE];  // K of the tile's keys (S layout)
  __shared__ __attribute__((aligned(1024))) char vt_lds[KTILE];  // V of the tile's keys (S layout)
  __shared__ __attribute__((aligned(1024))) char qk0[2][TILE];   // per group: Q (S layout), two buffers
  __shared__ __attribute__((aligned(1024))) char qk1[2][TILE];
  __shared__ __attribute__((aligned(1024))) char ok0[2][TILE];   // per group: dO (S layout)
  __shared__ __attribute__((aligned(1024))) char ok1[2][TILE];
  __shared__ __attribute__((aligned(256))) float sts0[2][2 * BQ];  // per group: log2 LSE, then -D, of the step's rows
  __shared__ __attribute__((aligned(256))) float sts1[2][2 * BQ];
  __shared__ int red[2][KW];

  if (p.plan[2] != BQ || p.plan[5] != KW) return;
  const int item = blockIdx.x / p.n_hg;
  const int kvh = blockIdx.x - item * p.n_hg;
  if (item >= p.plan[0]) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0], ktile = entry[1];
  const int part = entry[2] & 0xffff, parts = entry[2] >> 16;
  const int slot = entry[3];
  if (parts > 1 && (slot < 0 || slot + part >= p.slots)) return;  // a partial slot outside the workspace
  const int keys_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int delta = lk - lq;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kw = wave & (KW - 1), rs = wave / KW;
  const int col = lane & 31, half = lane >> 5;

  // this lane's key and the query rows that see it
  const int key = ktile * keys_per_tile + kw * 32 + col;
  const bool valid = key < lk;
  const KeyRows seen = key_rows_seen(p, key, valid, qa, lq, delta);
  const int rlo = seen.lo, rhi = seen.hi, srl = seen.sl, srh = seen.sh;
  const int wlo = seen.wlo, whi = seen.whi, wflo = seen.wflo, wfhi = seen.wfhi;
  if (lane == 0 && rs == 0) {  // group 1 holds the same keys
    red[0][kw] = wlo;
    red[1][kw] = whi;
  }
  // K and V of the tile's keys into LDS (keys past the sequence read as zeros)
  {
    const int rows = min(lk - ktile * keys_per_tile, KT);
    const uint16_t* kb = p.k + (int64_t)(ka + ktile * keys_per_tile) * p.sk_t + (int64_t)kvh * p.sk_h;
    const uint16_t* vb = p.v + (int64_t)(ka + ktile * keys_per_tile) * p.sv_t + (int64_t)kvh * p.sv_h;
#pragma unroll
    for (int r = 0; r < KINSTS; ++r) {
      int row, colm;
      s_dma_source<D>(wave * KINSTS + r, lane, &row, &colm);
      dma_16b(kb, rows * (int)p.sk_t * 2, (KA_LDS char*)kt_lds + (wave * KINSTS + r) * 1024,
              (uint32_t)(row * p.sk_t + colm) * 2u);
      dma_16b(vb, rows * (int)p.sv_t * 2, (KA_LDS char*)vt_lds + (wave * KINSTS + r) * 1024,
              (uint32_t)(row * p.sv_t + colm) * 2u);
    }
  }
  __syncthreads();
  int qlo = INT32_MAX, qhi = INT32_MIN;
#pragma unroll
  for (int w = 0; w < KW; ++w) {
    qlo = min(qlo, red[0][w]);
    qhi = max(qhi, red[1][w]);
  }
  qlo = __builtin_amdgcn_readfirstlane(qlo);
  qhi = __builtin_amdgcn_readfirstlane(qhi);
  const int r_first = qlo < qhi ? (qlo / BQ) * BQ : 0;
  const int n_rsteps = qlo < qhi ? (qhi - r_first + BQ - 1) / BQ : 0;
  const int all_steps = n_rsteps * p.group;
  const int s_begin = parts > 1 ? (int)((int64_t)part * all_steps / parts) : 0;
  const int n_steps = parts > 1 ? (int)((int64_t)(part + 1) * all_steps / parts) - s_begin : all_steps;
  const int my_steps = n_steps > rs ? (n_steps - rs + 1) / 2 : 0;  // this group's: s_begin + rs + 2 i
  const int n_iter = (n_steps + 1) / 2;

  const int gofs = rs * TILE;  // this group's buffers in the two-group arrays
  uint32_t qk_off[INSTS], ok_off[INSTS];
#pragma unroll
  for (int r = 0; r < INSTS; ++r) {
    int row, colm;
    s_dma_source<D>(kw * INSTS + r, lane, &row, &colm);
    qk_off[r] = (uint32_t)(row * p.sq_t + colm) * 2u;
    ok_off[r] = (uint32_t)(row * p.sdo_t + colm) * 2u;
  }
  // the steps in bwd_dkdv_kernel's order (rows downwards, then the group's next head), each group taking every other
  const int r_last = r_first + (n_rsteps - 1) * BQ;
  const int h0 = kvh * p.group;
  const int64_t q_step = (int64_t)BQ * p.sq_t, o_step = (int64_t)BQ * p.sdo_t;
  const int64_t q_wrap = p.sq_h + n_rsteps * q_step, o_wrap = p.sdo_h + n_rsteps * o_step;
  const int64_t st_wrap = 2 * p.total_q + (int64_t)n_rsteps * BQ;
  const int h_begin = n_rsteps > 0 ? s_begin / n_rsteps : 0;
  const int r_begin = r_last - (s_begin - h_begin * n_rsteps) * BQ;
  int c_r0 = r_begin;
  const uint16_t* c_q = p.q + (int64_t)(qa + r_begin) * p.sq_t + (int64_t)(h0 + h_begin) * p.sq_h;
  const uint16_t* c_o = p.dout + (int64_t)(qa + r_begin) * p.sdo_t + (int64_t)(h0 + h_begin) * p.sdo_h;
  const float* c_st = p.stats + (int64_t)(h0 + h_begin) * 2 * p.total_q + qa + r_begin;
  auto advance = [&]() {
    c_r0 -= BQ;
    c_q -= q_step;
    c_o -= o_step;
    c_st -= BQ;
    if (c_r0 < r_first) {  // the group's next head
      c_r0 = r_last;
      c_q += q_wrap;
      c_o += o_wrap;
      c_st += st_wrap;
    }
  };
  auto next_row = [&](int r) { return r == r_first ? r_last : r - BQ; };
  int r_cur = r_begin;
  if (rs == 1 && n_steps > 1) {
    advance();
    r_cur = next_row(r_cur);
  }
  auto copy_step = [&](KA_LDS char* tqk, KA_LDS char* tok, KA_LDS float* tst) {
    const int rows = min(lq - c_r0, BQ);
    const uint16_t* qs = c_q;
    const uint16_t* os = c_o;
    const float* src = c_st;
    advance();
    advance();
#pragma unroll
    for (int r = 0; r < INSTS; ++r) {
      const int at = gofs + (kw * INSTS + r) * 1024;
      dma_16b(qs, rows * (int)p.sq_t * 2, tqk + at, qk_off[r]);
      dma_16b(os, rows * (int)p.sdo_t * 2, tok + at, ok_off[r]);
    }
    if (kw == KW - 1) {  // 32 log2 LSE (lanes 0-31) then 32 -D (lanes 32-63), 4 B per lane; zeros past the stats
      const __amdgpu_buffer_rsrc_t rsrc =
          __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (int)(p.total_q + rows) * 4, kBufferFlags);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (KA_LDS void*)(tst + 2 * BQ * rs), 4,
                                               (uint32_t)((lane >> 5) * p.total_q + (lane & 31)) * 4u, 0, 0, 0);
    }
  };
  // the group's buffers are [rs] of the two-group arrays: its offset rides in the lanes' read offsets, so the
  // buffers' bases stay constants (a per-group base register left the reads' constant offsets unfolded: spills)
  const int q_read[2] = {gofs + s_offset<D>(key_row(col), half), gofs + s_offset<D>(key_row(col), 2 + half)};
  const int k_read[2] = {s_offset<D>(kw * 32 + col, half), s_offset<D>(kw * 32 + col, 2 + half)};
  const int t_read[2] = {gofs + s_tr_base(lane, 0), gofs + s_tr_base(lane, 1)};
  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  const float c = p.c;
  const KA_LDS char* const kt = (const KA_LDS char*)kt_lds;
  const KA_LDS char* const vt = (const KA_LDS char*)vt_lds;
  KA_LDS char* const tqk0 = (KA_LDS char*)qk0;
  KA_LDS char* const tqk1 = (KA_LDS char*)qk1;
  KA_LDS char* const tok0 = (KA_LDS char*)ok0;
  KA_LDS char* const tok1 = (KA_LDS char*)ok1;
  KA_LDS float* const tst0 = (KA_LDS float*)sts0;
  KA_LDS float* const tst1 = (KA_LDS float*)sts1;
  if (my_steps > 0) copy_step(tqk0, tok0, tst0);
  wait_vmcnt<0>();
  __syncthreads();

  auto step = [&](int i, const KA_LDS char* tqk, const KA_LDS char* tok, const KA_LDS float* tst, KA_LDS char* nqk,
                  KA_LDS char* nok, KA_LDS float* nst) {
    if (i + 1 < my_steps) copy_step(nqk, nok, nst);
    const int r0 = r_cur;
    r_cur = next_row(next_row(r_cur));
    if (i < my_steps && r0 < whi && r0 + BQ > wlo) {
      const int(&qr)[2] = q_read, (&kr)[2] = k_read, (&tr)[2] = t_read;
      // dP starts from -D of this lane's result rows: the MFMAs leave dP - D
      f32x16 st = f32x16{}, dpt;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 nd = *(const KA_LDS f32x4*)(tst + BQ + 2 * BQ * rs + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) dpt[4 * u + e] = nd[e];
      }
#pragma unroll
      for (int dc = 0; dc < DC; ++dc) {
        const int at = (dc >> 1) * 1024;
        const bf16x8 a = *(const KA_LDS bf16x8*)(tqk + qr[dc & 1] + at);
        const bf16x8 kb = *(const KA_LDS bf16x8*)(kt + kr[dc & 1] + at);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kb, st, 0, 0, 0);
        const bf16x8 b = *(const KA_LDS bf16x8*)(tok + qr[dc & 1] + at);
        const bf16x8 vb = *(const KA_LDS bf16x8*)(vt + kr[dc & 1] + at);
        dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, vb, dpt, 0, 0, 0);
      }
      f32x4 ls[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        ls[u] = *(const KA_LDS f32x4*)(tst + 2 * BQ * rs + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
      float x[2 * KC * 4];
#pragma unroll
      for (int jj = 0; jj < 2 * KC * 4; ++jj) x[jj] = __builtin_fmaf(st[jj], c, -ls[jj >> 2][jj & 3]);
      if (!(r0 >= wflo && r0 + BQ <= wfhi)) {
#pragma unroll
        for (int jj = 0; jj < 2 * KC * 4; ++jj) {
          const int row = r0 + result_row(jj, half);
          const bool vis =
              ((unsigned)(row - rlo) < (unsigned)(rhi - rlo)) | ((unsigned)(row - srl) < (unsigned)(srh - srl));
          x[jj] = vis ? x[jj] : -INFINITY;
        }
      }
      bf16x8 pb[KC], dsb[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int jj = kc * 8 + t;
          const float pr = __builtin_amdgcn_exp2f(x[jj]);
          pb[kc][t] = (__bf16)pr;
          dsb[kc][t] = (__bf16)(pr * dpt[jj]);
        }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          bf16x4 ov[2], qv[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const int at = tr[rr] + kc * (D / 8) * 256 + db * 1024;
            ov[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(tok + at)));
            qv[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(tqk + at)));
          }
          const bf16x8 ao = __builtin_shufflevector(ov[0], ov[1], 0, 1, 2, 3, 4, 5, 6, 7);
          dv[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao, pb[kc], dv[db], 0, 0, 0);
          const bf16x8 aq = __builtin_shufflevector(qv[0], qv[1], 0, 1, 2, 3, 4, 5, 6, 7);
          dk[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, dsb[kc], dk[db], 0, 0, 0);
        }
      }
    }
    wait_vmcnt<0>();
    __syncthreads();
  };
  int i = 0;
  for (; i + 1 < n_iter; i += 2) {
    step(i, tqk0, tok0, tst0, tqk1, tok1, tst1);
    step(i + 1, tqk1, tok1, tst1, tqk0, tok0, tst0);
  }
  if (i < n_iter) step(i, tqk0, tok0, tst0, tqk1, tok1, tst1);

  // group 1's sums to group 0 through the K and V tiles (no longer read): dK, then dV, 16 KiB per wave
  KA_LDS f32x4* const xs = (KA_LDS f32x4*)((kw < 2 ? (KA_LDS char*)kt_lds : (KA_LDS char*)vt_lds) + (kw & 1) * 16384) +
                           lane;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    f32x16(&acc)[DB] = which == 0 ? dk : dv;
    if (rs == 1) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          xs[(db * 4 + g4) * 64] = f32x4{acc[db][g4 * 4], acc[db][g4 * 4 + 1], acc[db][g4 * 4 + 2], acc[db][g4 * 4 + 3]};
    }
    __syncthreads();
    if (rs == 0) {
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const f32x4 y = xs[(db * 4 + g4) * 64];
          acc[db][g4 * 4] += y.x;
          acc[db][g4 * 4 + 1] += y.y;
          acc[db][g4 * 4 + 2] += y.z;
          acc[db][g4 * 4 + 3] += y.w;
        }
    }
    __syncthreads();
  }
  if (rs == 1) return;

  if (parts > 1) {  // one part of a split tile: fp32 dK (before the scale) and dV for bwd_merge_kernel
    float* base = p.partial + bwd_partial_base(slot, part, p.n_hg, kvh, KT, D) + (kw * 32 + col) * D + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        *(float4*)(base + db * 32 + g4 * 8) = float4{dk[db][g4 * 4], dk[db][g4 * 4 + 1], dk[db][g4 * 4 + 2],
                                                     dk[db][g4 * 4 + 3]};
        *(float4*)(base + KT * D + db * 32 + g4 * 8) = float4{dv[db][g4 * 4], dv[db][g4 * 4 + 1],
                                                              dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3]};
      }
    return;
  }
  if (valid) {  // lane (col, half) holds d = db*32 + (j/4)*8 + half*4 + j%4 of its key
    uint16_t* kq = p.dk + (int64_t)(ka + key) * p.sdk_t + (int64_t)kvh * p.sdk_h + half * 4;
    uint16_t* vq = p.dv + (int64_t)(ka + key) * p.sdv_t + (int64_t)kvh * p.sdv_h + half * 4;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 a;
        a[0] = pack_bf16(dk[db][g4 * 4] * p.scale, dk[db][g4 * 4 + 1] * p.scale);
        a[1] = pack_bf16(dk[db][g4 * 4 + 2] * p.scale, dk[db][g4 * 4 + 3] * p.scale);
        *(u32x2*)(kq + db * 32 + g4 * 8) = a;
        u32x2 b;
        b[0] = pack_bf16(dv[db][g4 * 4], dv[db][g4 * 4 + 1]);
        b[1] = pack_bf16(dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3]);
        *(u32x2*)(vq + db * 32 + g4 * 8) = b;
      }
  }
}

// ---- the split key tiles' merge: dK = scale * sum_p dK_p, dV = sum_p dV_p, summed in part order. Thread per (split
// tile, key/value head, key, dK or dV, 4 elements of D), in a grid-stride loop over a fixed grid.
constexpr int kBwdMergeThreads = 256;
constexpr int kBwdMergeBlocks = 1024;

template <int D>
__global__ __launch_bounds__(kBwdMergeThreads) void bwd_merge_kernel(BwdParams p) {
  constexpr int KT = 32 * kBwdWaves, C4 = D / 4;
  const int64_t units = (int64_t)p.plan[4] * p.n_hg * KT * 2 * C4;
  const int64_t stride = (int64_t)p.n_hg * KT * 2 * D;  // floats between consecutive slots
  for (int64_t idx = (int64_t)blockIdx.x * kBwdMergeThreads + threadIdx.x; idx < units;
       idx += (int64_t)gridDim.x * kBwdMergeThreads) {
    const int d = (int)(idx % C4) * 4;
    const int64_t r = idx / C4;
    const int which = (int)(r % 2);  // 0: dK, 1: dV
    const int key_l = (int)((r / 2) % KT);
    const int64_t mh = r / (2 * KT);
    const int merge = (int)(mh / p.n_hg), kvh = (int)(mh - (int64_t)merge * p.n_hg);
    const int32_t* e = p.plan + kPlanHeader + kMergeInts * merge;
    const int seg = e[0], tile = e[1], parts = e[2], slot = e[3];
    if (slot < 0 || parts < 2 || slot + parts > p.slots) continue;
    const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
    const int key = tile * p.plan[1] + key_l;
    if (key >= lk) continue;
    const float* x = p.partial + bwd_partial_base(slot, 0, p.n_hg, kvh, KT, D) + which * KT * D + key_l * D + d;
    float4 sum = *(const float4*)x;
    for (int q = 1; q < parts; ++q) {
      const float4 y = *(const float4*)(x + q * stride);
      sum.x += y.x;
      sum.y += y.y;
      sum.z += y.z;
      sum.w += y.w;
    }
    u32x2 out;
    if (which == 0) {
      out[0] = pack_bf16(sum.x * p.scale, sum.y * p.scale);
      out[1] = pack_bf16(sum.z * p.scale, sum.w * p.scale);
      *(u32x2*)(p.dk + (int64_t)(ka + key) * p.sdk_t + (int64_t)kvh * p.sdk_h + d) = out;
    } else {
      out[0] = pack_bf16(sum.x, sum.y);
      out[1] = pack_bf16(sum.z, sum.w);
      *(u32x2*)(p.dv + (int64_t)(ka + key) * p.sdv_t + (int64_t)kvh * p.sdv_h + d) = out;
    }
  }
}

// ---- launch

template <int D>
static hipError_t launch_bwd_d(const BwdParams& p, const Geometry& gq, const Geometry& gk, int32_t* plan_q,
                               int32_t* plan_k, int64_t items_q, int64_t items_k, int64_t tiles_k, int merges_k,
                               hipStream_t stream) {
  // the rows' statistics come from the dQ kernel (no separate pass below head size 512)
  hipError_t e;
  BwdParams pq = p;
  pq.plan = plan_q;
  pq.ng = gq.ng;
  pq.n_hg = gq.n_hg;
  if (items_q > 0)
    hipLaunchKernelGGL(bwd_dq_kernel<D>, dim3((unsigned)(items_q * gq.n_hg)), dim3(64 * bwd_q_waves(D)), 0, stream,
                       pq);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  BwdParams pk = p;
  pk.plan = plan_k;
  pk.ng = 1;
  pk.n_hg = gk.n_hg;
  const dim3 grid((unsigned)(items_k * gk.n_hg));
  if (items_k > 0) {
    if (D == 128 && KA_BWD2) {
      if constexpr (D == 128) hipLaunchKernelGGL(bwd_dkdv2_kernel<D>, grid, dim3(2 * 64 * kBwdWaves), 0, stream, pk);
    } else if (D == 128 && tiles_k * gk.n_hg >= kSplitKeyTiles) {
      if constexpr (D == 128) {
        hipLaunchKernelGGL((bwd_dkdv_kernel<D, 1>), grid, dim3(64 * kBwdWaves), 0, stream, pk);
        hipLaunchKernelGGL((bwd_dkdv_kernel<D, 2>), grid, dim3(64 * kBwdWaves), 0, stream, pk);
      }
    } else {
      hipLaunchKernelGGL((bwd_dkdv_kernel<D, 3>), grid, dim3(64 * kBwdWaves), 0, stream, pk);
    }
  }
  e = hipGetLastError();
  if (D > 128 || e != hipSuccess || items_k <= 0 || merges_k <= 0) return e;
  const int64_t blocks = ((int64_t)merges_k * gk.n_hg * 32 * kBwdWaves * 2 * (D / 4) + kBwdMergeThreads - 1) /
                         kBwdMergeThreads;
  hipLaunchKernelGGL(bwd_merge_kernel<D>, dim3((unsigned)(blocks < kBwdMergeBlocks ? blocks : kBwdMergeBlocks)),
                     dim3(kBwdMergeThreads), 0, stream, pk);
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdParams& p, int head_dim, const Geometry& gq, const Geometry& gk, int32_t* plan_q,
                      int32_t* plan_k, int64_t items_q, int64_t items_k, int tiles_q, int merges_q, int tiles_k,
                      int merges_k, int32_t* tile_base_q, int32_t* tile_base_k, int n_seq, hipStream_t stream) {
  // the two work lists, in one planner launch: query tiles as the forward's, key tiles from the bounds swapped (a
  // key j sees query rows i with j - right <= i + delta <= j + left: the window mirrored)
  const PlanJob jobs[2] = {{p.q_cu, p.k_cu, gq, p.left, p.right, plan_q, tiles_q, merges_q, (int)items_q, tile_base_q},
                           {p.k_cu, p.q_cu, gk, p.right, p.left, plan_k, tiles_k, merges_k, (int)items_k, tile_base_k}};
  hipError_t e = launch_plan(jobs, 2, n_seq, stream);
  if (e != hipSuccess) return e;
  switch (head_dim) {
    case 64: return launch_bwd_d<64>(p, gq, gk, plan_q, plan_k, items_q, items_k, tiles_k, merges_k, stream);
    case 128: return launch_bwd_d<128>(p, gq, gk, plan_q, plan_k, items_q, items_k, tiles_k, merges_k, stream);
    case 256: return launch_bwd_d<256>(p, gq, gk, plan_q, plan_k, items_q, items_k, tiles_k, merges_k, stream);
    case 512: {
      const int64_t vectors = p.total_q * p.heads;  // one vector per wave of the statistics pass
      const int64_t blocks = vectors < 4 * 8192 ? (vectors + 3) / 4 : 8192;
      if (blocks > 0) hipLaunchKernelGGL(bwd_stats_kernel<512>, dim3((unsigned)blocks), dim3(256), 0, stream, p);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
      return launch_bwd_pair(p, gq, gk, plan_q, plan_k, items_q, items_k, stream);
    }
    default: return hipErrorInvalidValue;
  }
}

}  // namespace karpo
