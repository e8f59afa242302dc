// The backward at head size 512 (the 31B global layers) for gfx950: the arithmetic of attn_bwd.hip, with pairs of
// waves sharing 32 query vectors (dQ kernel) or 32 keys (dK, dV kernels) as the forward's 512 tiles do. One wave
// cannot hold a 512-wide operand row and accumulator row for 32 vectors (128 + 256 registers per lane for each), so
// each wave of a pair holds half of D: half of the operands in registers and half of the gradient accumulators. A
// step's S (and dP) is a sum over all of D: each wave computes the product over its half, the pair adds the two
// partials through LDS (low half + high half, in that order in both waves, so both hold bit-equal sums), both run the
// same softmax, and each accumulates its half of the gradient.
//
// LDS holds one stage of a step's tiles (32 rows x 512 bf16 = 32 KiB per layout, three layouts for dQ and dK), so
// copies are phased within the step instead of double-buffered: the row-operand tiles of step s + 1 are copied while
// step s runs its softmax and its gradient products (they were last read before the first barrier), and the
// transposed tile of step s + 1 while step s + 1 runs its S / dP products (it was last read before the third).
// Three barriers per step.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "bwd_common.h"
#include "internal.h"
#include "karpo_attn.h"
#include "mfma_common.h"
#include "plan_common.h"

namespace karpo {

constexpr int kPairWaves = 4;  // two pairs per workgroup
constexpr int kPairStep = 32;  // keys (dQ) or query rows (dK, dV) per step

// A wave's eight 1 KiB copy blocks per tile (blocks 8w .. 8w+7 of 32) at head size 512, as byte offsets from the
// tile's first row (k_dma_source / v_dma_source of block 8w + r): the row-operand layout's advance 64 B per block;
// the transposed layout's advance 256 B per block, and four rows further from block 4 on. One or two registers per
// layout instead of eight (checked against the per-block formulas for every wave, lane and block).
__device__ __forceinline__ uint32_t k_block_base(int wave, int lane, int64_t stride) {
  int key, colm;
  k_dma_source<512>(wave * 8, lane, &key, &colm);
  return (uint32_t)(key * stride + colm) * 2u;
}
__device__ __forceinline__ uint32_t v_block_base(int wave, int lane, int64_t stride) {
  int key, colm;
  v_dma_source<512>(wave * 8, lane, &key, &colm);
  return (uint32_t)(key * stride + colm) * 2u;
}
__device__ __forceinline__ uint32_t k_block(uint32_t base, int r) { return base + (uint32_t)r * 64u; }
__device__ __forceinline__ uint32_t v_block(uint32_t base, int64_t stride, int r) {
  return base + (uint32_t)(r >> 2) * (uint32_t)(8 * stride) + (uint32_t)(r & 3) * 256u;
}

// The pair's partial S (q4 0-3) and dP (q4 4-7) of one wave: 32 floats per lane as 8 f32x4 [q4][lane].
__device__ __forceinline__ void exchange_write(KA_LDS f32x4* slot, int lane, const f32x16& a, const f32x16& b,
                                               bool with_b) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    slot[q4 * 64 + lane] = f32x4{a[4 * q4], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]};
    if (with_b) slot[(q4 + 4) * 64 + lane] = f32x4{b[4 * q4], b[4 * q4 + 1], b[4 * q4 + 2], b[4 * q4 + 3]};
  }
}
// Adds the partner's partials: low half (wave dh = 0) + high half, in that order in both waves.
__device__ __forceinline__ void exchange_add(const KA_LDS f32x4* other, int lane, int dh, f32x16& a, f32x16& b,
                                             bool with_b) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const f32x4 o = other[q4 * 64 + lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float mine = a[4 * q4 + e];
      a[4 * q4 + e] = dh ? o[e] + mine : mine + o[e];
    }
    if (with_b) {
      const f32x4 ob = other[(q4 + 4) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float mine = b[4 * q4 + e];
        b[4 * q4 + e] = dh ? ob[e] + mine : mine + ob[e];
      }
    }
  }
}

// ---- dQ: query tiles of two pairs (64 query vectors), 32 keys per step
template <int D>
__global__ __launch_bounds__(64 * kPairWaves, 1) void bwd_dq_pair_kernel(BwdParams p) {
  constexpr int W = kPairWaves, BN = kPairStep;
  constexpr int DH = D / 2, QC = DH / 16, OB = DH / 32, KC = BN / 16;
  constexpr int TILE = BN * D * 2, INSTS = TILE / 1024 / W;
  static_assert(INSTS * W * 1024 == TILE, "every wave copies the same number of 1 KiB blocks per tile");
  __shared__ __attribute__((aligned(1024))) char kk_s[TILE];  // K, row-operand layout
  __shared__ __attribute__((aligned(1024))) char kv_s[TILE];  // K, transposed-read layout
  __shared__ __attribute__((aligned(1024))) char vk_s[TILE];  // V, row-operand layout
  __shared__ __attribute__((aligned(16))) f32x4 xch[W][8 * 64];
  __shared__ int red[2][W];

  if (p.plan[2] != BN || p.plan[5] != W) return;
  const int item = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item * p.n_hg;
  if (item >= p.plan[0]) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0], tile = entry[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int kvh = (hg * p.ng) / p.group;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int dh = wave & 1;  // which half of D this wave holds

  const int vec = (wave >> 1) * 32 + col;
  const int off = vec / p.ng;
  const int pos = tile * p.plan[1] + off;
  const int head = hg * p.ng + (vec - off * p.ng);
  const bool valid = pos < lq;
  LaneBounds b = query_bounds(p, qa, lq, lk, pos);
  b.reduce_wave();
  if (lane == 0) {
    red[0][wave] = b.wlo;
    red[1][wave] = b.whi;
  }
  // this wave's half of Q and dO as B operands (elements dh*DH + c*16 + half*8 .. +8), the row's log2 LSE and D
  bf16x8 qop[QC], dop[QC];
  float lse2 = INFINITY, dsum = 0.f;
  {
    const uint16_t* qp = p.q + (int64_t)(qa + pos) * p.sq_t + (int64_t)head * p.sq_h + dh * DH + half * 8;
    const uint16_t* op = p.dout + (int64_t)(qa + pos) * p.sdo_t + (int64_t)head * p.sdo_h + dh * DH + half * 8;
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      u32x4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0};
      if (valid) {
        x = *(const u32x4*)(qp + c * 16);
        y = *(const u32x4*)(op + c * 16);
      }
      qop[c] = __builtin_bit_cast(bf16x8, x);
      dop[c] = __builtin_bit_cast(bf16x8, y);
    }
    if (valid) {
      lse2 = p.stats[((int64_t)head * 2) * p.total_q + qa + pos];
      dsum = p.stats[((int64_t)head * 2 + 1) * p.total_q + qa + pos];
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

  static_assert(D == 512 && INSTS == 8, "the block offsets below are those of head size 512");
  const uint32_t kk_off = k_block_base(wave, lane, p.sk_t), vk_off = k_block_base(wave, lane, p.sv_t);
  const uint32_t kv_off = v_block_base(wave, lane, p.sk_t);
  KA_LDS char* const kk = (KA_LDS char*)kk_s;
  KA_LDS char* const kv = (KA_LDS char*)kv_s;
  KA_LDS char* const vk = (KA_LDS char*)vk_s;
  // two copy cursors (the row-operand tiles and the transposed one are copied at different points of a step)
  const int64_t k_step = (int64_t)BN * p.sk_t, v_step = (int64_t)BN * p.sv_t;
  const uint16_t* kbase = p.k + (int64_t)kvh * p.sk_h + (int64_t)(ka + j_first) * p.sk_t;
  const uint16_t* vbase = p.v + (int64_t)kvh * p.sv_h + (int64_t)(ka + j_first) * p.sv_t;
  int r_j0 = j_first, t_j0 = j_first;
  const uint16_t* r_k = kbase;
  const uint16_t* r_v = vbase;
  const uint16_t* t_k = kbase;
  auto copy_rows = [&]() {
    const int rows = min(lk - r_j0, BN);
#pragma unroll
    for (int r = 0; r < INSTS; ++r) {
      const int at = (wave * INSTS + r) * 1024;
      dma_16b(r_k, rows * (int)p.sk_t * 2, kk + at, k_block(kk_off, r));
      dma_16b(r_v, rows * (int)p.sv_t * 2, vk + at, k_block(vk_off, r));
    }
    r_j0 += BN;
    r_k += k_step;
    r_v += v_step;
  };
  auto copy_trans = [&]() {
    const int rows = min(lk - t_j0, BN);
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      dma_16b(t_k, rows * (int)p.sk_t * 2, kv + (wave * INSTS + r) * 1024, v_block(kv_off, p.sk_t, r));
    t_j0 += BN;
    t_k += k_step;
  };
  const int k_read = k_offset<D>(key_row(col), half) + dh * QC * 512;  // this wave's chunks of the key rows
  const int g = lane >> 4, jl = lane & 15;
  const int v_read = v_offset<D>(8 * (g >> 1) + (jl >> 2), 16 * (g & 1) + 4 * (jl & 3)) + dh * OB * 256;
  f32x16 acc[OB];
#pragma unroll
  for (int db = 0; db < OB; ++db) acc[db] = f32x16{};
  const float c = p.c;
  KA_LDS f32x4* const mine = (KA_LDS f32x4*)&xch[wave][0];
  const KA_LDS f32x4* const other = (const KA_LDS f32x4*)&xch[wave ^ 1][0];

  if (n_steps > 0) {
    copy_rows();
    copy_trans();
  }
  wait_vmcnt<0>();
  __syncthreads();
  int j0 = j_first;
  for (int s = 0; s < n_steps; ++s) {
    const bool act = j0 < b.whi && j0 + BN > b.wlo;  // both waves of a pair decide alike (same vectors)
    const bool ahead = s + 1 < n_steps;
    f32x16 st = f32x16{}, dpt = f32x16{};
    if (act) {  // partial S^T = K Q^T and dP^T = V dO^T over this wave's half of D
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
        const bf16x8 a = *(const KA_LDS bf16x8*)(kk + k_read + dc * 512);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], st, 0, 0, 0);
        const bf16x8 v = *(const KA_LDS bf16x8*)(vk + k_read + dc * 512);
        dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, dop[dc], dpt, 0, 0, 0);
      }
      exchange_write(mine, lane, st, dpt, true);
    }
    __syncthreads();  // 1: the step's row tiles are read and the partials written
    if (ahead) copy_rows();
    bf16x8 dsb[KC];
    if (act) {
      exchange_add(other, lane, dh, st, dpt, true);
      float x[KC][8];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t) x[kc][t] = __builtin_fmaf(st[kc * 8 + t], c, -lse2);
      if (!(j0 >= b.wflo && j0 + BN <= b.wfhi)) {  // one uniform branch around the masking
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int key = j0 + kc * 16 + half * 8 + t;
            const bool vis = ((unsigned)(key - b.lo) < (unsigned)(b.hi - b.lo)) |
                             ((unsigned)(key - b.sl) < (unsigned)(b.sh - b.sl));
            x[kc][t] = vis ? x[kc][t] : -INFINITY;
          }
      }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t)
          dsb[kc][t] = (__bf16)(__builtin_amdgcn_exp2f(x[kc][t]) * (dpt[kc * 8 + t] - dsum));
    }
    // the transposed tile of this step (copied at the end of the last step) has landed; the next step's row tiles
    // (just issued) may still be in flight
    if (ahead) wait_vmcnt<2 * INSTS>(); else wait_vmcnt<0>();
    __syncthreads();  // 2: every wave's part of the transposed tile is in LDS; the partners' partials are read
    if (act) {  // dQ^T (this wave's half of D) += K^T dS^T, K read transposed
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 kt[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            kt[rr] = __builtin_bit_cast(
                bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (KA_LDS s16x4*)(kv + v_read + (kc * 4 + rr) * (D / 16) * 128 + db * 256)));
          const bf16x8 a = __builtin_shufflevector(kt[0], kt[1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, dsb[kc], acc[db], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();  // the next step's row tiles
    __syncthreads();  // 3: the transposed tile is read; the next row tiles are in LDS
    if (ahead) copy_trans();
    j0 += BN;
  }

  if (valid) {  // lane (col, half) holds d = dh*DH + db*32 + (j/4)*8 + half*4 + j%4
    uint16_t* dp = p.dq + (int64_t)(qa + pos) * p.sdq_t + (int64_t)head * p.sdq_h + dh * DH + half * 4;
#pragma unroll
    for (int db = 0; db < OB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 w;
        w[0] = pack_bf16(acc[db][g4 * 4] * p.scale, acc[db][g4 * 4 + 1] * p.scale);
        w[1] = pack_bf16(acc[db][g4 * 4 + 2] * p.scale, acc[db][g4 * 4 + 3] * p.scale);
        *(u32x2*)(dp + db * 32 + g4 * 8) = w;
      }
  }
}

// ---- dK (MODE 2) or dV (MODE 1): key tiles of two pairs (64 keys), 32 query rows of one head per step, each head of
// the GQA group in turn, rows from the last step down (as attn_bwd.hip's key-stationary kernel)
template <int D, int MODE>
__global__ __launch_bounds__(64 * kPairWaves, 1) void bwd_dkdv_pair_kernel(BwdParams p) {
  static_assert(MODE == 1 || MODE == 2, "dV or dK");
  constexpr bool DV = MODE == 1, DK = MODE == 2;
  constexpr int W = kPairWaves, BQ = kPairStep;
  constexpr int DH = D / 2, QC = DH / 16, OB = DH / 32, KC = BQ / 16;
  constexpr int TILE = BQ * D * 2, INSTS = TILE / 1024 / W;
  static_assert(INSTS * W * 1024 == TILE, "every wave copies the same number of 1 KiB blocks per tile");
  constexpr int ROWS = INSTS * (DK ? 2 : 1);  // this wave's row-tile copies per step (the last wave adds the stats)
  __shared__ __attribute__((aligned(1024))) char qk_s[TILE];              // Q, row-operand layout
  __shared__ __attribute__((aligned(1024))) char ot_s[DK ? TILE : 1024];  // dO, row-operand layout (dK)
  __shared__ __attribute__((aligned(1024))) char tr_s[TILE];  // Q (dK) or dO (dV), transposed-read layout
  __shared__ __attribute__((aligned(256))) float st_s[2][2 * BQ];  // log2 LSE, then D, of a step's rows (by parity)
  __shared__ __attribute__((aligned(16))) f32x4 xch[W][8 * 64];
  __shared__ int red[2][W];

  if (p.plan[2] != BQ || p.plan[5] != W) return;
  const int item = blockIdx.x / p.n_hg;
  const int kvh = blockIdx.x - item * p.n_hg;
  if (item >= p.plan[0]) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0], ktile = entry[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int dh = wave & 1;

  const int key = ktile * p.plan[1] + (wave >> 1) * 32 + col;
  const bool valid = key < lk;
  LaneBounds b = key_bounds(p, qa, lq, lk, key);
  b.reduce_wave();
  if (lane == 0) {
    red[0][wave] = b.wlo;
    red[1][wave] = b.whi;
  }
  // this wave's half of K (and of V for dK) of the lane's key as B operands
  bf16x8 kop[QC], vop[QC];
  {
    const uint16_t* kp = p.k + (int64_t)(ka + key) * p.sk_t + (int64_t)kvh * p.sk_h + dh * DH + half * 8;
    const uint16_t* vp = p.v + (int64_t)(ka + key) * p.sv_t + (int64_t)kvh * p.sv_h + dh * DH + half * 8;
#pragma unroll
    for (int dc = 0; dc < QC; ++dc) {
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
  const int n_steps = n_rsteps * p.group;

  static_assert(D == 512 && INSTS == 8, "the block offsets below are those of head size 512");
  const uint32_t qk_off = k_block_base(wave, lane, p.sq_t), ok_off = k_block_base(wave, lane, p.sdo_t);
  const uint32_t tr_off = v_block_base(wave, lane, DK ? p.sq_t : p.sdo_t);
  KA_LDS char* const qk = (KA_LDS char*)qk_s;
  KA_LDS char* const ok = (KA_LDS char*)ot_s;
  KA_LDS char* const tr = (KA_LDS char*)tr_s;
  KA_LDS float* const st0 = (KA_LDS float*)&st_s[0][0];
  // cursors over (head, row step), rows from the last step down, then the group's next head (pointer increments)
  const int r_last = r_first + (n_rsteps - 1) * BQ;
  const int h0 = kvh * p.group;
  const int64_t q_step = (int64_t)BQ * p.sq_t, o_step = (int64_t)BQ * p.sdo_t;
  const int64_t q_wrap = p.sq_h + n_rsteps * q_step, o_wrap = p.sdo_h + n_rsteps * o_step;
  const int64_t st_wrap = 2 * p.total_q + (int64_t)n_rsteps * BQ;
  const uint32_t st_off = (uint32_t)((lane >> 5) * p.total_q + (lane & 31)) * 4u;
  const uint16_t* q0 = p.q + (int64_t)(qa + r_last) * p.sq_t + (int64_t)h0 * p.sq_h;
  const uint16_t* o0 = p.dout + (int64_t)(qa + r_last) * p.sdo_t + (int64_t)h0 * p.sdo_h;
  int r_r0 = r_last, r_par = 0, t_r0 = r_last;
  const uint16_t* r_q = q0;
  const uint16_t* r_o = o0;
  const float* r_st = p.stats + (int64_t)h0 * 2 * p.total_q + qa + r_last;
  const uint16_t* t_x = DK ? q0 : o0;  // the transposed tile's source (Q for dK, dO for dV)
  const int64_t t_step = DK ? q_step : o_step, t_wrap = DK ? q_wrap : o_wrap;
  const int64_t t_stride = DK ? p.sq_t : p.sdo_t;
  auto copy_rows = [&]() {  // Q rows (dO rows for dK) and the rows' statistics (into the step parity's slot)
    const int rows = min(lq - r_r0, BQ);
#pragma unroll
    for (int r = 0; r < INSTS; ++r) {
      const int at = (wave * INSTS + r) * 1024;
      dma_16b(r_q, rows * (int)p.sq_t * 2, qk + at, k_block(qk_off, r));
      if constexpr (DK) dma_16b(r_o, rows * (int)p.sdo_t * 2, ok + at, k_block(ok_off, r));
    }
    if (wave == W - 1) {  // 32 log2 LSE (lanes 0-31) then 32 D (lanes 32-63), 4 B per lane; zeros past the stats
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)r_st, (short)0, (int)(p.total_q + rows) * 4, kBufferFlags);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (KA_LDS void*)(st0 + r_par * 2 * BQ), 4, st_off, 0, 0, 0);
    }
    r_r0 -= BQ;
    r_q -= q_step;
    r_o -= o_step;
    r_st -= BQ;
    if (r_r0 < r_first) {
      r_r0 = r_last;
      r_q += q_wrap;
      r_o += o_wrap;
      r_st += st_wrap;
    }
    r_par ^= 1;
  };
  auto copy_trans = [&]() {
    const int rows = min(lq - t_r0, BQ);
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      dma_16b(t_x, rows * (int)t_stride * 2, tr + (wave * INSTS + r) * 1024, v_block(tr_off, t_stride, r));
    t_r0 -= BQ;
    t_x -= t_step;
    if (t_r0 < r_first) {
      t_r0 = r_last;
      t_x += t_wrap;
    }
  };
  auto wait_rows = [&](bool ahead) {  // at most the row copies just issued outstanding
    if (!ahead) {
      wait_vmcnt<0>();
    } else if (wave == W - 1) {
      wait_vmcnt<ROWS + 1>();
    } else {
      wait_vmcnt<ROWS>();
    }
  };
  const int q_read = k_offset<D>(key_row(col), half) + dh * QC * 512;
  const int g = lane >> 4, jl = lane & 15;
  const int v_read = v_offset<D>(8 * (g >> 1) + (jl >> 2), 16 * (g & 1) + 4 * (jl & 3)) + dh * OB * 256;
  f32x16 acc[OB];  // dK^T or dV^T, this wave's half of D
#pragma unroll
  for (int db = 0; db < OB; ++db) acc[db] = f32x16{};
  const float c = p.c;
  KA_LDS f32x4* const mine = (KA_LDS f32x4*)&xch[wave][0];
  const KA_LDS f32x4* const other = (const KA_LDS f32x4*)&xch[wave ^ 1][0];

  if (n_steps > 0) {
    copy_rows();
    copy_trans();
  }
  wait_vmcnt<0>();
  __syncthreads();
  int r0 = r_last, par = 0;
  for (int s = 0; s < n_steps; ++s) {
    const bool act = r0 < b.whi && r0 + BQ > b.wlo;
    const bool ahead = s + 1 < n_steps;
    f32x16 st = f32x16{}, dpt = f32x16{};
    if (act) {  // partial S = Q K^T (and dP = dO V^T) over this wave's half of D
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
        const bf16x8 a = *(const KA_LDS bf16x8*)(qk + q_read + dc * 512);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kop[dc], st, 0, 0, 0);
        if constexpr (DK) {
          const bf16x8 o = *(const KA_LDS bf16x8*)(ok + q_read + dc * 512);
          dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o, vop[dc], dpt, 0, 0, 0);
        }
      }
      exchange_write(mine, lane, st, dpt, DK);
    }
    __syncthreads();  // 1: the row tiles are read and the partials written
    if (ahead) copy_rows();  // the statistics go to the other parity's slot: this step's stay readable
    bf16x8 pb[KC];
    if (act) {
      exchange_add(other, lane, dh, st, dpt, DK);
      // the rows' statistics four at a time (registers u = jj / 4 hold rows (u/2)*16 + half*8 + (u%2)*4 ..)
      const KA_LDS float* tst = st0 + par * 2 * BQ;
      float x[2 * KC * 4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 ls = *(const KA_LDS f32x4*)(tst + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[4 * u + e] = __builtin_fmaf(st[4 * u + e], c, -ls[e]);
      }
      if (!(r0 >= b.wflo && r0 + BQ <= b.wfhi)) {
#pragma unroll
        for (int jj = 0; jj < 2 * KC * 4; ++jj) {
          const int row = r0 + (jj >> 3) * 16 + half * 8 + (jj & 7);
          const bool vis = ((unsigned)(row - b.lo) < (unsigned)(b.hi - b.lo)) |
                           ((unsigned)(row - b.sl) < (unsigned)(b.sh - b.sl));
          x[jj] = vis ? x[jj] : -INFINITY;
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {  // P (dV) or dS (dK), four registers at a time
        f32x4 ds = {};
        if constexpr (DK) ds = *(const KA_LDS f32x4*)(tst + BQ + (u >> 1) * 16 + half * 8 + (u & 1) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int jj = 4 * u + e;
          const float pr = __builtin_amdgcn_exp2f(x[jj]);
          pb[jj >> 3][jj & 7] = DK ? (__bf16)(pr * (dpt[jj] - ds[e])) : (__bf16)pr;
        }
      }
    }
    wait_rows(ahead);  // this step's transposed tile has landed
    __syncthreads();   // 2: every wave's part of it is in LDS; the partners' partials are read
    if (act) {  // dV^T += dO^T P or dK^T += Q^T dS, this wave's half of D, the operand read transposed
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 xt[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            xt[rr] = __builtin_bit_cast(
                bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (KA_LDS s16x4*)(tr + v_read + (kc * 4 + rr) * (D / 16) * 128 + db * 256)));
          const bf16x8 a = __builtin_shufflevector(xt[0], xt[1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[kc], acc[db], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();
    __syncthreads();  // 3: the transposed tile is read; the next row tiles and statistics are in LDS
    if (ahead) copy_trans();
    r0 = r0 == r_first ? r_last : r0 - BQ;
    par ^= 1;
  }

  if (valid) {  // lane (col, half) holds d = dh*DH + db*32 + (j/4)*8 + half*4 + j%4 of its key
    uint16_t* gp = DK ? p.dk + (int64_t)(ka + key) * p.sdk_t + (int64_t)kvh * p.sdk_h
                      : p.dv + (int64_t)(ka + key) * p.sdv_t + (int64_t)kvh * p.sdv_h;
    gp += dh * DH + half * 4;
    const float f = DK ? p.scale : 1.f;
#pragma unroll
    for (int db = 0; db < OB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 w;
        w[0] = pack_bf16(acc[db][g4 * 4] * f, acc[db][g4 * 4 + 1] * f);
        w[1] = pack_bf16(acc[db][g4 * 4 + 2] * f, acc[db][g4 * 4 + 3] * f);
        *(u32x2*)(gp + db * 32 + g4 * 8) = w;
      }
  }
}

hipError_t launch_bwd_pair(const BwdParams& p, const Geometry& gq, const Geometry& gk, int32_t* plan_q,
                           int32_t* plan_k, int64_t items_q, int64_t items_k, hipStream_t stream) {
  constexpr int D = 512;
  BwdParams pq = p;
  pq.plan = plan_q;
  pq.ng = gq.ng;
  pq.n_hg = gq.n_hg;
  if (items_q > 0)
    hipLaunchKernelGGL(bwd_dq_pair_kernel<D>, dim3((unsigned)(items_q * gq.n_hg)), dim3(64 * kPairWaves), 0, stream,
                       pq);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  BwdParams pk = p;
  pk.plan = plan_k;
  pk.ng = 1;
  pk.n_hg = gk.n_hg;
  if (items_k > 0) {
    const dim3 grid((unsigned)(items_k * gk.n_hg));
    hipLaunchKernelGGL((bwd_dkdv_pair_kernel<D, 1>), grid, dim3(64 * kPairWaves), 0, stream, pk);
    hipLaunchKernelGGL((bwd_dkdv_pair_kernel<D, 2>), grid, dim3(64 * kPairWaves), 0, stream, pk);
  }
  return hipGetLastError();
}

}  // namespace karpo
