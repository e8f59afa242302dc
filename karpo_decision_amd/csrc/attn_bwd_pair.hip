// The backward at head size 512 (the 31B global layers) for gfx950: the arithmetic of attn_bwd.hip, with pairs of
// waves sharing 32 query vectors (dQ kernel) or 32 keys (dK / dV kernel) as the forward's 512 tiles do. One wave
// cannot hold a 512-wide operand row and accumulator row for 32 vectors (128 + 256 registers per lane for each), so
// each wave of a pair holds half of D: half of the operands in registers and half of the gradient accumulators. A
// step's S (and dP) is a sum over all of D: each wave computes the product over its half and the pair adds the two
// partials through LDS (a sum of two terms, bit-equal in either order, so the sums agree wherever they are formed).
//
// dQ kernel: both waves of a pair add the whole step's partials and run the same softmax; two barriers per step, (1)
// after the S / dP products (the partials are written), (2) at its end. K, read as rows and transposed (S layout),
// has two buffers: the next step's is copied from the step's start, a whole step ahead of its use; V, read only by
// the products before barrier 1, has one, refilled for the next step right after barrier 1.
// dK / dV kernel: both gradients in one pass over Q and dO (both read as rows and transposed, two buffers each). The
// pair splits the softmax by row block, each wave receiving only the partner's partials of its 16 rows, and the two
// swap P and dS as bf16 MFMA operands: three barriers per step (partials written, P / dS written, end).
// 32 KiB per tile and buffer.
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
// tile's first row (s_dma_source of block 8w + r): they advance 64 B per block, so one register per tile holds them
// instead of eight (checked against the per-block formula for every wave, lane and block).
__device__ __forceinline__ uint32_t s_block_base(int wave, int lane, int64_t stride) {
  int row, colm;
  s_dma_source<512>(wave * 8, lane, &row, &colm);
  return (uint32_t)(row * stride + colm) * 2u;
}
__device__ __forceinline__ uint32_t s_block(uint32_t base, int r) { return base + (uint32_t)r * 64u; }

// The pair's partial S (q4 0-3) and dP (q4 4-7) of one wave: 32 floats per lane as 8 f32x4 [q4][lane].
__device__ __forceinline__ void exchange_write(KA_LDS f32x4* slot, int lane, const f32x16& a, const f32x16& b,
                                               bool with_b) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    slot[q4 * 64 + lane] = f32x4{a[4 * q4], a[4 * q4 + 1], a[4 * q4 + 2], a[4 * q4 + 3]};
    if (with_b) slot[(q4 + 4) * 64 + lane] = f32x4{b[4 * q4], b[4 * q4 + 1], b[4 * q4 + 2], b[4 * q4 + 3]};
  }
}
// Adds the partner's partials (a sum of two terms: bit-equal in both waves, addition commutes exactly).
__device__ __forceinline__ void exchange_add(const KA_LDS f32x4* other, int lane, f32x16& a, f32x16& b, bool with_b) {
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const f32x4 o = other[q4 * 64 + lane];
#pragma unroll
    for (int e = 0; e < 4; ++e) a[4 * q4 + e] += o[e];
    if (with_b) {
      const f32x4 ob = other[(q4 + 4) * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) b[4 * q4 + e] += ob[e];
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
  __shared__ __attribute__((aligned(1024))) char k0_s[TILE];  // K of even steps (S layout: rows and transposed)
  __shared__ __attribute__((aligned(1024))) char k1_s[TILE];  // K of odd steps
  __shared__ __attribute__((aligned(1024))) char v_s[TILE];   // V (S layout, read as rows)
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
  float lse2 = INFINITY, ndsum = 0.f;  // the row's log2 LSE and -D (the statistics pass's)
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
      ndsum = p.stats[((int64_t)head * 2 + 1) * p.total_q + qa + pos];
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
  const uint32_t k_off = s_block_base(wave, lane, p.sk_t), v_off = s_block_base(wave, lane, p.sv_t);
  KA_LDS char* const k0 = (KA_LDS char*)k0_s;
  KA_LDS char* const k1 = (KA_LDS char*)k1_s;
  KA_LDS char* const vt = (KA_LDS char*)v_s;
  // copy cursors (K is copied at a step's start, V after its first barrier, both for the next step)
  const int64_t k_step = (int64_t)BN * p.sk_t, v_step = (int64_t)BN * p.sv_t;
  int ck_j0 = j_first, cv_j0 = j_first;
  const uint16_t* c_k = p.k + (int64_t)kvh * p.sk_h + (int64_t)(ka + j_first) * p.sk_t;
  const uint16_t* c_v = p.v + (int64_t)kvh * p.sv_h + (int64_t)(ka + j_first) * p.sv_t;
  auto copy_k = [&](KA_LDS char* dst) {
    const int rows = min(lk - ck_j0, BN);
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      dma_16b(c_k, rows * (int)p.sk_t * 2, dst + (wave * INSTS + r) * 1024, s_block(k_off, r));
    ck_j0 += BN;
    c_k += k_step;
  };
  auto copy_v = [&]() {
    const int rows = min(lk - cv_j0, BN);
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      dma_16b(c_v, rows * (int)p.sv_t * 2, vt + (wave * INSTS + r) * 1024, s_block(v_off, r));
    cv_j0 += BN;
    c_v += v_step;
  };
  // row reads of this wave's chunk dh*32 + 2 dc + half: k_read[dc & 1] + (dc >> 1) * 1024; transposed reads of its
  // columns dh*256 + db*32 ..: t_read[rr] + kc * (D/8) * 256 + (dh * 8 + db) * 1024
  const int k_read[2] = {s_offset<D>(key_row(col), half) + dh * 8192,
                         s_offset<D>(key_row(col), 2 + half) + dh * 8192};
  const int t_read[2] = {s_tr_base(lane, 0) + dh * 8192, s_tr_base(lane, 1) + dh * 8192};
  f32x16 acc[OB];
#pragma unroll
  for (int db = 0; db < OB; ++db) acc[db] = f32x16{};
  const float c = p.c;
  KA_LDS f32x4* const mine = (KA_LDS f32x4*)&xch[wave][0];
  const KA_LDS f32x4* const other = (const KA_LDS f32x4*)&xch[wave ^ 1][0];

  if (n_steps > 0) {
    copy_k(k0);
    copy_v();
  }
  wait_vmcnt<0>();
  __syncthreads();
  int j0 = j_first;
  auto step = [&](int s, const KA_LDS char* kt, KA_LDS char* kn) {
    const bool act = j0 < b.whi && j0 + BN > b.wlo;  // both waves of a pair decide alike (same vectors)
    const bool ahead = s + 1 < n_steps;
    if (ahead) copy_k(kn);  // its buffer was last read before the previous step's second barrier
    f32x16 st = f32x16{}, dpt = f32x16{};
    if (act) {  // partial S^T = K Q^T and dP^T = V dO^T over this wave's half of D
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
        const int at = k_read[dc & 1] + (dc >> 1) * 1024;
        const bf16x8 a = *(const KA_LDS bf16x8*)(kt + at);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], st, 0, 0, 0);
        const bf16x8 v = *(const KA_LDS bf16x8*)(vt + at);
        dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, dop[dc], dpt, 0, 0, 0);
      }
      exchange_write(mine, lane, st, dpt, true);
    }
    __syncthreads();  // 1: V is read and the partials written
    if (ahead) copy_v();
    if (act) {
      exchange_add(other, lane, st, dpt, true);
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
      bf16x8 dsb[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int t = 0; t < 8; ++t)
          dsb[kc][t] = (__bf16)(__builtin_amdgcn_exp2f(x[kc][t]) * (dpt[kc * 8 + t] + ndsum));
      // dQ^T (this wave's half of D) += K^T dS^T, K read transposed
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 kx[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            kx[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                    (KA_LDS s16x4*)(kt + t_read[rr] + kc * (D / 8) * 256 + db * 1024)));
          const bf16x8 a = __builtin_shufflevector(kx[0], kx[1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, dsb[kc], acc[db], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();  // the next step's K and V
    __syncthreads();  // 2: they are in LDS; this step's K and the partners' partials are read
    j0 += BN;
  };
  int s = 0;
  for (; s + 1 < n_steps; s += 2) {
    step(s, k0, k1);
    step(s + 1, k1, k0);
  }
  if (s < n_steps) step(s, k0, k1);

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

// ---- dK and dV: key tiles of two pairs (64 keys), 32 query rows of one head per step, each head of the GQA group in
// turn, rows from the last step down (as attn_bwd.hip's key-stationary kernel). A wave holds half of D of both
// accumulators (2 x 128 registers) and of K and V. The pair splits a step's softmax by row block: wave dh computes P
// and dS of rows dh*16 .. +16 from its own and the partner's partial S and dP of those rows, and the two
// swap their P and dS (bf16, the MFMA operands) through LDS: 24 KiB of exchange instead of 32, so Q and dO (read as
// rows and transposed) both get two buffers.
template <int D>
__global__ __launch_bounds__(64 * kPairWaves, 1) void bwd_dkdv_pair_kernel(BwdParams p) {
  constexpr int W = kPairWaves, BQ = kPairStep;
  constexpr int DH = D / 2, QC = DH / 16, OB = DH / 32, KC = BQ / 16;
  static_assert(KC == 2, "the waves of a pair take one 16-row block of a step each");
  constexpr int TILE = BQ * D * 2, INSTS = TILE / 1024 / W;
  static_assert(INSTS * W * 1024 == TILE, "every wave copies the same number of 1 KiB blocks per tile");
  __shared__ __attribute__((aligned(1024))) char q0_s[TILE];  // Q of even steps (S layout: rows for S, transposed for dK)
  __shared__ __attribute__((aligned(1024))) char q1_s[TILE];  // Q of odd steps
  __shared__ __attribute__((aligned(1024))) char o0_s[TILE];  // dO of even steps (S layout: rows for dP, transposed for dV)
  __shared__ __attribute__((aligned(1024))) char o1_s[TILE];  // dO of odd steps
  __shared__ __attribute__((aligned(256))) float st_s[2][2 * BQ];  // log2 LSE, then -D, of a step's rows (by parity)
  __shared__ __attribute__((aligned(16))) f32x4 xch[W][4 * 64];    // partial S and dP of the partner's row block
  __shared__ __attribute__((aligned(16))) bf16x8 pxch[W][2 * 64];  // P and dS of the wave's row block
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
  // this wave's half of K and V of the lane's key as B operands
  bf16x8 kop[QC], vop[QC];
  {
    const uint16_t* kp = p.k + (int64_t)(ka + key) * p.sk_t + (int64_t)kvh * p.sk_h + dh * DH + half * 8;
    const uint16_t* vp = p.v + (int64_t)(ka + key) * p.sv_t + (int64_t)kvh * p.sv_h + dh * DH + half * 8;
#pragma unroll
    for (int dc = 0; dc < QC; ++dc) {
      u32x4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0};
      if (valid) {
        x = *(const u32x4*)(kp + dc * 16);
        y = *(const u32x4*)(vp + dc * 16);
      }
      kop[dc] = __builtin_bit_cast(bf16x8, x);
      vop[dc] = __builtin_bit_cast(bf16x8, y);
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
  const uint32_t q_off = s_block_base(wave, lane, p.sq_t), o_off = s_block_base(wave, lane, p.sdo_t);
  KA_LDS char* const q0 = (KA_LDS char*)q0_s;
  KA_LDS char* const q1 = (KA_LDS char*)q1_s;
  KA_LDS char* const o0 = (KA_LDS char*)o0_s;
  KA_LDS char* const o1 = (KA_LDS char*)o1_s;
  KA_LDS float* const st0 = (KA_LDS float*)&st_s[0][0];
  KA_LDS float* const st1 = (KA_LDS float*)&st_s[1][0];
  // copy cursor over (head, row step), rows from the last step down, then the group's next head (pointer increments)
  const int r_last = r_first + (n_rsteps - 1) * BQ;
  const int h0 = kvh * p.group;
  const int64_t q_step = (int64_t)BQ * p.sq_t, o_step = (int64_t)BQ * p.sdo_t;
  const int64_t q_wrap = p.sq_h + n_rsteps * q_step, o_wrap = p.sdo_h + n_rsteps * o_step;
  const int64_t st_wrap = 2 * p.total_q + (int64_t)n_rsteps * BQ;
  const uint32_t st_off = (uint32_t)((lane >> 5) * p.total_q + (lane & 31)) * 4u;
  int c_r0 = r_last;
  const uint16_t* c_q = p.q + (int64_t)(qa + r_last) * p.sq_t + (int64_t)h0 * p.sq_h;
  const uint16_t* c_o = p.dout + (int64_t)(qa + r_last) * p.sdo_t + (int64_t)h0 * p.sdo_h;
  const float* c_st = p.stats + (int64_t)h0 * 2 * p.total_q + qa + r_last;
  // Q, dO and the rows' statistics of the cursor's step; the cursor moves on
  auto copy_step = [&](KA_LDS char* dq_, KA_LDS char* do_, KA_LDS float* dst) {
    const int rows = min(lq - c_r0, BQ);
#pragma unroll
    for (int r = 0; r < INSTS; ++r) {
      const int at = (wave * INSTS + r) * 1024;
      dma_16b(c_q, rows * (int)p.sq_t * 2, dq_ + at, s_block(q_off, r));
      dma_16b(c_o, rows * (int)p.sdo_t * 2, do_ + at, s_block(o_off, r));
    }
    if (wave == W - 1) {  // 32 log2 LSE (lanes 0-31) then 32 -D (lanes 32-63), 4 B per lane; zeros past the stats
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void*)c_st, (short)0, (int)(p.total_q + rows) * 4, kBufferFlags);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (KA_LDS void*)dst, 4, st_off, 0, 0, 0);
    }
    c_r0 -= BQ;
    c_q -= q_step;
    c_o -= o_step;
    c_st -= BQ;
    if (c_r0 < r_first) {
      c_r0 = r_last;
      c_q += q_wrap;
      c_o += o_wrap;
      c_st += st_wrap;
    }
  };
  // row reads of this wave's chunk dh*32 + 2 dc + half: row_read[dc & 1] + (dc >> 1) * 1024; transposed reads of its
  // columns dh*256 + db*32 ..: t_read[rr] + kc * (D/8) * 256 + db * 1024
  const int row_read[2] = {s_offset<D>(key_row(col), half) + dh * 8192,
                           s_offset<D>(key_row(col), 2 + half) + dh * 8192};
  const int t_read[2] = {s_tr_base(lane, 0) + dh * 8192, s_tr_base(lane, 1) + dh * 8192};
  f32x16 dk[OB], dv[OB];  // dK^T and dV^T, this wave's half of D
#pragma unroll
  for (int db = 0; db < OB; ++db) {
    dk[db] = f32x16{};
    dv[db] = f32x16{};
  }
  const float c = p.c;
  KA_LDS f32x4* const mine = (KA_LDS f32x4*)&xch[wave][0];
  const KA_LDS f32x4* const other = (const KA_LDS f32x4*)&xch[wave ^ 1][0];
  KA_LDS bf16x8* const pmine = (KA_LDS bf16x8*)&pxch[wave][0];
  const KA_LDS bf16x8* const pother = (const KA_LDS bf16x8*)&pxch[wave ^ 1][0];

  if (n_steps > 0) copy_step(q0, o0, st0);
  wait_vmcnt<0>();
  __syncthreads();
  int r0 = r_last;
  auto step = [&](int s, const KA_LDS char* qt, const KA_LDS char* ot, const KA_LDS float* tst, KA_LDS char* qn,
                  KA_LDS char* on, KA_LDS float* sn) {
    const bool act = r0 < b.whi && r0 + BQ > b.wlo;  // both waves of a pair decide alike (same keys)
    if (s + 1 < n_steps) copy_step(qn, on, sn);  // their buffers were last read before the previous step's end
    f32x16 st = f32x16{}, dpt = f32x16{};
    if (act) {  // partial S = Q K^T and dP = dO V^T over this wave's half of D
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
        const int at = row_read[dc & 1] + (dc >> 1) * 1024;
        const bf16x8 a = *(const KA_LDS bf16x8*)(qt + at);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kop[dc], st, 0, 0, 0);
        const bf16x8 o = *(const KA_LDS bf16x8*)(ot + at);
        dpt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(o, vop[dc], dpt, 0, 0, 0);
      }
      // registers 8 kc .. 8 kc + 7 hold rows kc*16 + half*8 .. +8: the partner's block (kc = 1 - dh) to it (a
      // wave-uniform branch, so each wave moves only the 16 registers it sends)
      if (dh) {
        mine[lane] = f32x4{st[0], st[1], st[2], st[3]};
        mine[64 + lane] = f32x4{st[4], st[5], st[6], st[7]};
        mine[128 + lane] = f32x4{dpt[0], dpt[1], dpt[2], dpt[3]};
        mine[192 + lane] = f32x4{dpt[4], dpt[5], dpt[6], dpt[7]};
      } else {
        mine[lane] = f32x4{st[8], st[9], st[10], st[11]};
        mine[64 + lane] = f32x4{st[12], st[13], st[14], st[15]};
        mine[128 + lane] = f32x4{dpt[8], dpt[9], dpt[10], dpt[11]};
        mine[192 + lane] = f32x4{dpt[12], dpt[13], dpt[14], dpt[15]};
      }
    }
    __syncthreads();  // 1: the partials are written
    bf16x8 pm, dm;
    if (act) {  // this wave's block: S and dP summed over D, P and dS of rows r0 + dh*16 + half*8 + t
      const f32x4 x0 = other[lane], x1 = other[64 + lane], x2 = other[128 + lane], x3 = other[192 + lane];
      float sv[8], pv[8];  // a sum of two terms (bit-equal in either order)
      if (dh) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[e] = st[8 + e] + x0[e];
          sv[4 + e] = st[12 + e] + x1[e];
          pv[e] = dpt[8 + e] + x2[e];
          pv[4 + e] = dpt[12 + e] + x3[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[e] = st[e] + x0[e];
          sv[4 + e] = st[4 + e] + x1[e];
          pv[e] = dpt[e] + x2[e];
          pv[4 + e] = dpt[4 + e] + x3[e];
        }
      }
      const KA_LDS float* rs = tst + dh * 16 + half * 8;
      const f32x4 l0 = *(const KA_LDS f32x4*)rs, l1 = *(const KA_LDS f32x4*)(rs + 4);
      const f32x4 d0 = *(const KA_LDS f32x4*)(rs + BQ), d1 = *(const KA_LDS f32x4*)(rs + BQ + 4);
      float x[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = __builtin_fmaf(sv[e], c, -l0[e]);
        x[4 + e] = __builtin_fmaf(sv[4 + e], c, -l1[e]);
      }
      if (!(r0 >= b.wflo && r0 + BQ <= b.wfhi)) {  // one uniform branch around the masking
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int row = r0 + dh * 16 + half * 8 + t;
          const bool vis = ((unsigned)(row - b.lo) < (unsigned)(b.hi - b.lo)) |
                           ((unsigned)(row - b.sl) < (unsigned)(b.sh - b.sl));
          x[t] = vis ? x[t] : -INFINITY;
        }
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float pr = __builtin_amdgcn_exp2f(x[t]);
        pm[t] = (__bf16)pr;
        dm[t] = (__bf16)(pr * (pv[t] + (t < 4 ? d0[t] : d1[t - 4])));  // d0, d1: -D
      }
      pmine[lane] = pm;
      pmine[64 + lane] = dm;
    }
    __syncthreads();  // 2: P and dS of both blocks are written
    if (act) {
      const bf16x8 po = pother[lane], dso = pother[64 + lane];
      bf16x8 pb[KC], dsb[KC];
      if (dh) {
        pb[0] = po;
        pb[1] = pm;
        dsb[0] = dso;
        dsb[1] = dm;
      } else {
        pb[0] = pm;
        pb[1] = po;
        dsb[0] = dm;
        dsb[1] = dso;
      }
      // dV^T += dO^T P and dK^T += Q^T dS, this wave's half of D, dO and Q read transposed
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 ox[2], qx[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) {
            const int at = t_read[rr] + kc * (D / 8) * 256 + db * 1024;
            ox[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(ot + at)));
            qx[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((KA_LDS s16x4*)(qt + at)));
          }
          const bf16x8 ao = __builtin_shufflevector(ox[0], ox[1], 0, 1, 2, 3, 4, 5, 6, 7);
          dv[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ao, pb[kc], dv[db], 0, 0, 0);
          const bf16x8 aq = __builtin_shufflevector(qx[0], qx[1], 0, 1, 2, 3, 4, 5, 6, 7);
          dk[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, dsb[kc], dk[db], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();  // the next step's tiles and statistics
    __syncthreads();  // 3: they are in LDS; this step's tiles and the exchanges are read
    r0 = r0 == r_first ? r_last : r0 - BQ;
  };
  int s = 0;
  for (; s + 1 < n_steps; s += 2) {
    step(s, q0, o0, st0, q1, o1, st1);
    step(s + 1, q1, o1, st1, q0, o0, st0);
  }
  if (s < n_steps) step(s, q0, o0, st0, q1, o1, st1);

  if (valid) {  // lane (col, half) holds d = dh*DH + db*32 + (j/4)*8 + half*4 + j%4 of its key
    uint16_t* kq = p.dk + (int64_t)(ka + key) * p.sdk_t + (int64_t)kvh * p.sdk_h + dh * DH + half * 4;
    uint16_t* vq = p.dv + (int64_t)(ka + key) * p.sdv_t + (int64_t)kvh * p.sdv_h + dh * DH + half * 4;
#pragma unroll
    for (int db = 0; db < OB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        u32x2 a, w;
        a[0] = pack_bf16(dk[db][g4 * 4] * p.scale, dk[db][g4 * 4 + 1] * p.scale);
        a[1] = pack_bf16(dk[db][g4 * 4 + 2] * p.scale, dk[db][g4 * 4 + 3] * p.scale);
        *(u32x2*)(kq + db * 32 + g4 * 8) = a;
        w[0] = pack_bf16(dv[db][g4 * 4], dv[db][g4 * 4 + 1]);
        w[1] = pack_bf16(dv[db][g4 * 4 + 2], dv[db][g4 * 4 + 3]);
        *(u32x2*)(vq + db * 32 + g4 * 8) = w;
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
    hipLaunchKernelGGL(bwd_dkdv_pair_kernel<D>, grid, dim3(64 * kPairWaves), 0, stream, pk);
  }
  return hipGetLastError();
}

}  // namespace karpo
