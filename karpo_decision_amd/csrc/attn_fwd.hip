// Packed varlen attention forward for gfx950 (MI355X): bf16 MFMA, fp32 online softmax, per-tile masks.
//
// Algorithm (the same arithmetic as the reference's Triton kernel, families/gemma/triton_attention.py:53-84, and the
// per-sequence SDPA path it replaces, families/gemma/packed.py:195-220): for each query, a running maximum m and sum l
// in the exp2 domain (logit * scale * log2 e), P = exp2(logit - m) rounded to bf16 for the P.V product, the output
// accumulated in fp32 and divided by l at the end. l sums the bf16-rounded P that the P.V product uses, so numerator
// and denominator carry the same weights. Masks (causal / window / image span, varlen alignment of
// tests/test_gemma_blocks.py:28-43) are evaluated per element only on key steps that cut through a wave's queries.
//
// Mapping onto a CU. One work item = one query tile x one head group, over all or one part of the tile's key steps:
//   * each wave holds 32 query vectors (position, head) of the tile in registers as MFMA B operands; the waves of a
//     workgroup share one K/V stream (wide tiles: 12 waves at head_dim 128, three per SIMD, so one wave's softmax
//     VALU work runs beside another wave's MFMAs; 8 at 256; 4 at 64; small tiles for packs of short sequences: 4
//     waves, three workgroups per CU at 128, two at 256), or a workgroup is one wave (narrow tiles for decode-shaped
//     packs, several workgroups per CU);
//   * per step, BN keys of K and V are copied global -> LDS by the DMA path (buffer_load ... lds, 16 B per lane),
//     double buffered, the next step's copy in flight while this step computes;
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: a lane owns one query column, so the row max and sum are in-lane plus
//     one v_permlane32_swap between the two half-waves;
//   * K rows are fed to the MFMA in the order that swaps bits 2 and 3 of the row index, which makes each lane's 8
//     consecutive S^T registers hold 8 consecutive keys, so the P registers are directly the B operand of
//     O^T = V^T P^T; the V^T operand comes from the V tile through ds_read_b64_tr_b16;
//   * LDS tiles are blocked so that every 16 lanes of an LDS read touch one contiguous 256-byte run (conflict-free on
//     the 64 banks): K as [16-key block][16-byte chunk][16 keys], V as [4-key group][16-wide d block][4 keys][16 d];
//     every per-step address is a lane base plus an immediate offset;
//   * the running maximum is only raised when a step's maximum exceeds it by more than a factor 2^8 (exact: the final
//     division by l cancels any common factor), so O is rescaled on few steps; at logit scales of order one (a
//     peaked softmax) it is kept exact instead (p.tau, chosen by the host);
//   * a part of a split tile stores its unnormalised fp32 O, running maximum m and sum l; merge_kernel combines the
//     parts as O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p with M = max_p m_p;
//   * at head_dim 512 one wave cannot hold 32 vectors' O (256 fp32 per lane) beside their Q operands, so a pair of
//     waves shares the vectors, each with half of D: each computes S^T over its half, the pair adds the two partials
//     through LDS (in the step's K tile, which every wave has finished reading), both run the same softmax, and each
//     multiplies P into its half of V.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"
#include "karpo_attn.h"
#include "mfma_common.h"
#include "plan_common.h"

// The file builds in two units: unit 0 (this file) holds every kernel but the head-size-128 wide and long tiles,
// which attn_fwd_128.hip builds as unit 1 under another machine-scheduler strategy; each instantiation is built in
// exactly one unit, so no kernel name is registered twice.
#ifndef KA_FWD_UNIT
#define KA_FWD_UNIT 0
#endif

namespace karpo {

// Per head size and tile shape (TileShape of plan_common.h): waves (W), keys per step (BN) and waves per SIMD the
// registers are budgeted for (OCC). Wide: D=64 4-wave workgroups, four per CU; D=128 one 12-wave workgroup per CU
// (three waves per SIMD) sharing one 32-key K/V stream (64-key steps in the long shape), 32 KiB LDS (64 KiB); D=256
// one 8-wave workgroup per CU, 64 KiB LDS; D=512 one 8-wave workgroup (four pairs, two waves per SIMD), 128 KiB LDS.
// Small: 4-wave workgroups, three per CU at D=128 (32 KiB LDS each), two at D=256 (64 KiB). Narrow: one wave per
// workgroup (a pair at D=512), 32 KiB LDS (64 KiB at D=256, 128 KiB at D=512), LDS-limited to five (two, one) per CU.
// s_barrier without the fence __syncthreads adds (which waits for every outstanding copy)
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

// The maximum of 16 scores as a tree of depth three (v_max3 nodes): the serial chain would be eight deep.
__device__ __forceinline__ float max16(const f32x16& v) {
  const float t0 = fmaxf(fmaxf(v[0], v[1]), v[2]), t1 = fmaxf(fmaxf(v[3], v[4]), v[5]);
  const float t2 = fmaxf(fmaxf(v[6], v[7]), v[8]), t3 = fmaxf(fmaxf(v[9], v[10]), v[11]);
  const float t4 = fmaxf(fmaxf(v[12], v[13]), v[14]);
  return fmaxf(fmaxf(fmaxf(t0, t1), t2), fmaxf(fmaxf(t3, t4), v[15]));
}

template <int D, int SHAPE> struct TileCfg {
  static constexpr int W = tile_waves(D, SHAPE);
  static constexpr int BN = tile_keys(D, SHAPE);
  static constexpr int QB = tile_blocks(D, SHAPE);  // 32-vector query blocks per wave
  static constexpr int OCC = SHAPE == kNarrow ? (D >= 256 ? 1 : 2)
                             : SHAPE == kDual ? 2
                             : D == 512       ? 2
                             : D == 64        ? 4
                             : D == 128       ? 3
                                              : 2;
  static constexpr bool PAIR = D == 512;  // a pair of waves per 32 query vectors, each with half of D
};

// ---- fused prologue / epilogue arithmetic (in fp32, rounding to bf16 where the reference's tensors are bf16)

__device__ __forceinline__ float sigmoid(float g) { return 1.f / (1.f + __expf(-g)); }

// The query prologue on chunks c0 .. c0 + NC of one lane's half of a query vector (x[i] holds elements
// (c0 + i) * 16 + half * 8 .. +8 of the row at `row`, pack row `qrow`): RMSNorm over the whole vector (the lane 32
// away holds the other half; in a pair, the other wave's chunks are read from the row), then rotation by halves of
// the first rope_dim elements, the partner chunk (d +- rope_dim / 2) read again from the row. Branch-free per chunk:
// every address is clamped in bounds and selects discard what does not apply, so the loads of a group of chunks
// issue together (one memory latency per group, not per chunk). Without a weight the host points q_norm_w at
// readable memory; the weight factor is wm * weight[d] + wa (WEIGHT: 1, 0; ONE_PLUS: 1, 1; PLAIN: 0, 1).
template <int DC, int RC>
__device__ __forceinline__ void query_prologue_regs(const Params& p, int64_t qrow, int half, float r, float wm,
                                                    float wa, bool norm, u32x4 (&x)[DC]);

template <int D, int NC>
__device__ __forceinline__ void query_prologue(const Params& p, const uint16_t* row, int64_t qrow, int half, int c0,
                                               u32x4 (&x)[NC]) {
  constexpr int DC = D / 16;
  constexpr int G = NC < 2 ? NC : 2;  // chunks per group of loads
  const bool norm = p.q_norm != KARPO_NORM_NONE;
  const float wm = (p.q_norm == KARPO_NORM_WEIGHT || p.q_norm == KARPO_NORM_ONE_PLUS) ? 1.f : 0.f;
  const float wa = (p.q_norm == KARPO_NORM_ONE_PLUS || p.q_norm == KARPO_NORM_PLAIN) ? 1.f : 0.f;
  const bool rot = p.rope_cos != nullptr;
  const int rd = rot ? p.rope_dim : 0, rh = rd >> 1;
  float r = 1.f;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NC; ++i)  // this wave's chunks (compile-time indices keep x in registers)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(bf16_at(x[i], e), bf16_at(x[i], e), ss);
#pragma unroll
    for (int i = 0; i < DC - NC; ++i) {  // a pair's other half, from the row
      const u32x4 v = *(const u32x4*)(row + ((c0 == 0 ? NC : 0) + i) * 16 + half * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(bf16_at(v, e), bf16_at(v, e), ss);
    }
    r = 1.f / __builtin_sqrtf(half_swap_sum(ss) * (1.f / D) + p.q_eps);
  }
  if constexpr (NC == DC && D <= 128) {  // the whole half-vector in registers (spare ones): rotate in place
    switch (rd) {
      case 0: query_prologue_regs<DC, 0>(p, qrow, half, r, wm, wa, norm, x); return;
      case 32: query_prologue_regs<DC, 2>(p, qrow, half, r, wm, wa, norm, x); return;
      case 64: if constexpr (DC >= 4) { query_prologue_regs<DC, 4>(p, qrow, half, r, wm, wa, norm, x); return; }
      break;
      case 128: if constexpr (DC >= 8) { query_prologue_regs<DC, 8>(p, qrow, half, r, wm, wa, norm, x); return; }
      break;
      case 256: if constexpr (DC >= 16) { query_prologue_regs<DC, 16>(p, qrow, half, r, wm, wa, norm, x); return; }
      break;
      default: break;  // other widths: the general path below
    }
  }
  const uint16_t* cr = rot ? p.rope_cos + qrow * p.rope_stride : nullptr;
  const uint16_t* sr = rot ? p.rope_sin + qrow * p.rope_stride : nullptr;
#pragma unroll
  for (int g0 = 0; g0 < NC; g0 += G) {
    u32x4 wv[G], pw[G], pr[G], cv[G], sv[G];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int d0 = (c0 + g0 + j) * 16 + half * 8;
      const bool in = d0 < rd;
      const int dp = in ? (d0 < rh ? d0 + rh : d0 - rh) : d0;
      wv[j] = *(const u32x4*)(p.q_norm_w + d0);
      if (rot) {
        pw[j] = *(const u32x4*)(p.q_norm_w + dp);
        pr[j] = *(const u32x4*)(row + dp);
        cv[j] = *(const u32x4*)(cr + (in ? d0 : 0));
        sv[j] = *(const u32x4*)(sr + (in ? d0 : 0));
      }
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int d0 = (c0 + g0 + j) * 16 + half * 8;
      const bool in = d0 < rd;
      const float sgn = d0 < rh ? -1.f : 1.f;
      float n[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float h = bf16_at(x[g0 + j], e);
        n[e] = norm ? round_bf16(h * r * __builtin_fmaf(wm, bf16_at(wv[j], e), wa)) : h;
      }
      if (rot) {
#pragma clang fp contract(off)  // x cos + rot(x) sin: both products rounded, then the sum, as the reference
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float hp = bf16_at(pr[j], e);
          const float np = norm ? round_bf16(hp * r * __builtin_fmaf(wm, bf16_at(pw[j], e), wa)) : hp;
          const float y = n[e] * bf16_at(cv[j], e) + sgn * np * bf16_at(sv[j], e);
          n[e] = in ? y : n[e];
        }
      }
#pragma unroll
      for (int t = 0; t < 4; ++t) x[g0 + j][t] = pack_bf16(n[2 * t], n[2 * t + 1]);
    }
  }
}

// The prologue when one lane holds all of its half-vector (no pair) and the rotated width is RC * 16 elements
// (compile time): normalise every chunk in place, then rotate chunks i < RC / 2 with i + RC / 2 in registers (the
// partner of element d is d +- RC * 8, the same position RC / 2 chunks away). No partner loads or recomputed norms.
template <int DC, int RC>
__device__ __forceinline__ void query_prologue_regs(const Params& p, int64_t qrow, int half, float r, float wm,
                                                    float wa, bool norm, u32x4 (&x)[DC]) {
  if (norm) {
#pragma unroll
    for (int i = 0; i < DC; ++i) {
      const u32x4 wv = *(const u32x4*)(p.q_norm_w + i * 16 + half * 8);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        x[i][t] = pack_bf16(bf16_at(x[i], 2 * t) * r * __builtin_fmaf(wm, bf16_at(wv, 2 * t), wa),
                            bf16_at(x[i], 2 * t + 1) * r * __builtin_fmaf(wm, bf16_at(wv, 2 * t + 1), wa));
    }
  }
  if constexpr (RC > 0) {
    static_assert(RC % 2 == 0 && RC <= DC, "rotate an even number of chunks");
    const uint16_t* cr = p.rope_cos + qrow * p.rope_stride + half * 8;
    const uint16_t* sr = p.rope_sin + qrow * p.rope_stride + half * 8;
#pragma unroll
    for (int i = 0; i < RC / 2; ++i) {
      const u32x4 c0 = *(const u32x4*)(cr + i * 16), s0 = *(const u32x4*)(sr + i * 16);
      const u32x4 c1 = *(const u32x4*)(cr + (i + RC / 2) * 16), s1 = *(const u32x4*)(sr + (i + RC / 2) * 16);
      u32x4 lo, hi;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        float a[2], b[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma clang fp contract(off)  // x cos + rot(x) sin: both products rounded, then the sum, as the reference
          const int e = 2 * t + u;
          const float n0 = bf16_at(x[i], e), n1 = bf16_at(x[i + RC / 2], e);
          a[u] = n0 * bf16_at(c0, e) - n1 * bf16_at(s0, e);
          b[u] = n1 * bf16_at(c1, e) + n0 * bf16_at(s1, e);
        }
        lo[t] = pack_bf16(a[0], a[1]);
        hi[t] = pack_bf16(b[0], b[1]);
      }
      x[i] = lo;
      x[i + RC / 2] = hi;
    }
  }
}

// Four output elements of one query: bf16(o), then the gate's bf16(bf16(o) * sigmoid(g)) when there is one.
__device__ __forceinline__ u32x2 output4(float o0, float o1, float o2, float o3, const uint16_t* gate4) {
  if (gate4 != nullptr) {
    const u32x2 g = *(const u32x2*)gate4;
    const u32x4 gv = {g[0], g[1], 0, 0};
    o0 = round_bf16(o0) * sigmoid(bf16_at(gv, 0));
    o1 = round_bf16(o1) * sigmoid(bf16_at(gv, 1));
    o2 = round_bf16(o2) * sigmoid(bf16_at(gv, 2));
    o3 = round_bf16(o3) * sigmoid(bf16_at(gv, 3));
  }
  u32x2 w;
  w[0] = pack_bf16(o0, o1);
  w[1] = pack_bf16(o2, o3);
  return w;
}

template <int D, int SHAPE, bool GATHER>
__global__ __launch_bounds__((64 * TileCfg<D, SHAPE>::W), (TileCfg<D, SHAPE>::OCC)) void attn_fwd_kernel(Params p) {
  constexpr int W = TileCfg<D, SHAPE>::W;  // waves of the workgroup
  constexpr int BN = TileCfg<D, SHAPE>::BN;
  constexpr bool PAIR = TileCfg<D, SHAPE>::PAIR;
  constexpr int QB = TileCfg<D, SHAPE>::QB;  // 32-vector query blocks per wave
  constexpr int DC = D / 16;       // 16-wide head-dim chunks of the QK^T contraction
  constexpr int DB = D / 32;       // 32-row head-dim blocks of O^T
  constexpr int QC = PAIR ? DC / 2 : DC;  // chunks of Q this wave holds (half of D in a pair)
  constexpr int OB = PAIR ? DB / 2 : DB;  // blocks of O^T this wave accumulates
  constexpr int KB = BN / 32;      // 32-key blocks of S^T
  constexpr int KC = BN / 16;      // 16-key chunks of the PV contraction
  constexpr int TILE = BN * D * 2;  // bytes of one K or V tile
  constexpr int BLKS = TILE / 1024;               // 1 KiB DMA instructions per K or V tile
  constexpr int INSTS = (BLKS + W - 1) / W;       // per wave (the last waves may issue fewer)
  static_assert(BLKS >= 1, "a tile holds at least one DMA instruction");
  static_assert(!PAIR || QB == 1, "a pair holds one query block");

  // K/V buffers: NB - 1 steps of copies in flight. One-wave tiles that stream their keys (decode-shaped packs, HBM
  // bound) keep three steps in flight in 64 KiB (two workgroups per CU: 96 KiB of copies in flight per CU instead of
  // five workgroups' 80; the markers layer's attention kernel 115.9 -> 109.6 us, planned two per CU either way); the
  // others two buffers. The deeper ring counts its own copies to wait for one step's, so it is only built where every
  // copy instruction is issued unconditionally (one wave, no row table).
  constexpr int NB = kv_buffers(D, SHAPE, GATHER);
  static_assert(NB == 2 || (W == 1 && BLKS == INSTS), "the ring waits on a fixed count of its wave's copies");
  constexpr int CPS = 2 * INSTS;  // copy instructions per step of a one-wave tile (K and V)
  static_assert(NB == 2 || (NB - 2) * CPS <= 63, "vmcnt counts at most 63 outstanding operations");
  // separate arrays per buffer: the compiler then sees that a step's copy never writes the tiles it reads
  __shared__ __attribute__((aligned(1024))) char k_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds2[NB > 2 ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char v_lds2[NB > 2 ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char k_lds3[NB > 3 ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char v_lds3[NB > 3 ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char k_lds4[NB > 4 ? TILE : 16];
  __shared__ __attribute__((aligned(1024))) char v_lds4[NB > 4 ? TILE : 16];
  // a pair's exchange of partial S^T: 16 floats per lane and wave (32 KiB for the 8-wave tile, so the tile's LDS is
  // exactly 160 KiB)
  __shared__ __attribute__((aligned(16))) f32x4 xch[PAIR ? W : 1][PAIR ? 4 * 64 : 1];
  // the workgroup's key envelope (unused, so not allocated, by one-wave workgroups; in the exchange slots for pairs,
  // read by every wave before the barrier that precedes the first exchange)
  __shared__ int red_s[PAIR ? 1 : 2][PAIR ? 1 : W];
  int(*red)[W];
  if constexpr (PAIR)
    red = (int(*)[W])&xch[0][0];
  else
    red = red_s;

  // a plan made for another tile shape is not run (its rows stay unwritten)
  if (p.plan[2] != BN || p.plan[5] != W) return;
  const int n_items = p.plan[0];
  const int item = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item * p.n_hg;
  if (item >= n_items) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0];
  const int tile = entry[1];
  const int part = entry[2] & 0xffff, parts = entry[2] >> 16;
  const int slot = entry[3];
  if (parts > 1 && (slot < 0 || slot + part >= p.slots)) return;  // a partial slot outside the workspace
  const int rows_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int kvh = (hg * p.ng) / p.group;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int dh = PAIR ? (wave & 1) : 0;  // in a pair: which half of D this wave holds

  // ---- this lane's query vectors (one per block): position, head, visible key ranges. With two blocks per wave the
  // registers hold the operands and accumulators of both: the key ranges wait in LDS for the masked steps, and the
  // vectors' rows are worked out again for the store from a copy of the lane index the compiler cannot see through
  // (so it keeps no set-up value live across the key loop).
  constexpr bool KEYS_IN_LDS = QB > 1;
  __shared__ int4 keys_lds[KEYS_IN_LDS ? QB * W * 64 : 1];
  int vec[QB], pos[QB], head[QB];
  bool valid[QB];
  int lo[QB], hi[QB], sl[QB], sh[QB];
  auto lane_query = [&](int b, int column) {
    vec[b] = lane_vector(wave, b, column, PAIR, QB);
    const int off = vec[b] / p.ng;
    pos[b] = tile * rows_per_tile + off;
    head[b] = hg * p.ng + (vec[b] - off * p.ng);
    valid[b] = pos[b] < lq;
  };
  int wlo = INT32_MAX, whi = INT32_MIN, wflo = INT32_MIN, wfhi = INT32_MAX;
#pragma unroll
  for (int b = 0; b < QB; ++b) {
    lane_query(b, col);
    lo[b] = hi[b] = sl[b] = sh[b] = 0;
    if (valid[b]) {
      const LaneKeys lk_ = lane_keys(pos[b], qa, lq, lk, p.left, p.right, p.spans, p.n_spans);
      lo[b] = lk_.lo;
      hi[b] = lk_.hi;
      sl[b] = lk_.sl;
      sh[b] = lk_.sh;
      wflo = max(wflo, lo[b]);
      wfhi = min(wfhi, hi[b]);
      if (lo[b] < hi[b]) {
        wlo = min(wlo, lo[b]);
        whi = max(whi, hi[b]);
      }
      if (sl[b] < sh[b]) {
        wlo = min(wlo, sl[b]);
        whi = max(whi, sh[b]);
      }
    }
    if constexpr (KEYS_IN_LDS) keys_lds[b * W * 64 + tid] = int4{lo[b], hi[b], sl[b], sh[b]};
  }
  wlo = __builtin_amdgcn_readfirstlane(wave_min(wlo));
  whi = __builtin_amdgcn_readfirstlane(wave_max(whi));
  wflo = __builtin_amdgcn_readfirstlane(wave_max(wflo));
  wfhi = __builtin_amdgcn_readfirstlane(wave_min(wfhi));
  if constexpr (W > 1) {
    if (lane == 0) {
      red[0][wave] = wlo;
      red[1][wave] = whi;
    }
  }

  // this wave's chunks of its queries (a pair's second wave: the second half of D), with the prologue applied;
  // loaded under the first K/V copy's latency (a pair loads them before: its norm also streams the other half's
  // chunks)
  bf16x8 qop[QB][QC];
  auto load_q = [&]() {
#pragma unroll
    for (int b = 0; b < QB; ++b) {
      const uint16_t* qrow = p.q + (int64_t)(qa + pos[b]) * p.sq_t + (int64_t)head[b] * p.sq_h;
      u32x4 x[QC];
#pragma unroll
      for (int i = 0; i < QC; ++i) {
        x[i] = u32x4{0, 0, 0, 0};
        if (valid[b]) x[i] = *(const u32x4*)(qrow + half * 8 + (dh * QC + i) * 16);
      }
      if (p.q_norm != KARPO_NORM_NONE || p.rope_cos != nullptr) {
        if (valid[b]) query_prologue<D, QC>(p, qrow, (int64_t)(qa + pos[b]), half, dh * QC, x);
        if (p.q_out != nullptr && valid[b] && part == 0) {  // the attention's query, once per (row, head)
          uint16_t* qo = p.q_out + (int64_t)(qa + pos[b]) * p.sqo_t + (int64_t)head[b] * p.sqo_h + half * 8;
#pragma unroll
          for (int i = 0; i < QC; ++i) *(u32x4*)(qo + (dh * QC + i) * 16) = x[i];
        }
      }
#pragma unroll
      for (int i = 0; i < QC; ++i) qop[b][i] = __builtin_bit_cast(bf16x8, x[i] ^ p.qsign);
    }
  };
  if constexpr (PAIR) load_q();
  int klo = wlo, khi = whi;
  if constexpr (W > 1) {
    __syncthreads();
#pragma unroll
    for (int w = 0; w < W; ++w) {
      klo = min(klo, red[0][w]);
      khi = max(khi, red[1][w]);
    }
    klo = __builtin_amdgcn_readfirstlane(klo);
    khi = __builtin_amdgcn_readfirstlane(khi);
  }
  int j_first, n_steps;  // the envelope's steps, or this part's share of them (possibly none)
  part_steps(klo, khi, BN, part, parts, &j_first, &n_steps);

  // ---- DMA: per instruction a lane's byte offset inside the step's rows (fixed for the kernel). Each step's rows
  // are one buffer resource starting at the step's first key row, sized to the rows that exist: reads past the
  // sequence's last key return zeros, so no per-step address arithmetic runs on the VALU.
  // Gathered keys (GATHER): a lane's row comes from the row table; the table entries of the step a copy issues are
  // loaded one step ahead (the end-of-step wait covers them), rows past the sequence or outside [0, total_k) get an
  // offset past the buffer and read as zeros.
  const uint16_t* kbase = p.k + (int64_t)kvh * p.sk_h + (GATHER ? 0 : (int64_t)ka * p.sk_t);
  const uint16_t* vbase = p.v + (int64_t)kvh * p.sv_h + (GATHER ? 0 : (int64_t)ka * p.sv_t);
  constexpr int GI = GATHER ? INSTS : 1;
  uint32_t k_voff[INSTS], v_voff[INSTS];
  int k_key[GI], v_key[GI], k_row[GI], v_row[GI];
#pragma unroll
  for (int r = 0; r < INSTS; ++r) {
    int key, colm;
    k_dma_source<D>(wave * INSTS + r, lane, &key, &colm);
    if constexpr (GATHER) {
      k_key[r] = key;
      k_voff[r] = (uint32_t)colm * 2u;
    } else {
      k_voff[r] = (uint32_t)(key * p.sk_t + colm) * 2u;
    }
    v_dma_source<D>(wave * INSTS + r, lane, &key, &colm);
    if constexpr (GATHER) {
      v_key[r] = key;
      v_voff[r] = (uint32_t)colm * 2u;
    } else {
      v_voff[r] = (uint32_t)(key * p.sv_t + colm) * 2u;
    }
  }
  auto fetch_rows = [&](int j0) {  // GATHER: the table rows of step j0's copy
    if constexpr (GATHER) {
#pragma unroll
      for (int r = 0; r < INSTS; ++r) {
        k_row[r] = j0 + k_key[r] < lk ? p.k_rows[ka + j0 + k_key[r]] : -1;
        v_row[r] = j0 + v_key[r] < lk ? p.k_rows[ka + j0 + v_key[r]] : -1;
      }
    }
  };
  auto gathered = [&](int row, uint32_t colb, int64_t stride, uint32_t bytes) -> uint32_t {
    return gather_offset(row, p.total_k, (uint32_t)(stride * 2), colb, bytes);
  };
  // copies run in step order: the step's first key row pointers advance by increments (no per-step multiply)
  const uint16_t* c_k = kbase + (GATHER ? 0 : (int64_t)j_first * p.sk_t);
  const uint16_t* c_v = vbase + (GATHER ? 0 : (int64_t)j_first * p.sv_t);
  const int64_t k_step = GATHER ? 0 : (int64_t)BN * p.sk_t, v_step = GATHER ? 0 : (int64_t)BN * p.sv_t;
  // one-wave tiles (decode-shaped packs) stream their sequence's keys once: on the markers layer the attention kernel
  // 109.5 -> 108.5 us and its merge 5.6 -> 5.0 us (the partials stay in L2)
  constexpr int AUX = SHAPE == kNarrow && !GATHER ? kCopyStream : 0;
  auto copy_k = [&](int j0, KA_LDS char* kt) {
    const int rows = min(lk - j0, BN);
    const uint16_t* ks = c_k;
    c_k += k_step;
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      if (BLKS % W == 0 || wave * INSTS + r < BLKS) {
        if constexpr (GATHER)
          dma_16b(ks, (int)p.k_bytes, kt + (wave * INSTS + r) * 1024, gathered(k_row[r], k_voff[r], p.sk_t, p.k_bytes));
        else
          dma_16b<AUX>(ks, rows * (int)p.sk_t * 2, kt + (wave * INSTS + r) * 1024, k_voff[r]);
      }
  };
  auto copy_v = [&](int j0, KA_LDS char* vt) {
    const int rows = min(lk - j0, BN);
    const uint16_t* vs = c_v;
    c_v += v_step;
#pragma unroll
    for (int r = 0; r < INSTS; ++r)
      if (BLKS % W == 0 || wave * INSTS + r < BLKS) {
        if constexpr (GATHER)
          dma_16b(vs, (int)p.v_bytes, vt + (wave * INSTS + r) * 1024, gathered(v_row[r], v_voff[r], p.sv_t, p.v_bytes));
        else
          dma_16b<AUX>(vs, rows * (int)p.sv_t * 2, vt + (wave * INSTS + r) * 1024, v_voff[r]);
      }
  };
  auto copy_step = [&](int j0, KA_LDS char* kt, KA_LDS char* vt) {
    copy_k(j0, kt);
    copy_v(j0, vt);
  };

  // ---- LDS read bases (per lane) for the MFMA operands (a pair's second wave starts at the second half of D)
  const int k_read = k_offset<D>(key_row(col), half) + dh * QC * 512;  // + kb * (2 * D/8 * 256) + dc * 512
  const int g = lane >> 4, jl = lane & 15;
  const int v_read =
      v_offset<D>(8 * (g >> 1) + (jl >> 2), 16 * (g & 1) + 4 * (jl & 3)) + dh * OB * 256;  // + kc, rr, db offsets

  f32x16 acc[QB][OB];
#pragma unroll
  for (int b = 0; b < QB; ++b)
#pragma unroll
    for (int db = 0; db < OB; ++db) acc[b][db] = f32x16{};
  // the running maximum starts finite: before the first visible key exp2(logit - m) is exp2(-inf) = 0 all the same,
  // and a rescale from it multiplies zeros (a part that sees no key stores m = -1e30 and l = 0: the merge gives it
  // weight 1 over zero sums, so an empty row still comes out 0 with LSE -inf)
  float m[QB], l[QB];
#pragma unroll
  for (int b = 0; b < QB; ++b) {
    m[b] = -1e30f;
    l[b] = 0.f;
  }
  const float c = p.c;
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};

  // buffer i of the ring (i a constant once the loops below unroll; a two-buffer kernel never names the others, so
  // they are not allocated)
  auto kbuf = [&](int i) -> KA_LDS char* {
    if constexpr (NB > 2) {
      switch (i) {
        case 2: return (KA_LDS char*)k_lds2;
        case 3: return (KA_LDS char*)k_lds3;
        case 4: return (KA_LDS char*)k_lds4;
        default: break;
      }
    }
    return i == 0 ? (KA_LDS char*)k_lds0 : (KA_LDS char*)k_lds1;
  };
  auto vbuf = [&](int i) -> KA_LDS char* {
    if constexpr (NB > 2) {
      switch (i) {
        case 2: return (KA_LDS char*)v_lds2;
        case 3: return (KA_LDS char*)v_lds3;
        case 4: return (KA_LDS char*)v_lds4;
        default: break;
      }
    }
    return i == 0 ? (KA_LDS char*)v_lds0 : (KA_LDS char*)v_lds1;
  };
  // waits until the copies of step s + 1 have landed, given that the ones of steps up to s + NB - 1 were issued
  // after them (the ring: exactly CPS instructions per issued step)
  auto wait_next = [&](int s) {
    if constexpr (NB == 2) {
      wait_vmcnt<0>();
    } else {
      const int later = min(NB - 2, n_steps - 2 - s);  // steps issued after step s + 1
      if (later >= 3) wait_vmcnt<3 * CPS>();
      else if (later == 2) wait_vmcnt<2 * CPS>();
      else if (later == 1) wait_vmcnt<CPS>();
      else wait_vmcnt<0>();
    }
  };
  KA_LDS char* const kt0 = (KA_LDS char*)k_lds0;
  KA_LDS char* const kt1 = (KA_LDS char*)k_lds1;
  KA_LDS char* const vt0 = (KA_LDS char*)v_lds0;
  KA_LDS char* const vt1 = (KA_LDS char*)v_lds1;
  // prologue: the first NB - 1 steps in flight (and the next one's table rows), wait for the first
  if constexpr (NB == 2) {
    if (n_steps > 0) {
      fetch_rows(j_first);
      copy_step(j_first, kt0, vt0);
      if (n_steps > 1) fetch_rows(j_first + BN);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NB - 1; ++i)
      if (i < n_steps) copy_step(j_first + i * BN, kbuf(i), vbuf(i));
  }
  if constexpr (!PAIR) load_q();
  wait_next(-1);
  __syncthreads();

  // S^T of a step's keys (st zeroed by the caller), K from the tile kt
  auto qk_products = [&](const KA_LDS char* kt, f32x16 (&st)[QB][KB]) {
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const bf16x8 a = *(const KA_LDS bf16x8*)(kt + k_read + kb * (2 * (D / 8) * 256) + dc * 512);
#pragma unroll
          for (int b = 0; b < QB; ++b)  // one K operand read feeds every query block
            st[b][kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[b][dc], st[b][kb], 0, 0, 0);
        }
      }
  };
  // the step's masks, softmax and P.V products (V from the tile vt) on its S^T
  auto softmax_pv = [&](int j0, const KA_LDS char* vt, f32x16 (&st)[QB][KB]) {
      bf16x8 pb[QB][KC];
      if (!(j0 >= wflo && j0 + BN <= wfhi)) {  // some query of this wave does not see every key of the step
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          int klo_ = lo[b], khi_ = hi[b], ksl = sl[b], ksh = sh[b];
          if constexpr (KEYS_IN_LDS) {
            const int4 kk = keys_lds[b * W * 64 + tid];
            klo_ = kk.x;
            khi_ = kk.y;
            ksl = kk.z;
            ksh = kk.w;
          }
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
              const int key = j0 + kb * 32 + (jj >> 3) * 16 + half * 8 + (jj & 7);
              const bool vis = ((unsigned)(key - klo_) < (unsigned)(khi_ - klo_)) |
                               ((unsigned)(key - ksl) < (unsigned)(ksh - ksl));
              st[b][kb][jj] = vis ? st[b][kb][jj] : -INFINITY;
            }
        }
      }
      // each block's row maximum (with two blocks a tree of depth three per 16 scores, the blocks side by side: 32k
      // layer 7.06 -> 6.94 ms; the one-block tiles keep the chain, which measured as fast or faster there), then one
      // uniform branch for the rare steps where some block raises its running maximum
      float mt[QB];
      bool need[QB], any = false;
#pragma unroll
      for (int b = 0; b < QB; ++b) {
        float mx = -INFINITY;
        if constexpr (QB > 1) {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb) mx = fmaxf(mx, max16(st[b][kb]));
        } else {
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) mx = fmaxf(mx, st[b][kb][jj]);
        }
        mt[b] = half_swap_max(mx) * c;
        need[b] = mt[b] > m[b] + p.tau;
        any |= need[b];
      }
      if (QB == 1 || __builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
        for (int b = 0; b < QB; ++b) {
          if (__builtin_amdgcn_ballot_w64(need[b])) {  // raise the running maximum (rare after the first steps)
            const float mn = need[b] ? mt[b] : m[b];
            const float alpha = need[b] ? __builtin_amdgcn_exp2f(m[b] - mn) : 1.f;  // from the start value: 0
            m[b] = mn;
            l[b] *= alpha;
#pragma unroll
            for (int db = 0; db < OB; ++db) acc[b][db] *= alpha;
          }
        }
      }
#pragma unroll
      for (int b = 0; b < QB; ++b) {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
          for (int t = 0; t < 8; t += 2) {
            const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[b][kc >> 1][(kc & 1) * 8 + t], c, -m[b]));
            const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[b][kc >> 1][(kc & 1) * 8 + t + 1], c, -m[b]));
            const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
            pb[b][kc][t] = pr[0];
            pb[b][kc][t + 1] = pr[1];
            l[b] = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, l[b], false);  // l sums the bf16 P the product uses
          }
        }
      }
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 pv[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            pv[rr] = __builtin_bit_cast(
                bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (KA_LDS s16x4*)(vt + v_read + (kc * 4 + rr) * (D / 16) * 128 + db * 256)));
          const bf16x8 a = __builtin_shufflevector(pv[0], pv[1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
          for (int b = 0; b < QB; ++b)  // one V operand read feeds every query block
            acc[b][db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[b][kc], acc[b][db], 0, 0, 0);
        }
      }
  };

  // step s: copy step s + NB - 1 into (kn, vn) while computing on (kt, vt); then wait for step s + 1's copy
  auto step = [&](int s, const KA_LDS char* kt, const KA_LDS char* vt, KA_LDS char* kn, KA_LDS char* vn) {
    const int j0 = j_first + s * BN;
    if (s + NB - 1 < n_steps) copy_step(j0 + (NB - 1) * BN, kn, vn);
    if (GATHER && s + NB < n_steps) fetch_rows(j0 + NB * BN);
    const bool active = j0 < whi && j0 + BN > wlo;  // wave-uniform: some query of this wave sees a key of the step
    if (PAIR || active) {  // a pair enters together (its barriers), each wave computes only when active
    f32x16 st[QB][KB];
#pragma unroll
    for (int b = 0; b < QB; ++b)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) st[b][kb] = f32x16{};
    if (active) qk_products(kt, st);
    if constexpr (PAIR) {
      // the pair adds its two partial S^T through LDS: each wave's 16 floats per lane go to its 4 KiB exchange slot
      // (read by the partner after the barrier; written again only after the step's end barrier)
      static_assert(KB == 1, "one 32-key block per step");
      KA_LDS f32x4* slot = (KA_LDS f32x4*)&xch[wave][0] + lane;
      const KA_LDS f32x4* other = (const KA_LDS f32x4*)&xch[wave ^ 1][0] + lane;
      if (active) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          slot[q4 * 64] = f32x4{st[0][0][4 * q4], st[0][0][4 * q4 + 1], st[0][0][4 * q4 + 2], st[0][0][4 * q4 + 3]};
      }
      __syncthreads();
      if (active) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {  // a sum of two terms: equal in both waves (addition commutes exactly)
          const f32x4 o = other[q4 * 64];
          st[0][0][4 * q4] += o.x;
          st[0][0][4 * q4 + 1] += o.y;
          st[0][0][4 * q4 + 2] += o.z;
          st[0][0][4 * q4 + 3] += o.w;
        }
      }
    }
    if (active) softmax_pv(j0, vt, st);
    }
    wait_next(s);
    __syncthreads();
  };
  int s = 0;
  if constexpr (NB == 2) {
    for (; s + 1 < n_steps; s += 2) {
      step(s, kt0, vt0, kt1, vt1);
      step(s + 1, kt1, vt1, kt0, vt0);
    }
    if (s < n_steps) step(s, kt0, vt0, kt1, vt1);
  } else {  // the ring unrolled NB times: step s computes on buffer s % NB and copies into (s + NB - 1) % NB
    for (; s + NB - 1 < n_steps; s += NB) {
#pragma unroll
      for (int i = 0; i < NB; ++i)
        step(s + i, kbuf(i), vbuf(i), kbuf((i + NB - 1) % NB), vbuf((i + NB - 1) % NB));
    }
#pragma unroll
    for (int i = 0; i < NB - 1; ++i)
      if (s + i < n_steps) step(s + i, kbuf(i), vbuf(i), kbuf((i + NB - 1) % NB), vbuf((i + NB - 1) % NB));
  }

  // ---- store: lane (col, half) holds d = db*32 + (j/4)*8 + half*4 + j%4 of its query vectors
  if constexpr (QB > 1) {
    int column = col;
    asm volatile("" : "+v"(column));  // opaque: the rows below are recomputed, not kept from the set-up
#pragma unroll
    for (int b = 0; b < QB; ++b) lane_query(b, column);
  }
#pragma unroll
  for (int b = 0; b < QB; ++b) {
    const float lt = half_swap_sum(l[b]);
    if (parts > 1) {  // one part of a split tile: unnormalised fp32 O, m and l for merge_kernel
      constexpr int V = tile_vectors(D, SHAPE);
      float* base = p.partial + partial_base(slot, part, p.n_hg, hg, V, D);
      float* op = base + (int64_t)vec[b] * D + dh * (D / 2) + half * 4;
#pragma unroll
      for (int db = 0; db < OB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          float4 x = {acc[b][db][g4 * 4], acc[b][db][g4 * 4 + 1], acc[b][db][g4 * 4 + 2], acc[b][db][g4 * 4 + 3]};
          *(float4*)(op + db * 32 + g4 * 8) = x;
        }
      if (half == 0 && dh == 0) {
        base[V * D + vec[b]] = m[b];
        base[V * D + V + vec[b]] = lt;
      }
      continue;
    }
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (valid[b] && p.lse != nullptr && half == 0 && dh == 0)  // ln(2^m * l): m is in the log2 domain of scale * q.k
      p.lse[(int64_t)head[b] * p.lse_stride + qa + pos[b]] =
          lt > 0.f ? (m[b] + __log2f(lt)) * 0.69314718055994531f : -INFINITY;
    if (valid[b]) {
      uint16_t* op = p.o + (int64_t)(qa + pos[b]) * p.so_t + (int64_t)head[b] * p.so_h + dh * (D / 2) + half * 4;
      const uint16_t* gp = p.gate != nullptr ? p.gate + (int64_t)(qa + pos[b]) * p.sg_t + (int64_t)head[b] * p.sg_h +
                                                   dh * (D / 2) + half * 4
                                             : nullptr;
#pragma unroll
      for (int db = 0; db < OB; ++db) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          *(u32x2*)(op + db * 32 + g4 * 8) =
              output4(acc[b][db][g4 * 4] * inv, acc[b][db][g4 * 4 + 1] * inv, acc[b][db][g4 * 4 + 2] * inv,
                      acc[b][db][g4 * 4 + 3] * inv, gp != nullptr ? gp + db * 32 + g4 * 8 : nullptr);
        }
      }
    }
  }
}

#if KA_FWD_UNIT == 0
// ---- the head-size-512 wide tile as a ping-pong (calls without a row table)
//
// attn_fwd_kernel's pair tile runs its eight waves in lockstep: every SIMD does its two waves' QK^T halves together,
// then both softmaxes, then both P.V halves, two barriers per step. Here the four pairs form two groups that
// alternate, phase by phase, between an MFMA phase (this wave's half of QK^T of step s and of P.V of step s - 1, then
// its partial scores to its exchange slot) and a VALU phase (the partner's partial added, the step's softmax), so one
// group's MFMAs run beside the other's softmax. Pairs 0, 1 (waves 0-3) form group A, pairs 2, 3 group B: the waves of
// a workgroup are dealt to the SIMDs in turn, so waves w and w + 4 share one, one of each group (a different deal
// would cost speed, not correctness: every wave meets the same barriers, and a pair is always in one group). T(s)
// holds K(s) and V(s - 1) (both are read in iteration s); it is copied during iteration s - 1 into the buffer T(s - 2)
// left and waited for at that iteration's end. The phase barriers are bare s_barrier instructions (each wave waits for
// its own LDS work and copies explicitly), so the copies stay in flight across the middle barrier. The arithmetic is
// attn_fwd_kernel's but for the order in which l adds up a step's 16 P values (two partial sums).


__global__ __launch_bounds__(512, 2) void attn_fwd_pair_pp_kernel(Params p) {
  constexpr int D = 512, W = 8, BN = 32;
  constexpr int DC = D / 16, DB = D / 32;
  constexpr int QC = DC / 2, OB = DB / 2;  // this wave's half of D
  constexpr int KC = BN / 16;
  constexpr int TILE = BN * D * 2;        // 32 KiB
  constexpr int BLKS = TILE / 1024;       // 32
  constexpr int INSTS = BLKS / W;         // 4 per wave and tile
  static_assert(BLKS % W == 0, "every wave copies the same number of blocks");
  __shared__ __attribute__((aligned(1024))) char k_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char k_lds1[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds0[TILE];
  __shared__ __attribute__((aligned(1024))) char v_lds1[TILE];
  __shared__ __attribute__((aligned(16))) f32x4 xch[W][4 * 64];  // a wave's 16 partial scores per lane
  int(*red)[W] = (int(*)[W])&xch[0][0];                           // the envelope (read before the first exchange)
  auto kbuf = [&](int i) -> KA_LDS char* { return i == 0 ? (KA_LDS char*)k_lds0 : (KA_LDS char*)k_lds1; };
  auto vbuf = [&](int i) -> KA_LDS char* { return i == 0 ? (KA_LDS char*)v_lds0 : (KA_LDS char*)v_lds1; };

  if (p.plan[2] != BN || p.plan[5] != W) return;
  const int n_items = p.plan[0];
  const int item = blockIdx.x / p.n_hg;
  const int hg = blockIdx.x - item * p.n_hg;
  if (item >= n_items) return;
  const int32_t* entry = p.plan + p.plan[6] + kItemInts * item;
  const int seg = entry[0];
  const int tile = entry[1];
  const int part = entry[2] & 0xffff, parts = entry[2] >> 16;
  const int slot = entry[3];
  if (parts > 1 && (slot < 0 || slot + part >= p.slots)) return;
  const int rows_per_tile = p.plan[1];
  const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
  const int ka = p.k_cu[seg], lk = p.k_cu[seg + 1] - ka;
  const int kvh = (hg * p.ng) / p.group;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, half = lane >> 5;
  const int dh = wave & 1;
  const int grp = wave >> 2;
  const int vec = (wave >> 1) * 32 + col;
  const int off = vec / p.ng;
  const int pos = tile * rows_per_tile + off;
  const int head = hg * p.ng + (vec - off * p.ng);
  const bool valid = pos < lq;
  int lo = 0, hi = 0, sl = 0, sh = 0;
  int wlo = INT32_MAX, whi = INT32_MIN, wflo = INT32_MIN, wfhi = INT32_MAX;
  if (valid) {
    const LaneKeys lk_ = lane_keys(pos, qa, lq, lk, p.left, p.right, p.spans, p.n_spans);
    lo = lk_.lo;
    hi = lk_.hi;
    sl = lk_.sl;
    sh = lk_.sh;
    wflo = lo;
    wfhi = hi;
    if (lo < hi) {
      wlo = lo;
      whi = hi;
    }
    if (sl < sh) {
      wlo = min(wlo, sl);
      whi = max(whi, sh);
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

  bf16x8 qop[QC];
  {
    const uint16_t* qrow = p.q + (int64_t)(qa + pos) * p.sq_t + (int64_t)head * p.sq_h;
    u32x4 x[QC];
#pragma unroll
    for (int i = 0; i < QC; ++i) {
      x[i] = u32x4{0, 0, 0, 0};
      if (valid) x[i] = *(const u32x4*)(qrow + half * 8 + (dh * QC + i) * 16);
    }
    if (p.q_norm != KARPO_NORM_NONE || p.rope_cos != nullptr) {
      if (valid) query_prologue<D, QC>(p, qrow, (int64_t)(qa + pos), half, dh * QC, x);
      if (p.q_out != nullptr && valid && part == 0) {
        uint16_t* qo = p.q_out + (int64_t)(qa + pos) * p.sqo_t + (int64_t)head * p.sqo_h + half * 8;
#pragma unroll
        for (int i = 0; i < QC; ++i) *(u32x4*)(qo + (dh * QC + i) * 16) = x[i];
      }
    }
#pragma unroll
    for (int i = 0; i < QC; ++i) qop[i] = __builtin_bit_cast(bf16x8, x[i] ^ p.qsign);
  }
  __syncthreads();
  int klo = wlo, khi = whi;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    klo = min(klo, red[0][w]);
    khi = max(khi, red[1][w]);
  }
  klo = __builtin_amdgcn_readfirstlane(klo);
  khi = __builtin_amdgcn_readfirstlane(khi);
  int j_first, n_steps;
  part_steps(klo, khi, BN, part, parts, &j_first, &n_steps);

  const uint16_t* kbase = p.k + (int64_t)kvh * p.sk_h + (int64_t)ka * p.sk_t;
  const uint16_t* vbase = p.v + (int64_t)kvh * p.sv_h + (int64_t)ka * p.sv_t;
  // a wave's INSTS copy blocks of a tile share their rows: block r starts r * 64 bytes (K) / r * 256 bytes (V) after
  // block 0 in memory, so one offset register per tile kind
  uint32_t k_voff0, v_voff0;
  {
    int key, colm;
    k_dma_source<D>(wave * INSTS, lane, &key, &colm);
    k_voff0 = (uint32_t)(key * p.sk_t + colm) * 2u;
    v_dma_source<D>(wave * INSTS, lane, &key, &colm);
    v_voff0 = (uint32_t)(key * p.sv_t + colm) * 2u;
  }
  // T(t) = K(t), V(t - 1): running pointers, empty ranges past the ends (every wave issues 2 INSTS copies per T)
  const uint16_t* ck = kbase + (int64_t)j_first * p.sk_t;
  const uint16_t* cv = vbase + (int64_t)j_first * p.sv_t;
  const int64_t k_step = (int64_t)BN * p.sk_t, v_step = (int64_t)BN * p.sv_t;
  const int j_end = j_first + n_steps * BN;
  int jt = j_first;
  auto copy_T = [&](int b) {
    const int rk = jt < j_end ? min(lk - jt, BN) : 0;
    const int rv = jt > j_first && jt <= j_end ? min(lk - (jt - BN), BN) : 0;
#pragma unroll
    for (int r = 0; r < INSTS; ++r) {
      dma_16b(ck, rk * (int)p.sk_t * 2, kbuf(b) + (wave * INSTS + r) * 1024, k_voff0 + 64u * r);
      dma_16b(cv, rv * (int)p.sv_t * 2, vbuf(b) + (wave * INSTS + r) * 1024, v_voff0 + 256u * r);
    }
    if (jt < j_end) ck += k_step;
    if (jt > j_first && jt <= j_end) cv += v_step;
    jt += BN;
  };

  const int k_read = k_offset<D>(key_row(col), half) + dh * QC * 512;
  const int g = lane >> 4, jl = lane & 15;
  const int v_read = v_offset<D>(8 * (g >> 1) + (jl >> 2), 16 * (g & 1) + 4 * (jl & 3)) + dh * OB * 256;

  f32x16 acc[OB];
#pragma unroll
  for (int db = 0; db < OB; ++db) acc[db] = f32x16{};
  float m = -1e30f, l = 0.f;  // finite start, as attn_fwd_kernel
  const float c = p.c;
  const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
  f32x16 st;
  bf16x8 pb[KC];
  KA_LDS f32x4* my_slot = (KA_LDS f32x4*)&xch[wave][0] + lane;
  const KA_LDS f32x4* other_slot = (const KA_LDS f32x4*)&xch[wave ^ 1][0] + lane;

  auto active = [&](int t) {
    const int j0 = j_first + t * BN;
    return t >= 0 && t < n_steps && j0 < whi && j0 + BN > wlo;
  };
  // this wave's half of QK^T(s) and of P.V(s - 1), both on T(s) (buffer b); the partial scores go to the slot
  auto mfma_phase = [&](int s, int b) {
    const bool a0 = active(s), a1 = active(s - 1);
    const KA_LDS char* kt = kbuf(b);
    const KA_LDS char* vt = vbuf(b);
    if (a0) {
      st = f32x16{};
#pragma unroll
      for (int dc = 0; dc < QC; ++dc) {
        const bf16x8 a = *(const KA_LDS bf16x8*)(kt + k_read + dc * 512);
        st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qop[dc], st, 0, 0, 0);
      }
    }
    if (a1) {
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
        for (int db = 0; db < OB; ++db) {
          bf16x4 v2[2];
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            v2[rr] = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                    (KA_LDS s16x4*)(vt + v_read + (kc * 4 + rr) * (D / 16) * 128 + db * 256)));
          const bf16x8 a = __builtin_shufflevector(v2[0], v2[1], 0, 1, 2, 3, 4, 5, 6, 7);
          acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[kc], acc[db], 0, 0, 0);
        }
      }
    }
    if (a0) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) my_slot[q4 * 64] = f32x4{st[4 * q4], st[4 * q4 + 1], st[4 * q4 + 2], st[4 * q4 + 3]};
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the slot written, this phase's LDS reads done
  };
  // the full scores of step t (this wave's partial plus the partner's, equal in both waves: addition commutes),
  // then the softmax: both waves of a pair compute the same m, l and P
  auto valu_phase = [&](int t) {
    if (!active(t)) return;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x4 o = other_slot[q4 * 64];
      st[4 * q4] += o.x;
      st[4 * q4 + 1] += o.y;
      st[4 * q4 + 2] += o.z;
      st[4 * q4 + 3] += o.w;
    }
    const int j0 = j_first + t * BN;
    if (!(j0 >= wflo && j0 + BN <= wfhi)) {
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        const int key = j0 + (jj >> 3) * 16 + half * 8 + (jj & 7);
        const bool vis = ((unsigned)(key - lo) < (unsigned)(hi - lo)) | ((unsigned)(key - sl) < (unsigned)(sh - sl));
        st[jj] = vis ? st[jj] : -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) mx = fmaxf(mx, st[jj]);
    const float mt = half_swap_max(mx) * c;
    const bool need = mt > m + p.tau;
    if (__builtin_amdgcn_ballot_w64(need)) {
      const float mn = need ? mt : m;
      const float alpha = need ? __builtin_amdgcn_exp2f(m - mn) : 1.f;
      m = mn;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < OB; ++db) acc[db] *= alpha;
    }
    // l in two partial sums (one chain through l kept an array of this kernel in scratch memory)
    float psum[2] = {0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
#pragma unroll
      for (int t2 = 0; t2 < 8; t2 += 2) {
        const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kc * 8 + t2], c, -m));
        const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(st[kc * 8 + t2 + 1], c, -m));
        const bf16x2 pr = {(__bf16)e0, (__bf16)e1};
        pb[kc][t2] = pr[0];
        pb[kc][t2 + 1] = pr[1];
        psum[(t2 >> 1) & 1] = __builtin_amdgcn_fdot2_f32_bf16(pr, ones, psum[(t2 >> 1) & 1], false);
      }
    }
    l += psum[0] + psum[1];
  };

  // prologue: T(0) (K(0) only) landed; the envelope slots are read by every wave before the first exchange write
  if (n_steps > 0) copy_T(0);
  wait_vmcnt<0>();
  __syncthreads();
  if (n_steps > 0) {
    // iteration s on buffer b = s % 2: T(s + 1) into the other buffer (which held T(s - 1)), waited at the end
    auto iter_a = [&](int s, int b) {
      if (s + 1 <= n_steps) copy_T(b ^ 1);
      mfma_phase(s, b);
      bare_barrier();
      valu_phase(s);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      wait_vmcnt<0>();
      bare_barrier();
    };
    auto iter_b = [&](int s, int b) {
      if (s + 1 <= n_steps) copy_T(b ^ 1);
      valu_phase(s - 1);
      __builtin_amdgcn_s_waitcnt(0xc07f);
      bare_barrier();
      mfma_phase(s, b);
      wait_vmcnt<0>();
      bare_barrier();
    };
    if (grp == 0) {
      int s = 0;
      for (; s + 1 <= n_steps; s += 2) {
        iter_a(s, 0);
        iter_a(s + 1, 1);
      }
      if (s <= n_steps) iter_a(s, 0);
    } else {
      int s = 0;
      for (; s + 1 <= n_steps; s += 2) {
        iter_b(s, 0);
        iter_b(s + 1, 1);
      }
      if (s <= n_steps) iter_b(s, 0);
    }
  }

  const float lt = half_swap_sum(l);
  if (parts > 1) {
    constexpr int V = 32 * W / 2;
    float* base = p.partial + partial_base(slot, part, p.n_hg, hg, V, D);
    float* op = base + (int64_t)vec * D + dh * (D / 2) + half * 4;
#pragma unroll
    for (int db = 0; db < OB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        float4 x = {acc[db][g4 * 4], acc[db][g4 * 4 + 1], acc[db][g4 * 4 + 2], acc[db][g4 * 4 + 3]};
        *(float4*)(op + db * 32 + g4 * 8) = x;
      }
    if (half == 0 && dh == 0) {
      base[V * D + vec] = m;
      base[V * D + V + vec] = lt;
    }
    return;
  }
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (valid && p.lse != nullptr && half == 0 && dh == 0)
    p.lse[(int64_t)head * p.lse_stride + qa + pos] = lt > 0.f ? (m + __log2f(lt)) * 0.69314718055994531f : -INFINITY;
  if (valid) {
    uint16_t* op = p.o + (int64_t)(qa + pos) * p.so_t + (int64_t)head * p.so_h + dh * (D / 2) + half * 4;
    const uint16_t* gp = p.gate != nullptr
                             ? p.gate + (int64_t)(qa + pos) * p.sg_t + (int64_t)head * p.sg_h + dh * (D / 2) + half * 4
                             : nullptr;
#pragma unroll
    for (int db = 0; db < OB; ++db) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        *(u32x2*)(op + db * 32 + g4 * 8) =
            output4(acc[db][g4 * 4] * inv, acc[db][g4 * 4 + 1] * inv, acc[db][g4 * 4 + 2] * inv,
                    acc[db][g4 * 4 + 3] * inv, gp != nullptr ? gp + db * 32 + g4 * 8 : nullptr);
      }
    }
  }
}
#endif  // KA_FWD_UNIT == 0

// ---- merge: the parts of split tiles. Thread per (split tile, head group, query vector, 4 head-dim elements), in a
// grid-stride loop over a fixed grid, so every load of a thread is independent and the launch costs little when the
// plan splits nothing. The parts' running maxima go on a common M: O = sum_p 2^(m_p - M) O_p / sum_p 2^(m_p - M) l_p
// (0 when no part saw a key, as an unsplit tile writes).
constexpr int kMergeThreads = 256;
constexpr int kMergeBlocks = 1024;

template <int D, int W, int V>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(Params p) {
  constexpr int C4 = D / 4;
  if (p.plan[5] != W) return;
  const int64_t units = (int64_t)p.plan[4] * p.n_hg * V * C4;
  const int rows_per_tile = p.plan[1];
  const int64_t stride = (int64_t)p.n_hg * V * (D + 2);  // floats between consecutive slots
  for (int64_t idx = (int64_t)blockIdx.x * kMergeThreads + threadIdx.x; idx < units;
       idx += (int64_t)gridDim.x * kMergeThreads) {
    const int d = (int)(idx % C4) * 4;
    const int vec = (int)((idx / C4) % V);
    const int64_t mh = idx / ((int64_t)C4 * V);
    const int merge = (int)(mh / p.n_hg), hg = (int)(mh - (int64_t)merge * p.n_hg);
    const int32_t* e = p.plan + kPlanHeader + kMergeInts * merge;
    const int seg = e[0], tile = e[1], parts = e[2], slot = e[3];
    if (slot < 0 || parts < 2 || slot + parts > p.slots) continue;
    const int off = vec / p.ng;
    const int pos = tile * rows_per_tile + off;
    const int qa = p.q_cu[seg], lq = p.q_cu[seg + 1] - qa;
    if (pos >= lq) continue;
    const int head = hg * p.ng + (vec - off * p.ng);
    const float* first = p.partial + ((int64_t)slot * p.n_hg + hg) * (int64_t)V * (D + 2);
    float mx = -INFINITY;
    for (int q = 0; q < parts; ++q) mx = fmaxf(mx, first[q * stride + V * D + vec]);
    float4 num = {0.f, 0.f, 0.f, 0.f};
    float den = 0.f;
    if (mx != -INFINITY) {
      for (int q = 0; q < parts; ++q) {
        const float* b = first + q * stride;
        const float w = __builtin_amdgcn_exp2f(b[V * D + vec] - mx);
        const float4 x = *(const float4*)(b + (int64_t)vec * D + d);
        num.x += w * x.x;
        num.y += w * x.y;
        num.z += w * x.z;
        num.w += w * x.w;
        den += w * b[V * D + V + vec];
      }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    if (p.lse != nullptr && d == 0)
      p.lse[(int64_t)head * p.lse_stride + qa + pos] = den > 0.f ? (mx + __log2f(den)) * 0.69314718055994531f
                                                                  : -INFINITY;
    const uint16_t* gp =
        p.gate != nullptr ? p.gate + (int64_t)(qa + pos) * p.sg_t + (int64_t)head * p.sg_h + d : nullptr;
    *(u32x2*)(p.o + (int64_t)(qa + pos) * p.so_t + (int64_t)head * p.so_h + d) =
        output4(num.x * inv, num.y * inv, num.z * inv, num.w * inv, gp);
  }
}

#if KA_FWD_UNIT == 0
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

__device__ int64_t block_sum64(int64_t x, int64_t* scratch /* >= kPlanThreads/64 */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  if (lane == 0) scratch[wave] = x;
  __syncthreads();
  int64_t t = 0;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) t += scratch[w];
  __syncthreads();
  return t;
}

// The plan of karpo_attn.h from the device bounds, in three passes over the tiles: the pack's workgroup-steps (which
// set the split length), a histogram of part costs, and the scatter (descending cost order; split tiles' slots and
// merge entries in tile order). The host planner (plan.cpp) lists the same items; among equal costs the order here
// depends on atomics. Workgroup b plans job b (the backward's two work lists in one launch).
struct PlanJobs {
  PlanJob a, b;
};
__global__ __launch_bounds__(kPlanThreads) void plan_kernel(PlanJobs jobs, int n_seq) {
  const PlanJob job = blockIdx.x == 0 ? jobs.a : jobs.b;
  const int32_t* __restrict__ q_cu = job.q_cu;
  const int32_t* __restrict__ k_cu = job.k_cu;
  const Geometry g = job.g;
  const int left = job.left, right = job.right;
  int32_t* __restrict__ plan = job.plan;
  const int tiles_cap = job.tiles, merges_cap = job.merges, items_cap = job.items;
  int32_t* __restrict__ tile_base = job.tile_base;
  __shared__ int hist[kCostBuckets];
  __shared__ int scratch[kPlanThreads / 64 + 1];
  __shared__ int64_t scratch64[kPlanThreads / 64];
  const int tid = threadIdx.x;
  // the header's constant entries (an empty plan until the items are listed)
  if (tid == 0) {
    plan[0] = 0;
    plan[1] = g.rows;
    plan[2] = g.bn;
    plan[3] = g.ng;
    plan[4] = 0;
    plan[5] = g.waves;
    plan[6] = kPlanHeader;
    plan[7] = 0;
    plan[8] = n_seq;
    plan[9] = job.gather;
    plan[10] = g.shape;
    plan[11] = 0;
  }
  if (job.status != nullptr) {  // the bounds against the call's contract: a violation plans nothing
    int bad = 0;
    for (int i = tid; i < n_seq; i += kPlanThreads) {
      const int q0 = q_cu[i], q1 = q_cu[i + 1], k0 = k_cu[i], k1 = k_cu[i + 1];
      bad |= q0 < 0 || k0 < 0 || q1 < q0 || k1 < k0 || q1 - q0 > job.max_q || (int64_t)q1 > job.total_q ||
             (job.key_bound > 0 && (int64_t)k1 > job.key_bound);
    }
    int total;
    block_exclusive_scan(bad, &total, scratch);
    if (tid == 0) *job.status = total > 0 ? KARPO_ATTN_ERR_BOUNDS : KARPO_ATTN_OK;
    if (total > 0) return;
  }
  int carry = 0;
  for (int base = 0; base < n_seq; base += kPlanThreads) {
    const int i = base + tid;
    const int nt = i < n_seq ? (int)tiles_of(q_cu[i + 1] - q_cu[i], g.rows) : 0;
    int total;
    const int ex = block_exclusive_scan(nt, &total, scratch);
    if (i < n_seq) tile_base[i] = carry + ex;
    carry += total;
  }
  if (tid == 0) tile_base[n_seq] = carry;
  const int n_tiles = min(carry, tiles_cap);
  for (int b = tid; b < kCostBuckets; b += kPlanThreads) hist[b] = 0;
  __syncthreads();

  // tile f: its segment, index in the segment and key steps
  auto locate = [&](int f, int* seg, int* t) -> int64_t {
    int l0 = 0, l1 = n_seq;  // last segment whose first tile is at or before f
    while (l1 - l0 > 1) {
      const int mid = (l0 + l1) >> 1;
      if (tile_base[mid] <= f) l0 = mid; else l1 = mid;
    }
    *seg = l0;
    *t = f - tile_base[l0];
    const int lq = q_cu[l0 + 1] - q_cu[l0], lk = k_cu[l0 + 1] - k_cu[l0];
    return tile_steps(lq, lk, *t, g.rows, g.bn, left, right);
  };
  int64_t mine = 0;
  for (int f = tid; f < n_tiles; f += kPlanThreads) {
    int seg, t;
    mine += locate(f, &seg, &t);
  }
  const int64_t tau = split_tau(block_sum64(mine, scratch64) * g.n_hg, g.conc);

  int64_t counts = 0;  // split tiles (high 32 bits) and items (low) of this thread's tiles
  for (int f = tid; f < n_tiles; f += kPlanThreads) {
    int seg, t;
    const int64_t steps = locate(f, &seg, &t);
    const int parts = split_parts(steps, tau);
    atomicAdd(&hist[part_cost(steps, parts)], parts);
    counts += (parts > 1 ? (int64_t)1 << 32 : 0) + parts;
  }
  const int64_t both = block_sum64(counts, scratch64);
  // within the capacities by the split policy's bound; a plan that would not fit lists no items (never written)
  const int n_merges = (int)(both >> 32), n_items = (int)(both & 0xffffffff);
  const bool fits = n_merges <= merges_cap && n_items <= items_cap;
  const int first = kPlanHeader + kMergeInts * min(n_merges, merges_cap);
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
  int slot_carry = 0, merge_carry = 0;
  for (int base = 0; base < n_tiles; base += kPlanThreads) {
    const int f = base + tid;
    int seg = 0, t = 0, parts = 0;
    int64_t steps = 0;
    if (f < n_tiles) {
      steps = locate(f, &seg, &t);
      parts = split_parts(steps, tau);
    }
    const bool split = parts > 1;
    int slots_total, merges_total;
    const int slot = slot_carry + block_exclusive_scan(split ? parts : 0, &slots_total, scratch);
    const int merge = merge_carry + block_exclusive_scan(split ? 1 : 0, &merges_total, scratch);
    slot_carry += slots_total;
    merge_carry += merges_total;
    if (f >= n_tiles || !fits) continue;
    if (split) {
      int32_t* m = plan + kPlanHeader + kMergeInts * merge;
      m[0] = seg;
      m[1] = t;
      m[2] = parts;
      m[3] = slot;
    }
    const int at = atomicAdd(&hist[part_cost(steps, parts)], parts);
    for (int q = 0; q < parts; ++q) {
      int32_t* e = plan + first + kItemInts * (at + q);
      e[0] = seg;
      e[1] = t;
      e[2] = q | (parts << 16);
      e[3] = split ? slot : -1;
    }
  }
  if (tid == 0) {
    plan[0] = fits ? n_items : 0;
    plan[4] = fits ? n_merges : 0;
    plan[6] = fits ? first : kPlanHeader;
    plan[7] = fits ? slot_carry : 0;
    if (!fits && job.status != nullptr) *job.status = KARPO_ATTN_ERR_CAPACITY;  // unreachable within the contract
  }
}

// ---- karpo_attn_norm_rope: L = D / 8 lanes per (row, head) vector, 8 elements (16 B) per lane, 64 / L vectors per
// wave; the sum of squares reduces over the vector's lanes, and a rotation partner (d +- rope_dim / 2, a multiple of
// 16 elements away) comes from lane +- rope_dim / 16 of the same vector by a lane permute.
constexpr int kNormRopeWaves = 4;

template <int D>
__global__ __launch_bounds__(64 * kNormRopeWaves) void norm_rope_kernel(NormRopeParams p) {
  constexpr int L = D / 8, VPW = 64 / L;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / L, l = lane - sub * L, d0 = l * 8;
  const bool norm = p.norm != KARPO_NORM_NONE;
  const float wm = (p.norm == KARPO_NORM_WEIGHT || p.norm == KARPO_NORM_ONE_PLUS) ? 1.f : 0.f;
  const float wa = (p.norm == KARPO_NORM_ONE_PLUS || p.norm == KARPO_NORM_PLAIN) ? 1.f : 0.f;
  u32x4 wv = {0, 0, 0, 0};
  if (p.w != nullptr) wv = *(const u32x4*)(p.w + d0);
  const bool rot = p.cos != nullptr;
  const int rd = rot ? p.rope_dim : 0, rh = rd >> 1;
  const bool in = d0 < rd;
  const int src = sub * L + (in ? (d0 < rh ? l + rh / 8 : l - rh / 8) : l);  // the partner's lane
  const float sgn = d0 < rh ? -1.f : 1.f;
  for (int64_t v0 = ((int64_t)blockIdx.x * kNormRopeWaves + wave) * VPW; v0 < p.vectors;
       v0 += (int64_t)gridDim.x * kNormRopeWaves * VPW) {
    const int64_t v = v0 + sub;
    const bool ok = v < p.vectors;
    const int64_t row = ok ? v / p.heads : 0;
    const int head = ok ? (int)(v - row * p.heads) : 0;
    u32x4 x = {0, 0, 0, 0};
    if (ok) x = *(const u32x4*)(p.x + row * p.sx_t + (int64_t)head * p.sx_h + d0);
    float n[8];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(bf16_at(x, e), bf16_at(x, e), ss);
#pragma unroll
    for (int o = L / 2; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    const float r = norm ? 1.f / __builtin_sqrtf(ss * (1.f / D) + p.eps) : 1.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float h = bf16_at(x, e);
      n[e] = norm ? round_bf16(h * r * __builtin_fmaf(wm, bf16_at(wv, e), wa)) : h;
    }
    if (rot) {
      u32x4 cv = {0, 0, 0, 0}, sv = {0, 0, 0, 0};
      if (ok && in) {
        cv = *(const u32x4*)(p.cos + row * p.rope_stride + d0);
        sv = *(const u32x4*)(p.sin + row * p.rope_stride + d0);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
#pragma clang fp contract(off)  // x cos + rot(x) sin: both products rounded, then the sum, as the reference
        const float pn = __shfl(n[e], src);
        const float y = n[e] * bf16_at(cv, e) + sgn * pn * bf16_at(sv, e);
        n[e] = in ? y : n[e];
      }
    }
    if (ok) {
      u32x4 out;
#pragma unroll
      for (int t = 0; t < 4; ++t) out[t] = pack_bf16(n[2 * t], n[2 * t + 1]);
      *(u32x4*)(p.y + row * p.sy_t + (int64_t)head * p.sy_h + d0) = out;
    }
  }
}

hipError_t launch_norm_rope(const NormRopeParams& p, int head_dim, hipStream_t stream) {
  if (p.vectors <= 0) return hipSuccess;
  const int64_t per_block = (int64_t)kNormRopeWaves * (64 / (head_dim / 8));
  int64_t blocks = (p.vectors + per_block - 1) / per_block;
  if (blocks > 8192) blocks = 8192;
  const dim3 grid((unsigned)blocks), block(64 * kNormRopeWaves);
  switch (head_dim) {
    case 64: hipLaunchKernelGGL(norm_rope_kernel<64>, grid, block, 0, stream, p); break;
    case 128: hipLaunchKernelGGL(norm_rope_kernel<128>, grid, block, 0, stream, p); break;
    case 256: hipLaunchKernelGGL(norm_rope_kernel<256>, grid, block, 0, stream, p); break;
    case 512: hipLaunchKernelGGL(norm_rope_kernel<512>, grid, block, 0, stream, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

#endif  // KA_FWD_UNIT == 0

// ---- launch

// Whether a shape is built with a row table: every shape but the wide and long tiles at head sizes 128 and 256,
// which tile_shape never selects for a call with a row table.
constexpr bool gather_built(int d, int shape) {
  return !((d == 128 || d == 256) && (shape == kWide || shape == kLong || shape == kDual));
}

template <int D, int SHAPE>
static hipError_t launch_attn(const Params& p, int64_t items, int64_t merges, int n_hg, hipStream_t stream) {
  using Cfg = TileCfg<D, SHAPE>;
  if (p.k_rows != nullptr) {
    if constexpr (gather_built(D, SHAPE))
      hipLaunchKernelGGL((attn_fwd_kernel<D, SHAPE, true>), dim3((unsigned)(items * n_hg)), dim3(64 * Cfg::W), 0,
                         stream, p);
    else
      return hipErrorInvalidValue;
  } else {
#if KA_FWD_UNIT == 0
    if constexpr (D == 512 && SHAPE == kWide)
      hipLaunchKernelGGL(attn_fwd_pair_pp_kernel, dim3((unsigned)(items * n_hg)), dim3(64 * Cfg::W), 0, stream, p);
    else
#endif
      hipLaunchKernelGGL((attn_fwd_kernel<D, SHAPE, false>), dim3((unsigned)(items * n_hg)), dim3(64 * Cfg::W), 0,
                         stream, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || merges <= 0) return e;
  constexpr int64_t per_merge = (int64_t)tile_vectors(D, SHAPE) * (D / 4);  // threads of one head group
  const int64_t blocks = (merges * n_hg * per_merge + kMergeThreads - 1) / kMergeThreads;
  hipLaunchKernelGGL((merge_kernel<D, Cfg::W, tile_vectors(D, SHAPE)>),
                     dim3((unsigned)(blocks < kMergeBlocks ? blocks : kMergeBlocks)),
                     dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

#if KA_FWD_UNIT == 0
hipError_t launch_forward(const Params& p, int head_dim, const Geometry& g, int64_t items, int64_t merges,
                          hipStream_t stream) {
  if (items <= 0) return hipSuccess;
  switch (head_dim * 8 + g.shape) {  // the shapes tile_shape selects per head size
    case 64 * 8 + kWide: return launch_attn<64, kWide>(p, items, merges, g.n_hg, stream);
    case 64 * 8 + kNarrow: return launch_attn<64, kNarrow>(p, items, merges, g.n_hg, stream);
    case 128 * 8 + kWide: return launch_forward_128(p, kWide, items, merges, g.n_hg, stream);
    case 128 * 8 + kNarrow: return launch_attn<128, kNarrow>(p, items, merges, g.n_hg, stream);
    case 128 * 8 + kSmall: return launch_attn<128, kSmall>(p, items, merges, g.n_hg, stream);
    case 128 * 8 + kLong: return launch_forward_128(p, kLong, items, merges, g.n_hg, stream);
    case 128 * 8 + kDual: return launch_attn<128, kDual>(p, items, merges, g.n_hg, stream);
    case 256 * 8 + kWide: return launch_attn<256, kWide>(p, items, merges, g.n_hg, stream);
    case 256 * 8 + kNarrow: return launch_attn<256, kNarrow>(p, items, merges, g.n_hg, stream);
    case 256 * 8 + kSmall: return launch_attn<256, kSmall>(p, items, merges, g.n_hg, stream);
    case 512 * 8 + kWide: return launch_attn<512, kWide>(p, items, merges, g.n_hg, stream);
    case 512 * 8 + kNarrow: return launch_attn<512, kNarrow>(p, items, merges, g.n_hg, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_plan(const PlanJob* jobs, int n_jobs, int n_seq, hipStream_t stream) {
  if (n_jobs < 1 || n_jobs > 2) return hipErrorInvalidValue;
  const PlanJobs pj = {jobs[0], jobs[n_jobs - 1]};
  hipLaunchKernelGGL(plan_kernel, dim3((unsigned)n_jobs), dim3(kPlanThreads), 0, stream, pj, n_seq);
  return hipGetLastError();
}
#else
hipError_t launch_forward_128(const Params& p, int shape, int64_t items, int64_t merges, int n_hg,
                              hipStream_t stream) {
  if (shape == kWide) return launch_attn<128, kWide>(p, items, merges, n_hg, stream);
  if (shape == kLong) return launch_attn<128, kLong>(p, items, merges, n_hg, stream);
  return hipErrorInvalidValue;
}
#endif  // KA_FWD_UNIT

}  // namespace karpo
