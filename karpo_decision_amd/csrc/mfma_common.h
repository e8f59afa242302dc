// MFMA operand layouts, LDS tile layouts and small device helpers shared by the forward (attn_fwd.hip) and backward
// (attn_bwd.hip) kernels: bf16 32x32x16 MFMA tiles, K tiles read as MFMA row operands, V tiles read transposed
// (ds_read_b64_tr_b16), global -> LDS copies through buffer_load ... lds.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tile_addr.h"

namespace karpo {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
#define KA_LDS __attribute__((address_space(3)))
#define KA_GLOBAL __attribute__((address_space(1)))


// Buffer resource word 3 for raw 32-bit accesses (bounds-checked against num_records, zero past the end).
constexpr int kBufferFlags = 0x00020000;


// Row of the 32-key block that MFMA A-row r reads: bits 2 and 3 of r swapped.
__device__ __forceinline__ int key_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// Byte offsets inside the LDS tiles.
//   K: (key k, 16-byte chunk c of its D/8) at ((k / 16) * D/8 + c) * 256 + (k % 16) * 16
//   V: (key k, element d) at ((k / 4) * D/16 + d / 16) * 128 + (k % 4) * 32 + (d % 16) * 2
template <int D>
__device__ __forceinline__ int k_offset(int k, int c) { return ((k >> 4) * (D / 8) + c) * 256 + (k & 15) * 16; }
template <int D>
__device__ __forceinline__ int v_offset(int k, int d) {
  return ((k >> 2) * (D / 16) + (d >> 4)) * 128 + (k & 3) * 32 + (d & 15) * 2;
}

// The maximum over a lane and the lane 32 away. IEEE maximum (NaN-propagating): one v_maximum3_f32, where fmaxf would
// first quiet both swapped values.
__device__ __forceinline__ float half_swap_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
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

// The S layout: rows (keys, or query rows) staged once and read both as MFMA row operands (ds_read_b128, one row's
// 16-byte chunk per lane) and transposed (ds_read_b64_tr_b16, four rows of one column group per lane). Chunk c of
// row k sits at ((k / 16) * D/8 + c) * 256 + ((k % 16) ^ 4 (c % 4)) * 16: a 256 B run holds 16 rows' chunk c, with the
// rows' order XOR-swizzled by the chunk index, so the 16 lanes of a row read cover one run and the 32 lanes of a
// transposed read (four rows x chunks c .. c+3) cover 64 distinct banks.
template <int D>
__device__ __forceinline__ int s_offset(int k, int c) {
  return ((k >> 4) * (D / 8) + c) * 256 + (((k & 15) ^ ((c & 3) << 2)) * 16);
}
// Inverse of s_offset for byte offset blk * 1024 + lane * 16 (the copy's source row and first column).
template <int D>
__device__ __forceinline__ void s_dma_source(int blk, int lane, int* row, int* col) {
  const int b = blk * 4 + (lane >> 4);  // 256-byte run: (row block, chunk)
  const int c = b % (D / 8);
  *row = (b / (D / 8)) * 16 + ((lane & 15) ^ ((c & 3) << 2));
  *col = c * 8;
}
// Row-operand read of element chunk 2 dc + half of row k: s_offset(k, 2 dc + half) = base[dc & 1] + (dc >> 1) * 1024
// with base[i] = s_offset(k, 2 i + half).
// Transposed read (the A operand rows d = db*32 + lane%32 over rows kc*16 + (lane/32)*8 .. +8 of the step, two reads
// rr = 0, 1 of four rows each): this lane's address is s_tr_base(lane, rr) + kc * (D/8) * 256 + db * 1024.
__device__ __forceinline__ int s_tr_base(int lane, int rr) {
  const int g = lane >> 4, jl = lane & 15;
  const int c = 2 * (g & 1) + ((jl >> 1) & 1);  // chunk within the 32-column block (its index mod 4)
  return c * 256 + (((4 * rr + 8 * (g >> 1) + (jl >> 2)) ^ (c << 2)) * 16) + (jl & 1) * 8;
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited on): at most N vector-memory operations of this wave in flight.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Cache policy of a copy whose rows no other workgroup reads again (the instruction's nt bit: streamed through the
// caches). Only for such data: where other tiles re-read the rows from L2, it costs 7-24% (32k, 131k, Qwen layers).
constexpr int kCopyStream = 2;

// One 16-byte chunk per lane from `base + voff` (bounds-checked against `bytes`: zeros past it) to `lds + 16 * lane`,
// with cache policy AUX (0, or kCopyStream).
template <int AUX = 0>
__device__ __forceinline__ void dma_16b(const uint16_t* base, int bytes, KA_LDS char* lds, uint32_t voff) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, bytes, kBufferFlags);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (KA_LDS void*)lds, 16, voff, 0, 0, AUX);
}


// ---- bf16 packing

// Element e of 8 packed bf16.
__device__ __forceinline__ float bf16_at(const u32x4& v, int e) {
  const unsigned w = v[e >> 1];
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  return (unsigned)__builtin_bit_cast(uint16_t, (__bf16)a) | ((unsigned)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}

}  // namespace karpo
