// Per-lane visibility bounds shared by the backward kernels (attn_bwd.hip, attn_bwd_pair.hip): the forward's mask
// rule seen from a query vector (the keys it sees) and from a key (the query rows that see it).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.h"
#include "mfma_common.h"

namespace karpo {

// What one lane sees: [lo, hi) by the window, [sl, sh) by its span (empty ranges when none); and the wave's envelope
// reduced over its lanes: [wlo, whi) the union, [wflo, wfhi) the range every lane sees whole.
struct LaneBounds {
  int lo = 0, hi = 0, sl = 0, sh = 0;
  int wlo = INT32_MAX, whi = INT32_MIN, wflo = INT32_MIN, wfhi = INT32_MAX;

  __device__ void reduce_wave() {
    wlo = __builtin_amdgcn_readfirstlane(wave_min(wlo));
    whi = __builtin_amdgcn_readfirstlane(wave_max(whi));
    wflo = __builtin_amdgcn_readfirstlane(wave_max(wflo));
    wfhi = __builtin_amdgcn_readfirstlane(wave_min(wfhi));
  }
  __device__ void set_window(int a, int b) {
    if (b < a) b = a;
    lo = a;
    hi = b;
    wflo = a;
    wfhi = b;
    if (a < b) {
      wlo = a;
      whi = b;
    }
  }
  __device__ void add_span(int x, int y) {
    if (x < y) {
      sl = x;
      sh = y;
      wlo = min(wlo, x);
      whi = max(whi, y);
    }
  }
};

// The span [s0, s1) of query rows holding pack row `row`, or false.
__device__ inline bool span_of(const BwdParams& p, int row, int* s0, int* s1) {
  int l0 = 0, l1 = p.n_spans;
  while (l1 - l0 > 1) {
    const int mid = (l0 + l1) >> 1;
    if (p.spans[2 * mid] <= row) l0 = mid; else l1 = mid;
  }
  *s0 = p.spans[2 * l0];
  *s1 = p.spans[2 * l0 + 1];
  return *s0 <= row && row < *s1;
}

// Keys query `pos` of a sequence (first pack row qa, lq queries, lk keys) sees.
__device__ inline LaneBounds query_bounds(const BwdParams& p, int qa, int lq, int lk, int pos) {
  LaneBounds b;
  if (pos >= lq) return b;
  const int delta = lk - lq, ip = pos + delta;
  b.set_window(p.left < 0 ? 0 : max(0, ip - p.left),
               p.right < 0 ? lk : (int)min((int64_t)lk, (int64_t)ip + p.right + 1));
  int s0, s1;
  if (p.n_spans > 0 && span_of(p, qa + pos, &s0, &s1)) b.add_span(max(0, s0 - qa + delta), min(lk, s1 - qa + delta));
  return b;
}

// Query rows that see key `key` of a sequence: key - right <= i + delta <= key + left, or both in one span.
__device__ inline LaneBounds key_bounds(const BwdParams& p, int qa, int lq, int lk, int key) {
  LaneBounds b;
  if (key >= lk) return b;
  const int delta = lk - lq;
  b.set_window(p.right < 0 ? 0 : max(0, key - p.right - delta),
               p.left < 0 ? lq : (int)min((int64_t)lq, (int64_t)key + p.left - delta + 1));
  const int kq = key - delta;  // the key's position in query rows
  int s0, s1;
  if (p.n_spans > 0 && kq >= 0 && kq < lq && span_of(p, qa + kq, &s0, &s1)) b.add_span(max(0, s0 - qa), min(lq, s1 - qa));
  return b;
}

}  // namespace karpo
