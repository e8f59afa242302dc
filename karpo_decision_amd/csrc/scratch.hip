// karpo_attn_fwd_noalloc: the forward pass with its scratch (the device plan, the planner's tile bases and status
// word, the fp32 partials of split tiles) in a file-scope device array instead of a caller's workspace, for callers
// that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid it).
//
// The array lives in this translation unit's own code object, which HIP loads on a device the first time this entry
// point asks for the array's address there; from then on the device holds kScratchBytes until the process ends.
// Each device has its own copy at its own address, looked up once per device with that device current and kept here;
// host code never passes the array's name to a kernel (in host code it is a stand-in, not a device address).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "karpo_attn.h"

namespace {

// 144 MiB: the largest workspace any call needs (135.3 MB of partials at head size 256 or 512 with the wide tiles,
// plus the plan) for plans of up to a few million work items.
constexpr size_t kScratchBytes = size_t(144) << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_lock;
void* g_scratch[kMaxDevices] = {};

// The current device's copy of the array (its address looked up on the first call on that device).
int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KARPO_ATTN_ERR_LAUNCH;
  std::lock_guard<std::mutex> hold(g_lock);
  if (g_scratch[dev] == nullptr) {
    // the lookup loads this unit's code object on the device (once): not a stream operation, so a first call made
    // while this thread captures a graph relaxes the thread's capture mode around it, as lazily initialising
    // libraries do, and restores it
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return KARPO_ATTN_ERR_LAUNCH;
    void* ptr = nullptr;
    const hipError_t got = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return KARPO_ATTN_ERR_LAUNCH;
    if (got != hipSuccess || ptr == nullptr) return KARPO_ATTN_ERR_LAUNCH;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return KARPO_ATTN_OK;
}

}  // namespace

extern "C" int karpo_attn_fwd_noalloc(const KarpoAttnArgs* a, void* stream) {
  if (a == nullptr) return KARPO_ATTN_ERR_NULL;
  if (a->plan != nullptr && a->plan_header != nullptr && a->plan_header[4] == 0) {
    // a host plan that splits no tile needs no scratch: karpo_attn_fwd takes it without a workspace (and checks the
    // header against the call), so no size limit applies and the array is not touched
    KarpoAttnArgs b = *a;
    b.workspace = nullptr;
    b.workspace_bytes = 0;
    return karpo_attn_fwd(&b, stream);
  }
  size_t need = 0;
  const int st = karpo_attn_workspace_bytes(a, &need);
  if (st != KARPO_ATTN_OK) return st;
  if (need > kScratchBytes) return KARPO_ATTN_ERR_SCRATCH;  // before any HIP call
  if (a->total_q == 0 || a->n_seq == 0) return karpo_attn_fwd(a, stream);  // nothing to launch
  KarpoAttnArgs b = *a;
  const int got = scratch_address(&b.workspace);
  if (got != KARPO_ATTN_OK) return got;
  b.workspace_bytes = kScratchBytes;
  return karpo_attn_fwd(&b, stream);
}
