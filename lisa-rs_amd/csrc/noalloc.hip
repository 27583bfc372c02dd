// noalloc.hip — lisa_attention_decode_noalloc: lisa_attention_decode for
// callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, hosts that forbid hipMalloc). The slice partials live
// in `scratch`, a fixed array of this library's device code: every GPU the
// library runs on holds its own copy until the process ends. Calls on one GPU
// share that copy, so calls that overlap on one GPU (other streams, other
// threads) race; calls queued on one in-order stream do not. No part of the
// scratch needs clearing: every slice partial the merge reads is written by
// the same call's partial kernel.
#include <hip/hip_runtime.h>

#include <mutex>

#include "bridge.h"
#include "lisa_hip.h"

static __device__ __align__(256) unsigned char scratch[LISA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU, once resolved

// The address of this GPU's copy of `scratch`, resolved on the first call with
// the device current.
int scratch_for(int ordinal, void** out) {
  if (ordinal < 0 || ordinal >= kMaxDevices) return lisa_fail(LISA_E_ARG, "device ordinal %d out of range", ordinal);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch_ptr[ordinal]) {
    int prev = 0;
    LISA_TRY(lisa_hip_check(hipGetDevice(&prev), "hipGetDevice"));
    LISA_TRY(lisa_hip_check(hipSetDevice(ordinal), "hipSetDevice"));
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    (void)hipSetDevice(prev);
    LISA_TRY(lisa_hip_check(e, "hipGetSymbolAddress(scratch)"));
    if (!ptr) return lisa_fail(LISA_E_NOMEM, "scratch has no device address on device %d", ordinal);
    g_scratch_ptr[ordinal] = ptr;
  }
  *out = g_scratch_ptr[ordinal];
  return LISA_OK;
}

}  // namespace

extern "C" int lisa_attention_decode_noalloc(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* args) {
  if (!dev || !args) return lisa_fail(LISA_E_ARG, "lisa_attention_decode_noalloc: null argument");
  if (args->m_rows != 1 && args->m_rows != 3)
    return lisa_fail(LISA_E_ARG, "lisa_attention_decode_noalloc: m_rows %u is not 1 or 3", args->m_rows);
  const uint64_t need = lisa_attention_workspace_bytes(args->m_rows, args->max_pos);
  if (need > (uint64_t)LISA_NOALLOC_SCRATCH_BYTES)
    return lisa_fail(LISA_E_ARG,
                     "lisa_attention_decode_noalloc: %u rows up to position %u need %llu bytes of slice partials, "
                     "above the fixed scratch of %llu bytes",
                     args->m_rows, args->max_pos, (unsigned long long)need,
                     (unsigned long long)LISA_NOALLOC_SCRATCH_BYTES);
  void* ptr = nullptr;
  LISA_TRY(scratch_for(dev->ordinal, &ptr));
  return lisa_attention_launch(dev, mod, args, ptr);
}
