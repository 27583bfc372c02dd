// attention.cpp — one gated-attention decode layer's attention core as a
// standalone entry point (the partial/merge half of the reference's
// encode_attention, runner.rs:1426-1592; attention.metal:118-319, 520-641):
// q/k norm + partial RoPE, KV append, split-K slice partials over the live
// context and their flash merge with the output gate. The slice partials live
// in a workspace: the caller's, or one the library keeps per device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>

#include "bridge.h"
#include "lisa_hip.h"
#include "lisa_kernels.h"
#include "lisa_model.h"

namespace {

// per-row, per-slice floats of the partials: 24 heads x (256 outputs + max, denominator)
constexpr uint64_t kSliceFloats = (uint64_t)LISA_ATT_QH * (LISA_ATT_HD + 2);

uint32_t slices_of(const LisaAttnDecodeArgs* a) { return a->max_pos / LISA_ATT_SLICE + 1; }

}  // namespace

extern "C" uint64_t lisa_attention_workspace_bytes(uint32_t m_rows, uint32_t max_pos) {
  return (uint64_t)m_rows * ((uint64_t)max_pos / LISA_ATT_SLICE + 1) * kSliceFloats * sizeof(float);
}

// Checks the arguments and launches the two kernels with the partials at
// `part` (lisa_attention_workspace_bytes of them).
int lisa_attention_launch(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* a, void* part) {
  if (!dev || !mod || !a || !part) return lisa_fail(LISA_E_ARG, "attention decode: null argument");
  if (a->m_rows != 1 && a->m_rows != 3) return lisa_fail(LISA_E_ARG, "attention decode: m_rows %u is not 1 or 3", a->m_rows);
  if (!a->q_proj || !a->k_raw || !a->v_raw || !a->q_norm_w || !a->k_norm_w || !a->key_cache || !a->value_cache ||
      !a->pos || !a->gated)
    return lisa_fail(LISA_E_ARG, "attention decode: null tensor");
  if (a->capacity == 0 || a->max_pos >= a->capacity || a->max_pos + 1 < a->m_rows)
    return lisa_fail(LISA_E_CAPACITY, "attention decode: last row position %u outside capacity %u", a->max_pos,
                     a->capacity);
  const uint32_t slices = slices_of(a);
  if (slices > 1024) return lisa_fail(LISA_E_ARG, "attention decode: %u slices exceed the merge's 1024", slices);
  hipFunction_t part_fn, merge_fn;
  const bool m3 = a->m_rows == 3;
  LISA_TRY(lisa_hip_check(hipModuleGetFunction(&part_fn, mod->mod, m3 ? "lisa_attn_partial_m3" : "lisa_attn_partial_m1"),
                          "hipModuleGetFunction"));
  LISA_TRY(lisa_hip_check(hipModuleGetFunction(&merge_fn, mod->mod, m3 ? "lisa_attn_merge_m3" : "lisa_attn_merge_m1"),
                          "hipModuleGetFunction"));
  LisaAttnParams p{};
  p.q_proj = a->q_proj;
  p.k_raw = a->k_raw;
  p.v_raw = a->v_raw;
  p.q_norm_w = a->q_norm_w;
  p.k_norm_w = a->k_norm_w;
  p.key_cache = a->key_cache;
  p.value_cache = a->value_cache;
  p.part_o = static_cast<float*>(part);
  p.part_ml = static_cast<float*>(part) + (size_t)a->m_rows * LISA_ATT_QH * slices * LISA_ATT_HD;
  p.pos = a->pos;
  p.gated = a->gated;
  p.capacity = a->capacity;
  p.s_max = slices;
  void* args[1] = {&p};
  LISA_TRY(lisa_hip_check(hipModuleLaunchKernel(part_fn, slices, LISA_ATT_KVH, 1, LISA_ATT_PARTIAL_THREADS(a->m_rows),
                                                1, 1, 0, dev->stream, args, nullptr), "launch lisa_attn_partial"));
  return lisa_hip_check(hipModuleLaunchKernel(merge_fn, LISA_ATT_QH, a->m_rows, 1, 256, 1, 1, 0, dev->stream, args,
                                              nullptr), "launch lisa_attn_merge");
}

extern "C" int lisa_attention_decode(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* a,
                                     LisaBuffer* workspace) {
  if (!dev || !a) return lisa_fail(LISA_E_ARG, "lisa_attention_decode: null argument");
  const uint64_t need = lisa_attention_workspace_bytes(a->m_rows, a->max_pos);
  if (workspace) {
    if (workspace->len < need)
      return lisa_fail(LISA_E_ARG, "attention workspace of %zu bytes, %llu needed", workspace->len,
                       (unsigned long long)need);
    return lisa_attention_launch(dev, mod, a, workspace->ptr);
  }
  // the library's workspace for this device, grown on demand
  static std::mutex mu;
  std::lock_guard<std::mutex> lock(mu);
  if (dev->attn_ws_len < need) {
    if (dev->attn_ws) {
      LISA_TRY(lisa_hip_check(hipStreamSynchronize(dev->stream), "hipStreamSynchronize"));
      (void)hipFree(dev->attn_ws);
      dev->attn_ws = nullptr;
      dev->attn_ws_len = 0;
    }
    LISA_TRY(lisa_hip_check(hipMalloc(&dev->attn_ws, need), "hipMalloc attention workspace"));
    dev->attn_ws_len = need;
  }
  return lisa_attention_launch(dev, mod, a, dev->attn_ws);
}
