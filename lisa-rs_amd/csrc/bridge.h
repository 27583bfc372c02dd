// bridge.h — internal definitions of the opaque handles of lisa_hip.h, shared
// by device.cpp (the bridge) and runner.cpp (the runner built on it).
#ifndef LISA_BRIDGE_H
#define LISA_BRIDGE_H

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

// One timed launch of an eager profile pass: start/stop events attached to the
// kernel dispatch itself (hipExtModuleLaunchKernel), so the interval is the
// kernel's execution, as a kernel trace reports it.
struct LisaProfRec {
  int kind;
  hipEvent_t start, stop;
};

struct LisaDevice {
  int ordinal = 0;
  hipStream_t stream = nullptr;
  std::string name, arch;
  uint64_t total_mem = 0;
  int cu_count = 0;
  // set while a profile pass runs: every lisa_launch is timed and tagged
  std::vector<LisaProfRec>* prof = nullptr;
  int prof_kind = -1;
  // workspace of lisa_attention_decode called without one (grown on demand)
  void* attn_ws = nullptr;
  size_t attn_ws_len = 0;
};

struct LisaBuffer {
  LisaDevice* dev = nullptr;
  void* ptr = nullptr;
  size_t len = 0;
};

struct LisaModule {
  LisaDevice* dev;
  hipModule_t mod;
};

struct LisaFunction {
  hipFunction_t fn;
  std::string name;
};

struct LisaEncoder {
  LisaDevice* dev = nullptr;
  LisaFunction* fn = nullptr;
  std::vector<std::vector<uint8_t>> args;
};

struct LisaGraph {
  hipGraph_t graph;
  hipGraphExec_t exec;
};

struct LisaEvent {
  hipEvent_t ev;
};

int lisa_fail(int code, const char* fmt, ...);
int lisa_hip_check(hipError_t e, const char* what);
std::string lisa_library_dir();
// Launch a kernel taking one by-value argument block.
int lisa_launch(LisaDevice* d, LisaFunction* f, const void* params, size_t len, uint32_t gx, uint32_t gy,
                uint32_t gz, uint32_t tx, uint32_t ty, uint32_t tz);

struct LisaAttnDecodeArgs;
// Checks a decode-attention call and launches its partial and merge kernels
// with the slice partials at `part` (attention.cpp).
int lisa_attention_launch(LisaDevice* dev, LisaModule* mod, const LisaAttnDecodeArgs* a, void* part);

#define LISA_TRY(expr)          \
  do {                          \
    const int lisa_rc_ = (expr); \
    if (lisa_rc_) return lisa_rc_; \
  } while (0)

#endif  // LISA_BRIDGE_H
