// device.cpp — the HIP runtime bridge behind include/lisa_hip.h, the MI355X
// counterpart of the reference's Metal FFI (src/device/metal.rs). One device
// handle owns one in-order HIP stream; buffers are hipMalloc'd device memory;
// kernels come from a gfx950 code object loaded with hipModuleLoad and are
// launched with hipModuleLaunchKernel from index-ordered argument slots.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "bridge.h"

// From hip/hip_ext.h (C linkage in libamdhip64); declared here because the
// header's template helpers do not compile with the host C++ compiler.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX, uint32_t globalWorkSizeY,
                                               uint32_t globalWorkSizeZ, uint32_t localWorkSizeX,
                                               uint32_t localWorkSizeY, uint32_t localWorkSizeZ,
                                               size_t sharedMemBytes, hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent, hipEvent_t stopEvent,
                                               uint32_t flags);
#include "lisa_hip.h"

namespace {
thread_local std::string g_error;
}

int lisa_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int lisa_hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return LISA_OK;
  return lisa_fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

extern "C" const char* lisa_last_error(void) { return g_error.c_str(); }

// ---------------------------------------------------------------------------
// device
// ---------------------------------------------------------------------------
extern "C" int lisa_device_create(int ordinal, LisaDevice** out) {
  if (!out) return lisa_fail(LISA_E_ARG, "lisa_device_create: null out");
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= ordinal || ordinal < 0)
    return lisa_fail(LISA_E_ARG, "no HIP device %d (found %d)", ordinal, count);
  LISA_TRY(lisa_hip_check(hipSetDevice(ordinal), "hipSetDevice"));
  LisaDevice* d = new LisaDevice();
  d->ordinal = ordinal;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, ordinal) == hipSuccess) {
    d->name = prop.name;
    d->arch = prop.gcnArchName;
    d->total_mem = prop.totalGlobalMem;
    d->cu_count = prop.multiProcessorCount;
  }
  const int rc = lisa_hip_check(hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking), "hipStreamCreate");
  if (rc) {
    delete d;
    return rc;
  }
  *out = d;
  return LISA_OK;
}

extern "C" void lisa_device_free(LisaDevice* d) {
  if (!d) return;
  (void)hipSetDevice(d->ordinal);
  (void)hipStreamSynchronize(d->stream);
  if (d->attn_ws) (void)hipFree(d->attn_ws);
  (void)hipStreamDestroy(d->stream);
  delete d;
}

extern "C" int lisa_device_name(LisaDevice* d, char* buf, size_t len) {
  if (!d || !buf || !len) return lisa_fail(LISA_E_ARG, "lisa_device_name: bad argument");
  std::snprintf(buf, len, "%s (%s, %d CUs)", d->name.c_str(), d->arch.c_str(), d->cu_count);
  return LISA_OK;
}

extern "C" uint64_t lisa_device_max_working_set(LisaDevice* d) { return d ? d->total_mem : 0; }

extern "C" int lisa_device_synchronize(LisaDevice* d) {
  if (!d) return lisa_fail(LISA_E_ARG, "null device");
  return lisa_hip_check(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
}

// ---------------------------------------------------------------------------
// buffers
// ---------------------------------------------------------------------------
extern "C" int lisa_buffer_alloc(LisaDevice* d, size_t len, LisaBuffer** out) {
  if (!d || !out) return lisa_fail(LISA_E_ARG, "lisa_buffer_alloc: bad argument");
  LisaBuffer* b = new LisaBuffer();
  b->dev = d;
  b->len = len;
  if (len) {
    const int rc = lisa_hip_check(hipMalloc(&b->ptr, len), "hipMalloc");
    if (rc) {
      delete b;
      return rc;
    }
    int rz = lisa_hip_check(hipMemsetAsync(b->ptr, 0, len, d->stream), "hipMemsetAsync");
    if (!rz) rz = lisa_hip_check(hipStreamSynchronize(d->stream), "hipStreamSynchronize");
    if (rz) {
      (void)hipFree(b->ptr);
      delete b;
      return rz;
    }
  }
  *out = b;
  return LISA_OK;
}

extern "C" void lisa_buffer_free(LisaBuffer* b) {
  if (!b) return;
  if (b->ptr) {
    (void)hipStreamSynchronize(b->dev->stream);
    (void)hipFree(b->ptr);
  }
  delete b;
}

extern "C" uint64_t lisa_buffer_device_ptr(const LisaBuffer* b) { return b ? (uint64_t)(uintptr_t)b->ptr : 0; }
extern "C" size_t lisa_buffer_len(const LisaBuffer* b) { return b ? b->len : 0; }

extern "C" int lisa_buffer_write(LisaBuffer* b, size_t off, const void* src, size_t len) {
  if (!b || (!src && len) || off + len > b->len || off + len < off)
    return lisa_fail(LISA_E_ARG, "lisa_buffer_write: range [%zu,+%zu) outside buffer of %zu", off, len,
                     b ? b->len : 0);
  if (!len) return LISA_OK;
  LISA_TRY(lisa_hip_check(hipMemcpyAsync((char*)b->ptr + off, src, len, hipMemcpyHostToDevice, b->dev->stream),
                          "hipMemcpyAsync H2D"));
  return lisa_hip_check(hipStreamSynchronize(b->dev->stream), "hipStreamSynchronize");
}

extern "C" int lisa_buffer_read(LisaBuffer* b, size_t off, void* dst, size_t len) {
  if (!b || (!dst && len) || off + len > b->len || off + len < off)
    return lisa_fail(LISA_E_ARG, "lisa_buffer_read: range [%zu,+%zu) outside buffer of %zu", off, len,
                     b ? b->len : 0);
  if (!len) return LISA_OK;
  LISA_TRY(lisa_hip_check(hipMemcpyAsync(dst, (const char*)b->ptr + off, len, hipMemcpyDeviceToHost, b->dev->stream),
                          "hipMemcpyAsync D2H"));
  return lisa_hip_check(hipStreamSynchronize(b->dev->stream), "hipStreamSynchronize");
}

extern "C" int lisa_buffer_copy(LisaBuffer* dst, size_t doff, const LisaBuffer* src, size_t soff, size_t len) {
  if (!dst || !src || doff + len > dst->len || soff + len > src->len)
    return lisa_fail(LISA_E_ARG, "lisa_buffer_copy: range outside buffers");
  if (!len) return LISA_OK;
  return lisa_hip_check(hipMemcpyAsync((char*)dst->ptr + doff, (const char*)src->ptr + soff, len,
                                       hipMemcpyDeviceToDevice, dst->dev->stream),
                        "hipMemcpyAsync D2D");
}

// ---------------------------------------------------------------------------
// modules and functions
// ---------------------------------------------------------------------------
extern "C" int lisa_module_load(LisaDevice* d, const char* path, LisaModule** out) {
  if (!d || !path || !out) return lisa_fail(LISA_E_ARG, "lisa_module_load: bad argument");
  hipModule_t m;
  const hipError_t e = hipModuleLoad(&m, path);
  if (e != hipSuccess) return lisa_fail(LISA_E_NOMODULE, "hipModuleLoad(%s): %s", path, hipGetErrorString(e));
  *out = new LisaModule{d, m};
  return LISA_OK;
}

extern "C" int lisa_module_load_data(LisaDevice* d, const void* blob, size_t len, LisaModule** out) {
  if (!d || !blob || !len || !out) return lisa_fail(LISA_E_ARG, "lisa_module_load_data: bad argument");
  hipModule_t m;
  const hipError_t e = hipModuleLoadData(&m, blob);
  if (e != hipSuccess) return lisa_fail(LISA_E_NOMODULE, "hipModuleLoadData: %s", hipGetErrorString(e));
  *out = new LisaModule{d, m};
  return LISA_OK;
}

std::string lisa_library_dir() {
  Dl_info info;
  if (dladdr((void*)&lisa_library_dir, &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    const size_t slash = p.rfind('/');
    if (slash != std::string::npos) return p.substr(0, slash);
  }
  return ".";
}

extern "C" int lisa_module_load_default(LisaDevice* d, LisaModule** out) {
  const std::string path = lisa_library_dir() + "/lisa_kernels.hsaco";
  return lisa_module_load(d, path.c_str(), out);
}

extern "C" void lisa_module_free(LisaModule* m) {
  if (!m) return;
  (void)hipModuleUnload(m->mod);
  delete m;
}

extern "C" int lisa_function_get(LisaModule* m, const char* name, LisaFunction** out) {
  if (!m || !name || !out) return lisa_fail(LISA_E_ARG, "lisa_function_get: bad argument");
  hipFunction_t f;
  const hipError_t e = hipModuleGetFunction(&f, m->mod, name);
  if (e != hipSuccess) return lisa_fail(LISA_E_NOMODULE, "kernel %s not found: %s", name, hipGetErrorString(e));
  *out = new LisaFunction{f, name};
  return LISA_OK;
}

// ---------------------------------------------------------------------------
// encoder: argument slots by index, launch on dispatch
// ---------------------------------------------------------------------------
extern "C" int lisa_encoder_begin(LisaDevice* d, LisaEncoder** out) {
  if (!d || !out) return lisa_fail(LISA_E_ARG, "lisa_encoder_begin: bad argument");
  LisaEncoder* e = new LisaEncoder();
  e->dev = d;
  *out = e;
  return LISA_OK;
}

extern "C" int lisa_encoder_set_function(LisaEncoder* e, LisaFunction* f) {
  if (!e || !f) return lisa_fail(LISA_E_ARG, "lisa_encoder_set_function: bad argument");
  e->fn = f;
  e->args.clear();
  return LISA_OK;
}

static int set_slot(LisaEncoder* e, uint32_t index, const void* bytes, size_t len) {
  if (index >= 64) return lisa_fail(LISA_E_ARG, "argument index %u out of range", index);
  if (e->args.size() <= index) e->args.resize(index + 1);
  e->args[index].assign((const uint8_t*)bytes, (const uint8_t*)bytes + len);
  return LISA_OK;
}

extern "C" int lisa_encoder_set_buffer(LisaEncoder* e, uint32_t index, const LisaBuffer* b, uint64_t offset) {
  if (!e || !b || offset > b->len) return lisa_fail(LISA_E_ARG, "lisa_encoder_set_buffer: bad argument");
  const uint64_t p = (uint64_t)(uintptr_t)b->ptr + offset;
  return set_slot(e, index, &p, sizeof p);
}

extern "C" int lisa_encoder_set_bytes(LisaEncoder* e, uint32_t index, const void* bytes, size_t len) {
  if (!e || (!bytes && len)) return lisa_fail(LISA_E_ARG, "lisa_encoder_set_bytes: bad argument");
  return set_slot(e, index, bytes, len);
}

int lisa_launch(LisaDevice* d, LisaFunction* f, const void* params, size_t len, uint32_t gx, uint32_t gy,
                uint32_t gz, uint32_t tx, uint32_t ty, uint32_t tz) {
  (void)len;
  if (!gx || !gy || !gz) return LISA_OK;
  void* args[1] = {const_cast<void*>(params)};
  if (d->prof) {
    LisaProfRec rec{d->prof_kind, nullptr, nullptr};
    LISA_TRY(lisa_hip_check(hipEventCreate(&rec.start), "hipEventCreate"));
    LISA_TRY(lisa_hip_check(hipEventCreate(&rec.stop), "hipEventCreate"));
    d->prof->push_back(rec);
    // global work sizes are in work-items
    const hipError_t e = hipExtModuleLaunchKernel(f->fn, gx * tx, gy * ty, gz * tz, tx, ty, tz, 0, d->stream, args,
                                                  nullptr, rec.start, rec.stop, 0);
    if (e != hipSuccess) return lisa_fail((int)e, "launch %s: %s", f->name.c_str(), hipGetErrorString(e));
    return LISA_OK;
  }
  const hipError_t e = hipModuleLaunchKernel(f->fn, gx, gy, gz, tx, ty, tz, 0, d->stream, args, nullptr);
  if (e != hipSuccess) return lisa_fail((int)e, "launch %s: %s", f->name.c_str(), hipGetErrorString(e));
  return LISA_OK;
}

extern "C" int lisa_encoder_dispatch_groups(LisaEncoder* e, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t tx,
                                            uint32_t ty, uint32_t tz) {
  if (!e || !e->fn) return lisa_fail(LISA_E_ARG, "dispatch without a function");
  std::vector<void*> ptrs(e->args.size());
  for (size_t i = 0; i < e->args.size(); ++i) {
    if (e->args[i].empty()) return lisa_fail(LISA_E_ARG, "argument %zu of %s not bound", i, e->fn->name.c_str());
    ptrs[i] = e->args[i].data();
  }
  if (!gx || !gy || !gz) return LISA_OK;
  const hipError_t r = hipModuleLaunchKernel(e->fn->fn, gx, gy, gz, tx, ty, tz, 0, e->dev->stream,
                                             ptrs.empty() ? nullptr : ptrs.data(), nullptr);
  if (r != hipSuccess) return lisa_fail((int)r, "launch %s: %s", e->fn->name.c_str(), hipGetErrorString(r));
  return LISA_OK;
}

extern "C" int lisa_encoder_dispatch_threads(LisaEncoder* e, uint32_t nx, uint32_t ny, uint32_t nz, uint32_t tx,
                                             uint32_t ty, uint32_t tz) {
  if (!tx || !ty || !tz) return lisa_fail(LISA_E_ARG, "zero threadgroup size");
  return lisa_encoder_dispatch_groups(e, (nx + tx - 1) / tx, (ny + ty - 1) / ty, (nz + tz - 1) / tz, tx, ty, tz);
}

extern "C" int lisa_encoder_end(LisaEncoder* e, int wait) {
  if (!e) return lisa_fail(LISA_E_ARG, "null encoder");
  int rc = LISA_OK;
  if (wait) rc = lisa_hip_check(hipStreamSynchronize(e->dev->stream), "hipStreamSynchronize");
  delete e;
  return rc;
}

// ---------------------------------------------------------------------------
// graphs and events
// ---------------------------------------------------------------------------
extern "C" int lisa_capture_begin(LisaDevice* d) {
  if (!d) return lisa_fail(LISA_E_ARG, "null device");
  return lisa_hip_check(hipStreamBeginCapture(d->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

extern "C" int lisa_capture_end(LisaDevice* d, LisaGraph** out) {
  if (!d || !out) return lisa_fail(LISA_E_ARG, "lisa_capture_end: bad argument");
  hipGraph_t g;
  LISA_TRY(lisa_hip_check(hipStreamEndCapture(d->stream, &g), "hipStreamEndCapture"));
  hipGraphExec_t x;
  const int rc = lisa_hip_check(hipGraphInstantiate(&x, g, nullptr, nullptr, 0), "hipGraphInstantiate");
  if (rc) {
    (void)hipGraphDestroy(g);
    return rc;
  }
  *out = new LisaGraph{g, x};
  return LISA_OK;
}

extern "C" int lisa_graph_launch(LisaGraph* g, LisaDevice* d) {
  if (!g || !d) return lisa_fail(LISA_E_ARG, "lisa_graph_launch: bad argument");
  return lisa_hip_check(hipGraphLaunch(g->exec, d->stream), "hipGraphLaunch");
}

extern "C" void lisa_graph_free(LisaGraph* g) {
  if (!g) return;
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  delete g;
}

extern "C" int lisa_event_create(LisaEvent** out) {
  if (!out) return lisa_fail(LISA_E_ARG, "null out");
  LisaEvent* e = new LisaEvent();
  const int rc = lisa_hip_check(hipEventCreate(&e->ev), "hipEventCreate");
  if (rc) {
    delete e;
    return rc;
  }
  *out = e;
  return LISA_OK;
}

extern "C" void lisa_event_free(LisaEvent* e) {
  if (!e) return;
  (void)hipEventDestroy(e->ev);
  delete e;
}

extern "C" int lisa_event_record(LisaEvent* e, LisaDevice* d) {
  if (!e || !d) return lisa_fail(LISA_E_ARG, "lisa_event_record: bad argument");
  return lisa_hip_check(hipEventRecord(e->ev, d->stream), "hipEventRecord");
}

extern "C" int lisa_event_elapsed_ms(LisaEvent* a, LisaEvent* b, float* ms) {
  if (!a || !b || !ms) return lisa_fail(LISA_E_ARG, "lisa_event_elapsed_ms: bad argument");
  LISA_TRY(lisa_hip_check(hipEventSynchronize(b->ev), "hipEventSynchronize"));
  return lisa_hip_check(hipEventElapsedTime(ms, a->ev, b->ev), "hipEventElapsedTime");
}
