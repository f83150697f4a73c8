// runtime.hip -- device context, allocation, copies and status reporting of libtalos_hip.so.
//
// The reference keeps tensors in host f64 vectors (Tensor.data / Tensor.grad,
// src/autograd.rs:14-20) and runs ops synchronously on the calling thread. Here tensors live in
// device memory as fp32; the _f64 copies convert at the host/device boundary, and kernel entry
// points enqueue on the caller's stream (talos_stream_sync waits for them).
#include <mutex>
#include <cstdarg>
#include <vector>

#include "common.hpp"

namespace talos {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

const char* last_error() { return g_last_error.c_str(); }

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return TALOS_OK;
  set_error("%s failed: %s", what, hipGetErrorString(e));
  return TALOS_ERR_HIP;
}

// Per-thread completion mode of the kernel entry points (false: synchronous, the default).
static thread_local bool t_async = false;

int entry_done(int rc, hipStream_t s) {
  if (rc != TALOS_OK || t_async) return rc;
  return hip_status(hipStreamSynchronize(s), "kernel entry (synchronous mode): hipStreamSynchronize");
}

int launch_status(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return TALOS_OK;
  set_error("launch of %s failed: %s", kernel, hipGetErrorString(e));
  return TALOS_ERR_HIP;
}

// The caller-owned workspace of the kernel-level entry points on this thread.
static thread_local void* t_ws = nullptr;
static thread_local size_t t_ws_bytes = 0;
static thread_local size_t t_ws_high = 0;

size_t bound_workspace_bytes() { return t_ws ? t_ws_bytes : 0; }
void note_workspace_need(size_t bytes) {
  if (bytes > t_ws_high) t_ws_high = bytes;
}

int EntryScratch::acquire(size_t bytes, hipStream_t stream) {
  s = stream;
  if (bytes == 0) return TALOS_OK;
  note_workspace_need(bytes);
  if (t_ws && bytes <= t_ws_bytes) {
    ptr = t_ws;
    owned = false;
    return TALOS_OK;
  }
  TALOS_HIP(hipMallocAsync(&ptr, bytes, stream));
  owned = true;
  return TALOS_OK;
}

int EntryScratch::release() {
  if (!owned || !ptr) return TALOS_OK;
  const hipError_t e = hipFreeAsync(ptr, s);
  ptr = nullptr;
  owned = false;
  return hip_status(e, "hipFreeAsync");
}

static std::once_flag g_init_once;
static int g_init_status = TALOS_OK;
static std::string g_init_error;

int ensure_device() {
  std::call_once(g_init_once, [] {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
      g_init_status = TALOS_ERR_NO_DEVICE;
      g_init_error = std::string("no usable GPU (hipGetDeviceCount: ") +
                     (e == hipSuccess ? "0 devices" : hipGetErrorString(e)) + ")";
      return;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) == hipSuccess) {
      std::string arch = prop.gcnArchName;
      if (arch.rfind("gfx950", 0) != 0) {
        g_init_status = TALOS_ERR_NO_DEVICE;
        g_init_error = "device 0 is " + arch + "; this library is built for gfx950 (MI355X) only";
      }
    }
  });
  if (g_init_status != TALOS_OK) set_error("%s", g_init_error.c_str());
  return g_init_status;
}

// ---------------------------------------------------------------------------
// Per-launch profiler
// ---------------------------------------------------------------------------
struct ProfRec {
  std::string kernel;
  double flops, bytes;
  hipEvent_t a, b;
};
struct Profiler {
  bool enabled = false;
  std::string filter;
  std::vector<ProfRec> recs;
  std::vector<hipEvent_t> pool;
  size_t used = 0;
};

static thread_local Profiler* g_prof = nullptr;

Profiler* profiler_new() { return new Profiler(); }

void profiler_delete(Profiler* p) {
  if (!p) return;
  for (hipEvent_t e : p->pool) (void)hipEventDestroy(e);
  delete p;
}

void profiler_set_current(Profiler* p) { g_prof = p; }

static hipEvent_t next_event(Profiler* p) {
  if (p->used == p->pool.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    p->pool.push_back(e);
  }
  return p->pool[p->used++];
}

int prof_begin(hipStream_t s, const char* kernel, double flops, double bytes) {
  Profiler* p = g_prof;
  if (!p || !p->enabled) return -1;
  if (!p->filter.empty() && std::string(kernel).find(p->filter) == std::string::npos) return -1;
  hipEvent_t a = next_event(p), b = next_event(p);
  if (!a || !b) return -1;
  (void)hipEventRecord(a, s);
  p->recs.push_back(ProfRec{kernel, flops, bytes, a, b});
  return (int)p->recs.size() - 1;
}

void prof_end(hipStream_t s, int idx) {
  Profiler* p = g_prof;
  if (idx < 0 || !p || idx >= (int)p->recs.size()) return;
  (void)hipEventRecord(p->recs[idx].b, s);
}

}  // namespace talos

using namespace talos;

extern "C" {

int talos_profiler_enable(talos_profiler prof, int enable, const char* kernel_filter) {
  TALOS_NONNULL(prof);
  Profiler* p = reinterpret_cast<Profiler*>(prof);
  if (enable) {
    TALOS_DEVICE();
    TALOS_HIP(hipDeviceSynchronize());
    p->recs.clear();
    p->used = 0;
    p->filter = kernel_filter ? kernel_filter : "";
  }
  p->enabled = enable != 0;
  return TALOS_OK;
}

int talos_profiler_read(talos_profiler prof, talos_prof_record* out, int max_records, int* count) {
  TALOS_NONNULL(prof);
  TALOS_NONNULL(count);
  TALOS_DEVICE();
  Profiler* p = reinterpret_cast<Profiler*>(prof);
  *count = (int)p->recs.size();
  for (int i = 0; i < (int)p->recs.size() && i < max_records; ++i) {
    TALOS_NONNULL(out);
    const ProfRec& r = p->recs[i];
    TALOS_HIP(hipEventSynchronize(r.b));
    float ms = 0.f;
    TALOS_HIP(hipEventElapsedTime(&ms, r.a, r.b));
    snprintf(out[i].kernel, sizeof(out[i].kernel), "%s", r.kernel.c_str());
    out[i].flops = r.flops;
    out[i].bytes = r.bytes;
    out[i].ms = ms;
  }
  return TALOS_OK;
}

const char* talos_last_error(void) { return last_error(); }

const char* talos_version(void) { return "talos_hip 0.1 (gfx950)"; }

int talos_init(void) { return ensure_device(); }

int talos_device_count(int* count) {
  TALOS_NONNULL(count);
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *count = n;
  return TALOS_OK;
}

int talos_malloc(void** ptr, size_t bytes) {
  TALOS_NONNULL(ptr);
  TALOS_DEVICE();
  *ptr = nullptr;
  if (bytes == 0) return TALOS_OK;
  hipError_t e = hipMalloc(ptr, bytes);
  if (e != hipSuccess) {
    set_error("hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    *ptr = nullptr;
    return TALOS_ERR_ALLOC;
  }
  return TALOS_OK;
}

int talos_free(void* ptr) {
  if (ptr == nullptr) return TALOS_OK;
  TALOS_DEVICE();
  TALOS_HIP(hipFree(ptr));
  return TALOS_OK;
}

int talos_memcpy_h2d(void* dst, const void* src, size_t bytes, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_NONNULL(src);
  TALOS_DEVICE();
  TALOS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream)));
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  return TALOS_OK;
}

int talos_memcpy_d2h(void* dst, const void* src, size_t bytes, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_NONNULL(src);
  TALOS_DEVICE();
  TALOS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream)));
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  return TALOS_OK;
}

int talos_memcpy_d2d(void* dst, const void* src, size_t bytes, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_NONNULL(src);
  TALOS_DEVICE();
  TALOS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream)));
  return TALOS_OK;
}

int talos_memcpy_h2d_f64(float* dst, const double* src, size_t n, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_NONNULL(src);
  TALOS_DEVICE();
  std::vector<float> tmp(n);
  for (size_t i = 0; i < n; ++i) tmp[i] = (float)src[i];
  TALOS_HIP(hipMemcpyAsync(dst, tmp.data(), n * sizeof(float), hipMemcpyHostToDevice, as_stream(stream)));
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  return TALOS_OK;
}

int talos_memcpy_d2h_f64(double* dst, const float* src, size_t n, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_NONNULL(src);
  TALOS_DEVICE();
  std::vector<float> tmp(n);
  TALOS_HIP(hipMemcpyAsync(tmp.data(), src, n * sizeof(float), hipMemcpyDeviceToHost, as_stream(stream)));
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  for (size_t i = 0; i < n; ++i) dst[i] = (double)tmp[i];
  return TALOS_OK;
}

int talos_set_async(int on) {
  TALOS_REQUIRE(on == 0 || on == 1, TALOS_ERR_SHAPE, "%s: on must be 0 or 1", __func__);
  t_async = on != 0;
  return TALOS_OK;
}

int talos_get_async(void) { return t_async ? 1 : 0; }

int talos_stream_sync(talos_stream_t stream) {
  TALOS_DEVICE();
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  return TALOS_OK;
}

int talos_stream_create(talos_stream_t* stream) {
  TALOS_NONNULL(stream);
  TALOS_DEVICE();
  hipStream_t s = nullptr;
  TALOS_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = reinterpret_cast<talos_stream_t>(s);
  return TALOS_OK;
}

int talos_stream_destroy(talos_stream_t stream) {
  if (stream == nullptr) return TALOS_OK;
  TALOS_DEVICE();
  TALOS_HIP(hipStreamDestroy(as_stream(stream)));
  return TALOS_OK;
}

// Events for timing the work enqueued on a stream (bench.py measures kernels with these on
// the stream they run on).
int talos_event_create(void** ev) {
  TALOS_NONNULL(ev);
  TALOS_DEVICE();
  hipEvent_t e = nullptr;
  TALOS_HIP(hipEventCreate(&e));
  *ev = reinterpret_cast<void*>(e);
  return TALOS_OK;
}

int talos_event_destroy(void* ev) {
  if (ev == nullptr) return TALOS_OK;
  TALOS_DEVICE();
  TALOS_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  return TALOS_OK;
}

int talos_event_record(void* ev, talos_stream_t stream) {
  TALOS_NONNULL(ev);
  TALOS_DEVICE();
  TALOS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), as_stream(stream)));
  return TALOS_OK;
}

int talos_event_elapsed_ms(void* start, void* stop, float* ms) {
  TALOS_NONNULL(start);
  TALOS_NONNULL(stop);
  TALOS_NONNULL(ms);
  TALOS_DEVICE();
  TALOS_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(stop)));
  TALOS_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(stop)));
  return TALOS_OK;
}

int talos_workspace_bind(void* ptr, size_t bytes) {
  TALOS_REQUIRE(ptr != nullptr || bytes == 0, TALOS_ERR_NULL, "%s: null buffer of %zu bytes", __func__, bytes);
  TALOS_REQUIRE((reinterpret_cast<uintptr_t>(ptr) & 255) == 0, TALOS_ERR_SHAPE,
                "%s: the workspace must be 256-byte aligned", __func__);
  t_ws = bytes ? ptr : nullptr;
  t_ws_bytes = bytes;
  t_ws_high = 0;
  return TALOS_OK;
}

size_t talos_workspace_high_water(void) { return t_ws_high; }

size_t talos_workspace_bytes(void) { return bound_workspace_bytes(); }

int talos_device_info(char* name, size_t name_len, int* cu_count, int* clock_khz, size_t* total_mem) {
  TALOS_DEVICE();
  hipDeviceProp_t prop;
  TALOS_HIP(hipGetDeviceProperties(&prop, 0));
  // some drivers report no marketing name: fall back to the architecture and CU count
  if (name && name_len) {
    if (prop.name[0])
      snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
    else
      snprintf(name, name_len, "AMD GPU with %d CUs (%s)", prop.multiProcessorCount, prop.gcnArchName);
  }
  if (cu_count) *cu_count = prop.multiProcessorCount;
  if (clock_khz) *clock_khz = prop.clockRate;
  if (total_mem) *total_mem = prop.totalGlobalMem;
  return TALOS_OK;
}

}  // extern "C"
