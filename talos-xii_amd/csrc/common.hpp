// common.hpp -- internal helpers shared by the HIP translation units of libtalos_hip.so:
// status reporting, host-side argument validation and the small device utilities
// (wave64 reductions, f64 partial combination) every kernel family uses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/talos_hip.h"

namespace talos {

// Thread-local message of the last failure (talos_last_error).
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
const char* last_error();

// Lazily initialises the device context; returns TALOS_OK or TALOS_ERR_NO_DEVICE.
int ensure_device();

inline hipStream_t as_stream(talos_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Returns TALOS_ERR_HIP with the runtime's message when e != hipSuccess.
int hip_status(hipError_t e, const char* what);

// The last step of every kernel entry point. In the calling thread's default mode the entry is
// synchronous, as the reference's Tensor ops return finished results: it waits for its stream and
// returns the stream's error, if any. After talos_set_async(1) on the thread it returns rc as soon
// as the work is enqueued. A non-zero rc is returned at once in both modes.
int entry_done(int rc, hipStream_t s);

// Checks the launch that was just enqueued.
int launch_status(const char* kernel);

// Per-launch event profiling (talos_plan_profile): when a profiler is active on the calling
// thread, every kernel launch is bracketed by two HIP events on its stream and tagged with the
// kernel's name and its algorithmic flops / bytes.
struct Profiler;
Profiler* profiler_new();
void profiler_delete(Profiler* p);
void profiler_set_current(Profiler* p);  // thread-local; nullptr switches profiling off
int prof_begin(hipStream_t s, const char* kernel, double flops, double bytes);
void prof_end(hipStream_t s, int idx);

// Scratch of a kernel-level entry point: the workspace the caller bound on this thread
// (talos_workspace_bind) when it holds `bytes`, else a stream-ordered allocation that release()
// frees on the same stream. acquire(0) takes nothing.
struct EntryScratch {
  void* ptr = nullptr;
  bool owned = false;
  hipStream_t s = nullptr;
  int acquire(size_t bytes, hipStream_t stream);
  int release();
  ~EntryScratch() { (void)release(); }
};
// The bytes of the workspace bound on this thread (0 when none), and a note of a call's need
// for talos_workspace_high_water.
size_t bound_workspace_bytes();
void note_workspace_need(size_t bytes);

struct ProfScope {
  hipStream_t s;
  int idx;
  ProfScope(hipStream_t s_, const char* kernel, double flops, double bytes)
      : s(s_), idx(prof_begin(s_, kernel, flops, bytes)) {}
  ~ProfScope() { prof_end(s, idx); }
};

}  // namespace talos

// Host-side validation: every entry point checks its arguments before touching the device,
// so the error paths run on machines without a GPU.
#define TALOS_REQUIRE(cond, code, ...)   \
  do {                                   \
    if (!(cond)) {                       \
      ::talos::set_error(__VA_ARGS__);   \
      return (code);                     \
    }                                    \
  } while (0)

#define TALOS_NONNULL(p) TALOS_REQUIRE((p) != nullptr, TALOS_ERR_NULL, "%s: null pointer argument '%s'", __func__, #p)

#define TALOS_DEVICE()                          \
  do {                                          \
    int _rc = ::talos::ensure_device();         \
    if (_rc != TALOS_OK) return _rc;            \
  } while (0)

#define TALOS_HIP(call)                                         \
  do {                                                          \
    int _rc = ::talos::hip_status((call), #call);               \
    if (_rc != TALOS_OK) return _rc;                            \
  } while (0)

#define TALOS_LAUNCHED(name)                          \
  do {                                                \
    int _rc = ::talos::launch_status(name);           \
    if (_rc != TALOS_OK) return _rc;                  \
  } while (0)

namespace talos {

// ---------------------------------------------------------------------------
// Device utilities
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Block-wide sum for blockDim.x <= 1024 (multiple of 64); every thread gets the result.
// red must hold blockDim.x / 64 elements.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, nw = blockDim.x / kWave;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  T t = 0;
  for (int i = 0; i < nw; ++i) t += red[i];
  return t;
}

// Phi(x), the standard normal CDF, and e = exp(-x^2 / 2). erf(z) for z >= 0 by Abramowitz &
// Stegun 7.1.26 (Hastings): erf(z) = 1 - t (a1 + t (a2 + t (a3 + t (a4 + t a5)))) exp(-z^2),
// t = 1 / (1 + p z), |error| <= 1.5e-7; with z = |x| / sqrt(2), exp(-z^2) is the same
// exp(-x^2 / 2) the density needs, so GELU and its derivative take one exponential. The lower
// tail 0.5 erfc(z) is formed directly (no cancellation for x < 0). t is the hardware reciprocal
// (v_rcp_f32, about 1 ulp on [1, inf)): a correctly rounded one is the ten-instruction division
// sequence, a third of the epilogue's per-element work, for an error far below the formula's.
__device__ __forceinline__ float normal_cdf(float x, float* e) {
  const float z = fabsf(x) * 0.70710678118654752f;
  *e = __expf(-0.5f * x * x);  // hardware exp2 of the scaled argument: relative error ~|x^2| 2^-24
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.0f));
  const float poly =
      t * fmaf(t, fmaf(t, fmaf(t, fmaf(t, 1.061405429f, -1.453152027f), 1.421413741f), -0.284496736f), 0.254829592f);
  const float tail = 0.5f * poly * *e;  // P(X > |x|)
  return x >= 0.f ? 1.0f - tail : tail;
}
__device__ __forceinline__ float gelu_f(float x) {
  float e;
  return x * normal_cdf(x, &e);
}
// d/dx of x * Phi(x) = Phi(x) + x * phi(x)
__device__ __forceinline__ float gelu_d(float x) {
  float e;
  const float cdf = normal_cdf(x, &e);
  return cdf + x * (0.39894228040143268f * e);
}
// gelu(x) = x * Phi(x), and *d = gelu'(x), sharing the exponential
__device__ __forceinline__ float gelu_fd(float x, float* d) {
  float e;
  const float cdf = normal_cdf(x, &e);
  *d = cdf + x * (0.39894228040143268f * e);
  return x * cdf;
}

inline unsigned ceil_div(size_t a, size_t b) { return (unsigned)((a + b - 1) / b); }

// The last token of sample b of a [batch, S] token grid: row lens[b] - 1 with lens clamped to
// [1, S], or S - 1 without lens (last_token, src/transformer.rs:92-109).
__device__ __forceinline__ int last_row(const int32_t* lens, int b, int S) {
  if (lens == nullptr) return S - 1;
  const int L = lens[b];
  return (L < 1 ? 1 : (L > S ? S : L)) - 1;
}

}  // namespace talos
