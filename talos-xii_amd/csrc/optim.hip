// optim.hip -- the optimizer step of the training loop: Adam over a flat parameter buffer
// (src/ppo.rs:519-533) and the global-norm gradient clip that the DQN trainer applies first
// (src/dqn.rs:207-225).
//
// Both kernels are HBM-bound element-wise passes. Per parameter the Adam step reads the
// gradient (4 B), reads and writes the parameter, m and v (3 x 8 B): 28 B. The squared-norm
// pass reads the gradient once (4 B). Each thread handles four consecutive parameters with
// 16-byte loads and stores when every buffer is 16-byte aligned; the arithmetic runs in f64
// (the reference keeps m, v and the update in f64) and rounds to fp32 once, on the store.
#include <algorithm>
#include <cmath>

#include "common.hpp"

namespace talos {
namespace {

// Bounded number of f64 partial sums of the squared-norm pass (fixed partition: the result
// does not depend on timing).
constexpr int kSumsqParts = 512;

struct AdamArgs {
  double lr, b1, b2, omb1, omb2, eps, bc1, bc2, max_norm;
};

template <bool VEC>
__global__ __launch_bounds__(256) void sumsq_partial_kernel(size_t n, const float* __restrict__ g,
                                                            double* __restrict__ part) {
  __shared__ double red[4];
  double s = 0.0;
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  size_t tail = 0;
  if (VEC) {
    const size_t n4 = n / 4;
    const float4* g4 = reinterpret_cast<const float4*>(g);
    for (size_t i = tid; i < n4; i += stride) {
      const float4 x = g4[i];
      s += (double)x.x * x.x + (double)x.y * x.y + (double)x.z * x.z + (double)x.w * x.w;
    }
    tail = n4 * 4;
  }
  for (size_t i = tail + tid; i < n; i += stride) s += (double)g[i] * g[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ __launch_bounds__(512) void sumsq_final_kernel(int nparts, int accumulate, const double* __restrict__ part,
                                                          double* __restrict__ out) {
  __shared__ double red[8];
  double s = 0.0;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) s += part[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) out[0] = accumulate ? out[0] + s : s;
}

// One parameter: src/ppo.rs:526-530 with g already scaled by the clip coefficient
// (src/dqn.rs:226).
__device__ __forceinline__ void adam_one(float& p, float gf, float& m, float& v, const AdamArgs& a, double coef) {
  const double g = (double)gf * coef;
  const double mn = a.b1 * (double)m + a.omb1 * g;
  const double vn = a.b2 * (double)v + a.omb2 * g * g;
  const double m_hat = mn / a.bc1, v_hat = vn / a.bc2;
  p = (float)((double)p - a.lr * m_hat / (sqrt(v_hat) + a.eps));
  m = (float)mn;
  v = (float)vn;
}

template <bool CLIP, bool VEC>
__global__ __launch_bounds__(256) void adam_kernel(size_t n, float* __restrict__ p, const float* __restrict__ g,
                                                   float* __restrict__ m, float* __restrict__ v, AdamArgs a,
                                                   const double* __restrict__ sumsq) {
  double coef = 1.0;
  if (CLIP) {
    // src/dqn.rs:215-220: clip_coef = max_norm / ||g|| when ||g|| > max_norm (max_norm is 1.0 there)
    const double norm = sqrt(sumsq[0]);
    if (norm > a.max_norm) coef = a.max_norm / norm;
  }
  const size_t tid = (size_t)blockIdx.x * blockDim.x + threadIdx.x, stride = (size_t)gridDim.x * blockDim.x;
  size_t tail = 0;
  if (VEC) {
    const size_t n4 = n / 4;
    float4* p4 = reinterpret_cast<float4*>(p);
    float4* m4 = reinterpret_cast<float4*>(m);
    float4* v4 = reinterpret_cast<float4*>(v);
    const float4* g4 = reinterpret_cast<const float4*>(g);
    for (size_t i = tid; i < n4; i += stride) {
      float4 pp = p4[i], mm = m4[i], vv = v4[i];
      const float4 gg = g4[i];
      adam_one(pp.x, gg.x, mm.x, vv.x, a, coef);
      adam_one(pp.y, gg.y, mm.y, vv.y, a, coef);
      adam_one(pp.z, gg.z, mm.z, vv.z, a, coef);
      adam_one(pp.w, gg.w, mm.w, vv.w, a, coef);
      p4[i] = pp;
      m4[i] = mm;
      v4[i] = vv;
    }
    tail = n4 * 4;
  }
  for (size_t i = tail + tid; i < n; i += stride) adam_one(p[i], g[i], m[i], v[i], a, coef);
}

unsigned elementwise_grid(size_t units, unsigned cap) {
  const size_t b = (units + 255) / 256;
  return (unsigned)std::max<size_t>(1, std::min<size_t>(b, cap));
}

}  // namespace

int grad_sumsq_launch(size_t n, const float* g, int accumulate, double* sumsq, double* part, hipStream_t s) {
  const bool vec = ((uintptr_t)g & 15) == 0;
  const unsigned nparts = elementwise_grid(vec ? (n + 3) / 4 : n, kSumsqParts);
  {
    ProfScope ps(s, "sumsq_partial_kernel", 2.0 * n, 4.0 * n + 8.0 * nparts);
    if (vec)
      hipLaunchKernelGGL(sumsq_partial_kernel<true>, dim3(nparts), dim3(256), 0, s, n, g, part);
    else
      hipLaunchKernelGGL(sumsq_partial_kernel<false>, dim3(nparts), dim3(256), 0, s, n, g, part);
    TALOS_LAUNCHED("sumsq_partial_kernel");
  }
  ProfScope ps(s, "sumsq_final_kernel", (double)nparts, 8.0 * nparts + 16.0);
  hipLaunchKernelGGL(sumsq_final_kernel, dim3(1), dim3(512), 0, s, (int)nparts, accumulate, part, sumsq);
  TALOS_LAUNCHED("sumsq_final_kernel");
  return TALOS_OK;
}

int adam_launch(size_t n, float* p, const float* g, float* m, float* v, int t, double lr, double beta1, double beta2,
                double eps, const double* sumsq, double max_norm, hipStream_t s) {
  if (n == 0) return TALOS_OK;
  AdamArgs a;
  a.lr = lr;
  a.b1 = beta1;
  a.b2 = beta2;
  a.omb1 = 1.0 - beta1;
  a.omb2 = 1.0 - beta2;
  a.eps = eps;
  // src/ppo.rs:528-529: 1 - beta^t with t the step count after the increment (powi)
  a.bc1 = 1.0 - std::pow(beta1, t);
  a.bc2 = 1.0 - std::pow(beta2, t);
  a.max_norm = max_norm;
  const bool vec = ((uintptr_t)p & 15) == 0 && ((uintptr_t)g & 15) == 0 && ((uintptr_t)m & 15) == 0 &&
                   ((uintptr_t)v & 15) == 0;
  const unsigned grid = elementwise_grid(vec ? (n + 3) / 4 : n, 16384);
  ProfScope ps(s, "adam_kernel", 12.0 * n, 28.0 * n);
  if (sumsq) {
    if (vec)
      hipLaunchKernelGGL((adam_kernel<true, true>), dim3(grid), dim3(256), 0, s, n, p, g, m, v, a, sumsq);
    else
      hipLaunchKernelGGL((adam_kernel<true, false>), dim3(grid), dim3(256), 0, s, n, p, g, m, v, a, sumsq);
  } else {
    if (vec)
      hipLaunchKernelGGL((adam_kernel<false, true>), dim3(grid), dim3(256), 0, s, n, p, g, m, v, a, sumsq);
    else
      hipLaunchKernelGGL((adam_kernel<false, false>), dim3(grid), dim3(256), 0, s, n, p, g, m, v, a, sumsq);
  }
  TALOS_LAUNCHED("adam_kernel");
  return TALOS_OK;
}

size_t grad_sumsq_workspace_bytes() { return kSumsqParts * sizeof(double); }

}  // namespace talos

using namespace talos;

extern "C" {

size_t talos_grad_sumsq_workspace_bytes(void) { return grad_sumsq_workspace_bytes(); }

int talos_grad_sumsq_f32(size_t n, const float* grads, int accumulate, double* sumsq, double* workspace,
                         talos_stream_t stream) {
  TALOS_NONNULL(sumsq);
  TALOS_REQUIRE(n == 0 || grads != nullptr, TALOS_ERR_NULL, "%s: null pointer argument 'grads'", __func__);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  if (workspace) return grad_sumsq_launch(n, grads, accumulate, sumsq, workspace, s);
  EntryScratch ws;
  if (int rc = ws.acquire(grad_sumsq_workspace_bytes(), s)) return rc;
  const int rc = grad_sumsq_launch(n, grads, accumulate, sumsq, static_cast<double*>(ws.ptr), s);
  const int rel = ws.release();
  return entry_done(rc ? rc : rel, as_stream(stream));
}

int talos_adam_step_f32(size_t n, float* params, const float* grads, float* m, float* v, int t, double lr,
                        double beta1, double beta2, double eps, const double* sumsq, double max_norm,
                        talos_stream_t stream) {
  TALOS_REQUIRE(t >= 1, TALOS_ERR_SHAPE, "%s: step count t=%d must be >= 1 (the first step is t=1)", __func__, t);
  TALOS_REQUIRE(beta1 >= 0.0 && beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0, TALOS_ERR_SHAPE,
                "%s: betas (%g, %g) outside [0, 1)", __func__, beta1, beta2);
  TALOS_REQUIRE(!sumsq || max_norm > 0.0, TALOS_ERR_SHAPE, "%s: max_norm=%g must be > 0 when clipping", __func__,
                max_norm);
  if (n == 0) return TALOS_OK;
  TALOS_NONNULL(params);
  TALOS_NONNULL(grads);
  TALOS_NONNULL(m);
  TALOS_NONNULL(v);
  TALOS_DEVICE();
  const int rc = adam_launch(n, params, grads, m, v, t, lr, beta1, beta2, eps, sumsq, max_norm, as_stream(stream));
  return entry_done(rc, as_stream(stream));
}

}  // extern "C"
