// ppo_update.hip -- PPO::update on the device (src/ppo.rs:625-770): the f64 GAE and advantage
// normalisation prologue, then the epoch / minibatch / Adam loop with the KL early stop, over
// the PPO plan's minibatch entry.
//
// GAE is the backward linear recurrence A_t = d_t + c_t * A_{t+1} (c_t = gamma * lambda *
// (1 - done_t), A_len = 0). One workgroup of 1024 threads evaluates it as a scan: each thread
// composes the affine map of its contiguous chunk (x_lo = D + C * x_hi), a suffix scan over the
// 1024 maps in LDS gives every chunk the value entering it from the right, and each thread then
// replays its chunk. All arithmetic is f64, as in the reference; only the association of the
// products differs from its sequential loop.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "plans.hpp"

namespace talos {
namespace {

constexpr int kGaeThreads = 1024;

struct GaeArgs {
  int len;
  const double* rew;
  const double* val;
  const uint8_t* term;
  double r_mean, r_den, r_clip, gamma, gl;
  float* adv;
  float* ret;
  double* adv_raw;
};

// d_t and c_t of the recurrence (src/ppo.rs:653-667).
__device__ __forceinline__ void gae_terms(const GaeArgs& g, int t, double& d, double& c) {
  double r = (g.rew[t] - g.r_mean) / g.r_den;  // RunningMeanStd::normalize, src/ppo.rs:477-479
  r = fmin(fmax(r, -g.r_clip), g.r_clip);
  const double nonterm = g.term[t] ? 0.0 : 1.0;
  const double v_next = t + 1 < g.len ? g.val[t + 1] : 0.0;
  d = r + g.gamma * v_next * nonterm - g.val[t];
  c = g.gl * nonterm;
}

__global__ __launch_bounds__(kGaeThreads) void gae_kernel(GaeArgs g) {
  __shared__ double sc[kGaeThreads], sd[kGaeThreads];
  __shared__ double red[kGaeThreads / 64];
  const int t = threadIdx.x;
  const int chunk = (g.len + kGaeThreads - 1) / kGaeThreads;
  const int lo = min(g.len, t * chunk), hi = min(g.len, lo + chunk);
  // the chunk's map x_lo = D + C * x_hi
  double C = 1.0, D = 0.0;
  for (int i = hi - 1; i >= lo; --i) {
    double d, c;
    gae_terms(g, i, d, c);
    D = d + c * D;
    C = c * C;
  }
  sc[t] = C;
  sd[t] = D;
  __syncthreads();
  // inclusive suffix scan: map of chunks t .. end, (C1, D1) o (C2, D2) = (C1 C2, D1 + C1 D2)
  for (int off = 1; off < kGaeThreads; off <<= 1) {
    double c2 = 1.0, d2 = 0.0;
    if (t + off < kGaeThreads) {
      c2 = sc[t + off];
      d2 = sd[t + off];
    }
    __syncthreads();
    D = D + C * d2;
    C = C * c2;
    sc[t] = C;
    sd[t] = D;
    __syncthreads();
  }
  // the value entering this chunk from the right: A at index hi (0 past the end)
  const double x_hi = t + 1 < kGaeThreads ? sd[t + 1] : 0.0;
  // replay: A_t, the return and the sum for the mean
  double x = x_hi, sum = 0.0;
  for (int i = hi - 1; i >= lo; --i) {
    double d, c;
    gae_terms(g, i, d, c);
    x = d + c * x;
    sum += x;
    g.ret[i] = (float)(x + g.val[i]);
    if (g.adv_raw) g.adv_raw[i] = x;
  }
  const double mean = block_sum(sum, red) / (double)g.len;
  // population std + 1e-8 (src/ppo.rs:674-675)
  x = x_hi;
  double ss = 0.0;
  for (int i = hi - 1; i >= lo; --i) {
    double d, c;
    gae_terms(g, i, d, c);
    x = d + c * x;
    ss += (x - mean) * (x - mean);
  }
  const double stdv = sqrt(block_sum(ss, red) / (double)g.len) + 1e-8;
  x = x_hi;
  for (int i = hi - 1; i >= lo; --i) {
    double d, c;
    gae_terms(g, i, d, c);
    x = d + c * x;
    g.adv[i] = (float)((x - mean) / stdv);
  }
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Work buffer: stats (doubles) | adv[n] | ret[n] | grads[params] | loss[1]
struct UpdateWork {
  double* stats;
  float *adv, *ret, *grads, *loss;
  size_t bytes;
};
UpdateWork update_work(void* base, int n, size_t n_params) {
  const size_t o_adv = align_up(TALOS_PPO_NSTATS * sizeof(double));
  const size_t o_ret = o_adv + align_up((size_t)n * sizeof(float));
  const size_t o_grads = o_ret + align_up((size_t)n * sizeof(float));
  const size_t o_loss = o_grads + align_up(n_params * sizeof(float));
  UpdateWork w{};
  w.bytes = o_loss + align_up(sizeof(float));
  if (base != nullptr) {
    char* p = static_cast<char*>(base);
    w.stats = reinterpret_cast<double*>(p);
    w.adv = reinterpret_cast<float*>(p + o_adv);
    w.ret = reinterpret_cast<float*>(p + o_ret);
    w.grads = reinterpret_cast<float*>(p + o_grads);
    w.loss = reinterpret_cast<float*>(p + o_loss);
  }
  return w;
}

}  // namespace

int gae_launch(int len, const double* rewards, const double* values, const uint8_t* terminals, double r_mean,
               double r_var, double r_clip, double gamma, double lambda, float* adv, float* ret, double* adv_raw,
               hipStream_t s) {
  if (len == 0) return TALOS_OK;
  GaeArgs g;
  g.len = len;
  g.rew = rewards;
  g.val = values;
  g.term = terminals;
  g.r_mean = r_mean;
  g.r_den = std::sqrt(r_var) + 1e-8;
  g.r_clip = r_clip;
  g.gamma = gamma;
  g.gl = gamma * lambda;
  g.adv = adv;
  g.ret = ret;
  g.adv_raw = adv_raw;
  // three f64 passes over the rollout, 8 + 8 + 1 B read and 4 + 4 (+ 8) B written per step
  ProfScope ps(s, "gae_kernel", 30.0 * len, (double)len * (17.0 * 3.0 + 8.0 + (adv_raw ? 8.0 : 0.0)));
  hipLaunchKernelGGL(gae_kernel, dim3(1), dim3(kGaeThreads), 0, s, g);
  TALOS_LAUNCHED("gae_kernel");
  return TALOS_OK;
}

}  // namespace talos

using namespace talos;

extern "C" {

int talos_ppo_gae_f64(int len, const double* rewards, const double* values, const uint8_t* terminals, double r_mean,
                      double r_var, double r_clip, double gamma, double lambda, float* adv, float* ret,
                      double* adv_raw, talos_stream_t stream) {
  TALOS_REQUIRE(len >= 0, TALOS_ERR_SHAPE, "%s: len=%d < 0", __func__, len);
  TALOS_REQUIRE(r_var >= 0.0 && r_clip >= 0.0, TALOS_ERR_SHAPE, "%s: r_var and r_clip must be >= 0", __func__);
  if (len == 0) return TALOS_OK;
  TALOS_NONNULL(rewards);
  TALOS_NONNULL(values);
  TALOS_NONNULL(terminals);
  TALOS_NONNULL(adv);
  TALOS_NONNULL(ret);
  TALOS_DEVICE();
  const int rc = gae_launch(len, rewards, values, terminals, r_mean, r_var, r_clip, gamma, lambda, adv, ret, adv_raw,
                            as_stream(stream));
  return entry_done(rc, as_stream(stream));
}

size_t talos_ppo_update_work_bytes(talos_plan plan, int n) {
  const talos_ppo_cfg* c = ppo_plan_cfg(plan);
  if (c == nullptr || n < 0) return 0;
  return update_work(nullptr, n, talos_ppo_param_count(c)).bytes;
}

int talos_ppo_update_f32(talos_plan plan, talos_ppo_update_args* a, talos_ppo_update_result* result,
                         talos_stream_t stream) {
  const talos_ppo_cfg* c = ppo_plan_cfg(plan);
  TALOS_REQUIRE(c != nullptr, TALOS_ERR_HANDLE, "%s: not a ppo plan", __func__);
  TALOS_NONNULL(a);
  TALOS_REQUIRE(a->n >= 0 && a->k_epochs >= 0 && a->adam_t >= 0, TALOS_ERR_SHAPE,
                "%s: n, k_epochs and adam_t must be >= 0", __func__);
  if (result) *result = talos_ppo_update_result{};
  if (a->n == 0) return TALOS_OK;  // an empty memory returns at once (src/ppo.rs:626-628)
  TALOS_NONNULL(a->states);
  TALOS_NONNULL(a->actions);
  TALOS_NONNULL(a->old_logp);
  TALOS_NONNULL(a->rewards);
  TALOS_NONNULL(a->values);
  TALOS_NONNULL(a->terminals);
  TALOS_NONNULL(a->params);
  TALOS_NONNULL(a->adam_m);
  TALOS_NONNULL(a->adam_v);
  TALOS_NONNULL(a->work);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  const int n = a->n, B = c->batch;
  const size_t n_params = talos_ppo_param_count(c);
  const size_t state_stride = (size_t)c->seq * c->in_dim;
  UpdateWork w = update_work(a->work, n, n_params);

  int rc = gae_launch(n, a->rewards, a->values, a->terminals, a->reward_mean, a->reward_var, a->reward_clip,
                      a->gamma, a->lambda, w.adv, w.ret, nullptr, s);
  if (rc) return rc;
  int t = a->adam_t;
  talos_ppo_update_result res{};
  for (int epoch = 0; epoch < a->k_epochs; ++epoch) {
    for (int start = 0; start < n; start += B) {
      const int nb = std::min(B, n - start);
      rc = talos_ppo_minibatch_f32(plan, nb, a->params, a->states + start * state_stride,
                                   a->lengths ? a->lengths + start : nullptr, a->actions + start, w.adv + start,
                                   w.ret + start, a->old_logp + start, w.loss, w.grads, w.stats, start > 0, stream);
      if (rc) return rc;
      ++t;  // Adam::step increments t first (src/ppo.rs:520)
      rc = talos_adam_step_f32(n_params, a->params, w.grads, a->adam_m, a->adam_v, t, a->lr, 0.9, 0.999, 1e-8,
                               nullptr, 0.0, stream);
      if (rc) return rc;
    }
    double st[TALOS_PPO_NSTATS];
    TALOS_HIP(hipMemcpyAsync(st, w.stats, sizeof(st), hipMemcpyDeviceToHost, s));
    TALOS_HIP(hipStreamSynchronize(s));
    res.epochs_run = epoch + 1;
    const double cnt = st[TALOS_PPO_STAT_COUNT];
    res.approx_kl = cnt > 0 ? st[TALOS_PPO_STAT_KL] / cnt : 0.0;
    res.mean_loss = cnt > 0 ? (-st[TALOS_PPO_STAT_POLICY] + (double)c->value_coef * st[TALOS_PPO_STAT_VALUE] -
                               (double)c->entropy_coef * st[TALOS_PPO_STAT_ENTROPY]) / cnt
                            : 0.0;
    if (cnt > 0 && res.approx_kl > a->target_kl * 1.5) {  // src/ppo.rs:761-768
      res.stopped_early = 1;
      break;
    }
  }
  a->adam_t = t;
  if (result) *result = res;
  return entry_done(TALOS_OK, as_stream(stream));
}

}  // extern "C"
