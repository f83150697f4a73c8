/*
 * talos_oracle.cpp -- CPU f64 restatement of Talos-XII's autograd hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product links, loads or calls this file:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
 * checker of the HIP path or as the reported CPU baseline.
 *
 * What it restates (file:line in zayokami/Talos-XII, a Rust crate that cannot be built
 * here: no cargo/rustc and no vendored crates):
 *   - the tape: Tensor{data, grad, shape, _ctx}, Context{parents, backward_op},
 *     backward() with DFS topological order and an all-ones seed, zero_grad()
 *     (src/autograd.rs:14-20, 51-54, 145-196);
 *   - the ops matmul (:200-354), relu (:356-386), log/exp (:388-430), sum/mean (:433-482),
 *     broadcast (:484-509), broadcast_to_batch (:511-547), sin/cos/sqrt (:549-630),
 *     transpose (:632-739), clip (:741-768), reshape (:770-792), mse_loss (:1599-1603),
 *     Add/Sub/Mul/Div/Neg (:1606-1862) and Tensor::rand's LCG (:114-124);
 *   - Linear (src/nn.rs:20-35, 72-133) and RMSNorm (src/nn.rs:144-304);
 *   - RoPE (src/transformer.rs:219-337), scale_tensor / softmax / batched_matmul_qt_k /
 *     batched_matmul_probs_v / concat_last_dim (src/transformer.rs:877-1183), the MLA forward
 *     (src/transformer.rs:478-560) and the pre-norm block wiring (src/transformer.rs:71-90);
 *   - the PPO per-sample loss graph (src/ppo.rs:691-756) and the actor-critic heads
 *     (src/ppo.rs:246-300);
 *   - the optimizer step: Adam (src/ppo.rs:519-533) and the DQN optimizer's global-norm
 *     gradient clip (src/dqn.rs:207-226);
 *   - PPO::update's prologue: reward normalisation, GAE and advantage normalisation
 *     (src/ppo.rs:650-676).
 * Extensions the configurations need (each documented where defined): causal softmax mask,
 * GELU, explicit sequence positions for RoPE, a differentiable last-token gather, a standard
 * multi-head attention block, and a batched PPO loss with a closed-form backward.
 * Checker support, not in the reference: gradient magnitude sums (Tensor::mag, the sum of
 * |term| over each gradient element's terms), from which the parity tests derive the rounding
 * allowance of parameter gradients; pinned by their closed forms in tests/test_oracle.py.
 *
 * Parallelism mirrors the reference: row-parallel loops on one global pool sized to all host
 * cores (rayon's global pool), matmul's serial path below m*n*k < 32768 (src/autograd.rs:222).
 */
#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../include/talos_hip.h"

namespace orc {

// ---------------------------------------------------------------------------
// Global thread pool (rayon's global pool stand-in)
// ---------------------------------------------------------------------------
class Pool {
 public:
  static Pool& get() {
    static Pool p;
    return p;
  }
  int threads() const { return (int)workers_.size() + 1; }
  void set_threads(int n) {
    shutdown();
    start(n);
  }
  // Runs f(begin, end) over chunks of [0, n).
  void run(size_t n, const std::function<void(size_t, size_t)>& f) {
    if (n == 0) return;
    if (workers_.empty() || n == 1 || in_job_) {
      f(0, n);
      return;
    }
    auto job = std::make_shared<Job>();
    job->f = &f;
    job->n = n;
    size_t parts = (size_t)threads() * 4;
    job->chunk = std::max<size_t>(1, (n + parts - 1) / parts);
    job->nchunks = (n + job->chunk - 1) / job->chunk;
    job->pending.store(job->nchunks);
    {
      std::lock_guard<std::mutex> lk(m_);
      job_ = job;
      ++gen_;
    }
    cv_.notify_all();
    in_job_ = true;
    work(*job);
    in_job_ = false;
    std::unique_lock<std::mutex> lk(m_);
    done_cv_.wait(lk, [&] { return job->pending.load() == 0; });
    job_.reset();
  }
  ~Pool() { shutdown(); }

 private:
  struct Job {
    const std::function<void(size_t, size_t)>* f;
    size_t n, chunk, nchunks;
    std::atomic<size_t> next{0};
    std::atomic<size_t> pending{0};
  };
  Pool() {
    int n = (int)std::thread::hardware_concurrency();
    const char* e = getenv("ORACLE_THREADS");
    if (e && atoi(e) > 0) n = atoi(e);
    start(std::max(1, n));
  }
  void start(int n) {
    stop_ = false;
    for (int i = 0; i < n - 1; ++i) workers_.emplace_back([this] { loop(); });
  }
  void shutdown() {
    {
      std::lock_guard<std::mutex> lk(m_);
      stop_ = true;
      ++gen_;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
    workers_.clear();
  }
  void work(Job& j) {
    for (;;) {
      size_t c = j.next.fetch_add(1);
      if (c >= j.nchunks) break;
      size_t b = c * j.chunk, e = std::min(j.n, b + j.chunk);
      (*j.f)(b, e);
      if (j.pending.fetch_sub(1) == 1) {
        std::lock_guard<std::mutex> lk(m_);
        done_cv_.notify_all();
      }
    }
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      std::shared_ptr<Job> j;
      {
        std::unique_lock<std::mutex> lk(m_);
        cv_.wait(lk, [&] { return gen_ != seen; });
        seen = gen_;
        if (stop_) return;
        j = job_;
      }
      if (j) work(*j);
    }
  }
  std::vector<std::thread> workers_;
  std::mutex m_;
  std::condition_variable cv_, done_cv_;
  std::shared_ptr<Job> job_;
  uint64_t gen_ = 0;
  bool stop_ = false;
  bool in_job_ = false;
};

// Element-parallel loop; small ranges run inline (rayon splits adaptively).
template <class F>
static void par_for(size_t n, F f, size_t serial_below = 2048) {
  if (n < serial_below) {
    for (size_t i = 0; i < n; ++i) f(i);
    return;
  }
  std::function<void(size_t, size_t)> body = [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) f(i);
  };
  Pool::get().run(n, body);
}
// Row-parallel loop: one task per row (par_chunks_mut over rows).
template <class F>
static void par_rows(size_t rows, F f) {
  std::function<void(size_t, size_t)> body = [&](size_t b, size_t e) {
    for (size_t i = b; i < e; ++i) f(i);
  };
  Pool::get().run(rows, body);
}

// ---------------------------------------------------------------------------
// Tape (src/autograd.rs:14-20, 51-54)
// ---------------------------------------------------------------------------
using Vec = std::vector<double>;
using Shape = std::vector<size_t>;
struct Ctx;
struct Tensor {
  std::shared_ptr<Vec> data, grad;
  // Leaves created while magnitude tracking is on (parity-bound support, not part of the
  // reference): for each gradient element, the sum of |term| over every term the backward
  // closures add into it -- (|X|^T |G|)_ij for dW = X^T G, sum_r |g x_hat| for an RMSNorm gain,
  // sum_r |g| for a broadcast bias. An fp32 evaluation of the same sum errs by a small multiple
  // of 2^-24 of it; a dropped or misplaced term errs by a whole term.
  std::shared_ptr<Vec> mag;
  Shape shape;
  std::shared_ptr<Ctx> ctx;
  size_t numel() const { return data->size(); }
};
static bool g_track_mag = false;
// The magnitude buffer of a tracked tensor (nullptr when untracked).
static double* mag_of(const Tensor& t) { return t.mag ? t.mag->data() : nullptr; }
// While a closure runs: the magnitudes of the gradient it receives (its output's), or nullptr.
// Pass-through closures (reshape, transpose, the element-wise ops) forward them; reductions
// (matmul, an RMSNorm gain, a broadcast bias) start from |g| itself. A closure that keeps no
// magnitudes leaves its parents' at 0, so a magnitude is taken as at least |g|.
static const double* g_out_mag = nullptr;
static inline double mag_in(const Vec& g, size_t i) {
  return g_out_mag ? std::max(g_out_mag[i], std::fabs(g[i])) : std::fabs(g[i]);
}
using BackFn = std::function<void(const Vec& gout, std::vector<Tensor>& parents)>;
struct Ctx {
  std::vector<Tensor> parents;
  BackFn backward_op;
};

static size_t prod(const Shape& s) {
  size_t p = 1;
  for (size_t v : s) p *= v;
  return p;
}
static void require(bool c, const char* msg) {
  if (!c) throw std::runtime_error(msg);
}

// Tensor::new (src/autograd.rs:94-105)
static Tensor tnew(Vec data, Shape shape) {
  require(data.size() == prod(shape), "Data length must match shape");
  Tensor t;
  size_t n = data.size();
  t.data = std::make_shared<Vec>(std::move(data));
  t.grad = std::make_shared<Vec>(n, 0.0);
  t.shape = std::move(shape);
  return t;
}
// A leaf whose gradient magnitudes are tracked when tracking is on.
static Tensor tleaf(Vec data, Shape shape) {
  Tensor t = tnew(std::move(data), std::move(shape));
  if (g_track_mag) t.mag = std::make_shared<Vec>(t.numel(), 0.0);
  return t;
}
// Output tensor recorded on the tape.
static Tensor tout(Vec data, Shape shape, std::vector<Tensor> parents, BackFn fn) {
  Tensor t = tnew(std::move(data), std::move(shape));
  if (g_track_mag) t.mag = std::make_shared<Vec>(t.numel(), 0.0);
  t.ctx = std::make_shared<Ctx>();
  t.ctx->parents = std::move(parents);
  t.ctx->backward_op = std::move(fn);
  return t;
}
static Tensor tzeros(Shape s) { return tnew(Vec(prod(s), 0.0), s); }

// Tensor::rand (src/autograd.rs:114-124): 64-bit LCG; r = (x >> 33) / u32::MAX lies in
// [0, 0.5), so values cover only [min, (min+max)/2) -- kept bit-exact.
static Vec lcg_rand(size_t n, double mn, double mx, uint64_t seed) {
  Vec d(n);
  uint64_t x = seed;
  for (size_t i = 0; i < n; ++i) {
    x = x * 6364136223846793005ULL + 1ULL;
    double r = (double)(x >> 33) / (double)UINT32_MAX;
    d[i] = mn + r * (mx - mn);
  }
  return d;
}

// backward() (src/autograd.rs:145-184): topological order by DFS over parents, node
// identity = address of the grad buffer, seed every element of the root grad with 1.0,
// then run the closures in reverse order. Iterative DFS (same post-order as the recursion).
static void backward(const Tensor& root) {
  std::unordered_set<const void*> visited;
  std::vector<Tensor> topo;
  struct Frame {
    Tensor t;
    size_t next;
  };
  std::vector<Frame> stack;
  if (!visited.count(root.grad.get())) {
    visited.insert(root.grad.get());
    stack.push_back({root, 0});
  }
  while (!stack.empty()) {
    Frame& fr = stack.back();
    if (fr.t.ctx && fr.next < fr.t.ctx->parents.size()) {
      const Tensor& p = fr.t.ctx->parents[fr.next++];
      if (!visited.count(p.grad.get())) {
        visited.insert(p.grad.get());
        stack.push_back({p, 0});
      }
    } else {
      topo.push_back(fr.t);
      stack.pop_back();
    }
  }
  for (auto& v : *root.grad) v = 1.0;
  for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
    if (it->ctx) {
      const Vec& g = *it->grad;
      g_out_mag = it->mag ? it->mag->data() : nullptr;
      it->ctx->backward_op(g, it->ctx->parents);
      g_out_mag = nullptr;
    }
  }
}
static void zero_grad(const Tensor& t) {
  std::fill(t.grad->begin(), t.grad->end(), 0.0);
  if (t.mag) std::fill(t.mag->begin(), t.mag->end(), 0.0);
}
static Tensor detach(const Tensor& t) {
  Tensor d = t;
  d.ctx.reset();
  return d;
}

// ---------------------------------------------------------------------------
// CPU SIMD-shaped helpers (src/simd.rs:1-94): 4-wide with two accumulators like the
// AVX2/FMA kernels; the compiler vectorises these loops at -O3 -march=native.
// ---------------------------------------------------------------------------
static inline double dot_product(const double* a, const double* b, size_t n) {
  double s0[4] = {0, 0, 0, 0}, s1[4] = {0, 0, 0, 0};
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    for (int l = 0; l < 4; ++l) s0[l] += a[i + l] * b[i + l];
    for (int l = 0; l < 4; ++l) s1[l] += a[i + 4 + l] * b[i + 4 + l];
  }
  double s = 0;
  for (int l = 0; l < 4; ++l) s += s0[l] + s1[l];
  for (; i < n; ++i) s += a[i] * b[i];
  return s;
}
static inline void add_scaled_row(double* out, const double* row, double scale, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] += scale * row[i];
}

// ---------------------------------------------------------------------------
// Ops
// ---------------------------------------------------------------------------

// matmul (src/autograd.rs:200-354). Rank-1 lhs is a single row; out shape [n] then.
static Tensor matmul(const Tensor& a, const Tensor& b) {
  require(a.shape.size() <= 2 && b.shape.size() == 2, "matmul rank");
  size_t m, k;
  if (a.shape.size() == 1) {
    m = 1;
    k = a.shape[0];
  } else {
    m = a.shape[0];
    k = a.shape[1];
  }
  size_t k2 = b.shape[0], n = b.shape[1];
  require(k == k2, "MatMul dimension mismatch");
  Vec out(m * n, 0.0);
  const Vec& A = *a.data;
  const Vec& B = *b.data;
  auto row = [&](size_t r) {
    double* o = &out[r * n];
    for (size_t i = 0; i < k; ++i) add_scaled_row(o, &B[i * n], A[r * k + i], n);
  };
  if (m * n * k < 32768) {
    for (size_t r = 0; r < m; ++r) row(r);
  } else {
    par_rows(m, row);
  }
  Shape os = a.shape.size() == 1 ? Shape{n} : Shape{m, n};
  return tout(std::move(out), os, {a, b}, [m, k, n](const Vec& g, std::vector<Tensor>& p) {
    const Vec& A = *p[0].data;
    const Vec& B = *p[1].data;
    {
      // dL/dLHS = grad_out . RHS^T (dot products, :268-306)
      Vec& ga = *p[0].grad;
      auto r_fn = [&](size_t r) {
        for (size_t i = 0; i < k; ++i) ga[r * k + i] += dot_product(&g[r * n], &B[i * n], n);
      };
      if (m * k * n < 32768) {
        for (size_t r = 0; r < m; ++r) r_fn(r);
      } else {
        par_rows(m, r_fn);
      }
    }
    {
      // dL/dRHS = LHS^T . grad_out (axpy rows, skipping A == 0, :310-348)
      Vec& gb = *p[1].grad;
      auto i_fn = [&](size_t i) {
        double* o = &gb[i * n];
        for (size_t r = 0; r < m; ++r) {
          double s = A[r * k + i];
          if (s == 0.0) continue;
          add_scaled_row(o, &g[r * n], s, n);
        }
      };
      if (k * n * m < 32768) {
        for (size_t i = 0; i < k; ++i) i_fn(i);
      } else {
        par_rows(k, i_fn);
      }
    }
    // magnitudes of tracked operands: |dC| |B|^T and |A|^T |dC|
    if (double* ma = mag_of(p[0])) {
      par_rows(m, [&](size_t r) {
        for (size_t i = 0; i < k; ++i) {
          double s = 0;
          for (size_t j = 0; j < n; ++j) s += std::fabs(g[r * n + j]) * std::fabs(B[i * n + j]);
          ma[r * k + i] += s;
        }
      });
    }
    if (double* mb = mag_of(p[1])) {
      par_rows(k, [&](size_t i) {
        for (size_t r = 0; r < m; ++r) {
          double s = std::fabs(A[r * k + i]);
          if (s == 0.0) continue;
          for (size_t j = 0; j < n; ++j) mb[i * n + j] += s * std::fabs(g[r * n + j]);
        }
      });
    }
  });
}

// Generic elementwise unary op with the reference's backward closure.
template <class Fwd, class Bwd>
static Tensor unary(const Tensor& x, Fwd fwd, Bwd bwd) {
  const Vec& X = *x.data;
  Vec y(X.size());
  par_for(X.size(), [&](size_t i) { y[i] = fwd(X[i]); });
  return tout(std::move(y), x.shape, {x}, [bwd](const Vec& g, std::vector<Tensor>& p) {
    const Vec& X = *p[0].data;
    Vec& gx = *p[0].grad;
    par_for(gx.size(), [&](size_t i) { gx[i] += bwd(X[i], g[i]); });
  });
}
// relu (src/autograd.rs:356-386): grad passes where x > 0.
static Tensor relu(const Tensor& x) {
  return unary(x, [](double v) { return v > 0.0 ? v : 0.0; },
               [](double v, double g) { return v > 0.0 ? g : 0.0; });
}
// log (:388-413), exp (:415-439)
static Tensor tlog(const Tensor& x) {
  return unary(x, [](double v) { return std::log(v); }, [](double v, double g) { return g / v; });
}
static Tensor texp(const Tensor& x) {
  return unary(x, [](double v) { return std::exp(v); }, [](double v, double g) { return g * std::exp(v); });
}
// sin / cos / sqrt (:549-630)
static Tensor tsin(const Tensor& x) {
  return unary(x, [](double v) { return std::sin(v); }, [](double v, double g) { return g * std::cos(v); });
}
static Tensor tcos(const Tensor& x) {
  return unary(x, [](double v) { return std::cos(v); }, [](double v, double g) { return -g * std::sin(v); });
}
static Tensor tsqrt(const Tensor& x) {
  return unary(x, [](double v) { return std::sqrt(v); },
               [](double v, double g) { return v > 0.0 ? g * 0.5 / std::sqrt(v) : 0.0; });
}
// clip (:741-768): value clamped by max(min).min(max); grad passes where min <= x <= max.
static Tensor clip(const Tensor& x, double mn, double mx) {
  return unary(x, [mn, mx](double v) { return std::min(std::max(v, mn), mx); },
               [mn, mx](double v, double g) { return (v >= mn && v <= mx) ? g : 0.0; });
}
// Neg (:1828-1852)
static Tensor neg(const Tensor& x) {
  return unary(x, [](double v) { return -v; }, [](double, double g) { return -g; });
}
// scale_tensor (src/transformer.rs:1052-1072)
static Tensor scale_tensor(const Tensor& x, double s) {
  return unary(x, [s](double v) { return v * s; }, [s](double, double g) { return g * s; });
}
// GELU, exact erf form (extension: the reference has no GELU). gelu(x) = x * Phi(x);
// d/dx = Phi(x) + x * phi(x).
static double gelu_f(double v) { return 0.5 * v * (1.0 + std::erf(v / std::sqrt(2.0))); }
static double gelu_d(double v) {
  const double inv_sqrt_2pi = 0.3989422804014327;
  return 0.5 * (1.0 + std::erf(v / std::sqrt(2.0))) + v * inv_sqrt_2pi * std::exp(-0.5 * v * v);
}
static Tensor gelu(const Tensor& x) {
  return unary(x, [](double v) { return gelu_f(v); }, [](double v, double g) { return g * gelu_d(v); });
}

// sum (:433-458) and mean (:460-482)
static Tensor tsum(const Tensor& x) {
  double s = 0;
  for (double v : *x.data) s += v;
  return tout({s}, {1}, {x}, [](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    double gv = g[0];
    par_for(gx.size(), [&](size_t i) { gx[i] += gv; });
  });
}
static Tensor tmean(const Tensor& x) {
  size_t len = x.numel();
  double s = 0;
  for (double v : *x.data) s += v;
  return tout({s / (double)len}, {1}, {x}, [len](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    double gv = g[0] / (double)len;
    par_for(gx.size(), [&](size_t i) { gx[i] += gv; });
  });
}
// broadcast (:484-509): scalar [1] -> new_shape; backward sums.
static Tensor broadcast(const Tensor& x, Shape ns) {
  require(x.shape == Shape{1}, "Broadcast only supported for scalar (1) to N");
  size_t len = prod(ns);
  Vec d(len, (*x.data)[0]);
  return tout(std::move(d), ns, {x}, [](const Vec& g, std::vector<Tensor>& p) {
    double s = 0;
    for (double v : g) s += v;
    (*p[0].grad)[0] += s;
  });
}
// broadcast_to_batch (:511-547): repeat along a new leading dim; backward sums chunks.
static Tensor broadcast_to_batch(const Tensor& x, size_t batch) {
  const Vec& X = *x.data;
  size_t len = X.size();
  Vec d;
  d.reserve(len * batch);
  for (size_t b = 0; b < batch; ++b) d.insert(d.end(), X.begin(), X.end());
  Shape ns{batch};
  ns.insert(ns.end(), x.shape.begin(), x.shape.end());
  return tout(std::move(d), ns, {x}, [](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    size_t cs = gx.size();
    for (size_t c = 0; c + cs <= g.size(); c += cs)
      for (size_t i = 0; i < cs; ++i) gx[i] += g[c + i];
    if (double* mx = mag_of(p[0]))
      for (size_t c = 0; c + cs <= g.size(); c += cs)
        for (size_t i = 0; i < cs; ++i) mx[i] += std::fabs(g[c + i]);
  });
}
// transpose (:632-739): generic N-D swap of two dims, one coordinate vector per element
// as in the reference; backward is the inverse scatter-add.
static Tensor transpose(const Tensor& x, size_t d0, size_t d1) {
  const Shape& sh = x.shape;
  size_t rank = sh.size();
  require(d0 < rank && d1 < rank, "transpose dims");
  Shape ns = sh;
  std::swap(ns[d0], ns[d1]);
  size_t len = x.numel();
  std::vector<size_t> st(rank, 1), nst(rank, 1);
  for (size_t i = rank - 1; i-- > 0;) st[i] = st[i + 1] * sh[i + 1];
  for (size_t i = rank - 1; i-- > 0;) nst[i] = nst[i + 1] * ns[i + 1];
  const Vec& X = *x.data;
  Vec d(len, 0.0);
  for (size_t i = 0; i < len; ++i) {
    size_t t = i;
    std::vector<size_t> c(rank, 0);
    for (size_t k = 0; k < rank; ++k) {
      c[k] = t / nst[k];
      t %= nst[k];
    }
    std::swap(c[d0], c[d1]);
    size_t o = 0;
    for (size_t k = 0; k < rank; ++k) o += c[k] * st[k];
    d[i] = X[o];
  }
  return tout(std::move(d), ns, {x}, [d0, d1](const Vec& g, std::vector<Tensor>& p) {
    const Shape& sh = p[0].shape;
    size_t rank = sh.size();
    Shape ns = sh;
    std::swap(ns[d0], ns[d1]);
    std::vector<size_t> st(rank, 1), nst(rank, 1);
    for (size_t i = rank - 1; i-- > 0;) st[i] = st[i + 1] * sh[i + 1];
    for (size_t i = rank - 1; i-- > 0;) nst[i] = nst[i + 1] * ns[i + 1];
    Vec& gx = *p[0].grad;
    double* mx = mag_of(p[0]);
    for (size_t i = 0; i < g.size(); ++i) {
      size_t t = i;
      std::vector<size_t> c(rank, 0);
      for (size_t k = 0; k < rank; ++k) {
        c[k] = t / nst[k];
        t %= nst[k];
      }
      std::swap(c[d0], c[d1]);
      size_t o = 0;
      for (size_t k = 0; k < rank; ++k) o += c[k] * st[k];
      gx[o] += g[i];
      if (mx) mx[o] += mag_in(g, i);
    }
  });
}
// reshape (:770-792): copies the buffer; backward is identity accumulate.
static Tensor reshape(const Tensor& x, Shape ns) {
  require(prod(ns) == x.numel(), "Reshape dimension mismatch");
  return tout(*x.data, ns, {x}, [](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    par_for(gx.size(), [&](size_t i) { gx[i] += g[i]; });
    if (double* mx = mag_of(p[0])) par_for(gx.size(), [&](size_t i) { mx[i] += mag_in(g, i); });
  });
}

// Add / Sub / Mul / Div (:1606-1826). Mul and Div detect lhs aliasing rhs by the shared
// grad buffer and accumulate the combined derivative once (:1729-1737, 1792-1800).
enum Bin { ADD, SUB, MUL, DIV };
static Tensor binary(const Tensor& a, const Tensor& b, Bin op) {
  require(a.shape == b.shape, "binary op shape mismatch");
  const Vec& A = *a.data;
  const Vec& B = *b.data;
  Vec y(A.size());
  par_for(A.size(), [&](size_t i) {
    switch (op) {
      case ADD: y[i] = A[i] + B[i]; break;
      case SUB: y[i] = A[i] - B[i]; break;
      case MUL: y[i] = A[i] * B[i]; break;
      case DIV: y[i] = A[i] / B[i]; break;
    }
  });
  return tout(std::move(y), a.shape, {a, b}, [op](const Vec& g, std::vector<Tensor>& p) {
    const Vec& A = *p[0].data;
    const Vec& B = *p[1].data;
    Vec& ga = *p[0].grad;
    Vec& gb = *p[1].grad;
    bool alias = p[0].grad.get() == p[1].grad.get();
    if (op == ADD || op == SUB) {
      par_for(ga.size(), [&](size_t i) { ga[i] += g[i]; });
      double sg = op == ADD ? 1.0 : -1.0;
      par_for(gb.size(), [&](size_t i) { gb[i] += sg * g[i]; });
    } else if (op == MUL) {
      if (alias) {
        par_for(ga.size(), [&](size_t i) { ga[i] += g[i] * (A[i] + B[i]); });
      } else {
        par_for(ga.size(), [&](size_t i) { ga[i] += g[i] * B[i]; });
        par_for(gb.size(), [&](size_t i) { gb[i] += g[i] * A[i]; });
      }
    } else {
      if (alias) {
        par_for(ga.size(), [&](size_t i) { ga[i] += g[i] / B[i] - g[i] * A[i] / (B[i] * B[i]); });
      } else {
        par_for(ga.size(), [&](size_t i) { ga[i] += g[i] / B[i]; });
        par_for(gb.size(), [&](size_t i) { gb[i] -= g[i] * A[i] / (B[i] * B[i]); });
      }
    }
    // magnitudes of tracked operands: the output's, scaled by each operand's partial derivative
    double* ma = mag_of(p[0]);
    double* mb = alias ? nullptr : mag_of(p[1]);
    if (ma || mb)
      par_for(g.size(), [&](size_t i) {
        const double m = mag_in(g, i);
        double ta, tb;
        switch (op) {
          case ADD:
          case SUB: ta = tb = m; break;
          case MUL: ta = m * std::fabs(B[i]); tb = m * std::fabs(A[i]); break;
          default: ta = m / std::fabs(B[i]); tb = m * std::fabs(A[i] / (B[i] * B[i])); break;
        }
        if (ma) ma[i] += alias ? ta + tb : ta;
        if (mb) mb[i] += tb;
      });
  });
}
static Tensor add(const Tensor& a, const Tensor& b) { return binary(a, b, ADD); }
static Tensor sub(const Tensor& a, const Tensor& b) { return binary(a, b, SUB); }
static Tensor mul(const Tensor& a, const Tensor& b) { return binary(a, b, MUL); }
static Tensor tdiv(const Tensor& a, const Tensor& b) { return binary(a, b, DIV); }
// mse_loss (:1599-1603): mean((a - b)^2) with diff * diff taking the aliasing path.
static Tensor mse_loss(const Tensor& a, const Tensor& b) {
  Tensor d = sub(a, b);
  Tensor sq = mul(d, d);
  return tmean(sq);
}

// ---------------------------------------------------------------------------
// nn.rs modules
// ---------------------------------------------------------------------------

// Linear::forward (src/nn.rs:72-133), all shape branches kept.
struct Linear {
  Tensor weight;
  bool has_bias = false;
  Tensor bias;
  size_t in_f = 0, out_f = 0;
};
static Tensor linear_forward(const Linear& L, const Tensor& input) {
  size_t rank = input.shape.size();
  Tensor xf = input;
  bool flat = false;
  if (rank > 2) {
    size_t bd = 1;
    for (size_t i = 0; i + 1 < rank; ++i) bd *= input.shape[i];
    xf = reshape(input, {bd, L.in_f});
    flat = true;
  }
  Tensor outf = matmul(xf, L.weight);
  Tensor out = outf;
  if (flat) {
    Shape ns(input.shape.begin(), input.shape.end() - 1);
    ns.push_back(L.out_f);
    out = reshape(outf, ns);
  }
  if (L.has_bias) {
    const Tensor& b = L.bias;
    if (out.shape.size() == 2 && out.shape[0] > 1) {
      out = add(out, broadcast_to_batch(b, out.shape[0]));
    } else if (out.shape.size() > 2) {
      size_t total = out.numel();
      size_t bd = total / L.out_f;
      Tensor of = reshape(out, {bd, L.out_f});
      Tensor rf = add(of, broadcast_to_batch(b, bd));
      out = reshape(rf, out.shape);
    } else {
      if (out.shape != b.shape) {
        if (out.shape.size() == 2 && out.shape[0] == 1) {
          out = add(out, reshape(b, {1, L.out_f}));
        } else {
          out = add(out, b);
        }
      } else {
        out = add(out, b);
      }
    }
  }
  return out;
}

// RMSNorm forward/backward (src/nn.rs:182-296): caches rms per row and x_hat; the backward
// is hand-written, dw reduced per feature over all rows.
static Tensor rmsnorm(const Tensor& x, const Tensor& w, double eps) {
  size_t dim = x.shape.back();
  require(w.numel() == dim, "RMSNorm dim mismatch");
  const Vec& X = *x.data;
  const Vec& W = *w.data;
  size_t ne = X.size(), rows = ne / dim;
  Vec out(ne), xhat(ne), rms(rows);
  par_rows(rows, [&](size_t r) {
    size_t base = r * dim;
    double ss = 0;
    for (size_t i = 0; i < dim; ++i) ss += X[base + i] * X[base + i];
    double rm = std::sqrt(ss / (double)dim + eps);
    rms[r] = rm;
    for (size_t i = 0; i < dim; ++i) {
      double xh = X[base + i] / rm;
      xhat[base + i] = xh;
      out[base + i] = xh * W[i];
    }
  });
  auto rms_c = std::make_shared<Vec>(std::move(rms));
  auto xh_c = std::make_shared<Vec>(std::move(xhat));
  return tout(std::move(out), x.shape, {x, w}, [rms_c, xh_c, dim](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    Vec& gw = *p[1].grad;
    const Vec& W = *p[1].data;
    const Vec& rms = *rms_c;
    const Vec& xh = *xh_c;
    size_t rows = g.size() / dim;
    par_rows(rows, [&](size_t r) {
      size_t base = r * dim;
      double inv = 1.0 / rms[r];
      double dot = 0;
      for (size_t i = 0; i < dim; ++i) dot += g[base + i] * W[i] * xh[base + i];
      double md = dot / (double)dim;
      for (size_t i = 0; i < dim; ++i) gx[base + i] += inv * (g[base + i] * W[i] - xh[base + i] * md);
    });
    par_rows(dim, [&](size_t i) {
      double s = 0;
      for (size_t r = 0; r < rows; ++r) s += g[r * dim + i] * xh[r * dim + i];
      gw[i] += s;
    });
    if (double* mw = mag_of(p[1])) {
      par_rows(dim, [&](size_t i) {
        double s = 0;
        for (size_t r = 0; r < rows; ++r) s += std::fabs(g[r * dim + i] * xh[r * dim + i]);
        mw[i] += s;
      });
    }
  });
}

// RoPE (src/transformer.rs:219-337). The cache holds cos/sin(pos * theta_i),
// theta_i = 1 / base^(2i/dim), for pos < max_len; pairs (2i, 2i+1) are rotated; the
// position of a row is start_pos + (index along shape[-2]).
struct Rope {
  size_t dim = 0;
  double base = 10000.0;
  Vec cosc, sinc;
};
static Rope rope_new(size_t dim, size_t max_len, double base) {
  Rope r;
  r.dim = dim;
  r.base = base;
  for (size_t pos = 0; pos < max_len; ++pos)
    for (size_t i = 0; i < dim / 2; ++i) {
      double theta = 1.0 / std::pow(base, (double)(2 * i) / (double)dim);
      double ang = (double)pos * theta;
      r.cosc.push_back(std::cos(ang));
      r.sinc.push_back(std::sin(ang));
    }
  return r;
}
static Tensor rope_forward(const Rope& R, const Tensor& x, size_t start_pos) {
  size_t dim = x.shape.back();
  require(dim == R.dim, "rope dim");
  size_t seq = x.shape[x.shape.size() - 2];
  const Vec& X = *x.data;
  Vec out = X;
  size_t nb = X.size() / (seq * dim);
  require((start_pos + seq) * (dim / 2) <= R.cosc.size(), "rope position beyond cache");
  for (size_t b = 0; b < nb; ++b)
    for (size_t t = 0; t < seq; ++t) {
      size_t ci = (start_pos + t) * (dim / 2);
      size_t bi = b * seq * dim + t * dim;
      for (size_t i = 0; i < dim / 2; ++i) {
        double c = R.cosc[ci + i], s = R.sinc[ci + i];
        double r1 = X[bi + 2 * i], r2 = X[bi + 2 * i + 1];
        out[bi + 2 * i] = r1 * c - r2 * s;
        out[bi + 2 * i + 1] = r1 * s + r2 * c;
      }
    }
  auto cosc = std::make_shared<Vec>(R.cosc);
  auto sinc = std::make_shared<Vec>(R.sinc);
  return tout(std::move(out), x.shape, {x}, [cosc, sinc, dim, start_pos](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    const Shape& sh = p[0].shape;
    size_t seq = sh[sh.size() - 2];
    size_t nb = gx.size() / (seq * dim);
    for (size_t b = 0; b < nb; ++b)
      for (size_t t = 0; t < seq; ++t) {
        size_t ci = (start_pos + t) * (dim / 2);
        size_t bi = b * seq * dim + t * dim;
        for (size_t i = 0; i < dim / 2; ++i) {
          double c = (*cosc)[ci + i], s = (*sinc)[ci + i];
          double g1 = g[bi + 2 * i], g2 = g[bi + 2 * i + 1];
          gx[bi + 2 * i] += g1 * c + g2 * s;
          gx[bi + 2 * i + 1] += -g1 * s + g2 * c;
        }
      }
  });
}

// softmax along the last dim (src/transformer.rs:1074-1121). causal (extension): row r is
// query i = r mod seq_len of a square [seq_len, seq_len] score matrix and keys j > i are
// excluded (probability exactly 0, zero gradient).
static Tensor softmax(const Tensor& x, size_t seq_len, bool causal) {
  const Vec& X = *x.data;
  size_t rows = X.size() / seq_len;
  Vec y(X.size(), 0.0);
  par_rows(rows, [&](size_t r) {
    const double* row = &X[r * seq_len];
    size_t lim = causal ? (r % seq_len) + 1 : seq_len;
    double mx = -INFINITY;
    for (size_t j = 0; j < lim; ++j) mx = std::max(mx, row[j]);
    double s = 0;
    std::vector<double> e(lim);
    for (size_t j = 0; j < lim; ++j) {
      e[j] = std::exp(row[j] - mx);
      s += e[j];
    }
    for (size_t j = 0; j < lim; ++j) y[r * seq_len + j] = e[j] / s;
  });
  auto yc = std::make_shared<Vec>(y);
  return tout(std::move(y), x.shape, {x}, [yc, seq_len](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    const Vec& Y = *yc;
    size_t rows = g.size() / seq_len;
    par_rows(rows, [&](size_t r) {
      size_t b = r * seq_len;
      double sgy = 0;
      for (size_t i = 0; i < seq_len; ++i) sgy += g[b + i] * Y[b + i];
      for (size_t i = 0; i < seq_len; ++i) gx[b + i] += Y[b + i] * (g[b + i] - sgy);
    });
  });
}

// batched_matmul_qt_k (src/transformer.rs:877-958): S[b,i,j] = q[b,i,:] . k[b,j,:].
static Tensor bmm_qt_k(const Tensor& q, const Tensor& k, size_t B, size_t S, size_t D) {
  const Vec& Q = *q.data;
  const Vec& K = *k.data;
  Vec out(B * S * S);
  par_rows(B, [&](size_t b) {
    for (size_t i = 0; i < S; ++i)
      for (size_t j = 0; j < S; ++j)
        out[b * S * S + i * S + j] = dot_product(&Q[b * S * D + i * D], &K[b * S * D + j * D], D);
  });
  return tout(std::move(out), {B, S, S}, {q, k}, [B, S, D](const Vec& g, std::vector<Tensor>& p) {
    const Vec& Q = *p[0].data;
    const Vec& K = *p[1].data;
    Vec& gq = *p[0].grad;
    Vec& gk = *p[1].grad;
    par_rows(B, [&](size_t b) {
      size_t bd = b * S * D;
      for (size_t i = 0; i < S; ++i)
        for (size_t j = 0; j < S; ++j) {
          double gv = g[b * S * S + i * S + j];
          for (size_t d = 0; d < D; ++d) {
            gq[bd + i * D + d] += gv * K[bd + j * D + d];
            gk[bd + j * D + d] += gv * Q[bd + i * D + d];
          }
        }
    });
  });
}
// batched_matmul_probs_v (src/transformer.rs:961-1050): O[b,i,:] = sum_j P[b,i,j] V[b,j,:],
// skipping |p| < 1e-9 in the forward as the reference does.
static Tensor bmm_p_v(const Tensor& pr, const Tensor& v, size_t B, size_t S, size_t Dv) {
  const Vec& P = *pr.data;
  const Vec& V = *v.data;
  Vec out(B * S * Dv, 0.0);
  par_rows(B, [&](size_t b) {
    for (size_t i = 0; i < S; ++i) {
      double* o = &out[b * S * Dv + i * Dv];
      for (size_t j = 0; j < S; ++j) {
        double pv = P[b * S * S + i * S + j];
        if (std::fabs(pv) < 1e-9) continue;
        add_scaled_row(o, &V[b * S * Dv + j * Dv], pv, Dv);
      }
    }
  });
  return tout(std::move(out), {B, S, Dv}, {pr, v}, [B, S, Dv](const Vec& g, std::vector<Tensor>& p) {
    const Vec& P = *p[0].data;
    const Vec& V = *p[1].data;
    Vec& gp = *p[0].grad;
    Vec& gv = *p[1].grad;
    par_rows(B, [&](size_t b) {
      size_t bp = b * S * S, bv = b * S * Dv;
      for (size_t i = 0; i < S; ++i)
        for (size_t d = 0; d < Dv; ++d) {
          double gg = g[bv + i * Dv + d];
          for (size_t j = 0; j < S; ++j) {
            gp[bp + i * S + j] += gg * V[bv + j * Dv + d];
            gv[bv + j * Dv + d] += gg * P[bp + i * S + j];
          }
        }
    });
  });
}
// concat_last_dim (src/transformer.rs:1123-1183)
static Tensor concat_last(const Tensor& a, const Tensor& b) {
  size_t la = a.shape.back(), lb = b.shape.back();
  Shape bd(a.shape.begin(), a.shape.end() - 1);
  size_t rows = prod(bd);
  const Vec& A = *a.data;
  const Vec& B = *b.data;
  Vec out(rows * (la + lb));
  par_rows(rows, [&](size_t r) {
    std::copy(&A[r * la], &A[r * la] + la, &out[r * (la + lb)]);
    std::copy(&B[r * lb], &B[r * lb] + lb, &out[r * (la + lb) + la]);
  });
  Shape ns = bd;
  ns.push_back(la + lb);
  return tout(std::move(out), ns, {a, b}, [la, lb](const Vec& g, std::vector<Tensor>& p) {
    Vec& ga = *p[0].grad;
    Vec& gb = *p[1].grad;
    size_t rows = ga.size() / la;
    par_rows(rows, [&](size_t r) {
      for (size_t k = 0; k < la; ++k) ga[r * la + k] += g[r * (la + lb) + k];
      for (size_t k = 0; k < lb; ++k) gb[r * lb + k] += g[r * (la + lb) + la + k];
    });
    double* ma = mag_of(p[0]);
    double* mb = mag_of(p[1]);
    if (ma || mb)
      par_rows(rows, [&](size_t r) {
        if (ma)
          for (size_t k = 0; k < la; ++k) ma[r * la + k] += mag_in(g, r * (la + lb) + k);
        if (mb)
          for (size_t k = 0; k < lb; ++k) mb[r * lb + k] += mag_in(g, r * (la + lb) + la + k);
      });
  });
}
// last_token (src/transformer.rs:92-109) takes row S-1 of each sequence. The reference
// builds the result with Tensor::new, which cuts the graph (no gradient reaches the backbone).
// differentiable = true (extension) records a gather whose backward scatter-adds into row S-1.
static Tensor last_token(const Tensor& x, bool differentiable) {
  size_t B = x.shape[0], S = x.shape[1], D = x.shape[2];
  const Vec& X = *x.data;
  Vec out;
  out.reserve(B * D);
  for (size_t b = 0; b < B; ++b) {
    size_t st = b * S * D + (S - 1) * D;
    out.insert(out.end(), X.begin() + st, X.begin() + st + D);
  }
  if (!differentiable) return tnew(std::move(out), {B, D});
  return tout(std::move(out), {B, D}, {x}, [B, S, D](const Vec& g, std::vector<Tensor>& p) {
    Vec& gx = *p[0].grad;
    double* mx = mag_of(p[0]);
    for (size_t b = 0; b < B; ++b)
      for (size_t i = 0; i < D; ++i) {
        gx[b * S * D + (S - 1) * D + i] += g[b * D + i];
        if (mx) mx[b * S * D + (S - 1) * D + i] += mag_in(g, b * D + i);
      }
  });
}

// ---------------------------------------------------------------------------
// Parameters held as leaf tensors, loaded from / gathered to a flat layout.
// ---------------------------------------------------------------------------
struct Params {
  std::vector<Tensor> leaves;
  const double* src = nullptr;
  size_t off = 0;
  Tensor take(Shape s) {
    size_t n = prod(s);
    Vec d(src + off, src + off + n);
    off += n;
    Tensor t = tleaf(std::move(d), s);
    leaves.push_back(t);
    return t;
  }
  void grads(double* dst) const {
    size_t o = 0;
    for (auto& t : leaves) {
      std::copy(t.grad->begin(), t.grad->end(), dst + o);
      o += t.numel();
    }
  }
  // the gradient magnitudes of the leaves (zeros for an untracked leaf)
  void mags(double* dst) const {
    size_t o = 0;
    for (auto& t : leaves) {
      if (t.mag)
        std::copy(t.mag->begin(), t.mag->end(), dst + o);
      else
        std::fill(dst + o, dst + o + t.numel(), 0.0);
      o += t.numel();
    }
  }
};
static Linear make_linear(Params& P, size_t in, size_t out, bool bias) {
  Linear L;
  L.in_f = in;
  L.out_f = out;
  L.weight = P.take({in, out});
  if (bias) {
    L.has_bias = true;
    L.bias = P.take({out});
  }
  return L;
}

// ---------------------------------------------------------------------------
// MLA block (src/transformer.rs:478-557) with a pre-norm residual around it.
// ---------------------------------------------------------------------------
struct MlaCfg {
  int batch, seq, d_model, n_heads, kv_latent, rope_dim, head_dim, v_dim;
  int causal;       // extension
  int literal_rope; // 1: rotate q_r/k_r along shape[-2] of [B,S,H,R] (the head index) like the
                    // reference's training path; 0: rotate by the sequence position
  double eps, rope_base;
};
struct Mla {
  Tensor g;
  Linear w_dkv, w_uk, w_uv, w_q, w_kr, w_qr, w_o;
};
static Mla make_mla(Params& P, const MlaCfg& c) {
  Mla m;
  size_t d = c.d_model, H = c.n_heads;
  m.g = P.take({d});
  m.w_dkv = make_linear(P, d, c.kv_latent, false);
  m.w_uk = make_linear(P, c.kv_latent, H * c.head_dim, false);
  m.w_uv = make_linear(P, c.kv_latent, H * c.v_dim, false);
  m.w_q = make_linear(P, d, H * c.head_dim, false);
  m.w_kr = make_linear(P, d, H * c.rope_dim, false);
  m.w_qr = make_linear(P, d, H * c.rope_dim, false);
  m.w_o = make_linear(P, H * c.v_dim, d, false);
  return m;
}
static Tensor mla_forward(const Mla& m, const MlaCfg& c, const Rope& R, const Tensor& xin) {
  size_t B = c.batch, S = c.seq, H = c.n_heads, hd = c.head_dim, rd = c.rope_dim, vd = c.v_dim;
  Tensor x = rmsnorm(xin, m.g, c.eps);
  Tensor c_kv = linear_forward(m.w_dkv, x);
  Tensor k_c = linear_forward(m.w_uk, c_kv);
  Tensor v_c = linear_forward(m.w_uv, c_kv);
  Tensor k_r_flat = linear_forward(m.w_kr, x);
  Tensor q_c = linear_forward(m.w_q, x);
  Tensor q_r_flat = linear_forward(m.w_qr, x);
  Tensor k_r = reshape(k_r_flat, {B, S, H, rd});
  Tensor q_r = reshape(q_r_flat, {B, S, H, rd});
  Tensor k_rot, q_rot;
  if (c.literal_rope) {
    k_rot = rope_forward(R, k_r, 0);
    q_rot = rope_forward(R, q_r, 0);
  } else {
    k_rot = transpose(rope_forward(R, transpose(k_r, 1, 2), 0), 1, 2);
    q_rot = transpose(rope_forward(R, transpose(q_r, 1, 2), 0), 1, 2);
  }
  Tensor q = concat_last(reshape(q_c, {B, S, H, hd}), q_rot);
  Tensor k = concat_last(reshape(k_c, {B, S, H, hd}), k_rot);
  Tensor v = reshape(v_c, {B, S, H, vd});
  size_t td = hd + rd;
  Tensor qf = reshape(transpose(q, 1, 2), {B * H, S, td});
  Tensor kf = reshape(transpose(k, 1, 2), {B * H, S, td});
  Tensor vf = reshape(transpose(v, 1, 2), {B * H, S, vd});
  Tensor sc = bmm_qt_k(qf, kf, B * H, S, td);
  Tensor scs = scale_tensor(sc, 1.0 / std::sqrt((double)td));
  Tensor pr = softmax(scs, S, c.causal != 0);
  Tensor o = bmm_p_v(pr, vf, B * H, S, vd);
  o = reshape(transpose(reshape(o, {B, H, S, vd}), 1, 2), {B, S, H * vd});
  return add(xin, linear_forward(m.w_o, o));
}

// Pre-norm block (talos_block_cfg). Standard multi-head attention: the Wqkv[d,3d] parameter is
// split into three Linear(d,d) (columns q|k|v) whose gradients are packed back afterwards. MLA
// attention: the Mla module above (its gain g is the block's g1, its residual the block's first).
struct Block {
  bool mla_attn = false;
  Tensor g1, g2;
  Tensor wqkv;
  Linear wq, wk, wv, wo, w1, w2;
  Mla mla;
};
static MlaCfg mla_cfg_of(const talos_block_cfg& c, size_t batch, size_t seq) {
  return MlaCfg{(int)batch, (int)seq, c.d_model, c.n_heads, c.kv_latent, c.rope_dim, c.head_dim, c.v_dim,
                c.causal, 0, (double)c.eps, (double)c.rope_base};
}
// Width of the RoPE table of a block: the head for standard attention, the decoupled RoPE dims for MLA.
static size_t rope_dim_of(const talos_block_cfg& c) {
  return (size_t)(c.attention == TALOS_ATTN_MLA ? c.rope_dim : c.head_dim);
}
static size_t block_param_count(const talos_block_cfg& c) {
  size_t d = c.d_model, F = c.ffn_dim, H = c.n_heads;
  size_t mlp = d + d * F + F + F * d + d;
  if (c.attention == TALOS_ATTN_MLA) {
    size_t L = c.kv_latent, r = c.rope_dim, hd = c.head_dim, vd = c.v_dim;
    return d + d * L + L * H * hd + L * H * vd + d * H * hd + 2 * d * H * r + H * vd * d + mlp;
  }
  return d + 3 * d * d + d * d + mlp;
}
static Tensor split_cols(const Tensor& w, size_t c0, size_t nc) {
  size_t r = w.shape[0], C = w.shape[1];
  Vec d(r * nc);
  for (size_t i = 0; i < r; ++i)
    for (size_t j = 0; j < nc; ++j) d[i * nc + j] = (*w.data)[i * C + c0 + j];
  return tleaf(std::move(d), {r, nc});
}
static Block make_block(Params& P, const talos_block_cfg& c) {
  Block b;
  size_t d = c.d_model, F = c.ffn_dim;
  if (c.attention == TALOS_ATTN_MLA) {
    b.mla_attn = true;
    b.mla = make_mla(P, mla_cfg_of(c, c.batch, c.seq));
    b.g1 = b.mla.g;
    b.g2 = P.take({d});
    b.w1 = make_linear(P, d, F, true);
    b.w2 = make_linear(P, F, d, true);
    return b;
  }
  b.g1 = P.take({d});
  b.wqkv = P.take({d, 3 * d});
  b.wq.weight = split_cols(b.wqkv, 0, d);
  b.wk.weight = split_cols(b.wqkv, d, d);
  b.wv.weight = split_cols(b.wqkv, 2 * d, d);
  for (Linear* L : {&b.wq, &b.wk, &b.wv}) {
    L->in_f = d;
    L->out_f = d;
  }
  b.wo = make_linear(P, d, d, false);
  b.g2 = P.take({d});
  b.w1 = make_linear(P, d, F, true);
  b.w2 = make_linear(P, F, d, true);
  return b;
}
// After backward: pack the three split weight grads into the Wqkv leaf's grad.
static void block_pack_grads(Block& b) {
  if (b.mla_attn) return;
  size_t d = b.wq.in_f;
  Vec& G = *b.wqkv.grad;
  const Linear* L[3] = {&b.wq, &b.wk, &b.wv};
  for (int s = 0; s < 3; ++s)
    for (size_t i = 0; i < d; ++i)
      for (size_t j = 0; j < d; ++j) G[i * 3 * d + s * d + j] += (*L[s]->weight.grad)[i * d + j];
  if (b.wqkv.mag)
    for (int s = 0; s < 3; ++s)
      for (size_t i = 0; i < d; ++i)
        for (size_t j = 0; j < d; ++j) (*b.wqkv.mag)[i * 3 * d + s * d + j] += (*L[s]->weight.mag)[i * d + j];
}
static void block_zero_split_grads(Block& b) {
  if (b.mla_attn) return;
  zero_grad(b.wq.weight);
  zero_grad(b.wk.weight);
  zero_grad(b.wv.weight);
}

// Pre-norm block forward (wiring of src/transformer.rs:71-90 with the attention of
// src/transformer.rs:478-557, standard heads): x [B,S,d] -> out [B,S,d].
static Tensor block_mlp(const Block& b, const talos_block_cfg& c, const Tensor& h2) {
  Tensor xn2 = rmsnorm(h2, b.g2, c.eps);
  Tensor f1 = linear_forward(b.w1, xn2);
  f1 = c.activation == TALOS_ACT_RELU ? relu(f1) : gelu(f1);
  Tensor f2 = linear_forward(b.w2, f1);
  return add(h2, f2);
}
static Tensor block_forward(const Block& b, const talos_block_cfg& c, const Rope& R, const Tensor& x) {
  size_t B = x.shape[0], S = x.shape[1], d = c.d_model, H = c.n_heads, hd = c.head_dim;
  if (b.mla_attn) return block_mlp(b, c, mla_forward(b.mla, mla_cfg_of(c, B, S), R, x));
  Tensor xn = rmsnorm(x, b.g1, c.eps);
  auto heads = [&](const Linear& L, bool rot) {
    Tensor t = linear_forward(L, xn);                 // [B,S,d]
    t = reshape(t, {B, S, H, hd});
    t = transpose(t, 1, 2);                           // [B,H,S,hd]
    if (rot) t = rope_forward(R, t, 0);               // rotates along S (pos = sequence index)
    return reshape(t, {B * H, S, hd});
  };
  Tensor q = heads(b.wq, true), k = heads(b.wk, true), v = heads(b.wv, false);
  Tensor sc = bmm_qt_k(q, k, B * H, S, hd);
  Tensor scs = scale_tensor(sc, 1.0 / std::sqrt((double)hd));
  Tensor pr = softmax(scs, S, c.causal != 0);
  Tensor o = bmm_p_v(pr, v, B * H, S, hd);
  o = reshape(o, {B, H, S, hd});
  o = transpose(o, 1, 2);
  o = reshape(o, {B, S, d});
  return block_mlp(b, c, add(x, linear_forward(b.wo, o)));
}

// ---------------------------------------------------------------------------
// Policy network + PPO loss
// ---------------------------------------------------------------------------
static talos_block_cfg block_cfg_of(const talos_ppo_cfg& p) {
  talos_block_cfg c{};
  c.batch = p.batch;
  c.seq = p.seq;
  c.d_model = p.d_model;
  c.n_heads = p.n_heads;
  c.head_dim = p.head_dim;
  c.ffn_dim = p.ffn_dim;
  c.causal = p.causal;
  c.activation = p.activation;
  c.eps = p.eps;
  c.rope_base = p.rope_base;
  c.attention = p.attention;
  c.kv_latent = p.kv_latent;
  c.rope_dim = p.rope_dim;
  c.v_dim = p.v_dim;
  return c;
}
struct Policy {
  Linear embed;
  std::vector<Block> blocks;
  Tensor gf;
  Linear out_proj, actor, critic;
};
static Policy make_policy(Params& P, const talos_ppo_cfg& c) {
  Policy pol;
  pol.embed = make_linear(P, c.in_dim, c.d_model, true);
  talos_block_cfg bc = block_cfg_of(c);
  for (int l = 0; l < c.n_layers; ++l) pol.blocks.push_back(make_block(P, bc));
  pol.gf = P.take({(size_t)c.d_model});
  pol.out_proj = make_linear(P, c.d_model, c.d_model, true);
  pol.actor = make_linear(P, c.d_model, c.n_actions, true);
  pol.critic = make_linear(P, c.d_model, 1, true);
  return pol;
}
// Backbone (LuckTransformer::forward shape, src/transformer.rs:71-90) + last token:
// x [B,S,in] -> [B,d].
static Tensor policy_last_hidden(const Policy& pol, const talos_ppo_cfg& c, const Rope& R, const Tensor& x,
                                 bool diff_last) {
  talos_block_cfg bc = block_cfg_of(c);
  Tensor h = linear_forward(pol.embed, x);
  for (auto& b : pol.blocks) h = block_forward(b, bc, R, h);
  Tensor hf = rmsnorm(h, pol.gf, c.eps);
  Tensor o = linear_forward(pol.out_proj, hf);
  return last_token(o, diff_last);
}

// Per-sample PPO loss graph, op for op as src/ppo.rs:702-749 (logits [A], value [1]).
static Tensor ppo_sample_loss(const talos_ppo_cfg& c, const Tensor& logits, const Tensor& value, int action,
                              double old_logp, double advantage, double ret) {
  size_t A = (size_t)c.n_actions;
  double mx = -INFINITY;
  for (double v : *logits.data) mx = std::max(mx, v);
  Tensor exp_logits = texp(add(logits, tnew(Vec(A, -mx), {A})));
  Tensor sum_exp = tsum(exp_logits);
  Tensor lse = add(tlog(sum_exp), tnew({mx}, {1}));
  Vec mask(A, 0.0);
  mask[(size_t)action] = 1.0;
  Tensor maskt = tnew(mask, {A});
  Tensor log_probs = sub(logits, broadcast(lse, {A}));
  Tensor log_prob = tsum(mul(log_probs, maskt));
  Tensor log_ratio = sub(log_prob, tnew({old_logp}, {1}));
  Tensor ratio = texp(log_ratio);
  Tensor adv = tnew({advantage}, {1});
  Tensor surr1 = mul(ratio, adv);
  Tensor surr2 = mul(clip(ratio, 1.0 - c.clip_eps, 1.0 + c.clip_eps), adv);
  double s1 = (*surr1.data)[0], s2 = (*surr2.data)[0];
  Tensor policy_loss = s1 < s2 ? surr1 : surr2;
  Tensor v_loss = mse_loss(sub(value, tnew({ret}, {1})), tzeros({1}));
  Tensor pp = texp(log_probs);
  Tensor entropy = neg(tsum(mul(pp, log_probs)));
  return sub(add(neg(policy_loss), mul(v_loss, tnew({(double)c.value_coef}, {1}))),
             mul(entropy, tnew({(double)c.entropy_coef}, {1})));
}

// Batched PPO loss with a closed-form backward (extension used by the batched oracle;
// pinned against ppo_sample_loss). logits [B,A], values [B,1] -> mean loss [1].
// Per sample: lp = z - lse(z), ratio = exp(lp[a] - old), pol = min-by-value of ratio*adv and
// clip(ratio)*adv (ties take the clipped branch, src/ppo.rs:738-740), v = (value - ret)^2,
// ent = -sum p*lp; loss = -pol + cv*v - ce*ent.
// dz_k = [-gr*ratio*(delta_ka - p_k) + ce*p_k*(lp_k + ent)] / B, gr = d pol / d ratio;
// dvalue = 2*cv*(value - ret) / B.
static Tensor ppo_batched_loss(const talos_ppo_cfg& c, const Tensor& logits, const Tensor& values,
                               const std::vector<int>& actions, const Vec& old_logp, const Vec& adv,
                               const Vec& ret) {
  size_t B = logits.shape[0], A = logits.shape[1];
  const Vec& Z = *logits.data;
  const Vec& V = *values.data;
  auto dz = std::make_shared<Vec>(B * A);
  auto dv = std::make_shared<Vec>(B);
  double total = 0;
  for (size_t b = 0; b < B; ++b) {
    const double* z = &Z[b * A];
    double mx = -INFINITY;
    for (size_t j = 0; j < A; ++j) mx = std::max(mx, z[j]);
    double se = 0;
    for (size_t j = 0; j < A; ++j) se += std::exp(z[j] - mx);
    double lse = std::log(se) + mx;
    std::vector<double> lp(A), p(A);
    double ent = 0;
    for (size_t j = 0; j < A; ++j) {
      lp[j] = z[j] - lse;
      p[j] = std::exp(lp[j]);
      ent -= p[j] * lp[j];
    }
    int a = actions[b];
    double ratio = std::exp(lp[(size_t)a] - old_logp[b]);
    double s1 = ratio * adv[b];
    double lo = 1.0 - c.clip_eps, hi = 1.0 + c.clip_eps;
    double rc = std::min(std::max(ratio, lo), hi);
    double s2 = rc * adv[b];
    double pol, gr;
    if (s1 < s2) {
      pol = s1;
      gr = adv[b];
    } else {
      pol = s2;
      gr = (ratio >= lo && ratio <= hi) ? adv[b] : 0.0;
    }
    double vd = V[b] - ret[b];
    double loss = -pol + c.value_coef * vd * vd - c.entropy_coef * ent;
    total += loss;
    for (size_t k = 0; k < A; ++k) {
      double dk = (k == (size_t)a ? 1.0 : 0.0) - p[k];
      (*dz)[b * A + k] = (-gr * ratio * dk + c.entropy_coef * p[k] * (lp[k] + ent)) / (double)B;
    }
    (*dv)[b] = 2.0 * c.value_coef * vd / (double)B;
  }
  return tout({total / (double)B}, {1}, {logits, values}, [dz, dv](const Vec& g, std::vector<Tensor>& p) {
    Vec& gz = *p[0].grad;
    Vec& gv = *p[1].grad;
    for (size_t i = 0; i < gz.size(); ++i) gz[i] += g[0] * (*dz)[i];
    for (size_t i = 0; i < gv.size(); ++i) gv[i] += g[0] * (*dv)[i];
  });
}

// ---------------------------------------------------------------------------
// Rollout inference with the KV cache: LuckTransformer::forward_inference_step
// (src/transformer.rs:157-196), MultiHeadLatentAttention::forward_inference_cached (:688-805),
// prune_kv_cache (:807-840), KVCache (:400-426) and ActorCritic::step_inference_cached
// (src/ppo.rs:391-433). Plain f64 vectors, no tape, one token per call, as the reference.
// Extension: blocks with standard multi-head attention (q | k | v columns of Wqkv, RoPE over the
// whole head) and several layers, one cache per layer, with the same rules.
// ---------------------------------------------------------------------------
// Linear::forward_inference (src/nn.rs:37-70): out = b, then out += x_i * W[i, :] for each
// non-zero input in order.
static Vec linear_inf(const double* x, size_t in, size_t out, const double* W, const double* b) {
  Vec y(out, 0.0);
  if (b) std::copy(b, b + out, y.begin());
  for (size_t i = 0; i < in; ++i) {
    if (x[i] == 0.0) continue;
    add_scaled_row(y.data(), W + i * out, x[i], out);
  }
  return y;
}
// RMSNorm::forward_inference (src/nn.rs:159-180)
static Vec rmsnorm_inf(const Vec& x, const double* w, double eps) {
  double ss = 0.0;
  for (double v : x) ss += v * v;
  const double rms = std::sqrt(ss / (double)x.size() + eps);
  Vec y(x.size());
  for (size_t i = 0; i < x.size(); ++i) y[i] = (x[i] / rms) * w[i];
  return y;
}

struct KvCache {
  std::vector<Vec> k, v;  // per head: rows of dk / dv values appended in order
};
struct Decoder {
  talos_ppo_cfg c{};
  Vec p;
  Rope rope;
  std::vector<std::vector<KvCache>> cache;  // [env][layer]
};

// Rotation of the pairs (2i, 2i+1) of x[0 .. dim) at pos; positions whose table offset lies past
// the cache are left unrotated, as the reference's `continue` does (src/transformer.rs:718-721).
static void rope_inf(const Rope& R, double* x, size_t pos) {
  const size_t half = R.dim / 2, off = pos * half;
  if (off >= R.cosc.size()) return;
  for (size_t i = 0; i < half; ++i) {
    const double c = R.cosc[off + i], s = R.sinc[off + i];
    const double a = x[2 * i], b = x[2 * i + 1];
    x[2 * i] = a * c - b * s;
    x[2 * i + 1] = a * s + b * c;
  }
}

// One block on one token: h -> out, appending the token's keys / values to kv.
static Vec block_step(const Decoder& D, const double* P, const Vec& h, KvCache& kv, size_t pos) {
  const talos_ppo_cfg& c = D.c;
  const size_t d = c.d_model, H = c.n_heads, F = c.ffn_dim;
  const bool mla = c.attention == TALOS_ATTN_MLA;
  const size_t hd = c.head_dim, r = mla ? c.rope_dim : 0, vd = mla ? c.v_dim : hd, td = hd + r;
  size_t o = 0;
  const double* g1 = P + o;
  o += d;
  Vec xn = rmsnorm_inf(h, g1, c.eps);
  std::vector<Vec> q(H, Vec(td)), k(H, Vec(td)), v(H, Vec(vd));
  const double* Wo;
  if (mla) {
    const size_t L = c.kv_latent;
    const double *Wdkv = P + o, *Wuk = Wdkv + d * L, *Wuv = Wuk + L * H * hd, *Wq = Wuv + L * H * vd,
                 *Wkr = Wq + d * H * hd, *Wqr = Wkr + d * H * r;
    Wo = Wqr + d * H * r;
    o = (size_t)(Wo - P) + H * vd * d;
    Vec ckv = linear_inf(xn.data(), d, L, Wdkv, nullptr);
    Vec kc = linear_inf(ckv.data(), L, H * hd, Wuk, nullptr);
    Vec vc = linear_inf(ckv.data(), L, H * vd, Wuv, nullptr);
    Vec krf = linear_inf(xn.data(), d, H * r, Wkr, nullptr);
    Vec qc = linear_inf(xn.data(), d, H * hd, Wq, nullptr);
    Vec qrf = linear_inf(xn.data(), d, H * r, Wqr, nullptr);
    for (size_t hh = 0; hh < H; ++hh) {
      rope_inf(D.rope, &krf[hh * r], pos);
      rope_inf(D.rope, &qrf[hh * r], pos);
      for (size_t i = 0; i < hd; ++i) {
        q[hh][i] = qc[hh * hd + i];
        k[hh][i] = kc[hh * hd + i];
      }
      for (size_t i = 0; i < r; ++i) {
        q[hh][hd + i] = qrf[hh * r + i];
        k[hh][hd + i] = krf[hh * r + i];
      }
      for (size_t i = 0; i < vd; ++i) v[hh][i] = vc[hh * vd + i];
    }
  } else {
    const double* Wqkv = P + o;
    Wo = Wqkv + 3 * d * d;
    o += 3 * d * d + d * d;
    Vec qkv = linear_inf(xn.data(), d, 3 * d, Wqkv, nullptr);
    for (size_t hh = 0; hh < H; ++hh) {
      for (size_t i = 0; i < hd; ++i) {
        q[hh][i] = qkv[hh * hd + i];
        k[hh][i] = qkv[d + hh * hd + i];
        v[hh][i] = qkv[2 * d + hh * hd + i];
      }
      rope_inf(D.rope, q[hh].data(), pos);
      rope_inf(D.rope, k[hh].data(), pos);
    }
  }
  // append, then attend over every cached row (src/transformer.rs:764-805)
  for (size_t hh = 0; hh < H; ++hh) {
    kv.k[hh].insert(kv.k[hh].end(), k[hh].begin(), k[hh].end());
    kv.v[hh].insert(kv.v[hh].end(), v[hh].begin(), v[hh].end());
  }
  const size_t n = kv.k[0].size() / td;
  const double scale = 1.0 / std::sqrt((double)td);
  Vec att(H * vd, 0.0);
  for (size_t hh = 0; hh < H; ++hh) {
    Vec sc(n);
    for (size_t j = 0; j < n; ++j) sc[j] = dot_product(q[hh].data(), &kv.k[hh][j * td], td) * scale;
    double mx = -INFINITY;
    for (double x : sc) mx = std::max(mx, x);
    double sum = 0.0;
    for (double& x : sc) {
      x = std::exp(x - mx);
      sum += x;
    }
    for (double& x : sc) x *= 1.0 / sum;
    for (size_t j = 0; j < n; ++j) {
      if (std::fabs(sc[j]) < 1e-9) continue;
      add_scaled_row(&att[hh * vd], &kv.v[hh][j * vd], sc[j], vd);
    }
  }
  Vec ao = linear_inf(att.data(), H * vd, d, Wo, nullptr);
  Vec h2(d);
  for (size_t i = 0; i < d; ++i) h2[i] = h[i] + ao[i];
  const double* g2 = P + o;
  o += d;
  Vec xn2 = rmsnorm_inf(h2, g2, c.eps);
  const double *W1 = P + o, *b1 = W1 + d * F, *W2 = b1 + F, *b2 = W2 + F * d;
  Vec f1 = linear_inf(xn2.data(), d, F, W1, b1);
  for (double& x : f1) x = c.activation == TALOS_ACT_RELU ? (x < 0.0 ? 0.0 : x) : gelu_f(x);
  Vec f2 = linear_inf(f1.data(), F, d, W2, b2);
  Vec out(d);
  for (size_t i = 0; i < d; ++i) out[i] = h2[i] + f2[i];
  return out;
}

}  // namespace orc

// ===========================================================================
// C ABI (ctypes) for the tests and the CPU baseline
// ===========================================================================
using namespace orc;

static thread_local std::string g_err;
// Magnitude tracking for the duration of one model call whose dmag output is non-null.
struct TrackMag {
  bool prev;
  explicit TrackMag(bool on) : prev(g_track_mag) { g_track_mag = on; }
  ~TrackMag() { g_track_mag = prev; }
};

#define GUARD(...)                  \
  try {                             \
    __VA_ARGS__;                    \
    return 0;                       \
  } catch (const std::exception& e) { \
    g_err = e.what();               \
    return 1;                       \
  }

extern "C" {

const char* orc_last_error(void) { return g_err.c_str(); }
int orc_threads(void) { return Pool::get().threads(); }
void orc_set_threads(int n) { Pool::get().set_threads(n < 1 ? 1 : n); }

// --- handle table for tape-level tests -----------------------------------
static std::mutex g_hm;
static std::unordered_map<int64_t, Tensor> g_handles;
static int64_t g_next = 1;
static int64_t put(const Tensor& t) {
  std::lock_guard<std::mutex> lk(g_hm);
  int64_t h = g_next++;
  g_handles[h] = t;
  return h;
}
static Tensor get(int64_t h) {
  std::lock_guard<std::mutex> lk(g_hm);
  auto it = g_handles.find(h);
  if (it == g_handles.end()) throw std::runtime_error("bad handle");
  return it->second;
}

int64_t orc_tensor_new(const double* data, const int64_t* shape, int rank) {
  try {
    Shape s(shape, shape + rank);
    return put(tleaf(Vec(data, data + prod(s)), s));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_tensor_new_len(const double* data, int64_t len, const int64_t* shape, int rank) {
  try {
    Shape s(shape, shape + rank);
    return put(tleaf(Vec(data, data + len), s));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_tensor_rand(const int64_t* shape, int rank, double mn, double mx, uint64_t seed) {
  Shape s(shape, shape + rank);
  return put(tnew(lcg_rand(prod(s), mn, mx, seed), s));
}
void orc_tensor_free(int64_t h) {
  std::lock_guard<std::mutex> lk(g_hm);
  g_handles.erase(h);
}
void orc_free_all(void) {
  std::lock_guard<std::mutex> lk(g_hm);
  g_handles.clear();
}
int orc_tensor_rank(int64_t h) { return (int)get(h).shape.size(); }
void orc_tensor_shape(int64_t h, int64_t* out) {
  Tensor t = get(h);
  for (size_t i = 0; i < t.shape.size(); ++i) out[i] = (int64_t)t.shape[i];
}
int64_t orc_tensor_numel(int64_t h) { return (int64_t)get(h).numel(); }
void orc_tensor_data(int64_t h, double* out) {
  Tensor t = get(h);
  std::copy(t.data->begin(), t.data->end(), out);
}
void orc_tensor_grad(int64_t h, double* out) {
  Tensor t = get(h);
  std::copy(t.grad->begin(), t.grad->end(), out);
}
// Leaves created after orc_set_track_mag(1) carry gradient magnitudes (see Tensor::mag);
// orc_tensor_mag copies them (zeros for an untracked tensor).
void orc_set_track_mag(int on) { g_track_mag = on != 0; }
void orc_tensor_mag(int64_t h, double* out) {
  Tensor t = get(h);
  if (t.mag)
    std::copy(t.mag->begin(), t.mag->end(), out);
  else
    std::fill(out, out + t.numel(), 0.0);
}
int orc_tensor_has_ctx(int64_t h) { return get(h).ctx ? 1 : 0; }

#define UNARY_H(name, expr)            \
  int64_t name(int64_t h) {            \
    try {                              \
      Tensor x = get(h);               \
      return put(expr);                \
    } catch (const std::exception& e) { \
      g_err = e.what();                \
      return 0;                        \
    }                                  \
  }
UNARY_H(orc_relu, relu(x))
UNARY_H(orc_log, tlog(x))
UNARY_H(orc_exp, texp(x))
UNARY_H(orc_sin, tsin(x))
UNARY_H(orc_cos, tcos(x))
UNARY_H(orc_sqrt, tsqrt(x))
UNARY_H(orc_neg, neg(x))
UNARY_H(orc_sum, tsum(x))
UNARY_H(orc_mean, tmean(x))
UNARY_H(orc_gelu, gelu(x))
UNARY_H(orc_detach, detach(x))

#define BINARY_H(name, expr)           \
  int64_t name(int64_t ha, int64_t hb) { \
    try {                              \
      Tensor a = get(ha), b = get(hb);   \
      return put(expr);                \
    } catch (const std::exception& e) { \
      g_err = e.what();                \
      return 0;                        \
    }                                  \
  }
BINARY_H(orc_matmul, matmul(a, b))
BINARY_H(orc_add, add(a, b))
BINARY_H(orc_sub, sub(a, b))
BINARY_H(orc_mul, mul(a, b))
BINARY_H(orc_div, tdiv(a, b))
BINARY_H(orc_mse_loss, mse_loss(a, b))

int64_t orc_clip(int64_t h, double mn, double mx) {
  try {
    return put(clip(get(h), mn, mx));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_scale(int64_t h, double s) {
  try {
    return put(scale_tensor(get(h), s));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_broadcast(int64_t h, const int64_t* shape, int rank) {
  try {
    return put(broadcast(get(h), Shape(shape, shape + rank)));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_broadcast_to_batch(int64_t h, int64_t batch) {
  try {
    return put(broadcast_to_batch(get(h), (size_t)batch));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_transpose(int64_t h, int d0, int d1) {
  try {
    return put(transpose(get(h), (size_t)d0, (size_t)d1));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_reshape(int64_t h, const int64_t* shape, int rank) {
  try {
    return put(reshape(get(h), Shape(shape, shape + rank)));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_softmax(int64_t h, int64_t seq_len, int causal) {
  try {
    return put(softmax(get(h), (size_t)seq_len, causal != 0));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_rmsnorm(int64_t hx, int64_t hw, double eps) {
  try {
    return put(rmsnorm(get(hx), get(hw), eps));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_rope(int64_t hx, int64_t max_len, double base, int64_t start_pos) {
  try {
    Tensor x = get(hx);
    Rope R = rope_new(x.shape.back(), (size_t)max_len, base);
    return put(rope_forward(R, x, (size_t)start_pos));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_bmm_qt_k(int64_t hq, int64_t hk) {
  try {
    Tensor q = get(hq), k = get(hk);
    return put(bmm_qt_k(q, k, q.shape[0], q.shape[1], q.shape[2]));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_bmm_p_v(int64_t hp, int64_t hv) {
  try {
    Tensor p = get(hp), v = get(hv);
    return put(bmm_p_v(p, v, v.shape[0], v.shape[1], v.shape[2]));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_concat_last(int64_t ha, int64_t hb) {
  try {
    return put(concat_last(get(ha), get(hb)));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int64_t orc_last_token(int64_t h, int differentiable) {
  try {
    return put(last_token(get(h), differentiable != 0));
  } catch (const std::exception& e) {
    g_err = e.what();
    return 0;
  }
}
int orc_backward(int64_t h) { GUARD(backward(get(h))) }
int orc_zero_grad(int64_t h) { GUARD(zero_grad(get(h))) }

// RoPE table as the reference precomputes it (f64), for the bit-exact table check.
void orc_rope_table(int64_t max_len, int64_t dim, double base, double* cos_out, double* sin_out) {
  Rope R = rope_new((size_t)dim, (size_t)max_len, base);
  std::copy(R.cosc.begin(), R.cosc.end(), cos_out);
  std::copy(R.sinc.begin(), R.sinc.end(), sin_out);
}
void orc_lcg_rand(int64_t n, double mn, double mx, uint64_t seed, double* out) {
  Vec v = lcg_rand((size_t)n, mn, mx, seed);
  std::copy(v.begin(), v.end(), out);
}

// --- model-level oracles ---------------------------------------------------

// C1: Linear(in,out,bias) + MSE against y (nn.rs:72-133, autograd.rs:1599-1603).
int orc_linear_mse(int64_t rows, int64_t in_f, int64_t out_f, const double* x, const double* w, const double* b,
                   const double* y, double* loss, double* dx, double* dw, double* db) {
  GUARD({
    Tensor X = tnew(Vec(x, x + rows * in_f), {(size_t)rows, (size_t)in_f});
    Linear L;
    L.in_f = in_f;
    L.out_f = out_f;
    L.weight = tnew(Vec(w, w + in_f * out_f), {(size_t)in_f, (size_t)out_f});
    L.has_bias = true;
    L.bias = tnew(Vec(b, b + out_f), {(size_t)out_f});
    Tensor Y = tnew(Vec(y, y + rows * out_f), {(size_t)rows, (size_t)out_f});
    Tensor l = mse_loss(linear_forward(L, X), Y);
    backward(l);
    *loss = (*l.data)[0];
    std::copy(X.grad->begin(), X.grad->end(), dx);
    std::copy(L.weight.grad->begin(), L.weight.grad->end(), dw);
    std::copy(L.bias.grad->begin(), L.bias.grad->end(), db);
  })
}

// Row ops (C2): forward + backward of a single op with upstream gradient dy.
int orc_rmsnorm_fwd_bwd(int64_t rows, int64_t dim, double eps, const double* x, const double* w, const double* dy,
                        double* y, double* dx, double* dw) {
  GUARD({
    Tensor X = tnew(Vec(x, x + rows * dim), {(size_t)rows, (size_t)dim});
    Tensor W = tnew(Vec(w, w + dim), {(size_t)dim});
    Tensor Y = rmsnorm(X, W, eps);
    Tensor G = tnew(Vec(dy, dy + rows * dim), {(size_t)rows, (size_t)dim});
    Tensor l = tsum(mul(Y, G));
    backward(l);
    std::copy(Y.data->begin(), Y.data->end(), y);
    std::copy(X.grad->begin(), X.grad->end(), dx);
    std::copy(W.grad->begin(), W.grad->end(), dw);
  })
}
int orc_softmax_fwd_bwd(int64_t rows, int64_t cols, int causal, const double* x, const double* dy, double* y,
                        double* dx) {
  GUARD({
    Tensor X = tnew(Vec(x, x + rows * cols), {(size_t)rows, (size_t)cols});
    Tensor Y = softmax(X, (size_t)cols, causal != 0);
    Tensor G = tnew(Vec(dy, dy + rows * cols), {(size_t)rows, (size_t)cols});
    backward(tsum(mul(Y, G)));
    std::copy(Y.data->begin(), Y.data->end(), y);
    std::copy(X.grad->begin(), X.grad->end(), dx);
  })
}
// RoPE on x[n_seq, seq, heads, dim] with position = sequence index: the layout is moved to
// [n_seq, heads, seq, dim] so that the reference op rotates along the sequence.
int orc_rope_fwd_bwd(int64_t n_seq, int64_t seq, int64_t heads, int64_t dim, double base, int64_t start_pos,
                     const double* x, const double* dy, double* y, double* dx) {
  GUARD({
    Shape s{(size_t)n_seq, (size_t)seq, (size_t)heads, (size_t)dim};
    Tensor X = tnew(Vec(x, x + prod(s)), s);
    Rope R = rope_new((size_t)dim, (size_t)(start_pos + seq), base);
    Tensor Y = transpose(rope_forward(R, transpose(X, 1, 2), (size_t)start_pos), 1, 2);
    Tensor G = tnew(Vec(dy, dy + prod(s)), s);
    backward(tsum(mul(Y, G)));
    std::copy(Y.data->begin(), Y.data->end(), y);
    std::copy(X.grad->begin(), X.grad->end(), dx);
  })
}
// Attention core on q/k [B,S,H,dk], v [B,S,H,dv] (already projected/rotated): forward output
// o [B,S,H,dv] and gradients for loss = sum(o * dout).
int orc_attention_fwd_bwd(int64_t B, int64_t S, int64_t H, int64_t dk, int64_t dv, double scale, int causal,
                          const double* q, const double* k, const double* v, const double* dout, double* o,
                          double* dq, double* dk_out, double* dv_out) {
  GUARD({
    Shape sq{(size_t)B, (size_t)S, (size_t)H, (size_t)dk}, sv{(size_t)B, (size_t)S, (size_t)H, (size_t)dv};
    Tensor Q = tnew(Vec(q, q + prod(sq)), sq), K = tnew(Vec(k, k + prod(sq)), sq), V = tnew(Vec(v, v + prod(sv)), sv);
    size_t BH = (size_t)(B * H);
    Tensor qf = reshape(transpose(Q, 1, 2), {BH, (size_t)S, (size_t)dk});
    Tensor kf = reshape(transpose(K, 1, 2), {BH, (size_t)S, (size_t)dk});
    Tensor vf = reshape(transpose(V, 1, 2), {BH, (size_t)S, (size_t)dv});
    Tensor sc = scale_tensor(bmm_qt_k(qf, kf, BH, (size_t)S, (size_t)dk), scale);
    Tensor pr = softmax(sc, (size_t)S, causal != 0);
    Tensor of = bmm_p_v(pr, vf, BH, (size_t)S, (size_t)dv);
    Tensor O = transpose(reshape(of, {(size_t)B, (size_t)H, (size_t)S, (size_t)dv}), 1, 2);
    Tensor G = tnew(Vec(dout, dout + prod(sv)), sv);
    backward(tsum(mul(O, G)));
    std::copy(O.data->begin(), O.data->end(), o);
    std::copy(Q.grad->begin(), Q.grad->end(), dq);
    std::copy(K.grad->begin(), K.grad->end(), dk_out);
    std::copy(V.grad->begin(), V.grad->end(), dv_out);
  })
}

size_t orc_block_param_count(const talos_block_cfg* c) { return block_param_count(*c); }

// C3: one block fwd+bwd with loss = sum(out * gout).
// dmag (nullable): the magnitude sums of the parameter gradients (Tensor::mag), same layout.
int orc_block_fwd_bwd(const talos_block_cfg* c, const double* params, const double* x, const double* gout,
                      double* out, double* dparams, double* dx, double* dmag) {
  GUARD({
    TrackMag tm(dmag != nullptr);
    Params P;
    P.src = params;
    Block b = make_block(P, *c);
    Rope R = rope_new(rope_dim_of(*c), (size_t)c->seq, c->rope_base);
    Shape s{(size_t)c->batch, (size_t)c->seq, (size_t)c->d_model};
    Tensor X = tnew(Vec(x, x + prod(s)), s);
    Tensor O = block_forward(b, *c, R, X);
    Tensor G = tnew(Vec(gout, gout + prod(s)), s);
    backward(tsum(mul(O, G)));
    block_pack_grads(b);
    std::copy(O.data->begin(), O.data->end(), out);
    P.grads(dparams);
    if (dmag) P.mags(dmag);
    std::copy(X.grad->begin(), X.grad->end(), dx);
  })
}

size_t orc_ppo_param_count(const talos_ppo_cfg* c) {
  size_t d = c->d_model;
  size_t blk = block_param_count(block_cfg_of(*c));
  return c->in_dim * d + d + c->n_layers * blk + d + d * d + d + d * c->n_actions + c->n_actions + d + 1;
}

// C4 batched: backbone once over [B,S,in], differentiable last token, batched closed-form loss.
// Writes loss, logits [B,A], values [B], dparams.
int orc_ppo_fwd_bwd(const talos_ppo_cfg* c, const double* params, const double* states, const int32_t* actions,
                    const double* adv, const double* ret, const double* old_logp, double* loss, double* logits_out,
                    double* values_out, double* dparams, double* dmag) {
  GUARD({
    TrackMag tm(dmag != nullptr);
    Params P;
    P.src = params;
    Policy pol = make_policy(P, *c);
    Rope R = rope_new(rope_dim_of(block_cfg_of(*c)), (size_t)c->seq, c->rope_base);
    size_t B = c->batch, S = c->seq, I = c->in_dim;
    Tensor X = tnew(Vec(states, states + B * S * I), {B, S, I});
    Tensor last = policy_last_hidden(pol, *c, R, X, true);
    Tensor logits = linear_forward(pol.actor, last);
    Tensor values = linear_forward(pol.critic, last);
    std::vector<int> acts(actions, actions + B);
    Tensor l = ppo_batched_loss(*c, logits, values, acts, Vec(old_logp, old_logp + B), Vec(adv, adv + B),
                                Vec(ret, ret + B));
    backward(l);
    for (auto& b : pol.blocks) block_pack_grads(b);
    *loss = (*l.data)[0];
    if (logits_out) std::copy(logits.data->begin(), logits.data->end(), logits_out);
    if (values_out) std::copy(values.data->begin(), values.data->end(), values_out);
    P.grads(dparams);
    if (dmag) P.mags(dmag);
  })
}

// C4 reference-faithful: one batch-1 graph per sample, the backbone run separately for the
// actor and for the critic (src/ppo.rs:691-757), loss accumulated and divided by the batch
// length. diff_last = 0 reproduces the reference's graph cut at last_token (src/transformer.rs:92-109).
int orc_ppo_fwd_bwd_per_sample(const talos_ppo_cfg* c, const double* params, const double* states,
                               const int32_t* actions, const double* adv, const double* ret,
                               const double* old_logp, int diff_last, double* loss, double* dparams,
                               double* dmag) {
  GUARD({
    TrackMag tm(dmag != nullptr);
    Params P;
    P.src = params;
    Policy pol = make_policy(P, *c);
    Rope R = rope_new(rope_dim_of(block_cfg_of(*c)), (size_t)c->seq, c->rope_base);
    size_t B = c->batch, S = c->seq, I = c->in_dim, A = c->n_actions;
    Tensor acc = tzeros({1});
    for (size_t i = 0; i < B; ++i) {
      // ActorCritic::forward_actor / forward_critic (src/ppo.rs:266-300): a [S, in] state is
      // reshaped to [1, S, in]; the head output [1, n] is reshaped to [n].
      Tensor st = tnew(Vec(states + i * S * I, states + (i + 1) * S * I), {S, I});
      Tensor xa = reshape(st, {1, S, I});
      Tensor la = policy_last_hidden(pol, *c, R, xa, diff_last != 0);
      Tensor logits = reshape(linear_forward(pol.actor, la), {A});
      Tensor xc = reshape(st, {1, S, I});
      Tensor lc = policy_last_hidden(pol, *c, R, xc, diff_last != 0);
      Tensor value = reshape(linear_forward(pol.critic, lc), {1});
      Tensor l = ppo_sample_loss(*c, logits, value, actions[i], old_logp[i], adv[i], ret[i]);
      acc = add(acc, l);
    }
    Tensor fl = tdiv(acc, tnew({(double)B}, {1}));
    backward(fl);
    for (auto& b : pol.blocks) block_pack_grads(b);
    *loss = (*fl.data)[0];
    P.grads(dparams);
    if (dmag) P.mags(dmag);
  })
}

// Per-sample PPO loss graph on given logits/value (for pinning the batched closed form).
int orc_ppo_sample_loss(const talos_ppo_cfg* c, const double* logits, double value, int action, double old_logp,
                        double adv, double ret, double* loss, double* dlogits, double* dvalue) {
  GUARD({
    size_t A = c->n_actions;
    Tensor z = tnew(Vec(logits, logits + A), {A});
    Tensor v = tnew({value}, {1});
    Tensor l = ppo_sample_loss(*c, z, v, action, old_logp, adv, ret);
    backward(l);
    *loss = (*l.data)[0];
    std::copy(z.grad->begin(), z.grad->end(), dlogits);
    *dvalue = (*v.grad)[0];
  })
}
int orc_ppo_batched_loss(const talos_ppo_cfg* c, int64_t B, const double* logits, const double* values,
                         const int32_t* actions, const double* old_logp, const double* adv, const double* ret,
                         double* loss, double* dlogits, double* dvalues) {
  GUARD({
    size_t A = c->n_actions;
    Tensor z = tnew(Vec(logits, logits + B * A), {(size_t)B, A});
    Tensor v = tnew(Vec(values, values + B), {(size_t)B, 1});
    std::vector<int> acts(actions, actions + B);
    Tensor l = ppo_batched_loss(*c, z, v, acts, Vec(old_logp, old_logp + B), Vec(adv, adv + B), Vec(ret, ret + B));
    backward(l);
    *loss = (*l.data)[0];
    std::copy(z.grad->begin(), z.grad->end(), dlogits);
    std::copy(v.grad->begin(), v.grad->end(), dvalues);
  })
}

// C5: MLA block out = x + MLA(rmsnorm(x)) with loss = sum(out * gout).
// cfg: [batch, seq, d_model, n_heads, kv_latent, rope_dim, head_dim, v_dim, causal, literal_rope]
size_t orc_mla_param_count(const int32_t* ci) {
  size_t d = ci[2], H = ci[3], L = ci[4], r = ci[5], hd = ci[6], vd = ci[7];
  return d + d * L + L * H * hd + L * H * vd + d * H * hd + d * H * r + d * H * r + H * vd * d;
}
int orc_mla_fwd_bwd(const int32_t* ci, double eps, double base, const double* params, const double* x,
                    const double* gout, double* out, double* dparams, double* dx, double* dmag) {
  GUARD({
    TrackMag tm(dmag != nullptr);
    MlaCfg c{ci[0], ci[1], ci[2], ci[3], ci[4], ci[5], ci[6], ci[7], ci[8], ci[9], eps, base};
    Params P;
    P.src = params;
    Mla m = make_mla(P, c);
    size_t max_len = c.literal_rope ? (size_t)std::max(c.seq, c.n_heads) : (size_t)c.seq;
    Rope R = rope_new((size_t)c.rope_dim, max_len, base);
    Shape s{(size_t)c.batch, (size_t)c.seq, (size_t)c.d_model};
    Tensor X = tnew(Vec(x, x + prod(s)), s);
    Tensor O = mla_forward(m, c, R, X);
    Tensor G = tnew(Vec(gout, gout + prod(s)), s);
    backward(tsum(mul(O, G)));
    std::copy(O.data->begin(), O.data->end(), out);
    P.grads(dparams);
    if (dmag) P.mags(dmag);
    std::copy(X.grad->begin(), X.grad->end(), dx);
  })
}

// Adam::step (src/ppo.rs:519-533) over one flat parameter vector with f64 state; t is the step
// count after the increment (src/ppo.rs:520). When max_norm > 0 the gradient is first clipped by
// its global L2 norm as the DQN optimizer does (src/dqn.rs:207-226): the norm is summed in index
// order, and g is multiplied by max_norm / norm when norm > max_norm (max_norm = 1.0 there).
void orc_adam_step(int64_t n, double* p, const double* g, double* m, double* v, int t, double lr, double b1,
                   double b2, double eps, double max_norm) {
  double clip_coef = 1.0;
  if (max_norm > 0.0) {
    double total = 0.0;
    for (int64_t j = 0; j < n; ++j) total += g[j] * g[j];
    total = std::sqrt(total);
    if (total > max_norm) clip_coef = max_norm / total;
  }
  const double bc1 = 1.0 - std::pow(b1, t), bc2 = 1.0 - std::pow(b2, t);
  for (int64_t j = 0; j < n; ++j) {
    const double gj = g[j] * clip_coef;
    m[j] = b1 * m[j] + (1.0 - b1) * gj;
    v[j] = b2 * v[j] + (1.0 - b2) * gj * gj;
    const double m_hat = m[j] / bc1, v_hat = v[j] / bc2;
    p[j] -= lr * m_hat / (std::sqrt(v_hat) + eps);
  }
}

// PPO::update's advantage prologue (src/ppo.rs:650-676), sequential as the reference: rewards
// normalised by the reward normaliser (RunningMeanStd::normalize, src/ppo.rs:477-479) and clipped
// to [-r_clip, r_clip]; delta_t = r_t + gamma * V_{t+1} * nonterm_t - V_t with V_len = 0;
// A_t = delta_t + gamma * lambda * nonterm_t * A_{t+1}; ret = A + V; the advantages are then
// normalised by their mean and population std + 1e-8.
void orc_ppo_gae(int64_t len, const double* rewards, const double* values, const uint8_t* terminals, double r_mean,
                 double r_var, double r_clip, double gamma, double lambda, double* adv_raw, double* returns,
                 double* adv_norm) {
  double last = 0.0;
  for (int64_t t = len - 1; t >= 0; --t) {
    const double nr = std::min(std::max((rewards[t] - r_mean) / (std::sqrt(r_var) + 1e-8), -r_clip), r_clip);
    const double non_terminal = terminals[t] ? 0.0 : 1.0;
    const double val_next = t < len - 1 ? values[t + 1] : 0.0;
    const double delta = nr + gamma * val_next * non_terminal - values[t];
    const double gae = delta + gamma * lambda * non_terminal * last;
    adv_raw[t] = gae;
    returns[t] = gae + values[t];
    last = gae;
  }
  double sum = 0.0;
  for (int64_t t = 0; t < len; ++t) sum += adv_raw[t];
  const double mean = sum / (double)len;
  double ss = 0.0;
  for (int64_t t = 0; t < len; ++t) ss += (adv_raw[t] - mean) * (adv_raw[t] - mean);
  const double stdv = std::sqrt(ss / (double)len) + 1e-8;
  for (int64_t t = 0; t < len; ++t) adv_norm[t] = (adv_raw[t] - mean) / stdv;
}

// Rollout decoder (see the orc::Decoder comment): one cache per environment and layer.
void* orc_decoder_new(const talos_ppo_cfg* c, const double* params, int64_t max_seq_len, int64_t n_envs) {
  auto* D = new Decoder();
  D->c = *c;
  D->p.assign(params, params + orc_ppo_param_count(c));
  const size_t rw = c->attention == TALOS_ATTN_MLA ? (size_t)c->rope_dim : (size_t)c->head_dim;
  D->rope = rope_new(rw, (size_t)max_seq_len, c->rope_base);
  D->cache.assign((size_t)n_envs, std::vector<KvCache>((size_t)c->n_layers));
  for (auto& env : D->cache)
    for (auto& kv : env) {
      kv.k.assign((size_t)c->n_heads, Vec());
      kv.v.assign((size_t)c->n_heads, Vec());
    }
  return D;
}
void orc_decoder_free(void* h) { delete static_cast<Decoder*>(h); }
// One token of environment env at position start_pos: logits [A], value, hidden [d] (the
// out_proj output the heads read).
int orc_decoder_step(void* h, int64_t env, const double* token, int64_t start_pos, double* logits, double* value,
                     double* hidden) {
  GUARD({
    auto* D = static_cast<Decoder*>(h);
    const talos_ppo_cfg& c = D->c;
    const size_t d = c.d_model, A = c.n_actions;
    const double* P = D->p.data();
    Vec x = linear_inf(token, (size_t)c.in_dim, d, P, P + c.in_dim * d);
    size_t o = (size_t)c.in_dim * d + d;
    talos_block_cfg bc = block_cfg_of(c);
    const size_t blk = block_param_count(bc);
    for (int l = 0; l < c.n_layers; ++l) {
      x = block_step(*D, P + o, x, D->cache[(size_t)env][(size_t)l], (size_t)start_pos);
      o += blk;
    }
    Vec hf = rmsnorm_inf(x, P + o, c.eps);
    o += d;
    Vec out = linear_inf(hf.data(), d, d, P + o, P + o + d * d);
    o += d * d + d;
    Vec lg = linear_inf(out.data(), d, A, P + o, P + o + d * A);
    o += d * A + A;
    Vec val = linear_inf(out.data(), d, 1, P + o, P + o + d);
    if (logits) std::copy(lg.begin(), lg.end(), logits);
    if (value) *value = val[0];
    if (hidden) std::copy(out.begin(), out.end(), hidden);
  })
}
// prune_kv_cache: keep the newest max_len rows of every layer (src/transformer.rs:807-840).
void orc_decoder_prune(void* h, int64_t env, int64_t max_len) {
  auto* D = static_cast<Decoder*>(h);
  const bool mla = D->c.attention == TALOS_ATTN_MLA;
  const size_t td = (size_t)D->c.head_dim + (mla ? (size_t)D->c.rope_dim : 0);
  const size_t vd = mla ? (size_t)D->c.v_dim : (size_t)D->c.head_dim;
  for (auto& kv : D->cache[(size_t)env]) {
    const size_t cur = kv.k[0].size() / td;
    if (cur <= (size_t)max_len) continue;
    const size_t rm = cur - (size_t)max_len;
    for (size_t hh = 0; hh < kv.k.size(); ++hh) {
      kv.k[hh].erase(kv.k[hh].begin(), kv.k[hh].begin() + (std::ptrdiff_t)(rm * td));
      kv.v[hh].erase(kv.v[hh].begin(), kv.v[hh].begin() + (std::ptrdiff_t)(rm * vd));
    }
  }
}
void orc_decoder_clear(void* h, int64_t env) {
  for (auto& kv : static_cast<Decoder*>(h)->cache[(size_t)env])
    for (size_t hh = 0; hh < kv.k.size(); ++hh) {
      kv.k[hh].clear();
      kv.v[hh].clear();
    }
}
// Rows cached for (env, layer), oldest first: k [len, H, dk] and v [len, H, dv] when non-null.
int64_t orc_decoder_cache(void* h, int64_t env, int64_t layer, double* k, double* v) {
  auto* D = static_cast<Decoder*>(h);
  const bool mla = D->c.attention == TALOS_ATTN_MLA;
  const size_t H = (size_t)D->c.n_heads, td = (size_t)D->c.head_dim + (mla ? (size_t)D->c.rope_dim : 0);
  const size_t vd = mla ? (size_t)D->c.v_dim : (size_t)D->c.head_dim;
  const KvCache& kv = D->cache[(size_t)env][(size_t)layer];
  const size_t n = kv.k[0].size() / td;
  for (size_t j = 0; j < n; ++j)
    for (size_t hh = 0; hh < H; ++hh) {
      if (k) std::copy(&kv.k[hh][j * td], &kv.k[hh][j * td] + td, k + (j * H + hh) * td);
      if (v) std::copy(&kv.v[hh][j * vd], &kv.v[hh][j * vd] + vd, v + (j * H + hh) * vd);
    }
  return (int64_t)n;
}
// The action choice of ActorCritic::step / step_inference_cached (src/ppo.rs:311-346, 401-432)
// with the uniform draw r given: probabilities by max-subtracted exp (max starts at -1e9), then
// the first i with r < p_i, subtracting p_i otherwise. When no i qualifies (r at or past the
// rounded total) the index keeps its initial 0: the reference's `action_idx == ACTION_SPACE`
// fallback can never fire. *logp = ln p[a].
int orc_sample_action(const double* logits, int64_t A, double r, double* logp) {
  double mx = -1e9;
  for (int64_t i = 0; i < A; ++i)
    if (logits[i] > mx) mx = logits[i];
  Vec p((size_t)A);
  double sum = 0.0;
  for (int64_t i = 0; i < A; ++i) {
    p[(size_t)i] = std::exp(logits[i] - mx);
    sum += p[(size_t)i];
  }
  for (auto& x : p) x /= sum;
  int64_t a = 0;
  for (int64_t i = 0; i < A; ++i) {
    if (r < p[(size_t)i]) {
      a = i;
      break;
    }
    r -= p[(size_t)i];
  }
  if (a == A) a = A - 1;  // unreachable, kept as the reference writes it
  if (logp) *logp = std::log(p[(size_t)a]);
  return (int)a;
}

}  // extern "C"
