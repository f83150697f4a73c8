// test_tape.cpp -- the reference's own autograd tests, run through the device tape (tape.hpp) on the
// GPU, plus graphs compared element-wise with the f64 oracle (oracle/liboracle.so, the checker).
//
// Mirrors src/grad_check.rs:6-114 (graph detach / clear, matmul KAT, broadcast KAT, finite
// difference of x^2 sin x), src/transformer.rs:1191-1328 (reshape copies, transpose KAT, the MLA,
// RoPE and RMSNorm backward tests, the LuckTransformer integration test) and src/autograd.rs:
// 1868-1875 (scalar broadcast); beyond the reference's sign / non-zero checks every module graph is
// compared element-wise with the same graph built from the oracle's ops. A DQN training step
// (DuelingQNetwork and train_dqn's batched update, src/dqn.rs:68-107, 134-154, 515-576) runs on the
// tape unchanged and is checked the same way. Exit status 0 when every check passes; each failing
// check prints its name and values.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../talos-xii_amd/host/tape.hpp"

using talos::tape::Linear;
using talos::tape::LuckTransformer;
using talos::tape::MLAConfig;
using talos::tape::MultiHeadLatentAttention;
using talos::tape::Panic;
using talos::tape::RMSNorm;
using talos::tape::RoPE;
using talos::tape::Shape;
using talos::tape::Tensor;

extern "C" {
// oracle C ABI (oracle/talos_oracle.cpp)
const char* orc_last_error(void);
int64_t orc_tensor_new_len(const double* data, int64_t len, const int64_t* shape, int rank);
void orc_tensor_data(int64_t h, double* out);
void orc_tensor_grad(int64_t h, double* out);
void orc_set_track_mag(int on);
void orc_tensor_mag(int64_t h, double* out);
int64_t orc_matmul(int64_t a, int64_t b);
int64_t orc_add(int64_t a, int64_t b);
int64_t orc_sub(int64_t a, int64_t b);
int64_t orc_mul(int64_t a, int64_t b);
int64_t orc_div(int64_t a, int64_t b);
int64_t orc_relu(int64_t h);
int64_t orc_exp(int64_t h);
int64_t orc_log(int64_t h);
int64_t orc_sin(int64_t h);
int64_t orc_sqrt(int64_t h);
int64_t orc_neg(int64_t h);
int64_t orc_sum(int64_t h);
int64_t orc_mean(int64_t h);
int64_t orc_clip(int64_t h, double mn, double mx);
int64_t orc_broadcast_to_batch(int64_t h, int64_t batch);
int64_t orc_transpose(int64_t h, int d0, int d1);
int64_t orc_reshape(int64_t h, const int64_t* shape, int rank);
int64_t orc_mse_loss(int64_t a, int64_t b);
int orc_backward(int64_t h);
int orc_linear_mse(int64_t rows, int64_t in_f, int64_t out_f, const double* x, const double* w, const double* b,
                   const double* y, double* loss, double* dx, double* dw, double* db);
void orc_adam_step(int64_t n, double* p, const double* g, double* m, double* v, int t, double lr, double b1,
                   double b2, double eps, double max_norm);
int orc_rmsnorm_fwd_bwd(int64_t rows, int64_t dim, double eps, const double* x, const double* w, const double* dy,
                        double* y, double* dx, double* dw);
int64_t orc_scale(int64_t h, double s);
int64_t orc_softmax(int64_t h, int64_t seq_len, int causal);
int64_t orc_rmsnorm(int64_t hx, int64_t hw, double eps);
int64_t orc_rope(int64_t hx, int64_t max_len, double base, int64_t start_pos);
int64_t orc_bmm_qt_k(int64_t hq, int64_t hk);
int64_t orc_bmm_p_v(int64_t hp, int64_t hv);
int64_t orc_concat_last(int64_t ha, int64_t hb);
void orc_free_all(void);
int64_t orc_broadcast(int64_t h, const int64_t* shape, int rank);
}

static int g_fail = 0, g_pass = 0;

static void check(bool cond, const std::string& name) {
  if (cond) {
    ++g_pass;
  } else {
    ++g_fail;
    std::printf("FAIL %s\n", name.c_str());
  }
}

static bool near(double a, double b, double tol) { return std::fabs(a - b) < tol; }

// |got - ref| <= rtol |ref| + max(atol, kappa 2^-24 mag) element-wise: the fp32 rule of the parity
// tests. mag (optional) holds the oracle's magnitude sums of the gradient (sums of |term| over
// every term of each element, orc_tensor_mag); with it, elements that cancel far below their terms
// get the rounding allowance of an fp32 evaluation of the same sum (kappa = 32, tests/common.py
// GRAD_KAPPA), and the number of elements that needed it is printed.
constexpr double kGradKappa = 32.0;
static void close(const std::vector<double>& got, const std::vector<double>& ref, const std::string& name,
                  double rtol = 1e-4, double atol = 1e-5, const std::vector<double>* mag = nullptr) {
  if (got.size() != ref.size() || (mag && mag->size() != ref.size())) {
    check(false, name + " (size)");
    return;
  }
  double worst = 0.0;
  size_t wi = 0, needs_mag = 0;
  bool okay = true;
  for (size_t i = 0; i < got.size(); ++i) {
    const double allow = mag ? std::max(atol, kGradKappa * std::ldexp((*mag)[i], -24)) : atol;
    const double err = std::fabs(got[i] - ref[i]), bound = rtol * std::fabs(ref[i]) + allow;
    if (err > bound) okay = false;
    if (err > rtol * std::fabs(ref[i]) + atol) ++needs_mag;
    if (err - bound > worst) {
      worst = err - bound;
      wi = i;
    }
  }
  if (mag && needs_mag)
    std::printf("  %s: %zu / %zu elements need the magnitude allowance\n", name.c_str(), needs_mag, got.size());
  if (!okay) std::printf("  %s worst at %zu: got %.9g ref %.9g\n", name.c_str(), wi, got[wi], ref[wi]);
  check(okay, name);
}

static std::vector<double> rng_normal(size_t n, uint64_t& s) {
  std::vector<double> v(n);
  for (size_t i = 0; i < n; i += 2) {  // Box-Muller on a 64-bit LCG
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    const double u1 = ((s >> 11) + 1.0) / 9007199254740993.0;
    s = s * 6364136223846793005ULL + 1442695040888963407ULL;
    const double u2 = (s >> 11) / 9007199254740992.0;
    const double r = std::sqrt(-2.0 * std::log(u1));
    v[i] = (double)(float)(r * std::cos(2 * M_PI * u2));
    if (i + 1 < n) v[i + 1] = (double)(float)(r * std::sin(2 * M_PI * u2));
  }
  return v;
}

static int64_t onew(const std::vector<double>& d, const std::vector<int64_t>& shape) {
  return orc_tensor_new_len(d.data(), (int64_t)d.size(), shape.data(), (int)shape.size());
}
static std::vector<double> odata(int64_t h, size_t n) {
  std::vector<double> v(n);
  orc_tensor_data(h, v.data());
  return v;
}
static std::vector<double> ograd(int64_t h, size_t n) {
  std::vector<double> v(n);
  orc_tensor_grad(h, v.data());
  return v;
}

// src/grad_check.rs:6-27
static void test_autograd_memory_leak_fix() {
  Tensor a = Tensor::from_vec({2.0}, {1});
  Tensor b = a;
  for (int i = 0; i < 100; ++i) b = b * Tensor::from_vec({1.1}, {1});
  check(b._ctx != nullptr, "memory_leak_fix: graph kept");
  Tensor c = b.detach();
  check(c._ctx == nullptr, "memory_leak_fix: detach drops the graph");
  Tensor d = b;
  d.clear_graph();
  check(d._ctx == nullptr, "memory_leak_fix: clear_graph");
  b.backward();
  check(near(a.grad()[0], std::pow(1.1, 100), 1e-4 * std::pow(1.1, 100)), "memory_leak_fix: d b / d a = 1.1^100");
}

// src/grad_check.rs:30-63
static void test_grad_check_matmul() {
  Tensor a = Tensor::from_vec({2.0, 3.0, 4.0, 5.0}, {2, 2});
  Tensor x = Tensor::from_vec({1.0, 2.0}, {2, 1});
  Tensor y = a.matmul(x);
  Tensor loss = y.sum();
  loss.backward();
  const auto ag = a.grad(), xg = x.grad();
  check(near(xg[0], 6.0, 1e-6) && near(xg[1], 8.0, 1e-6), "grad_check_matmul: dx = [6, 8]");
  check(near(ag[0], 1.0, 1e-6) && near(ag[1], 2.0, 1e-6) && near(ag[2], 1.0, 1e-6) && near(ag[3], 2.0, 1e-6),
        "grad_check_matmul: dA = [[1, 2], [1, 2]]");
  check(near(loss.item(), 22.0, 1e-6), "grad_check_matmul: loss = 22");
}

// src/grad_check.rs:66-90
static void test_grad_check_broadcast() {
  Tensor x = Tensor::from_vec({1.0, 2.0}, {2});
  Tensor y = Tensor::from_vec({10.0}, {1});
  Tensor z = x + y.broadcast({2});
  Tensor loss = z.sum();
  loss.backward();
  const auto xg = x.grad(), yg = y.grad();
  check(near(xg[0], 1.0, 1e-6) && near(xg[1], 1.0, 1e-6), "grad_check_broadcast: dx = [1, 1]");
  check(near(yg[0], 2.0, 1e-6), "grad_check_broadcast: dy = 2");
}

// src/grad_check.rs:93-114: autograd of x^2 sin x against a central difference (eps 1e-6, f64)
static void test_numerical_gradient_check() {
  const double xv = 2.0, eps = 1e-6;
  Tensor x = Tensor::from_vec({xv}, {1});
  Tensor y = (x * x) * x.sin();
  y.backward();
  const double g_auto = x.grad()[0];
  auto f = [](double v) { return v * v * std::sin(v); };
  const double g_num = (f(xv + eps) - f(xv - eps)) / (2 * eps);
  std::printf("  numerical gradient: auto %.9f num %.9f\n", g_auto, g_num);
  check(std::fabs(g_auto - g_num) < 1e-4, "numerical_gradient_check");
}

// src/autograd.rs:1868-1875
static void test_broadcast_scalar() {
  Tensor t = Tensor::from_vec({5.0}, {1});
  Tensor b = t.broadcast({2, 2});
  check(b.shape == talos::tape::Shape({2, 2}) && b.data() == std::vector<double>({5, 5, 5, 5}), "broadcast_scalar");
}

// src/transformer.rs:1191-1209: reshape is a copy
static void test_tensor_reshape() {
  Tensor t = Tensor::from_vec({1.0, 2.0, 3.0, 4.0}, {2, 2});
  Tensor r = t.reshape({4});
  check(r.shape == talos::tape::Shape({4}) && r.data()[0] == 1.0, "tensor_reshape: data");
  t.set_data({10.0, 2.0, 3.0, 4.0});
  check(r.data()[0] == 1.0, "tensor_reshape: independent copy");
}

// src/transformer.rs:1211-1225, plus the backward (inverse permutation, added)
static void test_tensor_transpose() {
  Tensor t = Tensor::from_vec({1, 2, 3, 4, 5, 6}, {2, 3});
  Tensor tt = t.transpose(0, 1);
  check(tt.shape == talos::tape::Shape({3, 2}) && tt.data() == std::vector<double>({1, 4, 2, 5, 3, 6}),
        "tensor_transpose: data");
  Tensor w = Tensor::from_vec({1, 10, 100, 1000, 1e4, 1e5}, {3, 2});
  (tt * w).sum().backward();
  check(t.grad() == std::vector<double>({1, 100, 1e4, 10, 1000, 1e5}), "tensor_transpose: backward");
}

// src/transformer.rs:1283-1299 (non-zero grads) and the closed form of the oracle
static void test_rmsnorm_backward() {
  RMSNorm norm(4, 1e-5);
  Tensor x = Tensor::rand({2, 4}, 0.1, 1.0, 123);
  Tensor out = norm.forward(x);
  out.sum().backward();
  bool any_x = false, any_w = false;
  for (double g : x.grad()) any_x |= std::fabs(g) > 1e-6;
  for (double g : norm.weight.grad()) any_w |= std::fabs(g) > 1e-6;
  check(any_x && any_w, "rmsnorm_backward: gradients flow");
  // against the oracle with an all-ones upstream gradient
  const auto xd = x.data();
  std::vector<double> w(4, 1.0), dy(8, 1.0), y(8), dx(8), dw(4);
  orc_rmsnorm_fwd_bwd(2, 4, 1e-5, xd.data(), w.data(), dy.data(), y.data(), dx.data(), dw.data());
  close(out.data(), y, "rmsnorm vs oracle: y");
  close(x.grad(), dx, "rmsnorm vs oracle: dx");
  close(norm.weight.grad(), dw, "rmsnorm vs oracle: dgain");
}

// C1: Linear [256,64] . [64,64] + MSE through the tape, against the oracle
static void test_linear_mse_c1() {
  uint64_t s = 11;
  const auto xv = rng_normal(256 * 64, s), yv = rng_normal(256 * 64, s);
  Linear lin(64, 64, true, 42);  // Linear::new's Xavier draw (Tensor::rand)
  Tensor x = Tensor::from_vec(xv, {256, 64}), y = Tensor::from_vec(yv, {256, 64});
  Tensor loss = lin.forward(x).mse_loss(y);
  loss.backward();
  const auto wv = lin.weight.data(), bv = lin.bias.data();
  double lr;
  std::vector<double> dx(256 * 64), dw(64 * 64), db(64);
  orc_linear_mse(256, 64, 64, xv.data(), wv.data(), bv.data(), yv.data(), &lr, dx.data(), dw.data(), db.data());
  close({loss.item()}, {lr}, "linear_mse: loss");
  close(x.grad(), dx, "linear_mse: dX");
  close(lin.weight.grad(), dw, "linear_mse: dW");
  close(lin.bias.grad(), db, "linear_mse: db");
  // grads accumulate across backward calls until zero_grad (src/autograd.rs:191-196)
  Tensor loss2 = lin.forward(x).mse_loss(y);
  loss2.backward();
  std::vector<double> dw2(dw.size());
  for (size_t i = 0; i < dw.size(); ++i) dw2[i] = 2 * dw[i];
  close(lin.weight.grad(), dw2, "linear_mse: grads accumulate");
  lin.weight.zero_grad();
  check(lin.weight.grad() == std::vector<double>(64 * 64, 0.0), "linear_mse: zero_grad");
}

// A graph over every tape op, built the same way in the tape and in the oracle.
static void test_composite_graph() {
  uint64_t s = 5;
  const auto av = rng_normal(6 * 5, s), bv = rng_normal(5 * 4, s), cv = rng_normal(4, s), tv = rng_normal(6 * 4, s);
  // tape
  Tensor A = Tensor::from_vec(av, {6, 5}), B = Tensor::from_vec(bv, {5, 4}), C = Tensor::from_vec(cv, {4});
  Tensor T = Tensor::from_vec(tv, {6, 4});
  Tensor h = A.matmul(B) + C.broadcast_to_batch(6);
  Tensor u = h.relu() + (h.clip(-0.5, 0.5) * h.sin());
  Tensor e = u.transpose(0, 1).reshape({2, 12}).exp();
  Tensor q = (e / (e + e.sqrt())).log();
  Tensor z = q.reshape({6, 4}) - (-T);
  Tensor loss = z.mse_loss(T) + z.mean();
  loss.backward();
  // oracle
  const int64_t oA = onew(av, {6, 5}), oB = onew(bv, {5, 4}), oC = onew(cv, {4}), oT = onew(tv, {6, 4});
  const int64_t oh = orc_add(orc_matmul(oA, oB), orc_broadcast_to_batch(oC, 6));
  const int64_t ou = orc_add(orc_relu(oh), orc_mul(orc_clip(oh, -0.5, 0.5), orc_sin(oh)));
  const std::vector<int64_t> s212{2, 12}, s64{6, 4};
  const int64_t oe = orc_exp(orc_reshape(orc_transpose(ou, 0, 1), s212.data(), 2));
  const int64_t oq = orc_log(orc_div(oe, orc_add(oe, orc_sqrt(oe))));
  const int64_t oz = orc_sub(orc_reshape(oq, s64.data(), 2), orc_neg(oT));
  const int64_t ol = orc_add(orc_mse_loss(oz, oT), orc_mean(oz));
  if (orc_backward(ol) != 0) std::printf("oracle: %s\n", orc_last_error());
  close({loss.item()}, odata(ol, 1), "composite: loss");
  close(A.grad(), ograd(oA, 30), "composite: dA");
  close(B.grad(), ograd(oB, 20), "composite: dB");
  close(C.grad(), ograd(oC, 4), "composite: dC");
  close(T.grad(), ograd(oT, 24), "composite: dT");
}

// Adam over a Linear's parameters (src/ppo.rs:482-539), and the DQN variant with the global
// gradient-norm clip (src/dqn.rs:207-226): three training steps through the tape against the
// oracle's f64 Adam fed the same gradients. The target scale makes ||g|| > 1 in the clipped run.
static void run_adam(double max_norm, double target_scale, const std::string& tag) {
  uint64_t s = 23;
  const auto xv = rng_normal(32 * 16, s);
  auto yv = rng_normal(32 * 8, s);
  for (double& y : yv) y *= target_scale;
  Linear lin(16, 8, true, 7);
  Tensor x = Tensor::from_vec(xv, {32, 16}), y = Tensor::from_vec(yv, {32, 8});
  talos::tape::Adam opt(lin.parameters(), 1e-2, max_norm);
  auto flat = [&](bool grads) {
    std::vector<double> out;
    for (const Tensor& p : lin.parameters()) {
      const auto d = grads ? p.grad() : p.data();
      out.insert(out.end(), d.begin(), d.end());
    }
    return out;
  };
  const std::vector<double> p0 = flat(false);
  std::vector<double> pr = p0, m(p0.size(), 0.0), v(p0.size(), 0.0);
  bool clipped = false;
  for (int t = 1; t <= 3; ++t) {
    opt.zero_grad();
    lin.forward(x).mse_loss(y).backward();
    const std::vector<double> g = flat(true);
    double ss = 0.0;
    for (double gi : g) ss += gi * gi;
    clipped = clipped || std::sqrt(ss) > 1.0;
    opt.step();
    orc_adam_step((int64_t)pr.size(), pr.data(), g.data(), m.data(), v.data(), t, 1e-2, 0.9, 0.999, 1e-8, max_norm);
    const std::vector<double> got = flat(false);
    std::vector<double> dgot(got.size()), dref(got.size());
    for (size_t i = 0; i < got.size(); ++i) {
      dgot[i] = got[i] - p0[i];
      dref[i] = pr[i] - p0[i];
    }
    close(dgot, dref, tag + ": parameter delta after step " + std::to_string(t));
  }
  check(opt.t() == 3, tag + ": step count");
  if (max_norm > 0.0) check(clipped, tag + ": the clip engaged");
}

static void test_adam_ppo() { run_adam(0.0, 1.0, "adam"); }
static void test_adam_dqn_clip() { run_adam(1.0, 30.0, "adam+clip"); }

// ---------------------------------------------------------------------------------------------
// Oracle-side restatement of the module wiring (the checker): each op is the oracle's, each
// module's forward follows the reference function cited
// ---------------------------------------------------------------------------------------------
static int64_t oshape(int64_t h, const std::vector<int64_t>& shape) {
  return orc_reshape(h, shape.data(), (int)shape.size());
}
static int64_t onew_t(const Tensor& t) {
  std::vector<int64_t> sh(t.shape.begin(), t.shape.end());
  return onew(t.data(), sh);
}
// Linear::forward (src/nn.rs:72-133) on the oracle: flatten N-D input, x . W, reshape back, bias
static int64_t olinear(int64_t x, const std::vector<int64_t>& xshape, const Linear& L, int64_t w, int64_t b) {
  const size_t rank = xshape.size();
  int64_t xf = x;
  int64_t bd = 1;
  if (rank > 2) {
    for (size_t i = 0; i + 1 < rank; ++i) bd *= xshape[i];
    xf = oshape(x, {bd, (int64_t)L.in_features});
  }
  int64_t out = orc_matmul(xf, w);
  std::vector<int64_t> oshp;
  if (rank > 2) {
    oshp.assign(xshape.begin(), xshape.end() - 1);
    oshp.push_back((int64_t)L.out_features);
    out = oshape(out, oshp);
  } else if (rank == 2) {
    oshp = {xshape[0], (int64_t)L.out_features};
  } else {
    oshp = {(int64_t)L.out_features};
  }
  if (!L.has_bias) return out;
  if (oshp.size() == 2 && oshp[0] > 1) return orc_add(out, orc_broadcast_to_batch(b, oshp[0]));
  if (oshp.size() > 2) {
    int64_t n = 1;
    for (int64_t v : oshp) n *= v;
    const int64_t rows = n / (int64_t)L.out_features;
    return oshape(orc_add(oshape(out, {rows, (int64_t)L.out_features}), orc_broadcast_to_batch(b, rows)), oshp);
  }
  if (oshp.size() == 2) return orc_add(out, oshape(b, {1, (int64_t)L.out_features}));
  return orc_add(out, b);
}
struct OLin {
  const Linear* L;
  int64_t w, b;
};
static OLin olin(const Linear& L) { return {&L, onew_t(L.weight), L.has_bias ? onew_t(L.bias) : 0}; }
static int64_t ofwd(const OLin& o, int64_t x, const std::vector<int64_t>& xs) { return olinear(x, xs, *o.L, o.w, o.b); }
static std::vector<double> omag(int64_t h, size_t n) {
  std::vector<double> v(n);
  orc_tensor_mag(h, v.data());
  return v;
}
// with_mag: the oracle tensor was created under orc_set_track_mag(1), so its magnitude sums bound
// the comparison as well
static void close_grad(const Tensor& t, int64_t h, const std::string& name, bool with_mag = false) {
  const std::vector<double> m = with_mag ? omag(h, t.numel()) : std::vector<double>();
  close(t.grad(), ograd(h, t.numel()), name, 1e-4, 1e-5, with_mag ? &m : nullptr);
}

// MultiHeadLatentAttention::forward (src/transformer.rs:478-560) on the oracle
struct OMla {
  OLin dkv, uk, uv, q, kr, qr, o;
};
static OMla omla(const MultiHeadLatentAttention& m) {
  return {olin(m.w_dkv), olin(m.w_uk), olin(m.w_uv), olin(m.w_q), olin(m.w_kr), olin(m.w_qr), olin(m.w_o)};
}
static int64_t omla_forward(const OMla& w, const MLAConfig& c, int64_t x, int64_t B, int64_t S) {
  const int64_t H = (int64_t)c.num_heads, hd = (int64_t)c.v_head_dim, R = (int64_t)c.qk_rope_dim;
  const std::vector<int64_t> xs{B, S, (int64_t)c.dim}, cs{B, S, (int64_t)c.kv_lora_rank};
  const int64_t ckv = ofwd(w.dkv, x, xs);
  const int64_t kc = ofwd(w.uk, ckv, cs), vc = ofwd(w.uv, ckv, cs);
  const int64_t kr = ofwd(w.kr, x, xs), qc = ofwd(w.q, x, xs), qr = ofwd(w.qr, x, xs);
  const int64_t krr = orc_rope(oshape(kr, {B, S, H, R}), (int64_t)c.max_seq_len, 10000.0, 0);
  const int64_t qrr = orc_rope(oshape(qr, {B, S, H, R}), (int64_t)c.max_seq_len, 10000.0, 0);
  const int64_t q = orc_concat_last(oshape(qc, {B, S, H, hd}), qrr);
  const int64_t k = orc_concat_last(oshape(kc, {B, S, H, hd}), krr);
  const int64_t v = oshape(vc, {B, S, H, hd});
  const int64_t bh = B * H, tot = hd + R;
  const int64_t qf = oshape(orc_transpose(q, 1, 2), {bh, S, tot});
  const int64_t kf = oshape(orc_transpose(k, 1, 2), {bh, S, tot});
  const int64_t vf = oshape(orc_transpose(v, 1, 2), {bh, S, hd});
  const int64_t pr = orc_softmax(orc_scale(orc_bmm_qt_k(qf, kf), 1.0 / std::sqrt((double)tot)), S, 0);
  const int64_t att = orc_bmm_p_v(pr, vf);
  const int64_t merged = oshape(orc_transpose(oshape(att, {B, H, S, hd}), 1, 2), {B, S, H * hd});
  return ofwd(w.o, merged, {B, S, H * hd});
}
static void close_mla_grads(const MultiHeadLatentAttention& m, const OMla& w, const std::string& tag,
                            bool with_mag = false) {
  close_grad(m.w_dkv.weight, w.dkv.w, tag + " dW_dkv", with_mag);
  close_grad(m.w_uk.weight, w.uk.w, tag + " dW_uk", with_mag);
  close_grad(m.w_uv.weight, w.uv.w, tag + " dW_uv", with_mag);
  close_grad(m.w_q.weight, w.q.w, tag + " dW_q", with_mag);
  close_grad(m.w_kr.weight, w.kr.w, tag + " dW_kr", with_mag);
  close_grad(m.w_qr.weight, w.qr.w, tag + " dW_qr", with_mag);
  close_grad(m.w_o.weight, w.o.w, tag + " dW_o", with_mag);
}
static bool any_nonzero(const std::vector<double>& v, double tol = 0.0) {
  for (double g : v)
    if (std::fabs(g) > tol) return true;
  return false;
}

// src/transformer.rs:1228-1266 (MLA forward / backward), and the same graph on the oracle
static void test_mla_forward_backward() {
  MLAConfig c;
  c.dim = 16;
  c.num_heads = 2;
  c.q_lora_rank = 0;
  c.kv_lora_rank = 8;
  c.qk_rope_dim = 4;
  c.v_head_dim = 8;
  c.max_seq_len = 10;
  MultiHeadLatentAttention mla(c, 42);
  Tensor input = Tensor::rand({1, 3, 16}, -0.1, 0.1, 123);
  Tensor output = mla.forward(input);
  check(output.shape == Shape({1, 3, 16}), "mla_forward_backward: output shape");
  Tensor loss = output.mean();
  loss.backward();
  double sdkv = 0.0, suk = 0.0;
  for (double g : mla.w_dkv.weight.grad()) sdkv += g;
  for (double g : mla.w_uk.weight.grad()) suk += g;
  check(std::fabs(sdkv) > 0.0, "mla_forward_backward: W_DKV gradient is not zero");
  check(std::fabs(suk) > 0.0, "mla_forward_backward: W_UK gradient is not zero");
  const OMla w = omla(mla);
  const int64_t ox = onew_t(input);
  const int64_t oout = omla_forward(w, c, ox, 1, 3);
  const int64_t ol = orc_mean(oout);
  orc_backward(ol);
  close(output.data(), odata(oout, output.numel()), "mla vs oracle: out");
  close({loss.item()}, odata(ol, 1), "mla vs oracle: loss");
  close_grad(input, ox, "mla vs oracle: dx");
  close_mla_grads(mla, w, "mla vs oracle:");
  orc_free_all();
}

// The MLA of MLAConfig::deepseek_v2_lite (C5's attention) at batch 2, seq 8, on the tape and the
// oracle, loss = sum(out * G). The input is N(0, 0.1^2), the scale of the reference's own module
// tests (Tensor::rand(-0.1, 0.1)): Linear::new's Tensor::rand draws every weight from [-l, 0), so
// the projections of N(0, 1) rows at d = 512 share a large common component, the logits reach the
// hundreds and the softmax saturates; a probability that rounds to 1 in fp32 carries no gradient
// where the f64 oracle still holds one of order 1e-6.
static void test_mla_deepseek_lite() {
  const MLAConfig c = MLAConfig::deepseek_v2_lite();
  MultiHeadLatentAttention mla(c, 7);
  uint64_t s = 77;
  auto xv = rng_normal(2 * 8 * 512, s);
  const auto gv = rng_normal(2 * 8 * 512, s);
  for (double& v : xv) v = (double)(float)(0.1 * v);
  Tensor x = Tensor::from_vec(xv, {2, 8, 512}), G = Tensor::from_vec(gv, {2, 8, 512});
  Tensor out = mla.forward(x);
  Tensor loss = (out * G).sum();
  loss.backward();
  orc_set_track_mag(1);
  const OMla w = omla(mla);
  const int64_t ox = onew(xv, {2, 8, 512}), oG = onew(gv, {2, 8, 512});
  const int64_t oout = omla_forward(w, c, ox, 2, 8);
  const int64_t ol = orc_sum(orc_mul(oout, oG));
  orc_backward(ol);
  orc_set_track_mag(0);
  close(out.data(), odata(oout, out.numel()), "deepseek_lite mla: out");
  // sum(out * G) at d = 512 is unscaled: dx and the weight gradients hold elements that cancel far
  // below their terms, so they take the magnitude allowance (its use is printed)
  close_grad(x, ox, "deepseek_lite mla: dx", true);
  close_mla_grads(mla, w, "deepseek_lite mla:", true);
  orc_free_all();
}

// src/transformer.rs:1269-1281 (RoPE backward), and against the oracle's RoPE
static void test_rope_backward() {
  RoPE rope(4, 10);
  Tensor x = Tensor::rand({1, 2, 4}, -1.0, 1.0, 123);
  Tensor out = rope.forward(x, 0);
  out.sum().backward();
  check(any_nonzero(x.grad(), 1e-6), "rope_backward: x.grad is not zero");
  // a second input, rows along shape[-2] at start_pos 3, loss = sum(out * G)
  uint64_t s = 9;
  const auto yv = rng_normal(3 * 5 * 8, s), gv = rng_normal(3 * 5 * 8, s);
  Tensor y = Tensor::from_vec(yv, {3, 5, 8}), G = Tensor::from_vec(gv, {3, 5, 8});
  RoPE r8(8, 10);
  Tensor o8 = r8.forward(y, 3);
  (o8 * G).sum().backward();
  const int64_t oy = onew(yv, {3, 5, 8}), oG = onew(gv, {3, 5, 8});
  const int64_t oo = orc_rope(oy, 10, 10000.0, 3);
  orc_backward(orc_sum(orc_mul(oo, oG)));
  close(o8.data(), odata(oo, o8.numel()), "rope vs oracle: out");
  close_grad(y, oy, "rope vs oracle: dx");
  bool threw = false;
  try {
    r8.forward(y, 6);  // positions 6..10: the table holds 0..9
  } catch (const Panic&) {
    threw = true;
  }
  check(threw, "rope: a position past the table panics");
  orc_free_all();
}

// The attention helpers chained at a size where they run on the batched MFMA GEMM: scores, scale,
// softmax (plain and causal), probabilities . V and a concatenation, loss = sum(out * G)
static void test_attention_ops_chain() {
  for (int causal = 0; causal <= 1; ++causal) {
    uint64_t s = 31 + causal;
    const size_t b = 6, S = 20, D = 24, Dv = 16;
    const auto qv = rng_normal(b * S * D, s), kv = rng_normal(b * S * D, s), vv = rng_normal(b * S * Dv, s);
    const auto ev = rng_normal(b * S * 8, s), gv = rng_normal(b * S * (Dv + 8), s);
    Tensor q = Tensor::from_vec(qv, {b, S, D}), k = Tensor::from_vec(kv, {b, S, D});
    Tensor v = Tensor::from_vec(vv, {b, S, Dv}), e = Tensor::from_vec(ev, {b, S, 8});
    Tensor G = Tensor::from_vec(gv, {b, S, Dv + 8});
    using namespace talos::tape;
    Tensor p = softmax(scale_tensor(batched_matmul_qt_k(q, k, b, S, D), 0.2), S, causal != 0);
    Tensor o = concat_last_dim(batched_matmul_probs_v(p, v, b, S, Dv), e);
    Tensor loss = (o * G).sum();
    loss.backward();
    const int64_t oq = onew(qv, {6, 20, 24}), ok_ = onew(kv, {6, 20, 24}), ov = onew(vv, {6, 20, 16});
    const int64_t oe = onew(ev, {6, 20, 8}), oG = onew(gv, {6, 20, 24});
    const int64_t op = orc_softmax(orc_scale(orc_bmm_qt_k(oq, ok_), 0.2), 20, causal);
    const int64_t oo = orc_concat_last(orc_bmm_p_v(op, ov), oe);
    const int64_t ol = orc_sum(orc_mul(oo, oG));
    orc_backward(ol);
    const std::string tag = causal ? "attention ops (causal): " : "attention ops: ";
    close(p.data(), odata(op, p.numel()), tag + "probs");
    close(o.data(), odata(oo, o.numel()), tag + "out");
    close_grad(q, oq, tag + "dq");
    close_grad(k, ok_, tag + "dk");
    close_grad(v, ov, tag + "dv");
    close_grad(e, oe, tag + "de");
    orc_free_all();
  }
}

// src/transformer.rs:1302-1327 (LuckTransformer integration), and the whole backbone against the
// oracle: embed, RMSNorm, MLA, residual, RMSNorm, ReLU FFN, residual, RMSNorm, out_proj
static void test_luck_transformer_integration() {
  LuckTransformer t(8, 8, true, 42);
  Tensor x = Tensor::rand({1, 5, 8}, -0.1, 0.1, 123);
  Tensor out = t.forward(x);
  Tensor loss = out.mean();
  loss.backward();
  const auto params = t.parameters();
  check(params.size() > 10, "luck_transformer: many parameters");
  check(any_nonzero(t.embed.weight.grad()), "luck_transformer: embed grad present");
  check(any_nonzero(t.norm_1.weight.grad()), "luck_transformer: norm grad present");
  // the oracle graph on the same parameter values
  const OLin emb = olin(t.embed), f1 = olin(t.ffn_1), f2 = olin(t.ffn_2), op = olin(t.out_proj);
  const OMla w = omla(t.mla_layer);
  const int64_t g1 = onew_t(t.norm_1.weight), g2 = onew_t(t.norm_2.weight), gf = onew_t(t.norm_final.weight);
  const int64_t ox = onew_t(x);
  const int64_t h = ofwd(emb, ox, {1, 5, 8});
  const int64_t h2 = orc_add(h, omla_forward(w, t.mla_layer.config, orc_rmsnorm(h, g1, 1e-5), 1, 5));
  const int64_t a = orc_relu(ofwd(f1, orc_rmsnorm(h2, g2, 1e-5), {1, 5, 8}));
  const int64_t h3 = orc_add(h2, ofwd(f2, a, {1, 5, 16}));
  const int64_t oout = ofwd(op, orc_rmsnorm(h3, gf, 1e-5), {1, 5, 8});
  const int64_t ol = orc_mean(oout);
  orc_backward(ol);
  close(out.data(), odata(oout, out.numel()), "luck_transformer vs oracle: out");
  close_grad(x, ox, "luck_transformer vs oracle: dx");
  close_grad(t.embed.weight, emb.w, "luck_transformer vs oracle: d embed.W");
  close_grad(t.embed.bias, emb.b, "luck_transformer vs oracle: d embed.b");
  close_grad(t.norm_1.weight, g1, "luck_transformer vs oracle: d norm_1");
  close_mla_grads(t.mla_layer, w, "luck_transformer vs oracle:");
  close_grad(t.norm_2.weight, g2, "luck_transformer vs oracle: d norm_2");
  close_grad(t.ffn_1.weight, f1.w, "luck_transformer vs oracle: d ffn_1.W");
  close_grad(t.ffn_2.weight, f2.w, "luck_transformer vs oracle: d ffn_2.W");
  close_grad(t.norm_final.weight, gf, "luck_transformer vs oracle: d norm_final");
  close_grad(t.out_proj.weight, op.w, "luck_transformer vs oracle: d out_proj.W");
  close_grad(t.out_proj.bias, op.b, "luck_transformer vs oracle: d out_proj.b");
  // last_token cuts the graph, as the reference's Tensor::new does
  Tensor last = t.last_token(out);
  check(last.shape == Shape({1, 8}) && last._ctx == nullptr, "luck_transformer: last_token has no graph");
  const auto od = out.data(), ld = last.data();
  check(std::equal(ld.begin(), ld.end(), od.begin() + 4 * 8), "luck_transformer: last_token is row S - 1");
  orc_free_all();
}

// DuelingQNetwork (src/dqn.rs:31-107, 134-154) written against the tape exactly as the reference
// writes it against its Tensor: the consumer code is unchanged
struct DuelingQNetwork {
  Linear l1, l2, val_head, adv_head;
  explicit DuelingQNetwork(uint64_t seed)
      : l1(8, 64, true, seed), l2(64, 64, true, seed + 1), val_head(64, 1, true, seed + 2), adv_head(64, 5, true, seed + 3) {}
  Tensor forward(const Tensor& state) const {
    Tensor x = l1.forward(state).relu();
    x = l2.forward(x).relu();
    Tensor val = val_head.forward(x), adv = adv_head.forward(x);
    if (state.shape.size() == 2 && state.shape[0] > 1) {
      Tensor ones_1_5 = Tensor::from_vec(std::vector<double>(5, 1.0), {1, 5});
      Tensor val_expanded = val.matmul(ones_1_5);
      Tensor ones_5_1 = Tensor::from_vec(std::vector<double>(5, 0.2), {5, 1});
      Tensor mean_adv_expanded = adv.matmul(ones_5_1).matmul(ones_1_5);
      return val_expanded + adv - mean_adv_expanded;
    }
    Tensor mean_adv = adv.mean().broadcast({5});
    Tensor val_expanded = val.broadcast({5});
    Tensor neg_mean_adv = Tensor::zeros({5}) - mean_adv;
    return val_expanded + adv + neg_mean_adv;
  }
  std::vector<Tensor> parameters() const {
    std::vector<Tensor> p;
    for (const Linear* l : {&l1, &l2, &val_head, &adv_head})
      for (const Tensor& t : l->parameters()) p.push_back(t);
    return p;
  }
  void load_state_dict(const DuelingQNetwork& o) {
    const auto a = parameters(), b = o.parameters();
    for (size_t i = 0; i < a.size(); ++i) a[i].set_data(b[i].data());
  }
  void soft_update(const DuelingQNetwork& src, double tau) {
    const auto a = parameters(), b = src.parameters();
    for (size_t i = 0; i < a.size(); ++i) {
      auto t = a[i].data();
      const auto sv = b[i].data();
      for (size_t j = 0; j < t.size(); ++j) t[j] = t[j] * (1.0 - tau) + sv[j] * tau;
      a[i].set_data(t);
    }
  }
};

// The oracle's DuelingQNetwork forward on given parameter handles (the same wiring)
static int64_t oq_forward(const std::vector<OLin>& w, int64_t state, const std::vector<int64_t>& ss) {
  const int64_t B = ss.size() == 2 ? ss[0] : 1;
  const std::vector<int64_t> hs = ss.size() == 2 ? std::vector<int64_t>{B, 64} : std::vector<int64_t>{64};
  int64_t x = orc_relu(ofwd(w[0], state, ss));
  x = orc_relu(ofwd(w[1], x, hs));
  const int64_t val = ofwd(w[2], x, hs), adv = ofwd(w[3], x, hs);
  if (ss.size() == 2 && ss[0] > 1) {
    const int64_t o15 = onew(std::vector<double>(5, 1.0), {1, 5}), o51 = onew(std::vector<double>(5, 0.2), {5, 1});
    return orc_sub(orc_add(orc_matmul(val, o15), adv), orc_matmul(orc_matmul(adv, o51), o15));
  }
  const std::vector<int64_t> s5{5};
  const int64_t mean_adv = orc_broadcast(orc_mean(adv), s5.data(), 1);
  const int64_t val_e = orc_broadcast(val, s5.data(), 1);
  return orc_add(orc_add(val_e, adv), orc_sub(onew(std::vector<double>(5, 0.0), {5}), mean_adv));
}

// train_dqn's batched update (src/dqn.rs:515-576) on the tape, two steps, against the oracle:
// Q(s, a) through the action mask and ones(5, 1), double-DQN targets from the policy's argmax and
// the target network's value, MSE, backward, Adam with the global-norm clip, soft update 0.005
static void test_dqn_train_step() {
  const size_t B = 64;
  DuelingQNetwork policy(101), target(202);
  target.load_state_dict(policy);
  talos::tape::Adam opt(policy.parameters(), 1e-3, 1.0);
  uint64_t s = 55;
  for (int step = 1; step <= 2; ++step) {
    const auto sv = rng_normal(B * 8, s), nv = rng_normal(B * 8, s), rv = rng_normal(B, s);
    std::vector<double> mask(B * 5, 0.0), done(B, 0.0);
    for (size_t i = 0; i < B; ++i) {
      mask[i * 5 + (i * 7 + step) % 5] = 1.0;
      done[i] = (i % 9 == 0) ? 1.0 : 0.0;
    }
    const std::vector<double> p0 = [&] {
      std::vector<double> v;
      for (const Tensor& t : policy.parameters()) {
        const auto d = t.data();
        v.insert(v.end(), d.begin(), d.end());
      }
      return v;
    }();
    opt.zero_grad();
    Tensor batch_state = Tensor::from_vec(sv, {B, 8}), batch_next = Tensor::from_vec(nv, {B, 8});
    Tensor batch_mask = Tensor::from_vec(mask, {B, 5});
    Tensor q_values = policy.forward(batch_state);
    Tensor ones_5_1 = Tensor::from_vec(std::vector<double>(5, 1.0), {5, 1});
    Tensor q_actions = (q_values * batch_mask).matmul(ones_5_1);
    const auto q_eval = policy.forward(batch_next).data(), q_tgt = target.forward(batch_next).data();
    std::vector<double> tv(B);
    for (size_t i = 0; i < B; ++i) {
      size_t am = 0;
      for (size_t k = 1; k < 5; ++k)
        if (q_eval[i * 5 + k] > q_eval[i * 5 + am]) am = k;
      tv[i] = rv[i] + 0.99 * q_tgt[i * 5 + am] * (1.0 - done[i]);
    }
    Tensor loss = q_actions.mse_loss(Tensor::from_vec(tv, {B, 1}));
    loss.backward();
    // the oracle: same parameters, inputs and targets
    std::vector<OLin> w;
    for (const Linear* l : {&policy.l1, &policy.l2, &policy.val_head, &policy.adv_head}) w.push_back(olin(*l));
    const int64_t os = onew(sv, {64, 8}), om = onew(mask, {64, 5});
    const int64_t oqa = orc_matmul(orc_mul(oq_forward(w, os, {64, 8}), om), onew(std::vector<double>(5, 1.0), {5, 1}));
    const int64_t ol = orc_mse_loss(oqa, onew(tv, {64, 1}));
    orc_backward(ol);
    const std::string tag = "dqn step " + std::to_string(step) + ": ";
    close({loss.item()}, odata(ol, 1), tag + "loss");
    std::vector<double> g_ref;
    for (const OLin& o : w) {
      const auto gw = ograd(o.w, o.L->weight.numel()), gb = ograd(o.b, o.L->bias.numel());
      g_ref.insert(g_ref.end(), gw.begin(), gw.end());
      g_ref.insert(g_ref.end(), gb.begin(), gb.end());
    }
    std::vector<double> g_got;
    for (const Tensor& t : policy.parameters()) {
      const auto g = t.grad();
      g_got.insert(g_got.end(), g.begin(), g.end());
    }
    close(g_got, g_ref, tag + "parameter gradients");
    opt.step();
    // the oracle's clipped Adam from the same state, fed the oracle's gradients
    static std::vector<double> pr, m, v;
    if (step == 1) {
      pr = p0;
      m.assign(p0.size(), 0.0);
      v.assign(p0.size(), 0.0);
    }
    orc_adam_step((int64_t)pr.size(), pr.data(), g_ref.data(), m.data(), v.data(), step, 1e-3, 0.9, 0.999, 1e-8, 1.0);
    std::vector<double> p1, dgot(pr.size()), dref(pr.size());
    for (const Tensor& t : policy.parameters()) {
      const auto d = t.data();
      p1.insert(p1.end(), d.begin(), d.end());
    }
    for (size_t i = 0; i < pr.size(); ++i) {
      dgot[i] = p1[i] - p0[i];
      dref[i] = pr[i] - p0[i];
    }
    close(dgot, dref, tag + "Adam (clipped) parameter delta");
    pr = p1;  // continue from the device's parameters
    // soft update: target <- 0.995 target + 0.005 policy
    std::vector<double> t0;
    for (const Tensor& t : target.parameters()) {
      const auto d = t.data();
      t0.insert(t0.end(), d.begin(), d.end());
    }
    target.soft_update(policy, 0.005);
    std::vector<double> t1, t1r(t0.size());
    for (const Tensor& t : target.parameters()) {
      const auto d = t.data();
      t1.insert(t1.end(), d.begin(), d.end());
    }
    for (size_t i = 0; i < t0.size(); ++i) t1r[i] = t0[i] * 0.995 + p1[i] * 0.005;
    close(t1, t1r, tag + "soft update", 1e-6, 1e-7);
    orc_free_all();
  }
  check(opt.t() == 2, "dqn: two optimizer steps");
  // the single-state forward (src/dqn.rs:97-106) against the oracle
  uint64_t s2 = 3;
  const auto one = rng_normal(8, s2);
  Tensor q1 = policy.forward(Tensor::from_vec(one, {8}));
  check(q1.shape == Shape({5}), "dqn: single-state Q has shape [5]");
  std::vector<OLin> w;
  for (const Linear* l : {&policy.l1, &policy.l2, &policy.val_head, &policy.adv_head}) w.push_back(olin(*l));
  const int64_t oq1 = oq_forward(w, onew(one, {8}), {8});
  close(q1.data(), odata(oq1, 5), "dqn: single-state Q vs oracle");
  orc_free_all();
}

// Shape errors panic as the reference's assert! does (src/autograd.rs:209, 1611)
static void test_shape_errors_panic() {
  bool threw = false;
  try {
    Tensor::from_vec({1, 2, 3}, {2, 2});
  } catch (const Panic&) {
    threw = true;
  }
  check(threw, "panic: data length must match shape");
  threw = false;
  try {
    Tensor::zeros({2, 3}).matmul(Tensor::zeros({2, 3}));
  } catch (const Panic&) {
    threw = true;
  }
  check(threw, "panic: matmul dimension mismatch");
  threw = false;
  try {
    (void)(Tensor::zeros({2}) + Tensor::zeros({3}));
  } catch (const Panic&) {
    threw = true;
  }
  check(threw, "panic: add shape mismatch");
}

int main() {
  std::setvbuf(stdout, nullptr, _IONBF, 0);
  struct {
    const char* name;
    void (*fn)();
  } tests[] = {{"autograd_memory_leak_fix", test_autograd_memory_leak_fix},
               {"grad_check_matmul", test_grad_check_matmul},
               {"grad_check_broadcast", test_grad_check_broadcast},
               {"numerical_gradient_check", test_numerical_gradient_check},
               {"broadcast_scalar", test_broadcast_scalar},
               {"tensor_reshape", test_tensor_reshape},
               {"tensor_transpose", test_tensor_transpose},
               {"rmsnorm_backward", test_rmsnorm_backward},
               {"linear_mse_c1", test_linear_mse_c1},
               {"composite_graph", test_composite_graph},
               {"adam_ppo", test_adam_ppo},
               {"adam_dqn_clip", test_adam_dqn_clip},
               {"mla_forward_backward", test_mla_forward_backward},
               {"mla_deepseek_lite", test_mla_deepseek_lite},
               {"rope_backward", test_rope_backward},
               {"attention_ops_chain", test_attention_ops_chain},
               {"luck_transformer_integration", test_luck_transformer_integration},
               {"dqn_train_step", test_dqn_train_step},
               {"shape_errors_panic", test_shape_errors_panic}};
  for (auto& t : tests) {
    std::printf("test %s\n", t.name);
    try {
      t.fn();
    } catch (const std::exception& e) {
      check(false, std::string(t.name) + ": exception " + e.what());
    }
  }
  std::printf("%d passed, %d failed\n", g_pass, g_fail);
  return g_fail ? 1 : 0;
}
