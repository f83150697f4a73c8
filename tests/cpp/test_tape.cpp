// test_tape.cpp -- the reference's own autograd tests, run through the device tape (tape.hpp) on the
// GPU, plus graphs compared element-wise with the f64 oracle (oracle/liboracle.so, the checker).
//
// Mirrors src/grad_check.rs:6-114 (graph detach / clear, matmul KAT, broadcast KAT, finite
// difference of x^2 sin x), src/transformer.rs:1191-1225 and 1283-1299 (reshape copies, transpose
// KAT, RMSNorm backward) and src/autograd.rs:1868-1875 (scalar broadcast). Exit status 0 when
// every check passes; each failing check prints its name and values.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../talos-xii_amd/host/tape.hpp"

using talos::tape::Linear;
using talos::tape::Panic;
using talos::tape::RMSNorm;
using talos::tape::Tensor;

extern "C" {
// oracle C ABI (oracle/talos_oracle.cpp)
const char* orc_last_error(void);
int64_t orc_tensor_new_len(const double* data, int64_t len, const int64_t* shape, int rank);
void orc_tensor_data(int64_t h, double* out);
void orc_tensor_grad(int64_t h, double* out);
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

// |got - ref| <= rtol |ref| + atol element-wise (the fp32 rule of the parity tests)
static void close(const std::vector<double>& got, const std::vector<double>& ref, const std::string& name,
                  double rtol = 1e-4, double atol = 1e-5) {
  if (got.size() != ref.size()) {
    check(false, name + " (size)");
    return;
  }
  double worst = 0.0;
  size_t wi = 0;
  bool okay = true;
  for (size_t i = 0; i < got.size(); ++i) {
    const double err = std::fabs(got[i] - ref[i]), bound = rtol * std::fabs(ref[i]) + atol;
    if (err > bound) okay = false;
    if (err - bound > worst) {
      worst = err - bound;
      wi = i;
    }
  }
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
