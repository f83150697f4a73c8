// tape.cpp -- the host-side autograd tape (tape.hpp) over the C ABI of libtalos_hip.so.
//
// Every op enqueues its forward kernel on the default stream and records a closure that enqueues
// the backward kernels, which accumulate into the parents' device grads exactly where the
// reference's closures do (citations per op). Host reads (data(), grad(), item()) wait for the
// stream, so results are observed in program order as with the reference's synchronous ops.
#include "tape.hpp"

#include <algorithm>
#include <cmath>
#include <sstream>
#include <unordered_set>

#include "../../include/talos_hip.h"

namespace talos {
namespace tape {

namespace {

void ok(int rc, const char* what) {
  if (rc != TALOS_OK) throw Panic(std::string(what) + ": " + talos_last_error());
}

size_t prod(const Shape& s) {
  size_t n = 1;
  for (size_t v : s) n *= v;
  return n;
}

std::string shape_str(const Shape& s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  o << "]";
  return o.str();
}

void require(bool c, const std::string& msg) {
  if (!c) throw Panic(msg);
}

// The scratch of the library calls made by this thread's ops (split-K partials, reduction
// partials, attention rows): one device buffer bound on the thread's first op and held until the
// thread exits, so an op never allocates scratch per call (a split-K product splits fewer times
// rather than outgrow it). Every op runs on the null stream, so calls sharing it never overlap.
// A workspace the caller bound on this thread before its first op stays bound instead.
constexpr size_t kTapeWorkspaceBytes = size_t(16) << 20;
struct TapeWorkspace {
  void* ptr = nullptr;
  bool checked = false;
  ~TapeWorkspace() {  // thread exit: unbind and free (a pool thread that ends leaks nothing)
    if (ptr) {
      talos_workspace_bind(nullptr, 0);
      talos_free(ptr);
    }
  }
};
void bind_workspace_once() {
  thread_local TapeWorkspace ws;
  if (ws.checked) return;
  ws.checked = true;
  if (talos_workspace_bytes() > 0) return;
  void* p = nullptr;
  ok(talos_malloc(&p, kTapeWorkspaceBytes), "talos_malloc (tape workspace)");
  ws.ptr = p;
  ok(talos_workspace_bind(p, kTapeWorkspaceBytes), "talos_workspace_bind");
}

// A new tensor with zeroed grad; data left for the op to fill.
Tensor fresh(Shape shape) {
  bind_workspace_once();
  Tensor t;
  const size_t n = prod(shape);
  t.data_ = std::make_shared<Storage>(n);
  t.grad_ = std::make_shared<Storage>(n);
  ok(talos_fill_zero(t.grad_->ptr, n * sizeof(float), nullptr), "fill_zero");
  t.shape = std::move(shape);
  return t;
}

Tensor with_ctx(Tensor out, std::vector<Tensor> parents,
                std::function<void(const Tensor&, std::vector<Tensor>&)> fn) {
  auto ctx = std::make_shared<Context>();
  ctx->parents = std::move(parents);
  ctx->backward_op = std::move(fn);
  out._ctx = std::move(ctx);
  return out;
}

Tensor unary(const Tensor& x, int op, float p0 = 0.f, float p1 = 0.f) {
  Tensor out = fresh(x.shape);
  ok(talos_unary_fwd_f32(op, x.numel(), p0, p1, x.data_->ptr, out.data_->ptr, nullptr), "unary_fwd");
  return with_ctx(out, {x}, [op, p0, p1](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_unary_bwd_f32(op, o.numel(), p0, p1, p[0].data_->ptr, o.grad_->ptr, p[0].grad_->ptr, nullptr),
       "unary_bwd");
  });
}

Tensor binary(const Tensor& a, const Tensor& b, int op, const char* name) {
  require(a.shape == b.shape, std::string(name) + " shape mismatch: " + shape_str(a.shape) + " vs " + shape_str(b.shape));
  Tensor out = fresh(a.shape);
  ok(talos_binary_fwd_f32(op, a.numel(), a.data_->ptr, b.data_->ptr, out.data_->ptr, nullptr), name);
  return with_ctx(out, {a, b}, [op, name](const Tensor& o, std::vector<Tensor>& p) {
    // the same tensor on both sides (x * x) shares one grad buffer: the kernel adds both terms once
    ok(talos_binary_bwd_f32(op, o.numel(), p[0].data_->ptr, p[1].data_->ptr, o.grad_->ptr, p[0].grad_->ptr,
                            p[1].grad_->ptr, nullptr),
       name);
  });
}

}  // namespace

Storage::Storage(size_t count) : n(count) {
  void* p = nullptr;
  ok(talos_malloc(&p, (count ? count : 1) * sizeof(float)), "talos_malloc");
  ptr = static_cast<float*>(p);
}

Storage::~Storage() { talos_free(ptr); }

// ---------------------------------------------------------------------------
// Construction and host access (src/autograd.rs:94-143)
// ---------------------------------------------------------------------------
Tensor Tensor::from_vec(const std::vector<double>& data, Shape shape) {
  require(data.size() == prod(shape), "Data length must match shape");  // src/autograd.rs:96-100
  Tensor t = fresh(std::move(shape));
  if (!data.empty()) ok(talos_memcpy_h2d_f64(t.data_->ptr, data.data(), data.size(), nullptr), "memcpy_h2d_f64");
  return t;
}

Tensor Tensor::zeros(Shape shape) {
  Tensor t = fresh(std::move(shape));
  ok(talos_fill_zero(t.data_->ptr, t.numel() * sizeof(float), nullptr), "fill_zero");
  return t;
}

Tensor Tensor::rand(Shape shape, double min, double max, uint64_t seed) {
  const size_t n = prod(shape);
  std::vector<double> v(n);
  uint64_t x = seed;
  for (size_t i = 0; i < n; ++i) {
    x = x * 6364136223846793005ULL + 1ULL;
    const double r = (double)(x >> 33) / (double)UINT32_MAX;
    v[i] = min + r * (max - min);
  }
  return from_vec(v, std::move(shape));
}

std::vector<double> Tensor::data() const {
  std::vector<double> out(numel());
  if (!out.empty()) ok(talos_memcpy_d2h_f64(out.data(), data_->ptr, out.size(), nullptr), "memcpy_d2h_f64");
  return out;
}

std::vector<double> Tensor::grad() const {
  std::vector<double> out(numel());
  if (!out.empty()) ok(talos_memcpy_d2h_f64(out.data(), grad_->ptr, out.size(), nullptr), "memcpy_d2h_f64");
  return out;
}

void Tensor::set_data(const std::vector<double>& v) const {
  require(v.size() == numel(), "set_data length must match the tensor");
  if (!v.empty()) ok(talos_memcpy_h2d_f64(data_->ptr, v.data(), v.size(), nullptr), "memcpy_h2d_f64");
}

double Tensor::item() const {
  require(numel() == 1, "item() needs a single-element tensor");  // src/autograd.rs:140-143
  return data()[0];
}

Tensor Tensor::detach() const {
  Tensor t;
  t.data_ = data_;
  t.grad_ = grad_;
  t.shape = shape;
  return t;
}

void Tensor::zero_grad() const {
  ok(talos_fill_zero(grad_->ptr, numel() * sizeof(float), nullptr), "fill_zero");
}

// DFS topological order keyed by the grad storage, all-ones seed, closures in reverse order
// (src/autograd.rs:145-184).
void Tensor::backward() const {
  std::unordered_set<const Storage*> visited;
  std::vector<Tensor> topo;
  std::function<void(const Tensor&)> build = [&](const Tensor& t) {
    if (!visited.insert(t.grad_.get()).second) return;
    if (t._ctx)
      for (const Tensor& p : t._ctx->parents) build(p);
    topo.push_back(t);
  };
  build(*this);
  std::vector<double> ones(numel(), 1.0);
  ok(talos_memcpy_h2d_f64(grad_->ptr, ones.data(), ones.size(), nullptr), "memcpy_h2d_f64");
  for (auto it = topo.rbegin(); it != topo.rend(); ++it)
    if (it->_ctx) it->_ctx->backward_op(*it, it->_ctx->parents);
}

// ---------------------------------------------------------------------------
// Ops
// ---------------------------------------------------------------------------
// matmul (src/autograd.rs:200-354): [m,k] . [k,n]; a rank-1 left operand is a single row.
// Backward dA += dC . B^T and dB += A^T . dC (beta = 1: grads accumulate).
Tensor Tensor::matmul(const Tensor& other) const {
  require(shape.size() <= 2 && other.shape.size() == 2, "matmul expects a rank <= 2 lhs and a rank-2 rhs");
  const int m = shape.size() == 1 ? 1 : (int)shape[0];
  const int k = shape.size() == 1 ? (int)shape[0] : (int)shape[1];
  const int k2 = (int)other.shape[0], n = (int)other.shape[1];
  require(k == k2, "MatMul dimension mismatch");  // src/autograd.rs:209
  // a rank-1 left operand gives a rank-1 result [n] (src/autograd.rs:254-258)
  Tensor out = fresh(shape.size() == 1 ? Shape{(size_t)n} : Shape{(size_t)m, (size_t)n});
  ok(talos_gemm_f32(0, 0, m, n, k, 1.f, data_->ptr, k, other.data_->ptr, n, 0.f, out.data_->ptr, n, nullptr),
     "matmul");
  return with_ctx(out, {*this, other}, [m, n, k](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_gemm_f32(0, 1, m, k, n, 1.f, o.grad_->ptr, n, p[1].data_->ptr, n, 1.f, p[0].grad_->ptr, k, nullptr),
       "matmul dA");
    ok(talos_gemm_f32(1, 0, k, n, m, 1.f, p[0].data_->ptr, k, o.grad_->ptr, n, 1.f, p[1].grad_->ptr, n, nullptr),
       "matmul dB");
  });
}

Tensor Tensor::relu() const { return unary(*this, TALOS_RELU); }      // src/autograd.rs:356-386
Tensor Tensor::log() const { return unary(*this, TALOS_LOG); }        // :388-413
Tensor Tensor::exp() const { return unary(*this, TALOS_EXP); }        // :415-441
Tensor Tensor::sin() const { return unary(*this, TALOS_SIN); }        // :549-574
Tensor Tensor::cos() const { return unary(*this, TALOS_COS); }        // :576-601
Tensor Tensor::sqrt() const { return unary(*this, TALOS_SQRT); }      // :603-630
Tensor Tensor::gelu() const { return unary(*this, TALOS_GELU); }
Tensor Tensor::scale(double s) const { return unary(*this, TALOS_SCALE, (float)s); }
Tensor Tensor::clip(double min, double max) const {                   // :741-768
  return unary(*this, TALOS_CLIP, (float)min, (float)max);
}

// sum / mean (src/autograd.rs:443-482): f64-combined reduction; backward adds g (or g / n).
static Tensor reduce(const Tensor& x, double scale) {
  Tensor out = fresh({1});
  ok(talos_reduce_sum_f32(x.numel(), (float)scale, x.data_->ptr, out.data_->ptr, nullptr), "reduce_sum");
  return with_ctx(out, {x}, [scale](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_fill_add_f32(p[0].numel(), (float)scale, o.grad_->ptr, p[0].grad_->ptr, nullptr), "fill_add");
  });
}
Tensor Tensor::sum() const { return reduce(*this, 1.0); }
Tensor Tensor::mean() const { return reduce(*this, 1.0 / (double)numel()); }

// broadcast of a [1] tensor to new_shape (src/autograd.rs:484-509); backward sums the grad.
Tensor Tensor::broadcast(Shape new_shape) const {
  require(shape == Shape{1}, "Broadcast only supported for scalar (1) to N");
  Tensor out = fresh(std::move(new_shape));
  ok(talos_fill_zero(out.data_->ptr, out.numel() * sizeof(float), nullptr), "fill_zero");
  ok(talos_fill_add_f32(out.numel(), 1.f, data_->ptr, out.data_->ptr, nullptr), "broadcast");
  auto tmp = std::make_shared<Storage>(1);
  return with_ctx(out, {*this}, [tmp](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_reduce_sum_f32(o.numel(), 1.f, o.grad_->ptr, tmp->ptr, nullptr), "broadcast bwd");
    ok(talos_binary_fwd_f32(TALOS_ADD, 1, p[0].grad_->ptr, tmp->ptr, p[0].grad_->ptr, nullptr), "broadcast bwd");
  });
}

// broadcast_to_batch (src/autograd.rs:511-547): [..] -> [batch, ..]; backward sums over the batch.
Tensor Tensor::broadcast_to_batch(size_t batch_size) const {
  Shape ns{batch_size};
  ns.insert(ns.end(), shape.begin(), shape.end());
  Tensor out = fresh(ns);
  const int len = (int)numel();
  ok(talos_broadcast_rows_f32(batch_size, len, data_->ptr, out.data_->ptr, nullptr), "broadcast_to_batch");
  return with_ctx(out, {*this}, [batch_size, len](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_bias_grad_f32((int)batch_size, len, o.grad_->ptr, 1.f, p[0].grad_->ptr, nullptr), "broadcast_to_batch bwd");
  });
}

// transpose of two dims (src/autograd.rs:632-739); backward is the inverse permutation, added.
Tensor Tensor::transpose(size_t dim0, size_t dim1) const {
  require(dim0 < shape.size() && dim1 < shape.size(), "transpose dims out of range");
  Shape ns = shape;
  std::swap(ns[dim0], ns[dim1]);
  Tensor out = fresh(ns);
  std::vector<long long> in_shape(shape.begin(), shape.end());
  ok(talos_transpose_f32((int)shape.size(), in_shape.data(), (int)dim0, (int)dim1, data_->ptr, out.data_->ptr, 0,
                         nullptr),
     "transpose");
  return with_ctx(out, {*this}, [dim0, dim1](const Tensor& o, std::vector<Tensor>& p) {
    std::vector<long long> os(o.shape.begin(), o.shape.end());
    ok(talos_transpose_f32((int)os.size(), os.data(), (int)dim0, (int)dim1, o.grad_->ptr, p[0].grad_->ptr, 1,
                           nullptr),
       "transpose bwd");
  });
}

// reshape copies the data (src/autograd.rs:770-792); backward adds the grad as is.
Tensor Tensor::reshape(Shape new_shape) const {
  require(prod(new_shape) == numel(), "Reshape dimension mismatch");
  Tensor out = fresh(std::move(new_shape));
  ok(talos_memcpy_d2d(out.data_->ptr, data_->ptr, numel() * sizeof(float), nullptr), "reshape");
  return with_ctx(out, {*this}, [](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_binary_fwd_f32(TALOS_ADD, o.numel(), p[0].grad_->ptr, o.grad_->ptr, p[0].grad_->ptr, nullptr),
       "reshape bwd");
  });
}

// mse_loss = mean((self - target)^2) built from the ops, as src/autograd.rs:1599-1603 does.
Tensor Tensor::mse_loss(const Tensor& target) const {
  Tensor diff = *this - target;
  Tensor sq = diff * diff;
  return sq.mean();
}

Tensor operator+(const Tensor& a, const Tensor& b) { return binary(a, b, TALOS_ADD, "Add"); }   // :1606-1647
Tensor operator-(const Tensor& a, const Tensor& b) { return binary(a, b, TALOS_SUB, "Sub"); }   // :1656-1695
Tensor operator*(const Tensor& a, const Tensor& b) { return binary(a, b, TALOS_MUL, "Mul"); }   // :1704-1760
Tensor operator/(const Tensor& a, const Tensor& b) { return binary(a, b, TALOS_DIV, "Div"); }   // :1767-1825
Tensor operator-(const Tensor& a) { return unary(a, TALOS_NEG); }                               // :1832-1862

// ---------------------------------------------------------------------------
// Modules
// ---------------------------------------------------------------------------
Linear::Linear(size_t in, size_t out, bool bias, uint64_t seed)
    : has_bias(bias), in_features(in), out_features(out) {
  const double limit = std::sqrt(6.0 / (double)(in + out));
  weight = Tensor::rand({in, out}, -limit, limit, seed);
  if (bias) this->bias = Tensor::zeros({out});
}

Linear::Linear(Tensor w, Tensor b, bool hb)
    : weight(std::move(w)), bias(std::move(b)), has_bias(hb) {
  require(weight.shape.size() == 2, "Linear weight must be [in, out]");
  in_features = weight.shape[0];
  out_features = weight.shape[1];
}

// src/nn.rs:72-133: flatten N-D input to 2-D, x . W, reshape back, add the broadcast bias.
Tensor Linear::forward(const Tensor& input) const {
  const size_t rank = input.shape.size();
  Tensor xf = input;
  bool flat = false;
  if (rank > 2) {
    size_t bd = 1;
    for (size_t i = 0; i + 1 < rank; ++i) bd *= input.shape[i];
    xf = input.reshape({bd, in_features});
    flat = true;
  }
  Tensor out = xf.matmul(weight);
  if (flat) {
    Shape ns(input.shape.begin(), input.shape.end() - 1);
    ns.push_back(out_features);
    out = out.reshape(ns);
  }
  if (!has_bias) return out;
  if (out.shape.size() == 2 && out.shape[0] > 1) return out + bias.broadcast_to_batch(out.shape[0]);
  if (out.shape.size() > 2) {
    const size_t bd = out.numel() / out_features;
    Tensor of = out.reshape({bd, out_features});
    return (of + bias.broadcast_to_batch(bd)).reshape(out.shape);
  }
  if (out.shape.size() == 2) return out + bias.reshape({1, out_features});
  return out + bias;
}

std::vector<Tensor> Linear::parameters() const {
  std::vector<Tensor> p{weight};
  if (has_bias) p.push_back(bias);
  return p;
}

RMSNorm::RMSNorm(size_t dim, double e) : weight(Tensor::from_vec(std::vector<double>(dim, 1.0), {dim})), eps(e) {}

// src/nn.rs:183-300: forward caches the per-row 1/rms; the hand-written backward accumulates dx
// and dgain (reduced over all rows in f64).
Tensor RMSNorm::forward(const Tensor& x) const {
  const size_t dim = weight.numel();
  require(!x.shape.empty() && x.shape.back() == dim, "RMSNorm dim mismatch");
  const size_t rows = x.numel() / dim;
  Tensor out = fresh(x.shape);
  auto rstd = std::make_shared<Storage>(rows);
  ok(talos_rmsnorm_fwd_f32((int)rows, (int)dim, (float)eps, x.data_->ptr, weight.data_->ptr, out.data_->ptr,
                           rstd->ptr, nullptr),
     "rmsnorm_fwd");
  return with_ctx(out, {x, weight}, [rstd, rows, dim](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_rmsnorm_bwd_f32((int)rows, (int)dim, p[0].data_->ptr, p[1].data_->ptr, rstd->ptr, o.grad_->ptr, 1.f,
                             p[0].grad_->ptr, 1.f, p[1].grad_->ptr, nullptr),
       "rmsnorm_bwd");
  });
}

std::vector<Tensor> RMSNorm::parameters() const { return {weight}; }

// ---------------------------------------------------------------------------
// Attention ops (src/transformer.rs:877-1183)
// ---------------------------------------------------------------------------
// S[b] = Q[b] . K[b]^T on [b, seq, dim] buffers (batched_matmul_qt_k, :877-958): the batched GEMM
// with transB; backward dQ += G . K, dK += G^T . Q (beta 1: grads accumulate, :940-955).
Tensor batched_matmul_qt_k(const Tensor& q, const Tensor& k, size_t b, size_t seq, size_t dim) {
  require(q.numel() == b * seq * dim && k.numel() == b * seq * dim, "batched_matmul_qt_k: q / k size mismatch");
  Tensor out = fresh({b, seq, seq});
  const int S = (int)seq, D = (int)dim, B = (int)b;
  const long long sq = (long long)seq * dim, ss = (long long)seq * seq;
  ok(talos_gemm_batched_f32(0, 1, S, S, D, 1.f, q.data_->ptr, D, sq, k.data_->ptr, D, sq, 0.f, out.data_->ptr, S, ss, B,
                            nullptr),
     "batched_matmul_qt_k");
  return with_ctx(out, {q, k}, [S, D, B, sq, ss](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_gemm_batched_f32(0, 0, S, D, S, 1.f, o.grad_->ptr, S, ss, p[1].data_->ptr, D, sq, 1.f, p[0].grad_->ptr, D,
                              sq, B, nullptr),
       "batched_matmul_qt_k dQ");
    ok(talos_gemm_batched_f32(1, 0, S, D, S, 1.f, o.grad_->ptr, S, ss, p[0].data_->ptr, D, sq, 1.f, p[1].grad_->ptr, D,
                              sq, B, nullptr),
       "batched_matmul_qt_k dK");
  });
}

// O[b] = P[b] . V[b] (batched_matmul_probs_v, :961-1050); backward dP += G . V^T, dV += P^T . G.
Tensor batched_matmul_probs_v(const Tensor& probs, const Tensor& v, size_t b, size_t seq, size_t dim_v) {
  require(probs.numel() == b * seq * seq && v.numel() == b * seq * dim_v,
          "batched_matmul_probs_v: probs / v size mismatch");
  Tensor out = fresh({b, seq, dim_v});
  const int S = (int)seq, D = (int)dim_v, B = (int)b;
  const long long sv = (long long)seq * dim_v, ss = (long long)seq * seq;
  ok(talos_gemm_batched_f32(0, 0, S, D, S, 1.f, probs.data_->ptr, S, ss, v.data_->ptr, D, sv, 0.f, out.data_->ptr, D,
                            sv, B, nullptr),
     "batched_matmul_probs_v");
  return with_ctx(out, {probs, v}, [S, D, B, sv, ss](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_gemm_batched_f32(0, 1, S, S, D, 1.f, o.grad_->ptr, D, sv, p[1].data_->ptr, D, sv, 1.f, p[0].grad_->ptr, S,
                              ss, B, nullptr),
       "batched_matmul_probs_v dP");
    ok(talos_gemm_batched_f32(1, 0, S, D, S, 1.f, p[0].data_->ptr, S, ss, o.grad_->ptr, D, sv, 1.f, p[1].grad_->ptr, D,
                              sv, B, nullptr),
       "batched_matmul_probs_v dV");
  });
}

Tensor scale_tensor(const Tensor& t, double scale) { return t.scale(scale); }  // :1052-1072

// Row softmax (:1074-1121): the closure reads the forward's output (kept alive with the graph).
Tensor softmax(const Tensor& t, size_t seq_len, bool causal) {
  require(seq_len > 0 && t.numel() % seq_len == 0, "softmax: length is not a multiple of seq_len");
  Tensor out = fresh(t.shape);
  const int rows = (int)(t.numel() / seq_len), cols = (int)seq_len, c = causal ? 1 : 0;
  ok(talos_softmax_fwd_f32(rows, cols, c, t.data_->ptr, out.data_->ptr, nullptr), "softmax");
  std::shared_ptr<Storage> y = out.data_;
  return with_ctx(out, {t}, [rows, cols, c, y](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_softmax_bwd_f32(rows, cols, c, y->ptr, o.grad_->ptr, 1.f, p[0].grad_->ptr, nullptr), "softmax bwd");
  });
}

// concat_last_dim (:1123-1183); the backward adds each half of the gradient to its parent.
Tensor concat_last_dim(const Tensor& a, const Tensor& b) {
  require(!a.shape.empty() && a.shape.size() == b.shape.size() &&
              std::equal(a.shape.begin(), a.shape.end() - 1, b.shape.begin()),
          "concat_last_dim: leading dims differ");
  const size_t ca = a.shape.back(), cb = b.shape.back(), rows = ca ? a.numel() / ca : b.numel() / cb;
  Shape ns(a.shape.begin(), a.shape.end() - 1);
  ns.push_back(ca + cb);
  Tensor out = fresh(ns);
  ok(talos_concat_last_f32(rows, (int)ca, (int)cb, a.data_->ptr, b.data_->ptr, out.data_->ptr, nullptr), "concat");
  return with_ctx(out, {a, b}, [rows, ca, cb](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_concat_last_bwd_f32(rows, (int)ca, (int)cb, o.grad_->ptr, p[0].grad_->ptr, p[1].grad_->ptr, nullptr),
       "concat bwd");
  });
}

RoPE::RoPE(size_t d, size_t len) : dim(d), max_len(len) { require(d % 2 == 0, "RoPE dim must be even"); }

// RoPE::forward (:253-337): rows of shape[-1] = dim, the position of a row is start_pos + its index
// along shape[-2]; the backward rotates by -theta and adds.
Tensor RoPE::forward(const Tensor& x, size_t start_pos) const {
  require(x.shape.size() >= 2 && x.shape.back() == dim, "RoPE: the last dimension must equal the RoPE dim");
  const size_t T = x.shape[x.shape.size() - 2];
  require(start_pos + T <= max_len, "RoPE: position past the cached table (index out of bounds)");
  const int n_seq = (int)(T ? x.numel() / (T * dim) : 0), seq = (int)T, D = (int)dim, sp = (int)start_pos;
  const float b = (float)base;
  Tensor out = fresh(x.shape);
  ok(talos_rope_fwd_f32(n_seq, seq, 1, D, sp, b, x.data_->ptr, out.data_->ptr, nullptr), "rope");
  return with_ctx(out, {x}, [n_seq, seq, D, sp, b](const Tensor& o, std::vector<Tensor>& p) {
    ok(talos_rope_bwd_f32(n_seq, seq, 1, D, sp, b, o.grad_->ptr, 1.f, p[0].grad_->ptr, nullptr), "rope bwd");
  });
}

MLAConfig MLAConfig::deepseek_v2_lite() {  // src/transformer.rs:21-31
  MLAConfig c;
  c.dim = 512;
  c.num_heads = 8;
  c.q_lora_rank = 0;
  c.kv_lora_rank = 128;
  c.qk_rope_dim = 32;
  c.v_head_dim = 64;
  c.max_seq_len = 2048;
  return c;
}

// MultiHeadLatentAttention::new (:428-464): projections seeded seed .. seed + 6, no biases
MultiHeadLatentAttention::MultiHeadLatentAttention(const MLAConfig& c, uint64_t seed)
    : config(c),
      w_dkv(c.dim, c.kv_lora_rank, false, seed),
      w_uk(c.kv_lora_rank, c.num_heads * c.v_head_dim, false, seed + 1),
      w_uv(c.kv_lora_rank, c.num_heads * c.v_head_dim, false, seed + 2),
      w_q(c.dim, c.num_heads * c.v_head_dim, false, seed + 3),
      w_kr(c.dim, c.num_heads * c.qk_rope_dim, false, seed + 4),
      w_qr(c.dim, c.num_heads * c.qk_rope_dim, false, seed + 5),
      w_o(c.num_heads * c.v_head_dim, c.dim, false, seed + 6),
      rope(c.qk_rope_dim, c.max_seq_len) {}

std::vector<Tensor> MultiHeadLatentAttention::parameters() const {  // :466-476
  return {w_dkv.weight, w_uk.weight, w_uv.weight, w_q.weight, w_kr.weight, w_qr.weight, w_o.weight};
}

// MultiHeadLatentAttention::forward (:478-560), op for op.
Tensor MultiHeadLatentAttention::forward(const Tensor& x) const {
  require(x.shape.size() == 3, "MultiHeadLatentAttention expects [batch, seq, dim]");
  const size_t B = x.shape[0], S = x.shape[1], H = config.num_heads, hd = config.v_head_dim,
               R = config.qk_rope_dim;
  const Tensor c_kv = w_dkv.forward(x);
  const Tensor k_c = w_uk.forward(c_kv), v_c = w_uv.forward(c_kv);
  const Tensor k_r_flat = w_kr.forward(x);
  const Tensor q_c = w_q.forward(x), q_r_flat = w_qr.forward(x);
  // RoPE on [B, S, H, R]: rows are indexed along H, the reference's shape[-2]
  const Tensor k_r_rot = rope.forward(k_r_flat.reshape({B, S, H, R}), 0);
  const Tensor q_r_rot = rope.forward(q_r_flat.reshape({B, S, H, R}), 0);
  const Tensor q = concat_last_dim(q_c.reshape({B, S, H, hd}), q_r_rot);
  const Tensor k = concat_last_dim(k_c.reshape({B, S, H, hd}), k_r_rot);
  const Tensor v = v_c.reshape({B, S, H, hd});
  const size_t bh = B * H, total = hd + R;
  const Tensor q_flat = q.transpose(1, 2).reshape({bh, S, total});
  const Tensor k_flat = k.transpose(1, 2).reshape({bh, S, total});
  const Tensor v_flat = v.transpose(1, 2).reshape({bh, S, hd});
  const Tensor scores = batched_matmul_qt_k(q_flat, k_flat, bh, S, total);
  const Tensor probs = softmax(scale_tensor(scores, 1.0 / std::sqrt((double)total)), S);
  const Tensor att = batched_matmul_probs_v(probs, v_flat, bh, S, hd);
  const Tensor merged = att.reshape({B, H, S, hd}).transpose(1, 2).reshape({B, S, H * hd});
  return w_o.forward(merged);
}

// LuckTransformer::new (:48-69): the MLA's config is fixed by hidden_dim
static MLAConfig luck_mla_config(size_t hidden) {
  MLAConfig c;
  c.dim = hidden;
  c.num_heads = 4;
  c.q_lora_rank = 0;
  c.kv_lora_rank = 32;
  c.qk_rope_dim = 16;
  c.v_head_dim = hidden / 4;
  c.max_seq_len = 256;
  return c;
}

LuckTransformer::LuckTransformer(size_t in_dim, size_t hidden, bool, uint64_t seed)
    : embed(in_dim, hidden, true, seed),
      norm_1(hidden, 1e-5),
      mla_layer(luck_mla_config(hidden), seed + 10),
      norm_2(hidden, 1e-5),
      ffn_1(hidden, hidden * 2, true, seed + 20),
      ffn_2(hidden * 2, hidden, true, seed + 30),
      norm_final(hidden, 1e-5),
      out_proj(hidden, hidden, true, seed + 40) {}

Tensor LuckTransformer::forward(const Tensor& x) const {  // :71-90
  const Tensor h = embed.forward(x);
  const Tensor h2 = h + mla_layer.forward(norm_1.forward(h));
  const Tensor f2 = ffn_2.forward(ffn_1.forward(norm_2.forward(h2)).relu());
  const Tensor h3 = h2 + f2;
  return out_proj.forward(norm_final.forward(h3));
}

Tensor LuckTransformer::last_token(const Tensor& x, bool differentiable) const {  // :92-109
  require(x.shape.size() == 3 && x.shape[1] > 0, "last_token expects [batch, seq, dim]");
  const size_t B = x.shape[0], S = x.shape[1], d = x.shape[2];
  Tensor out = fresh({B, d});
  for (size_t b = 0; b < B; ++b)
    ok(talos_memcpy_d2d(out.data_->ptr + b * d, x.data_->ptr + (b * S + S - 1) * d, d * sizeof(float), nullptr),
       "last_token");
  if (!differentiable) return out;
  return with_ctx(out, {x}, [B, S, d](const Tensor& o, std::vector<Tensor>& p) {
    for (size_t b = 0; b < B; ++b) {
      float* row = p[0].grad_->ptr + (b * S + S - 1) * d;
      ok(talos_binary_fwd_f32(TALOS_ADD, d, row, o.grad_->ptr + b * d, row, nullptr), "last_token bwd");
    }
  });
}

std::vector<Tensor> LuckTransformer::parameters() const {  // :205-215
  std::vector<Tensor> p;
  for (const Module* m : std::initializer_list<const Module*>{&embed, &norm_1, &mla_layer, &norm_2, &ffn_1, &ffn_2,
                                                              &norm_final, &out_proj}) {
    const auto q = m->parameters();
    p.insert(p.end(), q.begin(), q.end());
  }
  return p;
}

// ---------------------------------------------------------------------------
// Adam (src/ppo.rs:482-539; src/dqn.rs:173-246)
// ---------------------------------------------------------------------------
Adam::Adam(std::vector<Tensor> params, double lr, double max_grad_norm)
    : params_(std::move(params)), lr_(lr), max_norm_(max_grad_norm) {
  for (const Tensor& p : params_) {  // zero state, as Adam::new's vec![0.0; len]
    m_.push_back(std::make_unique<Storage>(p.numel()));
    v_.push_back(std::make_unique<Storage>(p.numel()));
    ok(talos_fill_zero(m_.back()->ptr, p.numel() * sizeof(float), nullptr), "fill_zero");
    ok(talos_fill_zero(v_.back()->ptr, p.numel() * sizeof(float), nullptr), "fill_zero");
  }
  if (max_norm_ > 0.0) {  // the norm and the partial sums behind it, allocated once
    void* p = nullptr;
    ok(talos_malloc(&p, sizeof(double) + talos_grad_sumsq_workspace_bytes()), "talos_malloc");
    sumsq_ = static_cast<double*>(p);
  }
}

Adam::~Adam() {
  if (sumsq_) talos_free(sumsq_);
}

void Adam::step() {
  ++t_;
  if (sumsq_) {  // src/dqn.rs:207-214: one norm over every parameter's gradient
    for (size_t i = 0; i < params_.size(); ++i)
      ok(talos_grad_sumsq_f32(params_[i].numel(), params_[i].grad_->ptr, i > 0, sumsq_, sumsq_ + 1, nullptr),
         "grad_sumsq");
  }
  for (size_t i = 0; i < params_.size(); ++i) {
    const Tensor& p = params_[i];
    ok(talos_adam_step_f32(p.numel(), p.data_->ptr, p.grad_->ptr, m_[i]->ptr, v_[i]->ptr, (int)t_, lr_, beta1, beta2,
                           eps, sumsq_, max_norm_, nullptr),
       "adam_step");
  }
}

void Adam::zero_grad() const {
  for (const Tensor& p : params_) p.zero_grad();
}

}  // namespace tape
}  // namespace talos
