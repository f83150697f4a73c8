// tape.hpp -- host-side autograd tape over the C ABI of libtalos_hip.so.
//
// Mirrors the reference's Rust Tensor API (src/autograd.rs:14-20, 51-54, 94-196 and the ops of
// :200-792, 1599-1862) and the Linear / RMSNorm modules (src/nn.rs:11-304), with tensors held in
// device memory as fp32 and every op and backward closure executed by the library's kernels:
//
//   reference (Rust)                         here (C++)
//   Tensor::new(data, shape)                 Tensor::from_vec(data, shape)
//   Tensor::zeros / rand / detach / item     Tensor::zeros / rand / detach / item
//   t.backward() / zero_grad / clear_graph   t.backward() / zero_grad / clear_graph
//   t.data.read() / t.grad.read()            t.data() / t.grad()  (f64 host copies)
//   matmul relu log exp sum mean broadcast   same names
//   broadcast_to_batch sin cos sqrt transpose clip reshape mse_loss
//   a + b, a - b, a * b, a / b, -a           same operators
//   MLA's batched_matmul_qt_k / _probs_v,    free functions of the same names
//   scale_tensor, softmax, concat_last_dim
//   RoPE, MLAConfig, MultiHeadLatentAttention, LuckTransformer  same names (src/transformer.rs)
//   Adam::new(params, lr) / step / zero_grad  Adam(params, lr[, max_grad_norm]) / step / zero_grad
//
// Semantics kept: grads accumulate (+=) and only zero_grad clears them; backward() seeds every
// element of the root's grad with 1.0 and runs the closures in reverse DFS topological order,
// visiting each tensor (identified by its grad storage) once; x * x with the same tensor on both
// sides accumulates 2x.g once. Shape errors throw talos::tape::Panic where the reference panics
// (assert!), and a failing kernel call throws with the library's message.
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace talos {
namespace tape {

struct Panic : std::runtime_error {
  explicit Panic(const std::string& m) : std::runtime_error(m) {}
};

using Shape = std::vector<size_t>;

// A device buffer of n fp32 values (freed with the last reference).
struct Storage {
  float* ptr = nullptr;
  size_t n = 0;
  explicit Storage(size_t n);
  ~Storage();
  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
};

class Tensor;
struct Context {
  std::vector<Tensor> parents;
  // receives the output tensor (its grad is grad_out) and the parents
  std::function<void(const Tensor& out, std::vector<Tensor>& parents)> backward_op;
};

class Tensor {
 public:
  std::shared_ptr<Storage> data_;
  std::shared_ptr<Storage> grad_;
  Shape shape;
  std::shared_ptr<Context> _ctx;

  static Tensor from_vec(const std::vector<double>& data, Shape shape);  // Tensor::new
  static Tensor zeros(Shape shape);
  // Tensor::rand: the reference's LCG x = x * 6364136223846793005 + 1, r = (x >> 33) / u32::MAX
  // (src/autograd.rs:114-124), evaluated in f64 and stored as fp32
  static Tensor rand(Shape shape, double min, double max, uint64_t seed);

  size_t numel() const { return data_ ? data_->n : 0; }
  std::vector<double> data() const;  // Tensor.data.read()
  std::vector<double> grad() const;  // Tensor.grad.read()
  void set_data(const std::vector<double>& v) const;  // Tensor.data.write() = v
  double item() const;
  Tensor detach() const;  // shares data and grad, drops the graph
  void clear_graph() { _ctx.reset(); }
  void zero_grad() const;
  void backward() const;

  Tensor matmul(const Tensor& other) const;
  Tensor relu() const;
  Tensor log() const;
  Tensor exp() const;
  Tensor sum() const;
  Tensor mean() const;
  Tensor broadcast(Shape new_shape) const;
  Tensor broadcast_to_batch(size_t batch_size) const;
  Tensor sin() const;
  Tensor cos() const;
  Tensor sqrt() const;
  Tensor transpose(size_t dim0, size_t dim1) const;
  Tensor clip(double min, double max) const;
  Tensor reshape(Shape new_shape) const;
  Tensor mse_loss(const Tensor& target) const;
  // extensions used by the configurations (no reference counterpart): GELU and a scale
  Tensor gelu() const;
  Tensor scale(double s) const;
};

Tensor operator+(const Tensor& a, const Tensor& b);
Tensor operator-(const Tensor& a, const Tensor& b);
Tensor operator*(const Tensor& a, const Tensor& b);
Tensor operator/(const Tensor& a, const Tensor& b);
Tensor operator-(const Tensor& a);

// Module (src/nn.rs:6-9)
struct Module {
  virtual ~Module() = default;
  virtual Tensor forward(const Tensor& input) const = 0;
  virtual std::vector<Tensor> parameters() const = 0;
};

// Linear (src/nn.rs:11-142): y = x . W + b with W stored [in, out]; N-D inputs are flattened to
// [rows, in] and the result reshaped back; the bias is broadcast over the rows.
struct Linear : Module {
  Tensor weight, bias;
  bool has_bias = true;
  size_t in_features = 0, out_features = 0;
  // Xavier-uniform limit sqrt(6/(in+out)) drawn with Tensor::rand, as Linear::new does (src/nn.rs:20-35)
  Linear(size_t in, size_t out, bool bias, uint64_t seed);
  Linear(Tensor weight, Tensor bias, bool has_bias);
  Tensor forward(const Tensor& input) const override;
  std::vector<Tensor> parameters() const override;
};

// RMSNorm (src/nn.rs:144-304): y = x / sqrt(mean(x^2) + eps) * w over the last dimension.
struct RMSNorm : Module {
  Tensor weight;
  double eps = 1e-5;
  explicit RMSNorm(size_t dim, double eps = 1e-5);
  Tensor forward(const Tensor& x) const override;
  std::vector<Tensor> parameters() const override;
};

// ---------------------------------------------------------------------------------------------
// Attention ops: the helpers of MultiHeadLatentAttention (src/transformer.rs:877-1183), free
// functions here since they use no module state
// ---------------------------------------------------------------------------------------------
// q, k [b, seq, dim] -> scores [b, seq, seq], s[b,i,j] = q[b,i,:] . k[b,j,:]
// (batched_matmul_qt_k, :877-958); backward dq += g . k, dk += g^T . q
Tensor batched_matmul_qt_k(const Tensor& q, const Tensor& k, size_t b, size_t seq, size_t dim);
// probs [b, seq, seq], v [b, seq, dim_v] -> [b, seq, dim_v] (batched_matmul_probs_v, :961-1050);
// backward dp += g . v^T, dv += p^T . g. The reference skips |p| < 1e-9 in the forward product;
// every probability is multiplied here (the difference is below 1e-9 per term)
Tensor batched_matmul_probs_v(const Tensor& probs, const Tensor& v, size_t b, size_t seq, size_t dim_v);
// t * scale (scale_tensor, :1052-1072)
Tensor scale_tensor(const Tensor& t, double scale);
// softmax over consecutive rows of seq_len with max subtraction (softmax, :1074-1121); the
// backward reads the saved output. causal = true (extension, no reference counterpart): row r is
// query r mod seq_len and keys past it get probability 0
Tensor softmax(const Tensor& t, size_t seq_len, bool causal = false);
// [.., ca] ++ [.., cb] -> [.., ca + cb] (concat_last_dim, :1123-1183)
Tensor concat_last_dim(const Tensor& a, const Tensor& b);

// RoPE (src/transformer.rs:219-337): interleaved pairs (2i, 2i+1) of the last dimension rotated by
// pos * base^(-2i/dim), pos = start_pos + the index along shape[-2]; the cos / sin table is
// evaluated in f64 for max_len positions (the library rounds it to fp32), and a position at or past
// max_len panics as the reference's table index does
struct RoPE {
  size_t dim = 0, max_len = 0;
  double base = 10000.0;
  RoPE(size_t dim, size_t max_len);
  Tensor forward(const Tensor& x, size_t start_pos) const;
};

// MLAConfig (src/transformer.rs:9-33)
struct MLAConfig {
  size_t dim = 0, num_heads = 0, q_lora_rank = 0, kv_lora_rank = 0, qk_rope_dim = 0, v_head_dim = 0,
         max_seq_len = 0;
  static MLAConfig deepseek_v2_lite();  // dim 512, 8 heads, kv latent 128, rope 32, v 64, 2048
};

// MultiHeadLatentAttention (src/transformer.rs:374-560): the latent down / up projections, the
// decoupled RoPE parts (rotated by RoPE::forward on [B, S, H, R], so position = head index as in
// the reference), per-head concatenation, the [B*H, S, hd + R] attention through the ops above with
// scale 1/sqrt(hd + R), and W_o. No biases. Parameters in the reference's order.
struct MultiHeadLatentAttention : Module {
  MLAConfig config;
  Linear w_dkv, w_uk, w_uv, w_q, w_kr, w_qr, w_o;
  RoPE rope;
  MultiHeadLatentAttention(const MLAConfig& config, uint64_t seed);  // seeds seed .. seed + 6
  Tensor forward(const Tensor& x) const override;  // x [B, S, dim]
  std::vector<Tensor> parameters() const override;
};

// LuckTransformer (src/transformer.rs:35-109, 200-216): embed -> RMSNorm -> MLA -> + residual ->
// RMSNorm -> Linear(d, 2d) + ReLU -> Linear(2d, d) -> + residual -> RMSNorm -> out_proj, with the
// MLA of LuckTransformer::new (4 heads, kv latent 32, rope 16, v_head_dim = d / 4, 256 positions)
struct LuckTransformer : Module {
  Linear embed;
  RMSNorm norm_1;
  MultiHeadLatentAttention mla_layer;
  RMSNorm norm_2;
  Linear ffn_1, ffn_2;
  RMSNorm norm_final;
  Linear out_proj;
  LuckTransformer(size_t in_dim, size_t hidden_dim, bool bias, uint64_t seed);
  Tensor forward(const Tensor& x) const override;  // x [B, S, in_dim] -> [B, S, hidden_dim]
  // [B, S, d] -> [B, d], row S - 1 of each sequence, built as a new tensor without a graph as the
  // reference does (no gradient reaches x); differentiable = true (extension) records a gather
  // whose backward adds the rows' gradient into row S - 1
  Tensor last_token(const Tensor& x, bool differentiable = false) const;
  std::vector<Tensor> parameters() const override;
};

// Adam (src/ppo.rs:482-539): Adam::new(params, lr), step(), zero_grad(), set_lr(); b1 = 0.9,
// b2 = 0.999, eps = 1e-8. m and v are fp32 device buffers beside each parameter; step()
// increments t and runs the library's fused Adam kernel once per parameter tensor. With
// max_grad_norm > 0 it is the DQN optimizer (src/dqn.rs:173-246, max_grad_norm = 1.0): one f64
// squared-norm pass over every parameter's grad first, then each kernel scales its gradient by
// max_grad_norm / ||g|| when ||g|| > max_grad_norm.
class Adam {
 public:
  Adam(std::vector<Tensor> params, double lr, double max_grad_norm = 0.0);
  ~Adam();
  Adam(const Adam&) = delete;
  Adam& operator=(const Adam&) = delete;
  void step();
  void zero_grad() const;
  void set_lr(double lr) { lr_ = lr; }
  size_t t() const { return t_; }
  double beta1 = 0.9, beta2 = 0.999, eps = 1e-8;

 private:
  std::vector<Tensor> params_;
  std::vector<std::unique_ptr<Storage>> m_, v_;
  double* sumsq_ = nullptr;  // clipping only: the norm, then the partial-sum workspace
  size_t t_ = 0;
  double lr_, max_norm_;
};

}  // namespace tape
}  // namespace talos
