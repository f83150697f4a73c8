/*
 * talos_hip.h -- C ABI of the MI355X (gfx950) autograd hot path for Talos-XII's
 * transformer and linear policy layers.
 *
 * Every entry point takes plain pointers and sizes. Device pointers are fp32 buffers
 * allocated with talos_malloc or any HIP allocator. Streams are hipStream_t passed as void*;
 * NULL is the null (default) stream. Calls are synchronous by default, as the reference's
 * Tensor ops are (src/autograd.rs:200-354 return finished host vectors): a kernel entry point
 * enqueues its work on the stream, waits for the stream and returns the stream's error, if any.
 * talos_set_async(1) turns the calling thread's kernel entries into their asynchronous forms,
 * which return as soon as the work is enqueued (talos_stream_sync or a synchronous copy waits),
 * as GPU libraries do; code that captures a HIP graph must use that mode. The host <-> device
 * copies are synchronous in both modes.
 * Status codes: 0 on success, a talos_status otherwise; talos_last_error() returns a
 * thread-local message for the last failure. Arguments are validated on the host before any
 * launch, so every error path below can be exercised on a machine without a GPU.
 *
 * Reference citations are file:line in zayokami/Talos-XII (Rust crate, src/).
 */
#ifndef TALOS_HIP_H
#define TALOS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* talos_stream_t;

enum talos_status {
  TALOS_OK = 0,
  TALOS_ERR_SHAPE = 1,       /* shape / stride / size mismatch (reference: assert! panics, autograd.rs:96-100, 209) */
  TALOS_ERR_NULL = 2,        /* null pointer argument */
  TALOS_ERR_DTYPE = 3,       /* unsupported dtype, op code or layout enum */
  TALOS_ERR_NO_DEVICE = 4,   /* no usable GPU */
  TALOS_ERR_HIP = 5,         /* HIP runtime error (message carries hipGetErrorString) */
  TALOS_ERR_ALLOC = 6,       /* device allocation failed */
  TALOS_ERR_HANDLE = 7,      /* invalid or freed handle */
  TALOS_ERR_UNSUPPORTED = 8, /* configuration outside what the kernels cover (message says which limit) */
  TALOS_ERR_IO = 9,          /* a checkpoint file could not be opened, read or written */
  TALOS_ERR_FORMAT = 10      /* malformed checkpoint contents (truncated, bad JSON, wrong value types) */
};

/* ------------------------------------------------------------------------- */
/* Runtime                                                                    */
/* ------------------------------------------------------------------------- */

/* Thread-local message describing the last non-zero status on this thread. */
const char* talos_last_error(void);
/* Library version string. */
const char* talos_version(void);
/* Initialises the HIP device context once per process (std::call_once). */
int talos_init(void);
/* Number of visible GPUs (0 on a machine without one; returns TALOS_OK). */
int talos_device_count(int* count);
int talos_malloc(void** ptr, size_t bytes);
int talos_free(void* ptr);
/* Host<->device copies. The _f64 variants convert between the reference's f64
 * host vectors (Tensor.data / Tensor.grad, autograd.rs:14-20) and fp32 device buffers. */
int talos_memcpy_h2d(void* dst, const void* src, size_t bytes, talos_stream_t stream);
int talos_memcpy_d2h(void* dst, const void* src, size_t bytes, talos_stream_t stream);
/* Device-to-device copy, enqueued on the stream. */
int talos_memcpy_d2d(void* dst, const void* src, size_t bytes, talos_stream_t stream);
int talos_memcpy_h2d_f64(float* dst, const double* src, size_t n, talos_stream_t stream);
int talos_memcpy_d2h_f64(double* dst, const float* src, size_t n, talos_stream_t stream);
/* Zero-fills with a kernel (no hipMemsetAsync, so it is safe inside a captured graph). */
int talos_fill_zero(void* dst, size_t bytes, talos_stream_t stream);
int talos_stream_sync(talos_stream_t stream);
/* Completion mode of the calling thread's kernel entry points: 0 (the default) synchronous,
 * 1 asynchronous (the *_async behaviour of a GPU library). No reference counterpart: the
 * reference's ops are always synchronous. talos_get_async returns the thread's mode. */
int talos_set_async(int on);
int talos_get_async(void);
/* Non-blocking stream at the default priority. */
int talos_stream_create(talos_stream_t* stream);
int talos_stream_destroy(talos_stream_t stream);
/* Events for timing the work of a stream: elapsed_ms waits for stop. */
int talos_event_create(void** ev);
int talos_event_destroy(void* ev);
int talos_event_record(void* ev, talos_stream_t stream);
int talos_event_elapsed_ms(void* start, void* stop, float* ms);
/* Caller-owned scratch for the kernel-level entry points called from this thread: the split-K
 * partials of the GEMMs, the D rows of talos_attn_bwd_f32 and the f64 partial sums of the
 * reductions (talos_bias_grad_f32, talos_rmsnorm_bwd_f32, talos_reduce_sum_f32,
 * talos_grad_sumsq_f32 with a NULL workspace). A call whose scratch fits the bound buffer uses it
 * and allocates nothing; a GEMM whose split-K partials would not fit splits K fewer times (down to
 * no split) instead; any other call that needs more allocates and frees on its stream
 * (hipMallocAsync / hipFreeAsync), as every call does when nothing is bound. ptr must be device
 * memory, 256-byte aligned; NULL, 0 unbinds. The library never frees it, and calls that share one
 * binding must not overlap on the device (issue them on one stream). The reference has no
 * counterpart (its ops allocate host vectors per call, src/autograd.rs:262-264). */
int talos_workspace_bind(void* ptr, size_t bytes);
/* The largest scratch (bytes) a call on this thread asked for since the last bind. */
size_t talos_workspace_high_water(void);
/* Bytes of the workspace bound on this thread (0 when none). No reference counterpart: it lets a
 * layer above (the C++ tape) leave a caller's binding in place. */
size_t talos_workspace_bytes(void);
/* Name (with gfx arch), compute-unit count, peak clock (kHz) and memory of device 0. */
int talos_device_info(char* name, size_t name_len, int* cu_count, int* clock_khz, size_t* total_mem);

/* ------------------------------------------------------------------------- */
/* Kernel-level entry points (device pointers, fp32 unless stated)            */
/* ------------------------------------------------------------------------- */

/* C[M,N] = alpha * op(A) * op(B) + beta * C, row-major.
 * op(A) is A[M,K] (lda >= K) when transA == 0, or the transpose of A stored [K,M] (lda >= M).
 * op(B) is B[K,N] (ldb >= N) when transB == 0, or the transpose of B stored [N,K] (ldb >= K).
 * Replaces Tensor::matmul (autograd.rs:200-354): forward C = A.B is (0,0); the backward
 * dA += dC.B^T is (0,1) with beta 1 and dB += A^T.dC is (1,0) with beta 1 (grads accumulate,
 * autograd.rs:290, 330). beta must be 0 or 1. MFMA v_mfma_f32_32x32x2_f32 tiles; long-K
 * products with a small C are split over K with the partial tiles summed in f64. */
int talos_gemm_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                   const float* B, int ldb, float beta, float* C, int ldc, talos_stream_t stream);

/* Same contract, bf16-in / fp32-accumulate: A and B stay fp32 in memory and are rounded to bf16
 * (nearest even) as they are staged into LDS; products use v_mfma_f32_32x32x16_bf16 with fp32
 * accumulation and an fp32 C. No reference counterpart (the reference is f64 only,
 * autograd.rs:16-17): this is the optional bf16 variant of talos_gemm_f32. */
int talos_gemm_bf16acc_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                           const float* B, int ldb, float beta, float* C, int ldc, talos_stream_t stream);

/* Batched C_b = alpha * A_b . op(B_b) + beta * C_b for b in [0,batch) with element strides
 * sA, sB, sC between consecutive matrices (same trans conventions as talos_gemm_f32).
 * Replaces batched_matmul_qt_k (transformer.rs:877-958: S = Q.K^T is transB = 1) and
 * batched_matmul_probs_v (transformer.rs:961-1050: O = P.V is transB = 0) and their backward. */
int talos_gemm_batched_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                           long long sA, const float* B, int ldb, long long sB, float beta, float* C, int ldc,
                           long long sC, int batch, talos_stream_t stream);

/* db[cols] = beta * db + sum_rows dy[rows, cols]. Backward of broadcast_to_batch
 * (autograd.rs:530-544), i.e. the Linear bias gradient (nn.rs:96-101). Partials are
 * combined in f64. */
int talos_bias_grad_f32(int rows, int cols, const float* dy, float beta, float* db, talos_stream_t stream);

/* RMSNorm forward (nn.rs:182-230): rms = sqrt(mean(x^2) + eps), y = x / rms * w.
 * Saves rstd[rows] = 1/rms (the reference caches rms and x_hat, nn.rs:196-197; x_hat is
 * recomputed from x and rstd instead of being stored). */
int talos_rmsnorm_fwd_f32(int rows, int dim, float eps, const float* x, const float* w, float* y, float* rstd,
                          talos_stream_t stream);
/* RMSNorm backward (nn.rs:234-296): dx += rstd * (g*w - x_hat * mean(g*w*x_hat)),
 * dw += sum_rows g * x_hat. beta_dx / beta_dw in {0,1} select overwrite or accumulate. */
int talos_rmsnorm_bwd_f32(int rows, int dim, const float* x, const float* w, const float* rstd, const float* dy,
                          float beta_dx, float* dx, float beta_dw, float* dw, talos_stream_t stream);

/* Row softmax (transformer.rs:1074-1096) with max subtraction. causal != 0 adds the
 * causal mask: row r is query q = r mod cols, keys j > q get probability exactly 0
 * (extension; the reference has no mask). */
int talos_softmax_fwd_f32(int rows, int cols, int causal, const float* x, float* y, talos_stream_t stream);
/* dx = beta*dx + y * (g - sum(g*y)) (transformer.rs:1098-1117). Masked entries get 0. */
int talos_softmax_bwd_f32(int rows, int cols, int causal, const float* y, const float* dy, float beta, float* dx,
                          talos_stream_t stream);

/* Rotary embedding on x[n_seq, seq_len, heads, dim] (row-major, interleaved pairs
 * (2i, 2i+1)), position of token t is start_pos + t, theta_i = base^(-2i/dim) with the
 * cos/sin table computed in f64 and rounded to fp32 (transformer.rs:239-251, 255-292).
 * The reference's training path rotates by the index along shape[-2] (transformer.rs:262);
 * here the position is always the sequence index. */
int talos_rope_fwd_f32(int n_seq, int seq_len, int heads, int dim, int start_pos, float base, const float* x,
                       float* y, talos_stream_t stream);
/* Backward = rotation by -theta (transformer.rs:305-333): dx = beta*dx + R^T dy. */
int talos_rope_bwd_f32(int n_seq, int seq_len, int heads, int dim, int start_pos, float base, const float* dy,
                       float beta, float* dx, talos_stream_t stream);
/* Writes the fp32 cos/sin table [max_len, dim/2] the kernels use (bit-exact check). */
int talos_rope_table_f32(int max_len, int dim, float base, float* cos_out, float* sin_out, talos_stream_t stream);

/* Fused scaled-dot-product attention over q/k/v laid out [batch, seq, heads, dim]
 * with row strides ld_q/ld_k/ld_v/ld_o (elements between consecutive tokens), replacing
 * the chain transpose -> batched_matmul_qt_k -> scale_tensor -> softmax -> batched_matmul_probs_v
 * -> transpose (transformer.rs:519-557, 877-1121). Saves lse[batch, heads, seq] (natural
 * log-sum-exp of the scaled scores) for the backward. qk_dim <= 128, v_dim <= 128, seq <= 256. */
int talos_attn_fwd_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal,
                       const float* q, int ld_q, const float* k, int ld_k, const float* v, int ld_v,
                       float* o, int ld_o, float* lse, talos_stream_t stream);
/* Backward of talos_attn_fwd_f32: writes dq, dk, dv (overwrite) with the same layouts. */
int talos_attn_bwd_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal,
                       const float* q, int ld_q, const float* k, int ld_k, const float* v, int ld_v,
                       const float* o, int ld_o, const float* lse, const float* dout, int ld_do,
                       float* dq, int ld_dq, float* dk, int ld_dk, float* dv, int ld_dv, talos_stream_t stream);

/* Same contract and results as talos_attn_bwd_f32, allocating nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). For seq > 32 the backward keeps
 * D = rowsum(dO * O) of each (batch, head, query) row in a static device array of 2^20 rows (4 MiB,
 * which each GPU the library runs on holds until the process ends); batch * heads * seq above 2^20
 * is TALOS_ERR_UNSUPPORTED. Every call on one GPU shares that array: calls that overlap on one GPU
 * (on other streams or threads) race. */
int talos_attn_bwd_noalloc_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal,
                               const float* q, int ld_q, const float* k, int ld_k, const float* v, int ld_v,
                               const float* o, int ld_o, const float* lse, const float* dout, int ld_do, float* dq,
                               int ld_dq, float* dk, int ld_dk, float* dv, int ld_dv, talos_stream_t stream);

/* Element-wise ops of the tape (autograd.rs:356-792, 1606-1862). */
enum talos_unary_op {
  TALOS_RELU = 0, TALOS_LOG = 1, TALOS_EXP = 2, TALOS_SIN = 3, TALOS_COS = 4, TALOS_SQRT = 5,
  TALOS_NEG = 6, TALOS_SCALE = 7, TALOS_CLIP = 8, TALOS_GELU = 9, TALOS_COPY = 10
};
enum talos_binary_op { TALOS_ADD = 0, TALOS_SUB = 1, TALOS_MUL = 2, TALOS_DIV = 3 };
/* y = op(x); p0/p1 are the scale factor (SCALE) or [min,max] (CLIP). */
int talos_unary_fwd_f32(int op, size_t n, float p0, float p1, const float* x, float* y, talos_stream_t stream);
/* dx += dop(x) * dy, exactly the reference closures (e.g. relu passes where x > 0,
 * clip where min <= x <= max, sqrt only where x > 0). */
int talos_unary_bwd_f32(int op, size_t n, float p0, float p1, const float* x, const float* dy, float* dx,
                        talos_stream_t stream);
/* GELU (an extension: the reference has relu only, autograd.rs:356-386; the configurations'
 * MLPs use GELU): y = 0.5 x (1 + erf(x / sqrt(2))). The same function as op TALOS_GELU, with a
 * float4 kernel. */
int talos_gelu_fwd_f32(size_t n, const float* x, float* y, talos_stream_t stream);
/* dx = beta * dx + dy * (Phi(x) + x phi(x)), beta 0 (overwrite) or 1 (accumulate, as the tape's
 * grads do). */
int talos_gelu_bwd_f32(size_t n, const float* x, const float* dy, float beta, float* dx, talos_stream_t stream);
int talos_binary_fwd_f32(int op, size_t n, const float* a, const float* b, float* y, talos_stream_t stream);
/* da += d/da, db += d/db. When da == db (the same tensor on both sides, autograd.rs:1729, 1792)
 * the combined derivative is accumulated once. */
int talos_binary_bwd_f32(int op, size_t n, const float* a, const float* b, const float* dy, float* da, float* db,
                         talos_stream_t stream);
/* out[0] = scale * sum(x) (sum / mean, autograd.rs:433-482), partials combined in f64. */
int talos_reduce_sum_f32(size_t n, float scale, const float* x, float* out, talos_stream_t stream);
/* dx[i] += scale * g[0] (backward of sum / mean / broadcast-from-scalar). */
int talos_fill_add_f32(size_t n, float scale, const float* g, float* dx, talos_stream_t stream);
/* y[..] = x with dims dim0, dim1 swapped (autograd.rs:632-739). accumulate != 0 adds into y
 * (the backward scatter-add). rank <= 6. */
int talos_transpose_f32(int rank, const long long* shape, int dim0, int dim1, const float* x, float* y,
                        int accumulate, talos_stream_t stream);
/* out[rows, ca+cb] = [a | b] (concat_last_dim, transformer.rs:1123-1160); backward splits. */
int talos_concat_last_f32(size_t rows, int ca, int cb, const float* a, const float* b, float* out,
                          talos_stream_t stream);
int talos_concat_last_bwd_f32(size_t rows, int ca, int cb, const float* dout, float* da, float* db,
                              talos_stream_t stream);
/* out[rows, cols] = broadcast_to_batch of v[cols] (autograd.rs:511-528). */
int talos_broadcast_rows_f32(size_t rows, int cols, const float* v, float* out, talos_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Optimizer step                                                             */
/* ------------------------------------------------------------------------- */

/* sumsq[0] = (accumulate ? sumsq[0] : 0) + sum_i grads[i]^2, summed in f64: the global-norm
 * loop of the DQN optimizer (dqn.rs:207-214). sumsq is ONE device double; several parameter
 * tensors share one norm by calling this once per tensor with accumulate = 1 after the first.
 * workspace: NULL (the call allocates and frees its partial sums on the stream) or a device
 * buffer of talos_grad_sumsq_workspace_bytes() bytes, reused across calls on one stream.
 * Deterministic (fixed partition of the partial sums). */
size_t talos_grad_sumsq_workspace_bytes(void);
int talos_grad_sumsq_f32(size_t n, const float* grads, int accumulate, double* sumsq, double* workspace,
                         talos_stream_t stream);

/* One Adam step over n parameters, Adam::step (ppo.rs:519-533):
 *   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2;
 *   params -= lr * (m / (1 - b1^t)) / (sqrt(v / (1 - b2^t)) + eps)
 * t is the step count AFTER the reference's increment (1 on the first call; t < 1 is
 * TALOS_ERR_SHAPE). m and v are fp32 state, zero before the first step; the arithmetic runs in
 * f64 and rounds once on the store. The reference uses b1 = 0.9, b2 = 0.999, eps = 1e-8.
 * When sumsq != NULL (a device double from talos_grad_sumsq_f32) the gradient is first scaled by
 * the DQN global-norm clip (dqn.rs:215-226): c = max_norm / sqrt(*sumsq) if sqrt(*sumsq) >
 * max_norm, else 1 (the reference's max_norm is 1.0; max_norm <= 0 is TALOS_ERR_SHAPE).
 * params, grads, m and v must not overlap. */
int talos_adam_step_f32(size_t n, float* params, const float* grads, float* m, float* v, int t, double lr,
                        double beta1, double beta2, double eps, const double* sumsq, double max_norm,
                        talos_stream_t stream);

/* ------------------------------------------------------------------------- */
/* Fused model-level entry points                                             */
/* ------------------------------------------------------------------------- */

enum talos_activation { TALOS_ACT_GELU = 0, TALOS_ACT_RELU = 1 };

/* Attention of a block: standard multi-head attention with RoPE on all of q and k, or the
 * reference's multi-head latent attention (MultiHeadLatentAttention, transformer.rs:428-560). */
enum talos_attention { TALOS_ATTN_MHA = 0, TALOS_ATTN_MLA = 1 };

/* Pre-norm transformer block (the wiring of LuckTransformer::forward, transformer.rs:71-90):
 *   h2  = x + Wo . attn(rmsnorm(x; g1))
 *   out = h2 + W2 . act(rmsnorm(h2; g2) . W1 + b1) + b2
 * attention = TALOS_ATTN_MHA: [q|k|v] = rmsnorm(x; g1) . Wqkv, RoPE on q and k, head_dim per
 *   head, n_heads * head_dim == d_model. Parameter layout (fp32, contiguous, in this order),
 *   d = d_model, F = ffn_dim:
 *     g1[d] | Wqkv[d,3d] (columns q | k | v, heads contiguous) | Wo[d,d] | g2[d] |
 *     W1[d,F] | b1[F] | W2[F,d] | b2[d]
 * attention = TALOS_ATTN_MLA: the attention of talos_mla_cfg below (latent kv_latent, decoupled
 *   RoPE of rope_dim per head, content head_dim, value v_dim); with ReLU and F = 2d this is the
 *   reference block exactly. Parameter layout (the order of LuckTransformer::parameters,
 *   transformer.rs:205-215), H = n_heads, L = kv_latent, r = rope_dim, hd = head_dim, vd = v_dim:
 *     g1[d] | W_dkv[d,L] | W_uk[L,H*hd] | W_uv[L,H*vd] | W_q[d,H*hd] | W_kr[d,H*r] |
 *     W_qr[d,H*r] | W_o[H*vd,d] | g2[d] | W1[d,F] | b1[F] | W2[F,d] | b2[d]
 * Linear weights are stored [in, out] as in the reference (nn.rs:22). The MLA fields are ignored
 * (and may be left zero) for TALOS_ATTN_MHA. */
typedef struct talos_block_cfg {
  int batch;
  int seq;
  int d_model;
  int n_heads;
  int head_dim;   /* MHA: n_heads * head_dim == d_model; MLA: content q/k dims per head */
  int ffn_dim;
  int causal;     /* 1: causal attention mask */
  int activation; /* talos_activation */
  float eps;      /* RMSNorm eps */
  float rope_base;
  int attention;  /* talos_attention */
  int kv_latent;  /* MLA only */
  int rope_dim;   /* MLA only */
  int v_dim;      /* MLA only */
} talos_block_cfg;

size_t talos_block_param_count(const talos_block_cfg* cfg);

/* Policy network of the PPO actor-critic (ppo.rs:246-307): embed Linear(in,d)+b ->
 * n_layers blocks -> RMSNorm -> out_proj Linear(d,d)+b -> last token -> actor Linear(d,A)+b
 * and critic Linear(d,1)+b. Parameter layout:
 *   We[in,d] | be[d] | block_0 ... block_{L-1} (talos_block_cfg layout) | gf[d] |
 *   Wout[d,d] | bout[d] | Wa[d,A] | ba[A] | Wc[d,1] | bc[1]
 * The reference's ActorCritic (ActorCritic::new, ppo.rs:254-258 with LuckTransformer::new,
 * transformer.rs:48-69) is in_dim 8, d 64, one TALOS_ATTN_MLA layer (4 heads, latent 32, rope 16,
 * head_dim = v_dim = 16), ffn 128 ReLU, eps 1e-5, no causal mask, 5 actions; its parameter order
 * (ActorCritic::parameters, ppo.rs:302-307) is this layout. */
typedef struct talos_ppo_cfg {
  int batch;      /* samples per minibatch */
  int seq;        /* tokens per sample (all samples padded to seq) */
  int in_dim;     /* state features per token (8, sim.rs:347-356) */
  int d_model;
  int n_layers;
  int n_heads;
  int head_dim;
  int ffn_dim;
  int n_actions;
  int causal;
  int activation;
  float eps;
  float rope_base;
  float clip_eps;     /* 0.2, ppo.rs:17 */
  float value_coef;   /* 0.5, ppo.rs:20 */
  float entropy_coef; /* 0.01, ppo.rs:21 */
  int attention;      /* talos_attention of every block, with the MLA widths below */
  int kv_latent;
  int rope_dim;
  int v_dim;
} talos_ppo_cfg;

size_t talos_ppo_param_count(const talos_ppo_cfg* cfg);

/* MLA block (MultiHeadLatentAttention, transformer.rs:374-398, 428-560) with a pre-norm residual:
 *   out = x + W_o . attn([q_c | rope(q_r)], [k_c | rope(k_r)], v),  xn = rmsnorm(x; g),
 *   c_kv = xn . W_dkv, k_c = c_kv . W_uk, v = c_kv . W_uv, q_c = xn . W_q, q_r = xn . W_qr,
 *   k_r = xn . W_kr, per-head concatenation of content and RoPE dims, scale 1/sqrt(head_dim +
 *   rope_dim) (transformer.rs:542), RoPE position = sequence index. No biases (transformer.rs:441-460).
 * Parameter layout: g[d] | W_dkv[d,L] | W_uk[L,H*hd] | W_uv[L,H*vd] | W_q[d,H*hd] | W_kr[d,H*r] |
 *   W_qr[d,H*r] | W_o[H*vd,d]. */
/* TALOS_PREC_BF16: the projections' GEMMs, and the attention's QK^T, PV and gradient contractions
 * where seq > 64, seq % 4 == 0 and the head dims fit (32, 32), (64, 64) or (96, 64) (fused plans), take bf16
 * operands (nearest even) with fp32 accumulation; softmax, lse and the norm stay fp32. */
enum talos_precision { TALOS_PREC_FP32 = 0, TALOS_PREC_BF16 = 1 /* bf16-in / fp32-accumulate */ };
typedef struct talos_mla_cfg {
  int batch;
  int seq;
  int d_model;
  int n_heads;
  int kv_latent;
  int rope_dim;
  int head_dim;  /* content dims of q / k per head */
  int v_dim;
  int causal;
  int precision; /* talos_precision */
  float eps;
  float rope_base;
} talos_mla_cfg;

size_t talos_mla_param_count(const talos_mla_cfg* cfg);

/* Opaque plans own device workspace sized for one configuration. */
typedef struct talos_plan_s* talos_plan;

/* One pre-norm block forward + backward for loss = sum(out * gout):
 * writes out[batch*seq, d], dparams (same layout as params), dx. */
int talos_block_plan_create(const talos_block_cfg* cfg, talos_plan* plan);
int talos_block_fwd_bwd_f32(talos_plan plan, const float* params, const float* x, const float* gout, float* out,
                            float* dparams, float* dx, talos_stream_t stream);

/* PPO minibatch forward + backward (ppo.rs:686-757 for one minibatch, with the
 * backbone evaluated once and the last-token gather differentiable): states[batch, seq, in_dim],
 * actions[batch] (int32), adv/ret/old_logp[batch]. Writes the mean loss (device scalar,
 * loss_out[0]) and dparams (overwritten, same layout as params). */
int talos_ppo_plan_create(const talos_ppo_cfg* cfg, talos_plan* plan);
int talos_ppo_fwd_bwd_f32(talos_plan plan, const float* params, const float* states, const int32_t* actions,
                          const float* adv, const float* ret, const float* old_logp, float* loss_out,
                          float* dparams, talos_stream_t stream);
/* Forward only: logits[batch, A] and values[batch] of the policy (for old log-probs). */
int talos_ppo_forward_f32(talos_plan plan, const float* params, const float* states, float* logits,
                          float* values, talos_stream_t stream);

/* Sums over a minibatch's samples that talos_ppo_minibatch_f32 can write (device doubles):
 * approx_kl = (ratio - 1) - log_ratio (ppo.rs:726-729), the chosen surrogate, (V - ret)^2, the
 * entropy, and the sample count. */
enum talos_ppo_stat {
  TALOS_PPO_STAT_KL = 0,
  TALOS_PPO_STAT_POLICY = 1,
  TALOS_PPO_STAT_VALUE = 2,
  TALOS_PPO_STAT_ENTROPY = 3,
  TALOS_PPO_STAT_COUNT = 4,
  TALOS_PPO_NSTATS = 5
};

/* The minibatch entry of the update loop: n samples (1 <= n <= cfg.batch; the loss is the mean
 * over n, as ppo.rs:754-755 divides by chunk.len()). lengths (device int32[n], or NULL for all
 * seq) gives each sample's token count, Q5 of the reference's varying state lengths: the last
 * token of sample b is row lengths[b] - 1 and keys at or past lengths[b] are masked, so a
 * right-padded sample gives exactly its unpadded result (padding rows must hold finite values).
 * stats (device double[TALOS_PPO_NSTATS], or NULL) receives the sums above, added to its
 * contents when stats_accumulate != 0. loss (device float[1]) may be NULL. */
int talos_ppo_minibatch_f32(talos_plan plan, int n, const float* params, const float* states,
                            const int32_t* lengths, const int32_t* actions, const float* adv, const float* ret,
                            const float* old_logp, float* loss, float* dparams, double* stats,
                            int stats_accumulate, talos_stream_t stream);
/* The clipped PPO loss of a minibatch from the actor logits [n, n_actions] and critic values [n]
 * (replaces the per-sample loss graph of ppo.rs:702-749 and its mean, ppo.rs:754-755). Per sample,
 * in f64: logp = log_softmax(logits), ratio = exp(logp[action] - old_logp), surrogates ratio * adv
 * and clip(ratio, 1 - clip_eps, 1 + clip_eps) * adv, the smaller kept (ties take the clipped one);
 * loss = mean(-surrogate + value_coef (value - ret)^2 - entropy_coef H). loss (device float[1])
 * and stats (device double[TALOS_PPO_NSTATS], added into when stats_accumulate != 0) may each be
 * NULL, not both. An action outside [0, n_actions) makes the loss NaN (the reference panics).
 * n_actions may be any positive count here (the plans take at most 64). */
int talos_ppo_head_loss_fwd_f32(int n, int n_actions, float clip_eps, float value_coef, float entropy_coef,
                                const float* logits, const float* values, const int32_t* actions, const float* adv,
                                const float* ret, const float* old_logp, float* loss, double* stats,
                                int stats_accumulate, talos_stream_t stream);
/* Its gradient with respect to the logits and values (the closures of the same graph,
 * ppo.rs:702-755, in closed form): dlogits [n, n_actions] and dvalues [n] are overwritten; loss
 * (device float[1]) is written too when not NULL. A sample with an out-of-range action gets a
 * zero gradient. */
int talos_ppo_head_loss_bwd_f32(int n, int n_actions, float clip_eps, float value_coef, float entropy_coef,
                                const float* logits, const float* values, const int32_t* actions, const float* adv,
                                const float* ret, const float* old_logp, float* dlogits, float* dvalues, float* loss,
                                talos_stream_t stream);
/* Forward only for n samples with optional lengths (the rollout's log-probs and values). */
int talos_ppo_forward_n_f32(talos_plan plan, int n, const float* params, const float* states,
                            const int32_t* lengths, float* logits, float* values, talos_stream_t stream);

/* Advantages and returns of one rollout, the f64 prologue of PPO::update (ppo.rs:650-676):
 *   r_t   = clamp((rewards_t - r_mean) / (sqrt(r_var) + 1e-8), -r_clip, r_clip)
 *           (RunningMeanStd::normalize, ppo.rs:477-479; r_clip = 10 at ppo.rs:655)
 *   d_t   = r_t + gamma * V_{t+1} * (1 - done_t) - V_t,   V_len = 0
 *   A_t   = d_t + gamma * lambda * (1 - done_t) * A_{t+1}, A_len = 0
 *   ret_t = A_t + V_t;  adv_t = (A_t - mean(A)) / (std(A) + 1e-8)  (population std)
 * The reference uses gamma 0.99, lambda 0.95 (ppo.rs:18-19). rewards, values: device double[len];
 * terminals: device uint8[len] (0 / non-zero); adv, ret: device float[len] (the loss inputs);
 * adv_raw: device double[len] or NULL. The recursion runs as a parallel linear-recurrence scan in
 * f64 in one workgroup. */
int talos_ppo_gae_f64(int len, const double* rewards, const double* values, const uint8_t* terminals,
                      double r_mean, double r_var, double r_clip, double gamma, double lambda, float* adv,
                      float* ret, double* adv_raw, talos_stream_t stream);

/* PPO::update on the device (ppo.rs:625-770): GAE and advantage normalisation, then k_epochs
 * passes over the rollout in order (no shuffling, as the reference's indices.chunks), each a
 * minibatch forward + backward (talos_ppo_minibatch_f32, minibatch = the plan's batch, the last
 * chunk shorter) followed by one Adam step (talos_adam_step_f32, b = (0.9, 0.999), eps 1e-8). An
 * epoch whose mean approx_kl exceeds 1.5 * target_kl (0.015 at ppo.rs:678) ends the update
 * (ppo.rs:761-768). The host synchronises once per epoch, for the KL check. */
typedef struct talos_ppo_update_args {
  int n;                     /* samples in the rollout */
  const float* states;       /* device [n, seq, in_dim], right-padded when lengths != NULL */
  const int32_t* lengths;    /* device [n] or NULL */
  const int32_t* actions;    /* device [n] */
  const float* old_logp;     /* device [n]: the rollout policy's log-probs */
  const double* rewards;     /* device [n] */
  const double* values;      /* device [n]: the rollout's critic values */
  const uint8_t* terminals;  /* device [n] */
  double reward_mean, reward_var, reward_clip;  /* the reward normaliser's state; clip 10 */
  double gamma, lambda, target_kl;              /* 0.99, 0.95, 0.015 in the reference */
  int k_epochs;
  double lr;                 /* Adam::set_lr(current_lr), ppo.rs:630 */
  float* params;             /* device, updated in place */
  float* adam_m;             /* device, same size as params (zero before the first update) */
  float* adam_v;
  int adam_t;                /* Adam steps taken before this update; advanced by the update */
  void* work;                /* device, talos_ppo_update_work_bytes(plan, n) bytes */
} talos_ppo_update_args;
typedef struct talos_ppo_update_result {
  int epochs_run;            /* epochs completed, early stop included */
  int stopped_early;         /* 1 when the KL check ended the update */
  double approx_kl;          /* mean approx_kl of the last epoch run */
  double mean_loss;          /* mean over the last epoch's samples of the per-sample loss */
} talos_ppo_update_result;
size_t talos_ppo_update_work_bytes(talos_plan plan, int n);
int talos_ppo_update_f32(talos_plan plan, talos_ppo_update_args* args, talos_ppo_update_result* result,
                         talos_stream_t stream);

/* MLA block forward + backward for loss = sum(out * gout): writes out[batch*seq, d], dparams
 * (overwritten, same layout as params) and dx. */
int talos_mla_plan_create(const talos_mla_cfg* cfg, talos_plan* plan);
int talos_mla_fwd_bwd_f32(talos_plan plan, const float* params, const float* x, const float* gout, float* out,
                          float* dparams, float* dx, talos_stream_t stream);

int talos_plan_destroy(talos_plan plan);

/* ------------------------------------------------------------------------- */
/* Rollout inference with the KV cache                                        */
/* ------------------------------------------------------------------------- */
/* The policy's step on one new token per environment with a cache of earlier tokens
 * (LuckTransformer::forward_inference_step, transformer.rs:157-196;
 * MultiHeadLatentAttention::forward_inference_cached, transformer.rs:688-805), for n_envs
 * environments at once, each with its own cache, followed by prune_kv_cache to context_len rows
 * (transformer.rs:807-840; sim.rs:578 prunes after every step) and the action draw of
 * ActorCritic::step_inference_cached (ppo.rs:391-433). A step attends over the rows cached plus
 * the new token (at most context_len + 1), then keeps the newest context_len. RoPE rotates q / k at
 * the environment's position; positions >= max_seq_len (the reference's RoPE cache length, 0 selects
 * 256) are left unrotated as the reference's `continue` does (transformer.rs:718-721). The
 * configuration is any talos_ppo_cfg architecture (batch and seq are ignored); the decoder owns
 * the caches (n_envs * n_layers * n_heads * (context_len + 1) * (dk + dv) floats) and its
 * activations, so a step allocates nothing. For the reference ActorCritic's shape (in_dim 8, d 64,
 * MLA with 4 heads, latent 32, rope 16, head and value dims 16, ffn 128, 5 actions) and
 * context_len <= 16 the step is one kernel launch whose cache holds each token's latent row and
 * rotated k_rope rows instead (n_envs * n_layers * (context_len + 1) * (kv_latent + n_heads *
 * rope_dim) floats); the environment variable TALOS_DECODER_LAYERED=1 at creation selects the
 * general path instead. */
typedef struct talos_decoder_s* talos_decoder;
int talos_ppo_decoder_create(const talos_ppo_cfg* cfg, int n_envs, int context_len, int max_seq_len,
                             talos_decoder* dec);
/* One token for environments 0..n-1 (n <= n_envs), all device buffers: tokens [n, in_dim],
 * positions [n] (start_pos of each token), reset [n] (optional: nonzero clears that environment's
 * cache before the token, KVCache::clear for a new episode), uniforms [n] (the draws the reference
 * takes from rand::random; required for actions / logp). Outputs, each optional: logits [n, A],
 * values [n] (the critic on the same hidden state), actions [n] (int32), logp [n] (ln p of the
 * action). The action is the first i with r < p_i after subtracting the earlier p_j, or 0 when none
 * qualifies, as the reference's loop leaves it. */
int talos_ppo_decoder_step_f32(talos_decoder dec, int n, const float* params, const float* tokens,
                               const int32_t* positions, const uint8_t* reset, const float* uniforms, float* logits,
                               float* values, int32_t* actions, float* logp, talos_stream_t stream);
/* Host copy of one environment's cached rows of a layer, oldest first: k [len, n_heads, dk] and
 * v [len, n_heads, dv] (either may be NULL); *len = rows held. Waits for the device. A latent cache
 * is expanded to the reference's rows with the last step's parameters (k_h = [c.W_uk_h |
 * k_rope_h], v_h = c.W_uv_h, in f64 on the host), which must still be valid device memory. */
int talos_ppo_decoder_read_cache(talos_decoder dec, int layer, int env, float* k, float* v, int* len);
int talos_ppo_decoder_destroy(talos_decoder dec);

/* ------------------------------------------------------------------------- */
/* Checkpoints of the reference's ActorCritic                                 */
/* ------------------------------------------------------------------------- */
/* The two files of save_ppo_model / load_ppo_model (main.rs:123-166): "<path>.bin" in bincode 1.3
 * (its fixed-width little-endian encoding) and "<path>" in serde_json, both of ActorCritic
 * {backbone: LuckTransformer, actor_head, critic_head} (ppo.rs:246-251; transformer.rs:35-45,
 * 8-17, 374-398, 219-225; nn.rs:11-17, 144-149; Tensor as {data, shape}, autograd.rs:22-49).
 * params are HOST fp32 arrays in the talos_ppo_cfg layout (talos_ppo_param_count floats): saving
 * widens each value exactly to the file's f64, loading rounds each f64 to the nearest fp32. The
 * configuration must be one the format holds: TALOS_ATTN_MLA, n_layers 1 and head_dim == v_dim (the
 * reference's q/k content heads are v_head_dim wide, transformer.rs:410-425), else
 * TALOS_ERR_UNSUPPORTED. Loading checks every shape, in/out width, RMSNorm eps and the RoPE base
 * against cfg (TALOS_ERR_SHAPE on a mismatch) and leaves params unchanged on any failure. These
 * functions run on the host only and need no GPU. */
enum talos_checkpoint_format { TALOS_CKPT_BINCODE = 0, TALOS_CKPT_JSON = 1 };
/* Serialises into buf (cap bytes) and sets *size to the checkpoint's length; buf == NULL only
 * measures. max_seq_len is MLAConfig::max_seq_len, the length of the RoPE caches the file holds
 * (0 selects 256, LuckTransformer::new's value, transformer.rs:48-56). Non-finite values are
 * written as JSON null, as serde_json does (and its reader rejects them). */
int talos_ppo_checkpoint_encode(const talos_ppo_cfg* cfg, const float* params, int max_seq_len, int format,
                                uint8_t* buf, size_t cap, size_t* size);
int talos_ppo_checkpoint_decode(const talos_ppo_cfg* cfg, const uint8_t* buf, size_t size, int format,
                                float* params);
/* save_ppo_model: writes "<path>.bin", then "<path>" (each through a temporary file and a rename).
 * load_ppo_model: reads "<path>.bin", falling back to "<path>" when the binary is missing or does
 * not decode; TALOS_ERR_IO when neither file opens. */
int talos_ppo_checkpoint_save(const talos_ppo_cfg* cfg, const float* params, int max_seq_len, const char* path);
int talos_ppo_checkpoint_load(const talos_ppo_cfg* cfg, const char* path, float* params);

/* Per-launch profiling of a plan's entry points (the reference has only ad-hoc Instant timers
 * that print, src/dqn.rs:483-583 and src/autograd.rs:1877-1890). While enabled, every kernel the
 * plan launches is bracketed by two HIP events on its stream and recorded with the kernel's name
 * and its algorithmic flops and HBM bytes. kernel_filter (NULL = all) keeps only launches whose
 * kernel name contains it. Enabling clears earlier records (after a device synchronise). */
typedef struct talos_profiler_s* talos_profiler;
typedef struct talos_prof_record {
  char kernel[64];
  double flops;
  double bytes;
  float ms;
} talos_prof_record;
int talos_plan_profiler(talos_plan plan, talos_profiler* prof);
int talos_profiler_enable(talos_profiler prof, int enable, const char* kernel_filter);
/* Copies up to max_records records (waiting for their events); *count = records held. */
int talos_profiler_read(talos_profiler prof, talos_prof_record* out, int max_records, int* count);

#ifdef __cplusplus
}
#endif

#endif /* TALOS_HIP_H */
