// decode.hip -- rollout inference with the KV cache for many environments at once: one token per
// environment per call through the policy (LuckTransformer::forward_inference_step,
// src/transformer.rs:157-196; MultiHeadLatentAttention::forward_inference_cached, :688-805), the
// cache pruned to the context window after the step (prune_kv_cache, :807-840, called after every
// pull, src/sim.rs:578), and the action drawn as ActorCritic::step_inference_cached does
// (src/ppo.rs:391-433) with the caller's uniform draws.
//
// Each environment's cache is a ring of cap = window + 1 rows per layer and head: a step attends
// over the rows held plus the new token (at most window + 1), then the oldest row is dropped when
// more than window remain, as the reference appends first and prunes afterwards. Layout per
// layer: K [env][head][cap][dk], V [env][head][cap][dv], so a head's rows are contiguous; one
// length and ring start per environment serve every layer.
//
// The projections run as GEMMs over the n environments' rows (M = n); the cached attention is
// one wave per (environment, head): it rotates the new q / k at the environment's position,
// stores k / v into the ring and attends over the ring. Positions whose RoPE table entry lies
// past max_seq_len are not rotated, as the reference's inference path skips them
// (src/transformer.rs:718-721).
#include <algorithm>
#include <cmath>
#include <vector>

#include "gemm.hpp"
#include "plans.hpp"
#include "rowops.hpp"

struct talos_decoder_s {
  talos_ppo_cfg cfg{};
  talos_block_cfg bc{};
  int n_envs = 0, window = 0, cap = 0, max_seq_len = 0;
  int dk = 0, dv = 0, ow = 0;
  std::vector<void*> allocs;
  float *rcos = nullptr, *rsin = nullptr;
  std::vector<float*> kc, vc;  // per layer ring caches
  int32_t *len = nullptr, *head = nullptr;
  // activations over the n_envs rows
  float *x = nullptr, *y = nullptr, *xn = nullptr, *rstd = nullptr, *qkv = nullptr, *ckv = nullptr, *kcn = nullptr,
        *vn = nullptr, *qc = nullptr, *qr = nullptr, *kr = nullptr, *o = nullptr, *h2 = nullptr, *a = nullptr,
        *pout = nullptr, *logits = nullptr, *values = nullptr;
};

namespace talos {
namespace {

constexpr int kMaxWindow = 1023;  // ring rows <= 1024: the scores of one wave fit in LDS
constexpr int kDecodeWaves = 4;   // waves per 256-thread workgroup

int dec_alloc(talos_decoder_s* D, void** out, size_t bytes) {
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes ? bytes : 4);
  if (e != hipSuccess) {
    set_error("decoder allocation of %zu bytes failed: %s", bytes, hipGetErrorString(e));
    return TALOS_ERR_ALLOC;
  }
  D->allocs.push_back(p);
  *out = p;
  return TALOS_OK;
}
template <typename T>
int dec_alloc_n(talos_decoder_s* D, T** out, size_t n) {
  return dec_alloc(D, reinterpret_cast<void**>(out), n * sizeof(T));
}

void dec_free(talos_decoder_s* D) {
  for (void* p : D->allocs) (void)hipFree(p);
  D->allocs.clear();
}

struct DecAttnArgs {
  int n, H, a, b, dk, dv, cap, rope_off, rope_dim, max_pos;
  float scale;
  // q / k per head = [part a | part b]; part b may be empty (b = 0)
  const float *qa, *qb, *ka, *kb, *v;
  long long ldqa, ldqb, ldka, ldkb, ldv;
  const float *rcos, *rsin;
  const int32_t* pos;
  const int32_t* len;
  const int32_t* head;
  float* kcache;
  float* vcache;
  float* o;  // [n, H * dv]
};

// Element i of the (rotated) per-head vector [pa | pb] of one token.
__device__ __forceinline__ float head_elem(const float* pa, const float* pb, int a, int i) {
  return i < a ? pa[i] : pb[i - a];
}
__device__ __forceinline__ float rotated(const float* pa, const float* pb, int a, int i, const DecAttnArgs& g,
                                         int pos) {
  const float x = head_elem(pa, pb, a, i);
  const int rel = i - g.rope_off;
  if (rel < 0 || rel >= g.rope_dim || pos < 0 || pos >= g.max_pos) return x;
  const int half = g.rope_dim >> 1, m = rel >> 1;
  const float c = g.rcos[pos * half + m], s = g.rsin[pos * half + m];
  const int i0 = g.rope_off + 2 * m;
  const float x0 = head_elem(pa, pb, a, i0), x1 = head_elem(pa, pb, a, i0 + 1);
  // (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), src/transformer.rs:724-733
  return (rel & 1) ? fmaf(x0, s, x1 * c) : fmaf(x0, c, -x1 * s);
}

__global__ __launch_bounds__(256) void decode_attn_kernel(DecAttnArgs g) {
  __shared__ float s_q[kDecodeWaves][128], s_k[kDecodeWaves][128], s_v[kDecodeWaves][128];
  __shared__ float s_p[kDecodeWaves][kMaxWindow + 1];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int item = blockIdx.x * kDecodeWaves + wv;
  const bool active = item < g.n * g.H;  // every wave reaches every barrier
  const int e = active ? item / g.H : 0, h = active ? item % g.H : 0;
  int rows = 0, slot_new = 0;
  if (active) {
    const int pos = g.pos[e];
    const float* qa = g.qa + (long long)e * g.ldqa + (long long)h * g.a;
    const float* qb = g.qb + (long long)e * g.ldqb + (long long)h * g.b;
    const float* ka = g.ka + (long long)e * g.ldka + (long long)h * g.a;
    const float* kb = g.kb + (long long)e * g.ldkb + (long long)h * g.b;
    const float* vv = g.v + (long long)e * g.ldv + (long long)h * g.dv;
    const int L = g.len[e], hd0 = g.head[e];
    rows = L + 1;
    slot_new = (hd0 + L) % g.cap;
    float* krow = g.kcache + (((long long)e * g.H + h) * g.cap + slot_new) * g.dk;
    float* vrow = g.vcache + (((long long)e * g.H + h) * g.cap + slot_new) * g.dv;
    for (int i = lane; i < g.dk; i += 64) {
      s_q[wv][i] = rotated(qa, qb, g.a, i, g, pos);
      const float kv = rotated(ka, kb, g.a, i, g, pos);
      s_k[wv][i] = kv;
      krow[i] = kv;
    }
    for (int i = lane; i < g.dv; i += 64) {
      s_v[wv][i] = vv[i];
      vrow[i] = vv[i];
    }
  }
  __syncthreads();
  float mx = -INFINITY;
  if (active) {
    const int hd0 = g.head[e];
    const float* kbase = g.kcache + ((long long)e * g.H + h) * g.cap * g.dk;
    for (int j = lane; j < rows; j += 64) {
      float sc = 0.f;
      if (j == rows - 1) {  // the new row, from LDS
        for (int i = 0; i < g.dk; ++i) sc = fmaf(s_q[wv][i], s_k[wv][i], sc);
      } else {
        const float4* kr = reinterpret_cast<const float4*>(kbase + (long long)((hd0 + j) % g.cap) * g.dk);
        for (int i = 0; i < (g.dk >> 2); ++i) {
          const float4 k4 = kr[i];
          sc = fmaf(s_q[wv][4 * i], k4.x, sc);
          sc = fmaf(s_q[wv][4 * i + 1], k4.y, sc);
          sc = fmaf(s_q[wv][4 * i + 2], k4.z, sc);
          sc = fmaf(s_q[wv][4 * i + 3], k4.w, sc);
        }
      }
      sc *= g.scale;
      s_p[wv][j] = sc;
      mx = fmaxf(mx, sc);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  }
  __syncthreads();
  float sum = 0.f;
  if (active) {
    for (int j = lane; j < rows; j += 64) {
      const float p = __expf(s_p[wv][j] - mx);
      s_p[wv][j] = p;
      sum += p;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
  }
  __syncthreads();
  if (active) {
    const int hd0 = g.head[e];
    const float inv = 1.f / sum;
    const float* vbase = g.vcache + ((long long)e * g.H + h) * g.cap * g.dv;
    for (int i = lane; i < g.dv; i += 64) {
      float acc = 0.f;
      for (int j = 0; j < rows - 1; ++j) acc = fmaf(s_p[wv][j], vbase[(long long)((hd0 + j) % g.cap) * g.dv + i], acc);
      acc = fmaf(s_p[wv][rows - 1], s_v[wv][i], acc);
      g.o[(long long)e * g.H * g.dv + (long long)h * g.dv + i] = acc * inv;
    }
  }
}

// Cache bookkeeping of one environment per thread.
__global__ void decode_reset_kernel(int n, const uint8_t* __restrict__ reset, int32_t* __restrict__ len,
                                    int32_t* __restrict__ head) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n && reset[e]) {
    len[e] = 0;
    head[e] = 0;
  }
}
// After the step: the new row is held, then the oldest row dropped past the window.
__global__ void decode_advance_kernel(int n, int window, int cap, int32_t* __restrict__ len,
                                      int32_t* __restrict__ head) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const int l = len[e] + 1;
  if (l > window) {
    head[e] = (head[e] + 1) % cap;
    len[e] = window;
  } else {
    len[e] = l;
  }
}

// Probabilities in f64 with the reference's max start of -1e9, the first action whose
// probability exceeds the remaining draw (0 when none does: the reference's index starts at 0 and
// its ACTION_SPACE fallback never fires), ln p of the action (src/ppo.rs:401-432).
__global__ void decode_sample_kernel(int n, int A, const float* __restrict__ logits, const float* __restrict__ u,
                                     int32_t* __restrict__ actions, float* __restrict__ logp) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  const float* z = logits + (long long)e * A;
  double mx = -1e9;
  for (int i = 0; i < A; ++i) mx = fmax(mx, (double)z[i]);
  double sum = 0.0;
  for (int i = 0; i < A; ++i) sum += exp((double)z[i] - mx);
  double r = (double)u[e];
  int act = 0;
  for (int i = 0; i < A; ++i) {
    const double p = exp((double)z[i] - mx) / sum;
    if (r < p) {
      act = i;
      break;
    }
    r -= p;
  }
  if (actions) actions[e] = act;
  if (logp) logp[e] = (float)log(exp((double)z[act] - mx) / sum);
}

int dmm(hipStream_t s, int M, int N, int K, const float* A, long long lda, const float* B, long long ldb, float* C,
        long long ldc, const float* bias = nullptr, const float* resid = nullptr, long long ldr = 0,
        int act = GEMM_ACT_NONE) {
  GemmDesc g;
  g.M = M;
  g.N = N;
  g.K = K;
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.C = C;
  g.ldc = ldc;
  g.bias = bias;
  g.resid = resid;
  g.ldr = ldr;
  g.act = act;
  g.ksplit = 1;
  return gemm_launch(g, s);
}

int decode_step(talos_decoder_s* D, int n, const float* P, const float* tokens, const int32_t* pos,
                const uint8_t* reset, const float* uniforms, float* logits, float* values, int32_t* actions,
                float* logp, hipStream_t s) {
  const talos_ppo_cfg& c = D->cfg;
  talos_block_cfg bc = D->bc;
  bc.batch = n;
  bc.seq = 1;
  const PpoOff po = ppo_offsets(c);
  const int d = c.d_model, F = c.ffn_dim, H = c.n_heads, A = c.n_actions;
  const bool mla = c.attention == TALOS_ATTN_MLA;
  const unsigned eblocks = (unsigned)ceil_div((size_t)n, 256);
  int rc;
  if (reset) {
    hipLaunchKernelGGL(decode_reset_kernel, dim3(eblocks), dim3(256), 0, s, n, reset, D->len, D->head);
    TALOS_LAUNCHED("decode_reset_kernel");
  }
  if ((rc = dmm(s, n, d, c.in_dim, tokens, c.in_dim, P + po.we, d, D->x, d, P + po.be))) return rc;
  float *x = D->x, *y = D->y;
  size_t base = po.blocks;
  for (int l = 0; l < c.n_layers; ++l) {
    const BlockOff bo = block_offsets(bc, base);
    base = bo.end;
    if ((rc = rmsnorm_fwd_launch(n, d, c.eps, x, P + bo.g1, D->xn, D->rstd, s))) return rc;
    DecAttnArgs g{};
    g.n = n;
    g.H = H;
    g.dk = D->dk;
    g.dv = D->dv;
    g.cap = D->cap;
    g.max_pos = D->max_seq_len;
    g.scale = (float)(1.0 / std::sqrt((double)D->dk));
    g.rcos = D->rcos;
    g.rsin = D->rsin;
    g.pos = pos;
    g.len = D->len;
    g.head = D->head;
    g.kcache = D->kc[l];
    g.vcache = D->vc[l];
    g.o = D->o;
    if (mla) {
      const int Lt = c.kv_latent, r = c.rope_dim, hd = c.head_dim, vd = c.v_dim;
      const MlaW& w = bo.mla;
      if ((rc = dmm(s, n, Lt, d, D->xn, d, P + w.wdkv, Lt, D->ckv, Lt))) return rc;
      if ((rc = dmm(s, n, H * hd, Lt, D->ckv, Lt, P + w.wuk, H * hd, D->kcn, H * hd))) return rc;
      if ((rc = dmm(s, n, H * vd, Lt, D->ckv, Lt, P + w.wuv, H * vd, D->vn, H * vd))) return rc;
      if ((rc = dmm(s, n, H * hd, d, D->xn, d, P + w.wq, H * hd, D->qc, H * hd))) return rc;
      if ((rc = dmm(s, n, H * r, d, D->xn, d, P + w.wqr, H * r, D->qr, H * r))) return rc;
      if ((rc = dmm(s, n, H * r, d, D->xn, d, P + w.wkr, H * r, D->kr, H * r))) return rc;
      g.a = hd;
      g.b = r;
      g.qa = D->qc;
      g.ldqa = (long long)H * hd;
      g.qb = D->qr;
      g.ldqb = (long long)H * r;
      g.ka = D->kcn;
      g.ldka = (long long)H * hd;
      g.kb = D->kr;
      g.ldkb = (long long)H * r;
      g.v = D->vn;
      g.ldv = (long long)H * vd;
      g.rope_off = hd;
      g.rope_dim = r;
    } else {
      const int hd = c.head_dim;
      if ((rc = dmm(s, n, 3 * d, d, D->xn, d, P + bo.wqkv, 3 * d, D->qkv, 3 * d))) return rc;
      g.a = hd;
      g.b = 0;
      g.qa = D->qkv;
      g.ldqa = 3LL * d;
      g.qb = D->qkv;
      g.ldqb = 3LL * d;
      g.ka = D->qkv + d;
      g.ldka = 3LL * d;
      g.kb = D->qkv + d;
      g.ldkb = 3LL * d;
      g.v = D->qkv + 2 * d;
      g.ldv = 3LL * d;
      g.rope_off = 0;
      g.rope_dim = hd;
    }
    {
      // algorithmic bytes: the cached rows of K and V read, the new rows written, q / o
      ProfScope ps(s, "decode_attn_kernel", 4.0 * n * H * (double)D->cap * (D->dk + D->dv),
                   4.0 * n * H * ((double)D->cap * (D->dk + D->dv) + 2.0 * D->dk + 2.0 * D->dv));
      const unsigned blocks = (unsigned)ceil_div((size_t)n * H, kDecodeWaves);
      hipLaunchKernelGGL(decode_attn_kernel, dim3(blocks), dim3(64 * kDecodeWaves), 0, s, g);
      TALOS_LAUNCHED("decode_attn_kernel");
    }
    // h2 = x + o.Wo; out = h2 + act(rmsnorm(h2).W1 + b1).W2 + b2
    if ((rc = dmm(s, n, d, D->ow, D->o, D->ow, P + bo.wo, d, D->h2, d, nullptr, x, d))) return rc;
    if ((rc = rmsnorm_fwd_launch(n, d, c.eps, D->h2, P + bo.g2, D->xn, D->rstd, s))) return rc;
    if ((rc = dmm(s, n, F, d, D->xn, d, P + bo.w1, F, D->a, F, P + bo.b1, nullptr, 0,
                  c.activation == TALOS_ACT_GELU ? GEMM_ACT_GELU : GEMM_ACT_RELU)))
      return rc;
    if ((rc = dmm(s, n, d, F, D->a, F, P + bo.w2, d, y, d, P + bo.b2, D->h2, d))) return rc;
    std::swap(x, y);
  }
  hipLaunchKernelGGL(decode_advance_kernel, dim3(eblocks), dim3(256), 0, s, n, D->window, D->cap, D->len, D->head);
  TALOS_LAUNCHED("decode_advance_kernel");
  // final norm, out_proj, heads
  if ((rc = rmsnorm_fwd_launch(n, d, c.eps, x, P + po.gf, D->xn, D->rstd, s))) return rc;
  if ((rc = dmm(s, n, d, d, D->xn, d, P + po.wout, d, D->pout, d, P + po.bout))) return rc;
  float* lg = logits ? logits : D->logits;
  if ((rc = dmm(s, n, A, d, D->pout, d, P + po.wa, A, lg, A, P + po.ba))) return rc;
  if (values && (rc = dmm(s, n, 1, d, D->pout, d, P + po.wc, 1, values, 1, P + po.bc))) return rc;
  if (actions || logp) {
    hipLaunchKernelGGL(decode_sample_kernel, dim3(eblocks), dim3(256), 0, s, n, A, lg, uniforms, actions, logp);
    TALOS_LAUNCHED("decode_sample_kernel");
  }
  return TALOS_OK;
}

}  // namespace
}  // namespace talos

using namespace talos;

extern "C" {

int talos_ppo_decoder_create(const talos_ppo_cfg* cfg, int n_envs, int context_len, int max_seq_len,
                             talos_decoder* dec) {
  TALOS_NONNULL(cfg);
  TALOS_NONNULL(dec);
  *dec = nullptr;
  talos_ppo_cfg c = *cfg;
  // the architecture is checked as a one-token batch
  c.batch = 1;
  c.seq = 1;
  if (int rc = check_ppo_cfg(c)) return rc;
  TALOS_REQUIRE(n_envs >= 1, TALOS_ERR_SHAPE, "%s: n_envs=%d < 1", __func__, n_envs);
  TALOS_REQUIRE(context_len >= 1 && context_len <= kMaxWindow, TALOS_ERR_UNSUPPORTED,
                "%s: context_len=%d outside [1, %d]", __func__, context_len, kMaxWindow);
  TALOS_REQUIRE(max_seq_len >= 0, TALOS_ERR_SHAPE, "%s: max_seq_len=%d < 0", __func__, max_seq_len);
  const talos_block_cfg bc = block_cfg_of(c);
  const bool mla = c.attention == TALOS_ATTN_MLA;
  const int dk = mla ? c.head_dim + c.rope_dim : c.head_dim, dv = mla ? c.v_dim : c.head_dim;
  TALOS_REQUIRE(dk % 4 == 0 && dk <= 128 && dv <= 128, TALOS_ERR_UNSUPPORTED,
                "%s: head widths dk=%d (multiple of 4, <= 128) and dv=%d (<= 128)", __func__, dk, dv);
  const size_t cap = (size_t)context_len + 1;
  TALOS_REQUIRE((size_t)n_envs * c.n_heads * cap * 128 < (1ULL << 40), TALOS_ERR_UNSUPPORTED,
                "%s: cache too large", __func__);
  TALOS_DEVICE();
  auto* D = new talos_decoder_s();
  D->cfg = c;
  D->bc = bc;
  D->n_envs = n_envs;
  D->window = context_len;
  D->cap = (int)cap;
  D->max_seq_len = max_seq_len > 0 ? max_seq_len : 256;
  D->dk = dk;
  D->dv = dv;
  D->ow = attn_width(bc);
  const size_t n = (size_t)n_envs, d = c.d_model, F = c.ffn_dim, H = c.n_heads;
  int rc = 0;
  for (int l = 0; l < c.n_layers; ++l) {
    float *k = nullptr, *v = nullptr;
    rc |= dec_alloc_n(D, &k, n * H * cap * dk);
    rc |= dec_alloc_n(D, &v, n * H * cap * dv);
    D->kc.push_back(k);
    D->vc.push_back(v);
  }
  rc |= dec_alloc_n(D, &D->len, n);
  rc |= dec_alloc_n(D, &D->head, n);
  for (float** b : {&D->x, &D->y, &D->xn, &D->h2, &D->pout}) rc |= dec_alloc_n(D, b, n * d);
  rc |= dec_alloc_n(D, &D->rstd, n);
  rc |= dec_alloc_n(D, &D->a, n * F);
  rc |= dec_alloc_n(D, &D->o, n * D->ow);
  rc |= dec_alloc_n(D, &D->logits, n * c.n_actions);
  rc |= dec_alloc_n(D, &D->values, n);
  if (mla) {
    rc |= dec_alloc_n(D, &D->ckv, n * c.kv_latent);
    rc |= dec_alloc_n(D, &D->kcn, n * H * c.head_dim);
    rc |= dec_alloc_n(D, &D->qc, n * H * c.head_dim);
    rc |= dec_alloc_n(D, &D->vn, n * H * c.v_dim);
    rc |= dec_alloc_n(D, &D->qr, n * H * c.rope_dim);
    rc |= dec_alloc_n(D, &D->kr, n * H * c.rope_dim);
  } else {
    rc |= dec_alloc_n(D, &D->qkv, n * 3 * d);
  }
  std::vector<float> cs, sn;
  rope_table_host(D->max_seq_len, rope_width(bc), (double)c.rope_base, cs, sn);
  rc |= dec_alloc_n(D, &D->rcos, cs.size());
  rc |= dec_alloc_n(D, &D->rsin, sn.size());
  if (rc == TALOS_OK) {
    rc = hip_status(hipMemcpy(D->rcos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    if (rc == TALOS_OK)
      rc = hip_status(hipMemcpy(D->rsin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice), "hipMemcpy");
    // every cache starts empty
    if (rc == TALOS_OK) rc = hip_status(hipMemset(D->len, 0, n * 4), "hipMemset");
    if (rc == TALOS_OK) rc = hip_status(hipMemset(D->head, 0, n * 4), "hipMemset");
  }
  if (rc) {
    dec_free(D);
    delete D;
    return rc ? rc : TALOS_ERR_ALLOC;
  }
  *dec = D;
  return TALOS_OK;
}

int talos_ppo_decoder_step_f32(talos_decoder dec, int n, const float* params, const float* tokens,
                               const int32_t* positions, const uint8_t* reset, const float* uniforms, float* logits,
                               float* values, int32_t* actions, float* logp, talos_stream_t stream) {
  TALOS_REQUIRE(dec != nullptr, TALOS_ERR_HANDLE, "%s: null decoder", __func__);
  TALOS_REQUIRE(n >= 1 && n <= dec->n_envs, TALOS_ERR_SHAPE, "%s: n=%d outside [1, %d] (the decoder's n_envs)",
                __func__, n, dec->n_envs);
  TALOS_NONNULL(params);
  TALOS_NONNULL(tokens);
  TALOS_NONNULL(positions);
  TALOS_REQUIRE(uniforms != nullptr || (actions == nullptr && logp == nullptr), TALOS_ERR_NULL,
                "%s: actions / logp need the uniform draws", __func__);
  TALOS_DEVICE();
  return decode_step(dec, n, params, tokens, positions, reset, uniforms, logits, values, actions, logp,
                     as_stream(stream));
}

int talos_ppo_decoder_read_cache(talos_decoder dec, int layer, int env, float* k, float* v, int* len) {
  TALOS_REQUIRE(dec != nullptr, TALOS_ERR_HANDLE, "%s: null decoder", __func__);
  TALOS_REQUIRE(layer >= 0 && layer < dec->cfg.n_layers && env >= 0 && env < dec->n_envs, TALOS_ERR_SHAPE,
                "%s: layer %d / env %d out of range", __func__, layer, env);
  TALOS_NONNULL(len);
  TALOS_DEVICE();
  TALOS_HIP(hipDeviceSynchronize());
  int32_t L = 0, hd = 0;
  TALOS_HIP(hipMemcpy(&L, dec->len + env, 4, hipMemcpyDeviceToHost));
  TALOS_HIP(hipMemcpy(&hd, dec->head + env, 4, hipMemcpyDeviceToHost));
  *len = L;
  const int H = dec->cfg.n_heads, cap = dec->cap, dk = dec->dk, dv = dec->dv;
  std::vector<float> kr((size_t)H * cap * dk), vr((size_t)H * cap * dv);
  TALOS_HIP(hipMemcpy(kr.data(), dec->kc[layer] + (size_t)env * H * cap * dk, kr.size() * 4, hipMemcpyDeviceToHost));
  TALOS_HIP(hipMemcpy(vr.data(), dec->vc[layer] + (size_t)env * H * cap * dv, vr.size() * 4, hipMemcpyDeviceToHost));
  for (int j = 0; j < L; ++j) {
    const int slot = (hd + j) % cap;
    for (int h = 0; h < H; ++h) {
      if (k) std::copy_n(&kr[((size_t)h * cap + slot) * dk], dk, k + ((size_t)j * H + h) * dk);
      if (v) std::copy_n(&vr[((size_t)h * cap + slot) * dv], dv, v + ((size_t)j * H + h) * dv);
    }
  }
  return TALOS_OK;
}

int talos_ppo_decoder_destroy(talos_decoder dec) {
  if (dec == nullptr) return TALOS_OK;
  TALOS_DEVICE();
  (void)hipDeviceSynchronize();
  dec_free(dec);
  delete dec;
  return TALOS_OK;
}

}  // extern "C"
