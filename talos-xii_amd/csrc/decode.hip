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
// layer: V [env][head][cap][dv] and K [env][head][cap][dk] (layered step) or
// [env][head][dk / 4][cap][4] (one-launch step), so a head's rows are contiguous; one length and
// ring start per environment serve every layer. Positions whose RoPE table entry lies past
// max_seq_len are not rotated, as the reference's inference path skips them
// (src/transformer.rs:718-721).
//
// Two implementations of the step, chosen when the decoder is created:
//  * the one-launch step (decode_fused_kernel) for the shapes it is instantiated for: every
//    phase of the step in one kernel, 16 environments per workgroup;
//  * the layered step (decode_step) for any configuration: the projections as GEMMs over the n
//    environments' rows (M = n) and the cached attention as one wave per (environment, head),
//    which rotates the new q / k, stores k / v into the ring and attends over the ring.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <type_traits>
#include <vector>

#include "gemm.hpp"
#include "plans.hpp"
#include "rowops.hpp"
#include "rowtile.hpp"

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
  // the one-launch step (small policies): chosen at creation, with its LDS layout in floats
  // the one-launch step applies (chosen at creation); its caches hold latent and k_rope rows
  bool fused = false;
  size_t k_layer = 0, v_layer = 0;  // floats per layer of kc / vc
  const float* params = nullptr;     // the last step's parameters (read_cache expands latent rows)
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
__device__ void sample_action(const float* z, int A, float u, int32_t* action, float* logp) {
  double mx = -1e9;
  for (int i = 0; i < A; ++i) mx = fmax(mx, (double)z[i]);
  double sum = 0.0;
  for (int i = 0; i < A; ++i) sum += exp((double)z[i] - mx);
  double r = (double)u;
  int act = 0;
  for (int i = 0; i < A; ++i) {
    const double p = exp((double)z[i] - mx) / sum;
    if (r < p) {
      act = i;
      break;
    }
    r -= p;
  }
  if (action) *action = act;
  if (logp) *logp = (float)log(exp((double)z[act] - mx) / sum);
}
__global__ void decode_sample_kernel(int n, int A, const float* __restrict__ logits, const float* __restrict__ u,
                                     int32_t* __restrict__ actions, float* __restrict__ logp) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= n) return;
  sample_action(logits + (long long)e * A, A, u[e], actions ? actions + e : nullptr, logp ? logp + e : nullptr);
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

// ---- The one-launch step --------------------------------------------------------------------
// For the shapes it is instantiated for (the reference ActorCritic's, FusedShape below) and
// windows up to kFusedMaxWindow, the whole step is one kernel: a workgroup of four waves owns 16
// environments, keeps their activations in LDS through every layer and reads each weight once per
// workgroup from L2. The products run on the fp32 matrix cores with the 16 environments as the
// rows of one 16x16 tile; every dimension is a compile-time constant, so a lane issues all of its
// weight loads before the first product. The phases are those of the layered path (decode_step
// below), in the same order, separated by workgroup barriers instead of launches.
constexpr int kFusedMaxWindow = 16;  // the staged rows of 16 environments fit in LDS
constexpr int kFusedEnvs = kRowTileRows;  // the rows of a v_mfma_f32_16x16x4f32 tile
#ifndef TALOS_FUSED_WAVES
#define TALOS_FUSED_WAVES 8
#endif
constexpr int kFusedThreads = 64 * TALOS_FUSED_WAVES;  // two waves a SIMD hide each other's latency
typedef rt_gptr gptr_t;
typedef rt_lptr lptr_t;

template <int IN_, int D_, int H_, int HD_, int R_, int VD_, int LT_, int F_, int A_, bool MLA_>
struct FusedShape {
  static constexpr int IN = IN_, D = D_, H = H_, HD = HD_, R = R_, VD = VD_, LT = LT_, F = F_, A = A_;
  static constexpr bool MLA = MLA_;
  static constexpr int DK = MLA ? HD + R : HD, DV = MLA ? VD : HD;
  static constexpr int ROPE_OFF = MLA ? HD : 0, ROPE = MLA ? R : HD;
};
// ActorCritic::new (src/ppo.rs:254-258): in_dim 8, d 64, MLA with 4 heads (content 16, rope 16,
// value 16, latent 32), ffn 128, 5 actions
using RefActorCritic = FusedShape<8, 64, 4, 16, 16, 16, 32, 128, 5, true>;

template <class SH>
bool fused_shape_matches(const talos_ppo_cfg& c) {
  const bool mla = c.attention == TALOS_ATTN_MLA;
  return mla == SH::MLA && c.in_dim == SH::IN && c.d_model == SH::D && c.n_heads == SH::H &&
         c.head_dim == SH::HD && c.ffn_dim == SH::F && c.n_actions == SH::A &&
         (!mla || (c.rope_dim == SH::R && c.v_dim == SH::VD && c.kv_latent == SH::LT));
}

struct FusedArgs {
  int n, layers, cap, window, max_pos, relu;
  float eps, scale;
  const float* P;
  const float *tokens, *u;
  const int32_t* pos;
  const uint8_t* reset;
  float *logits, *values, *logp;
  int32_t* actions;
  int32_t *len, *head;
  float *kc, *vc;                // layer-major caches
  long long kc_layer, vc_layer;  // floats per layer
  const float *rcos, *rsin;
  // parameter offsets: embedding and heads; layer 0's block and the stride between layers
  long long we, be, gf, wout, bout, wa, ba, wc, bc, lstride;
  long long g1, g2, w1, b1, w2, b2, wo, wqkv, wdkv, wuk, wuv, wq, wkr, wqr;
};

// The row-tile products and norms of rowtile.hpp with this kernel's wave count.
template <int K, int N, int LDW, bool TRANS = false>
using FmmW = RowTileW<K, N, LDW, TRANS, kFusedThreads / 64>;
template <int K, int N, int LDX, int LDW, bool TRANS, class Out>
__device__ __forceinline__ void fmm_run(const float* X, const FmmW<K, N, LDW, TRANS>& wt, Out out) {
  rowtile_mm<K, N, LDX>(X, wt, out);
}
template <int D>
using NormG = RowGain<D>;
template <int D, int LD>
__device__ __forceinline__ void fnorm(const float* x, float* y, float eps, const NormG<D>& gn) {
  row_norm<D, LD>(x, y, eps, gn);
}

// The step of one workgroup. MLA attention runs in its absorbed form: the cache holds, per layer,
// environment and slot, the latent row c = x.W_dkv ([LT]) and the rotated k_rope rows of every
// head ([H][R]) instead of the per-head K and V of the reference (k_h = [c.W_uk_h | k_rope_h],
// v_h = c.W_uv_h, src/transformer.rs:706-781), which halves the bytes a step reads:
//   score_h(j) = (W_uk_h q_c_h) . c_j + q_rope_h . k_rope_h(j),
//   o_h = (sum_j p_h(j) c_j) . W_uv_h.
// Both are slot-minor, [env][LT / 4][cap] and [env][H][R / 4][cap] of float4, so a workgroup's
// rows are one contiguous block of each, copied into LDS with direct-to-LDS loads
// (global_load_lds_dwordx4) issued a phase or more before the attention: at the start for layer
// 0, after the previous layer's attention for the others.
template <class SH>
__global__ __launch_bounds__(kFusedThreads) void decode_fused_kernel(FusedArgs a) {
  static_assert(SH::MLA, "the one-launch step is instantiated for latent attention");
  constexpr int T = kFusedThreads, E = kFusedEnvs;
  constexpr int D = SH::D, H = SH::H, DK = SH::DK, DV = SH::DV, F = SH::F, A = SH::A, IN = SH::IN;
  constexpr int HD = SH::HD, R = SH::R, LT = SH::LT;
  constexpr int LDD = D + 4, LDQ = H * DK + 4, LDV = H * DV + 4, LDF = F + 4, LDI = IN + 4, LDC = LT + 4;
  constexpr int LDR = H * R + 4, LDA = H * LT + 4;
  constexpr int CAPM = kFusedMaxWindow + 1, NC4 = LT / 4, NR4 = R / 4;
  constexpr int CF4 = E * NC4 * CAPM, KF4 = E * H * NR4 * CAPM;  // float4s of the staged rows
  static_assert(CF4 % 64 == 0 && KF4 % 64 == 0, "whole wave copies");
  static_assert(LT % 16 == 0 && R % 4 == 0 && HD % 4 == 0 && LDA >= LDD, "layout");
  __shared__ __align__(16) float x[E * LDD], xn[E * LDD], qh[E * (LDQ > LDF ? LDQ : LDF)], qa[E * LDA];
  __shared__ __align__(16) float kr[E * LDR], ckv[E * LDC], o[E * LDV], tok[E * LDI], lg[E * A];
  __shared__ float pr[E * H * CAPM], inv[E * H];
  __shared__ __align__(16) float sc_c[CF4 * 4], sc_k[KF4 * 4];  // the held latent / k_rope rows
  __shared__ int slen[E], shead[E], spos[E];
  float* q = qh;     // [q_c | q_rope] per head
  float* hid = qh;   // the FFN rows reuse q's (dead after the attention) with stride LDF
  float* ctx = qa;   // sum_j p_h(j) c_j reuses W_uk_h q_c_h's rows (dead after the scores)
  float* pout = qa;  // the out_proj rows, with stride LDD
  const int env0 = blockIdx.x * E, tid = threadIdx.x, cap = a.cap, n_on = min(E, a.n - env0);
  const float* P = a.P;
  // copy the workgroup's held rows of layer l into sc_c / sc_k: the blocks are contiguous
  // (n_on * NC4 * cap and n_on * H * NR4 * cap float4s); a wave instruction fills 64 consecutive
  // float4s of LDS, a lane past the block re-reads the block's last float4 (in bounds)
  auto stage = [&](int l) {
    const int wave = tid >> 6, lane = tid & 63;
    const float4* gc = reinterpret_cast<const float4*>(a.kc + l * a.kc_layer) + (long long)env0 * NC4 * cap;
    const float4* gk = reinterpret_cast<const float4*>(a.vc + l * a.vc_layer) + (long long)env0 * H * NR4 * cap;
    const int nc = n_on * NC4 * cap, nk = n_on * H * NR4 * cap;
    for (int i = wave; i * 64 < nc; i += T / 64)
      __builtin_amdgcn_global_load_lds((gptr_t)(gc + min(i * 64 + lane, nc - 1)), (lptr_t)(sc_c + i * 256), 16, 0, 0);
    for (int i = wave; i * 64 < nk; i += T / 64)
      __builtin_amdgcn_global_load_lds((gptr_t)(gk + min(i * 64 + lane, nk - 1)), (lptr_t)(sc_k + i * 256), 16, 0, 0);
  };
  stage(0);
  if (tid < E) {
    const int e = env0 + tid;
    const bool on = e < a.n;
    int l = on ? a.len[e] : -1, h = on ? a.head[e] : 0;
    if (on && a.reset && a.reset[e]) {
      l = 0;
      h = 0;
    }
    slen[tid] = l;  // -1 marks an environment past n
    shead[tid] = h;
    spos[tid] = on ? a.pos[e] : -1;
  }
  for (int idx = tid; idx < E * IN; idx += T) {
    const int e = idx / IN, c = idx % IN;
    tok[e * LDI + c] = env0 + e < a.n ? a.tokens[(long long)(env0 + e) * IN + c] : 0.f;
  }
  // the first phases' weights and gains, in flight during the set-up
  FmmW<IN, D, D> w_emb;
  w_emb.load(P + a.we, P + a.be);
  NormG<D> gn;
  gn.load(P + a.g1);
  lds_barrier();
  // this thread's RoPE items (environment, head, pair) and their factors, reused by every layer;
  // positions outside the table are not rotated (src/transformer.rs:718-721)
  constexpr int HALF = R / 2, NROT = E * H * HALF, ROT_PER = (NROT + T - 1) / T;
  float rc[ROT_PER], rs[ROT_PER];
  bool rot[ROT_PER];
#pragma unroll
  for (int t = 0; t < ROT_PER; ++t) {
    const int idx = tid + t * T, e = idx / (H * HALF), m = idx % HALF;
    const int p = idx < NROT ? spos[e] : -1;
    rot[t] = p >= 0 && p < a.max_pos;
    rc[t] = rot[t] ? a.rcos[p * HALF + m] : 1.f;
    rs[t] = rot[t] ? a.rsin[p * HALF + m] : 0.f;
  }
  // the layer's products from x_norm: down-projection, q_c, q_rope, k_rope
  FmmW<D, LT, LT> w_dkv;
  FmmW<D, H * HD, H * HD> w_q;
  FmmW<D, H * R, H * R> w_qr, w_kr;
  auto load_in = [&](const float* B) {
    // tiles spread over the waves: q 0-3, q_rope 6,7,0,1, k_rope 2-5, W_dkv 4,5 (of 8)
    w_dkv.load(B + a.wdkv, nullptr, 4);
    w_q.load(B + a.wq, nullptr);
    w_qr.load(B + a.wqr, nullptr, 6);
    w_kr.load(B + a.wkr, nullptr, 2);
  };
  load_in(P);
  fmm_run<IN, D, LDI>(tok, w_emb, [&](int e, int n, float s) { x[e * LDD + n] = s; });
  lds_barrier();
  for (int l = 0; l < a.layers; ++l) {
    const float* B = P + l * a.lstride;
    // W_uk_h^T per head (q_c_h -> the latent space) and W_uv_h per head
    FmmW<HD, LT, H * HD, true> w_uk[H];
    FmmW<LT, DV, H * DV> w_uv[H];
#pragma unroll
    for (int h = 0; h < H; ++h) w_uk[h].load(B + a.wuk + h * HD, nullptr, 2 * h);
    fnorm<D, LDD>(x, xn, a.eps, gn);
    lds_barrier();
    fmm_run<D, LT, LDD>(xn, w_dkv, [&](int e, int n, float s) { ckv[e * LDC + n] = s; });
    fmm_run<D, H * HD, LDD>(xn, w_q, [&](int e, int n, float s) { q[e * LDQ + (n / HD) * DK + n % HD] = s; });
    fmm_run<D, H * R, LDD>(xn, w_qr, [&](int e, int n, float s) { q[e * LDQ + (n / R) * DK + HD + n % R] = s; });
    fmm_run<D, H * R, LDD>(xn, w_kr, [&](int e, int n, float s) { kr[e * LDR + n] = s; });
    lds_barrier();
#pragma unroll
    for (int h = 0; h < H; ++h) w_uv[h].load(B + a.wuv + h * DV, nullptr, 2 * h);
    // RoPE on the new q_rope / k_rope rows: (x0, x1) -> (x0 c - x1 s, x0 s + x1 c),
    // src/transformer.rs:724-733
#pragma unroll
    for (int t = 0; t < ROT_PER; ++t) {
      const int idx = tid + t * T;
      if (idx < NROT && rot[t]) {
        const int e = idx / (H * HALF), h = (idx / HALF) % H, m = idx % HALF;
        const int aq = e * LDQ + h * DK + HD + 2 * m, ak = e * LDR + h * R + 2 * m;
        const float q0 = q[aq], q1 = q[aq + 1], k0 = kr[ak], k1 = kr[ak + 1];
        q[aq] = fmaf(q0, rc[t], -q1 * rs[t]);
        q[aq + 1] = fmaf(q0, rs[t], q1 * rc[t]);
        kr[ak] = fmaf(k0, rc[t], -k1 * rs[t]);
        kr[ak + 1] = fmaf(k0, rs[t], k1 * rc[t]);
      }
    }
    // q_c_h -> W_uk_h q_c_h in the latent space (two tiles a head)
#pragma unroll
    for (int h = 0; h < H; ++h)
      fmm_run<HD, LT, LDQ>(q + h * DK, w_uk[h], [&](int e, int n, float s) { qa[e * LDA + h * LT + n] = s; });
    __builtin_amdgcn_s_waitcnt(kVmcnt0);  // this wave's row copies have landed in LDS
    lds_barrier();
    float* cc = a.kc + l * a.kc_layer;  // [env][LT / 4][cap] of float4
    float* kk = a.vc + l * a.vc_layer;  // [env][H][R / 4][cap] of float4
    // the new latent and k_rope rows into the ring slot after the held rows
    for (int idx = tid; idx < E * (NC4 + H * NR4); idx += T) {
      const int e = idx / (NC4 + H * NR4), c = idx % (NC4 + H * NR4);
      if (slen[e] < 0) continue;
      const int slot = (shead[e] + slen[e]) % cap;
      if (c < NC4)
        *reinterpret_cast<float4*>(cc + (((long long)(env0 + e) * NC4 + c) * cap + slot) * 4) =
            *reinterpret_cast<const float4*>(ckv + e * LDC + 4 * c);
      else
        *reinterpret_cast<float4*>(kk + (((long long)(env0 + e) * H * NR4 + (c - NC4)) * cap + slot) * 4) =
            *reinterpret_cast<const float4*>(kr + e * LDR + 4 * (c - NC4));
    }
    // scores of the held rows from LDS: a lane per (environment, head, slot), slot fastest, so a
    // wave's lanes read consecutive float4s of each quarter-row plane. A slot outside the held
    // rows (empty, or the new row's) is dropped.
    // (unrolled over the lane's items so their LDS reads are in flight together; the quotient
    // i / cap is taken in fp32 from (i + 0.5) / cap: i < 2^16 and cap <= 17 leave the rounding
    // error far below the 0.5 / cap margin)
    const float rcap = 1.0f / (float)cap;
#pragma unroll
    for (int it = 0; it < (E * H * CAPM + T - 1) / T; ++it) {
      const int i = tid + it * T;
      if (i >= n_on * H * cap) continue;
      const int eh = (int)(((float)i + 0.5f) * rcap), slot = i - eh * cap, e = eh / H, h = eh - e * H;
      const int hd0 = shead[e], j = slot - hd0 + (slot < hd0 ? cap : 0);
      if (j >= slen[e]) continue;
      const float4* cr = reinterpret_cast<const float4*>(sc_c) + e * NC4 * cap + slot;
      const float4* kq = reinterpret_cast<const float4*>(sc_k) + eh * NR4 * cap + slot;
      const float* qar = qa + e * LDA + h * LT;
      const float* qrr = q + e * LDQ + h * DK + HD;
      float sc = 0.f;
#pragma unroll
      for (int c = 0; c < NC4; ++c) {
        const float4 q4 = *reinterpret_cast<const float4*>(qar + 4 * c), c4 = cr[c * cap];
        sc = fmaf(q4.x, c4.x, sc);
        sc = fmaf(q4.y, c4.y, sc);
        sc = fmaf(q4.z, c4.z, sc);
        sc = fmaf(q4.w, c4.w, sc);
      }
#pragma unroll
      for (int c = 0; c < NR4; ++c) {
        const float4 q4 = *reinterpret_cast<const float4*>(qrr + 4 * c), k4 = kq[c * cap];
        sc = fmaf(q4.x, k4.x, sc);
        sc = fmaf(q4.y, k4.y, sc);
        sc = fmaf(q4.z, k4.z, sc);
        sc = fmaf(q4.w, k4.w, sc);
      }
      pr[eh * CAPM + j] = sc * a.scale;
    }
    // the new row's score, from LDS
    for (int idx = tid; idx < E * H; idx += T) {
      const int e = idx / H, h = idx % H;
      if (slen[e] < 0) continue;
      float sc = 0.f;
#pragma unroll
      for (int i = 0; i < LT; ++i) sc = fmaf(qa[e * LDA + h * LT + i], ckv[e * LDC + i], sc);
#pragma unroll
      for (int i = 0; i < R; ++i) sc = fmaf(q[e * LDQ + h * DK + HD + i], kr[e * LDR + h * R + i], sc);
      pr[idx * CAPM + slen[e]] = sc * a.scale;
    }
    lds_barrier();
    FmmW<H * DV, D, D> w_o;
    w_o.load(B + a.wo, nullptr);
    for (int idx = tid; idx < E * H; idx += T) {
      const int rows = slen[idx / H] + 1;
      float* p = pr + idx * CAPM;
      float sv[CAPM];
      float mx = -INFINITY, sum = 0.f;
#pragma unroll
      for (int j = 0; j < CAPM; ++j) {
        sv[j] = j < rows ? p[j] : -INFINITY;
        mx = fmaxf(mx, sv[j]);
      }
#pragma unroll
      for (int j = 0; j < CAPM; ++j) {
        if (j < rows) {
          const float ex = __expf(sv[j] - mx);
          p[j] = ex;
          sum += ex;
        }
      }
      inv[idx] = rows > 0 ? 1.f / sum : 0.f;
    }
    lds_barrier();
    // ctx_h = sum_j p_h(j) c_j from LDS: a lane per (environment, head, 4 latent columns)
    for (int idx = tid; idx < E * H * NC4; idx += T) {
      const int e = idx / (H * NC4), h = (idx / NC4) % H, c = idx % NC4;
      const int rows = slen[e] + 1, hd0 = shead[e];
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      if (rows > 0) {
        const float* p = pr + (e * H + h) * CAPM;
        const float4* cb = reinterpret_cast<const float4*>(sc_c) + (e * NC4 + c) * cap;
#pragma unroll
        for (int j = 0; j < kFusedMaxWindow; ++j) {
          if (j < rows - 1) {
            const int s = hd0 + j, slot = s - (s >= cap ? cap : 0);
            const float4 cv = cb[slot];
            const float pj = p[j];
            acc.x = fmaf(pj, cv.x, acc.x);
            acc.y = fmaf(pj, cv.y, acc.y);
            acc.z = fmaf(pj, cv.z, acc.z);
            acc.w = fmaf(pj, cv.w, acc.w);
          }
        }
        const float pl = p[rows - 1], iv = inv[e * H + h];
        const float4 cn = *reinterpret_cast<const float4*>(ckv + e * LDC + 4 * c);
        acc.x = fmaf(pl, cn.x, acc.x) * iv;
        acc.y = fmaf(pl, cn.y, acc.y) * iv;
        acc.z = fmaf(pl, cn.z, acc.z) * iv;
        acc.w = fmaf(pl, cn.w, acc.w) * iv;
      }
      *reinterpret_cast<float4*>(ctx + e * LDA + h * LT + 4 * c) = acc;
    }
    lds_barrier();
    if (l + 1 < a.layers) stage(l + 1);  // the staged rows are free: the next layer's copies fly
    // o_h = ctx_h . W_uv_h, a head per wave
#pragma unroll
    for (int h = 0; h < H; ++h)
      fmm_run<LT, DV, LDA>(ctx + h * LT, w_uv[h], [&](int e, int n, float s) { o[e * LDV + h * DV + n] = s; });
    lds_barrier();
    // h2 = x + o.Wo
    gn.load(B + a.g2);
    fmm_run<H * DV, D, LDV>(o, w_o, [&](int e, int n, float s) { x[e * LDD + n] = s + x[e * LDD + n]; });
    lds_barrier();
    FmmW<D, F, F> w_1;
    w_1.load(B + a.w1, B + a.b1);
    fnorm<D, LDD>(x, xn, a.eps, gn);
    lds_barrier();
    FmmW<F, D, D> w_2;
    w_2.load(B + a.w2, B + a.b2);
    const bool relu = a.relu;
    fmm_run<D, F, LDD>(xn, w_1, [&](int e, int n, float s) { hid[e * LDF + n] = relu ? fmaxf(s, 0.f) : gelu_f(s); });
    lds_barrier();
    // x = h2 + act(.).W2 + b2; the next layer's (or the final) gains and input products in flight
    const bool more = l + 1 < a.layers;
    gn.load(more ? B + a.lstride + a.g1 : P + a.gf);
    if (more) load_in(B + a.lstride);
    fmm_run<F, D, LDF>(hid, w_2, [&](int e, int n, float s) { x[e * LDD + n] = s + x[e * LDD + n]; });
    lds_barrier();
  }
  FmmW<D, D, D> w_out;
  w_out.load(P + a.wout, P + a.bout);
  fnorm<D, LDD>(x, xn, a.eps, gn);
  lds_barrier();
  FmmW<D, A, A> w_a;
  FmmW<D, 1, 1> w_c;
  w_a.load(P + a.wa, P + a.ba);
  if (a.values) w_c.load(P + a.wc, P + a.bc, 1);
  fmm_run<D, D, LDD>(xn, w_out, [&](int e, int n, float s) { pout[e * LDD + n] = s; });
  lds_barrier();
  {
    float* logits = a.logits;
    float* values = a.values;
    const int n_env = a.n;
    fmm_run<D, A, LDD>(pout, w_a, [&](int e, int n, float s) {
      lg[e * A + n] = s;
      if (logits && env0 + e < n_env) logits[(long long)(env0 + e) * A + n] = s;
    });
    if (values)
      fmm_run<D, 1, LDD>(pout, w_c, [&](int e, int n, float s) {
        if (env0 + e < n_env) values[env0 + e] = s;
      });
  }
  lds_barrier();
  if (tid < E && env0 + tid < a.n) {
    const int e = env0 + tid;
    if (a.actions || a.logp)
      sample_action(lg + tid * A, A, a.u[e], a.actions ? a.actions + e : nullptr, a.logp ? a.logp + e : nullptr);
    // the new row is held, then the oldest dropped past the window
    const int l = slen[tid] + 1;
    if (l > a.window) {
      a.head[e] = (shead[tid] + 1) % cap;
      a.len[e] = a.window;
    } else {
      a.head[e] = shead[tid];
      a.len[e] = l;
    }
  }
}

// The one-launch step applies: an instantiated shape and a window within kFusedMaxWindow.
bool fused_applies(const talos_ppo_cfg& c, int window) {
  return window <= kFusedMaxWindow && fused_shape_matches<RefActorCritic>(c);
}

int decode_step_fused(talos_decoder_s* D, int n, const float* P, const float* tokens, const int32_t* pos,
                      const uint8_t* reset, const float* uniforms, float* logits, float* values, int32_t* actions,
                      float* logp, hipStream_t s) {
  using SH = RefActorCritic;
  const talos_ppo_cfg& c = D->cfg;
  talos_block_cfg bc = D->bc;
  bc.batch = n;
  bc.seq = 1;
  const PpoOff po = ppo_offsets(c);
  const BlockOff b0 = block_offsets(bc, po.blocks);
  FusedArgs a{};
  a.n = n;
  a.layers = c.n_layers;
  a.cap = D->cap;
  a.window = D->window;
  a.max_pos = D->max_seq_len;
  a.relu = c.activation == TALOS_ACT_RELU;
  a.eps = c.eps;
  a.scale = (float)(1.0 / std::sqrt((double)D->dk));
  a.P = P;
  a.tokens = tokens;
  a.u = uniforms;
  a.pos = pos;
  a.reset = reset;
  a.logits = logits;
  a.values = values;
  a.logp = logp;
  a.actions = actions;
  a.len = D->len;
  a.head = D->head;
  a.kc = D->kc[0];
  a.vc = D->vc[0];
  a.kc_layer = (long long)D->k_layer;
  a.vc_layer = (long long)D->v_layer;
  a.rcos = D->rcos;
  a.rsin = D->rsin;
  a.we = po.we;
  a.be = po.be;
  a.gf = po.gf;
  a.wout = po.wout;
  a.bout = po.bout;
  a.wa = po.wa;
  a.ba = po.ba;
  a.wc = po.wc;
  a.bc = po.bc;
  a.lstride = (long long)(b0.end - po.blocks);
  a.g1 = b0.g1;
  a.g2 = b0.g2;
  a.w1 = b0.w1;
  a.b1 = b0.b1;
  a.w2 = b0.w2;
  a.b2 = b0.b2;
  a.wo = b0.wo;
  a.wqkv = b0.wqkv;
  a.wdkv = b0.mla.wdkv;
  a.wuk = b0.mla.wuk;
  a.wuv = b0.mla.wuv;
  a.wq = b0.mla.wq;
  a.wkr = b0.mla.wkr;
  a.wqr = b0.mla.wqr;
  const double d = SH::D, F = SH::F, H = SH::H, A = SH::A;
  const double attn_macs = SH::MLA ? d * SH::LT + SH::LT * H * (SH::HD + SH::DV) + d * H * (SH::HD + 2.0 * SH::R)
                                   : 3.0 * d * d;
  const double macs = SH::IN * d + c.n_layers * (attn_macs + H * SH::DV * d + 2.0 * d * F) + d * d + d * (A + 1);
  // algorithmic bytes: the held latent and k_rope rows read and the new rows written (every
  // layer), the weights once, tokens and positions in, logits / value / action / log-prob out
  const double cache = 4.0 * n * c.n_layers * (double)a.cap * (SH::LT + H * SH::R);
  ProfScope ps(s, "decode_fused_kernel", 2.0 * n * macs, cache + 4.0 * po.end + 4.0 * n * (SH::IN + A + 5));
  hipLaunchKernelGGL((decode_fused_kernel<SH>), dim3(ceil_div((size_t)n, kFusedEnvs)), dim3(kFusedThreads), 0, s,
                     a);
  TALOS_LAUNCHED("decode_fused_kernel");
  return TALOS_OK;
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
  // the one-launch step where its limits allow; TALOS_DECODER_LAYERED=1 keeps the layered path
  const char* layered = std::getenv("TALOS_DECODER_LAYERED");
  D->fused = fused_applies(c, context_len) && !(layered && layered[0] == '1');
  const size_t n = (size_t)n_envs, d = c.d_model, F = c.ffn_dim, H = c.n_heads;
  int rc = 0;
  {  // one layer-major block each for K and V (layered), or the latent and k_rope rows (one-launch)
    D->k_layer = D->fused ? n * cap * c.kv_latent : n * H * cap * dk;
    D->v_layer = D->fused ? n * cap * H * c.rope_dim : n * H * cap * dv;
    float *k = nullptr, *v = nullptr;
    rc |= dec_alloc_n(D, &k, (size_t)c.n_layers * D->k_layer);
    rc |= dec_alloc_n(D, &v, (size_t)c.n_layers * D->v_layer);
    for (int l = 0; rc == TALOS_OK && l < c.n_layers; ++l) {
      D->kc.push_back(k + (size_t)l * D->k_layer);
      D->vc.push_back(v + (size_t)l * D->v_layer);
    }
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
  dec->params = params;
  const hipStream_t s = as_stream(stream);
  const int rc = dec->fused
                     ? decode_step_fused(dec, n, params, tokens, positions, reset, uniforms, logits, values, actions, logp, s)
                     : decode_step(dec, n, params, tokens, positions, reset, uniforms, logits, values, actions, logp, s);
  return entry_done(rc, s);
}

int talos_ppo_decoder_read_cache(talos_decoder dec, int layer, int env, float* k, float* v, int* len) {
  TALOS_REQUIRE(dec != nullptr, TALOS_ERR_HANDLE, "%s: null decoder", __func__);
  TALOS_REQUIRE(layer >= 0 && layer < dec->cfg.n_layers && env >= 0 && env < dec->n_envs, TALOS_ERR_SHAPE,
                "%s: layer %d / env %d out of range", __func__, layer, env);
  TALOS_NONNULL(len);
  TALOS_DEVICE();
  TALOS_HIP(hipDeviceSynchronize());
  int32_t L = 0, hd0 = 0;
  TALOS_HIP(hipMemcpy(&L, dec->len + env, 4, hipMemcpyDeviceToHost));
  TALOS_HIP(hipMemcpy(&hd0, dec->head + env, 4, hipMemcpyDeviceToHost));
  *len = L;
  const int H = dec->cfg.n_heads, cap = dec->cap, dk = dec->dk, dv = dec->dv;
  if (dec->fused) {
    // latent rows c [LT / 4][slot][4] and k_rope rows [H][R / 4][slot][4] (slot-minor):
    // k_h = [c.W_uk_h | k_rope_h], v_h = c.W_uv_h with the last step's weights
    const talos_ppo_cfg& c = dec->cfg;
    const int Lt = c.kv_latent, R = c.rope_dim, hd = c.head_dim, vd = c.v_dim;
    std::vector<float> cr((size_t)cap * Lt), kr((size_t)cap * H * R);
    TALOS_HIP(hipMemcpy(cr.data(), dec->kc[layer] + (size_t)env * cap * Lt, cr.size() * 4, hipMemcpyDeviceToHost));
    TALOS_HIP(hipMemcpy(kr.data(), dec->vc[layer] + (size_t)env * cap * H * R, kr.size() * 4, hipMemcpyDeviceToHost));
    if (L == 0) return TALOS_OK;
    TALOS_REQUIRE(dec->params != nullptr, TALOS_ERR_HANDLE, "%s: no step has run", __func__);
    talos_block_cfg bc = dec->bc;
    bc.batch = 1;
    bc.seq = 1;
    size_t base = ppo_offsets(c).blocks;
    for (int l = 0; l < layer; ++l) base = block_offsets(bc, base).end;
    const MlaW w = block_offsets(bc, base).mla;
    std::vector<float> wuk((size_t)Lt * H * hd), wuv((size_t)Lt * H * vd);
    TALOS_HIP(hipMemcpy(wuk.data(), dec->params + w.wuk, wuk.size() * 4, hipMemcpyDeviceToHost));
    TALOS_HIP(hipMemcpy(wuv.data(), dec->params + w.wuv, wuv.size() * 4, hipMemcpyDeviceToHost));
    std::vector<float> cj(Lt);
    for (int j = 0; j < L; ++j) {
      const int slot = (hd0 + j) % cap;
      for (int t = 0; t < Lt; ++t) cj[t] = cr[((size_t)(t / 4) * cap + slot) * 4 + t % 4];
      for (int h = 0; h < H; ++h) {
        if (k) {
          float* kj = k + ((size_t)j * H + h) * dk;
          for (int i = 0; i < hd; ++i) {
            double sum = 0.0;
            for (int t = 0; t < Lt; ++t) sum += (double)cj[t] * wuk[(size_t)t * H * hd + h * hd + i];
            kj[i] = (float)sum;
          }
          for (int i = 0; i < R; ++i) kj[hd + i] = kr[(((size_t)h * (R / 4) + i / 4) * cap + slot) * 4 + i % 4];
        }
        if (v) {
          float* vj = v + ((size_t)j * H + h) * dv;
          for (int i = 0; i < vd; ++i) {
            double sum = 0.0;
            for (int t = 0; t < Lt; ++t) sum += (double)cj[t] * wuv[(size_t)t * H * vd + h * vd + i];
            vj[i] = (float)sum;
          }
        }
      }
    }
    return TALOS_OK;
  }
  std::vector<float> kr((size_t)H * cap * dk), vr((size_t)H * cap * dv);
  TALOS_HIP(hipMemcpy(kr.data(), dec->kc[layer] + (size_t)env * H * cap * dk, kr.size() * 4, hipMemcpyDeviceToHost));
  TALOS_HIP(hipMemcpy(vr.data(), dec->vc[layer] + (size_t)env * H * cap * dv, vr.size() * 4, hipMemcpyDeviceToHost));
  for (int j = 0; j < L; ++j) {
    const int slot = (hd0 + j) % cap;
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
