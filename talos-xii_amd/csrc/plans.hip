// plans.hip -- fused pre-norm transformer block and PPO policy forward + backward.
//
// A plan owns every device buffer one configuration needs (saved activations, gradient
// scratch, split-K partials, the RoPE table), so a training step allocates nothing.
//
// Block (talos_block_cfg; the wiring of LuckTransformer::forward, src/transformer.rs:71-90):
//   xn1 = rmsnorm(x; g1)                       rowops  (rstd saved)
//   standard attention (TALOS_ATTN_MHA):
//     qkv = xn1 . Wqkv, RoPE on the q|k columns GEMM, RoPE in the epilogue
//     o   = attention(q, k, v)                  fused attention (lse saved)
//   latent attention (TALOS_ATTN_MLA, MultiHeadLatentAttention::forward, src/transformer.rs:478-557):
//     c_kv = xn1 . W_dkv, k_c = c_kv . W_uk, v = c_kv . W_uv, q_c = xn1 . W_q,
//     q_r = xn1 . W_qr, k_r = xn1 . W_kr        GEMMs, RoPE in the q_r / k_r epilogues
//     q = [q_c | q_r], k = [k_c | k_r] per head concatenation
//     o   = attention(q, k, v), scale 1/sqrt(head_dim + rope_dim)
//   h2  = x + o . Wo                            GEMM, residual in the epilogue
//   xn2 = rmsnorm(h2; g2)
//   a   = act(xn2 . W1 + b1)                    GEMM, bias + activation epilogue; u saved: gelu' of
//                                               the pre-activation for GELU (the backward then
//                                               multiplies by it), the pre-activation for ReLU
//   out = h2 + a . W2 + b2                      GEMM, bias + residual epilogue
// and the backward in reverse, with weight gradients as split-K GEMMs (f64 partial sums) and
// the activation derivative / RoPE^T folded into the producing kernels.
//
// Policy (talos_ppo_cfg; ActorCritic, src/ppo.rs:246-307): embed Linear -> blocks -> last token
// -> RMSNorm -> out_proj -> actor / critic Linear heads -> clipped PPO loss (src/ppo.rs:691-756).
// The final RMSNorm and out_proj act on each token independently and only the last token of a
// sequence reaches the heads, so they run on the B last-token rows (same result as running them
// on all B*S tokens and gathering afterwards, as the reference does).
#include <cmath>
#include <cstdlib>
#include <vector>

#include "attention.hpp"
#include "gemm.hpp"
#include "plans.hpp"
#include "rowops.hpp"
#include "rowtile.hpp"

struct talos_plan_s {
  int kind = 0;  // 1 block, 2 ppo, 3 mla
  talos_block_cfg blk{};
  talos_ppo_cfg ppo{};
  std::vector<void*> allocs;
  // rope table [seq, rope width / 2] (the head for standard attention, rope_dim for MLA)
  float* rcos = nullptr;
  float* rsin = nullptr;
  // per layer saved activations; a latent-attention layer keeps c_kv, v and the concatenated
  // q / k in m instead of qkv
  struct MlaAct {
    float *ckv, *v, *q, *k;
  };
  struct Layer {
    float *x, *xn1, *rstd1, *qkv, *o, *lse, *h2, *xn2, *rstd2, *u, *a, *out;
    MlaAct m;
  };
  std::vector<Layer> layers;
  // backward scratch
  float *g_out = nullptr, *g_h2 = nullptr, *g_u = nullptr, *g_xn = nullptr, *g_o = nullptr, *g_qkv = nullptr,
        *g_x = nullptr;
  float* attn_ws = nullptr;
  float* gemm_ws = nullptr;
  size_t gemm_ws_bytes = 0;
  double* red_ws = nullptr;
  size_t red_ws_bytes = 0;
  // Block and PPO backward: the gain (and embedding) gradients' partial-sum combinations are held
  // back and run as one launch at the end (reduce_parts_batch_launch), each job's partials in a
  // slot of hold_ws (red_ws_bytes each) of its own until then
  double* hold_ws = nullptr;
  int hold_slots = 0, hold_next = 0;
  bool holding = false;
  std::vector<talos::PartsJob> held;
  // Block and MLA backward (one stream): the split-K weight gradients' combinations too, each
  // product's partials in a slot of hold_gws (gemm_ws_bytes each). Not the PPO plans': their
  // partials (64 MB a product at C4) would leave the Infinity Cache before the end.
  float* hold_gws = nullptr;
  int hold_gslots = 0, hold_gnext = 0;
  std::vector<talos::SplitJob> held_split;
  // The backward's side stream: weight-gradient products run there as soon as the main stream has
  // produced their operands, with their own split-K workspace, overlapping the main stream's
  // memory-bound kernels. Before the main stream overwrites a buffer such a product reads, it waits
  // for that product's event (readers); every entry point joins the side stream before returning.
  hipStream_t side = nullptr;
  float* gemm_ws2 = nullptr;
  hipEvent_t ev_fork = nullptr, ev_join = nullptr;
  struct Reader {
    const void* buf;
    hipEvent_t ev;
  };
  std::vector<Reader> readers;
  // ppo
  float *h0 = nullptr, *last = nullptr, *lastn = nullptr, *rstdf = nullptr, *pout = nullptr, *logits = nullptr,
        *values = nullptr, *g_logits = nullptr, *g_values = nullptr, *g_pout = nullptr, *g_lastn = nullptr,
        *g_last = nullptr;
  double* loss_ws = nullptr;
  // the last layer's MLP half on the last-token rows only: its inputs gathered from x and o,
  // its activations and the backward scratch, [batch, d] / [batch, F]
  struct LastRows {
    float *x, *o, *lse, *h2, *xn2, *rstd2, *u, *a, *g_u, *g_xn, *g_h2, *g_o;
    float *xn1, *q, *dq, *g_xnq;  // the last layer's query path on these rows (last-query attention)
    float *z, *uv;  // absorbed values: sum_j p_j xn1_j and Wv_h dO_h per (sample, head), [batch][H][d]
  } lr{};
  float* wpre = nullptr;  // absorbed values: the four heads' p_j^h on every row of the last layer, [M][4]
  const int32_t* lens = nullptr;  // per-sample lengths of the PPO call in progress (nullptr: all seq)
  int num_cu = 256;
  // TALOS_PLAN_UNFUSED=1 at creation: every fused alternative (row norms in GEMM epilogues, the
  // embedding + norm kernel, the fused heads, the last-row tail kernels) takes its separate-kernel
  // path instead; the same results, as the tests check at full size
  bool unfused = false;
  bool bf16 = false;  // bf16-in / fp32-accumulate GEMMs (MLA plans with TALOS_PREC_BF16)
  bool rowdot = true;  // MLA plans: the dO product forms the attention backward's D (TALOS_MLA_ROWDOT)
  talos::Profiler* prof = nullptr;
  // latent attention: the projections before concatenation and the attention gradients,
  // shared by all layers
  struct MlaScratch {
    float *dq, *dk, *dv, *dqc, *dqr, *dkc, *dkr, *dckv;
    float* ds = nullptr;  // the attention backward's dS rows (attn_bwd_ds_supported)
  } ms{};
  // bf16 MLA plans: bf16 copies of the fp32 tensors the bf16-in products read (an operand inside
  // [base, base + n) is read from copy + offset), each written by the step that writes the tensor
  // (the norm, a product's epilogue) or converted right after it (the attention's outputs and
  // gradients; the caller's weights and output gradient at the start of a call, whose bases are
  // set then)
  struct Shadow {
    const float* base;
    size_t n;
    uint16_t* copy;
  };
  std::vector<Shadow> shadows;
  uint16_t *p16 = nullptr, *g16 = nullptr;  // the copies of the caller's weights and output gradient
  talos_mla_cfg mla{};
};

namespace talos {

MlaDims mla_dims(const talos_block_cfg& c) {
  return MlaDims{c.batch, c.seq, c.d_model, c.n_heads, c.kv_latent, c.rope_dim, c.head_dim, c.v_dim, c.causal};
}
MlaDims mla_dims(const talos_mla_cfg& c) {
  return MlaDims{c.batch, c.seq, c.d_model, c.n_heads, c.kv_latent, c.rope_dim, c.head_dim, c.v_dim, c.causal};
}

MlaW mla_weights(const MlaDims& D, size_t base) {
  const size_t d = D.d, H = D.H, L = D.L, r = D.r, hd = D.hd, vd = D.vd;
  MlaW w;
  w.wdkv = base;
  w.wuk = w.wdkv + d * L;
  w.wuv = w.wuk + L * H * hd;
  w.wq = w.wuv + L * H * vd;
  w.wkr = w.wq + d * H * hd;
  w.wqr = w.wkr + d * H * r;
  w.wo = w.wqr + d * H * r;
  w.end = w.wo + H * vd * d;
  return w;
}

int attn_width(const talos_block_cfg& c) {
  return c.attention == TALOS_ATTN_MLA ? c.n_heads * c.v_dim : c.d_model;
}
int rope_width(const talos_block_cfg& c) {
  return c.attention == TALOS_ATTN_MLA ? c.rope_dim : c.head_dim;
}

BlockOff block_offsets(const talos_block_cfg& c, size_t base) {
  const size_t d = c.d_model, F = c.ffn_dim;
  BlockOff o{};
  o.g1 = base;
  if (c.attention == TALOS_ATTN_MLA) {
    o.mla = mla_weights(mla_dims(c), o.g1 + d);
    o.wo = o.mla.wo;
    o.g2 = o.mla.end;
  } else {
    o.wqkv = o.g1 + d;
    o.wo = o.wqkv + 3 * d * d;
    o.g2 = o.wo + d * d;
  }
  o.w1 = o.g2 + d;
  o.b1 = o.w1 + d * F;
  o.w2 = o.b1 + F;
  o.b2 = o.w2 + F * d;
  o.end = o.b2 + d;
  return o;
}

size_t block_params(const talos_block_cfg& c) { return block_offsets(c, 0).end; }

talos_block_cfg block_cfg_of(const talos_ppo_cfg& p) {
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

PpoOff ppo_offsets(const talos_ppo_cfg& c) {
  const size_t d = c.d_model;
  PpoOff o;
  o.we = 0;
  o.be = (size_t)c.in_dim * d;
  o.blocks = o.be + d;
  o.gf = o.blocks + (size_t)c.n_layers * block_params(block_cfg_of(c));
  o.wout = o.gf + d;
  o.bout = o.wout + d * d;
  o.wa = o.bout + d;
  o.ba = o.wa + d * (size_t)c.n_actions;
  o.wc = o.ba + c.n_actions;
  o.bc = o.wc + d;
  o.end = o.bc + 1;
  return o;
}

static size_t ppo_params(const talos_ppo_cfg& c) { return ppo_offsets(c).end; }

int check_block_cfg(const talos_block_cfg& c) {
  TALOS_REQUIRE(c.batch > 0 && c.seq > 0 && c.d_model > 0 && c.n_heads > 0 && c.head_dim > 0 && c.ffn_dim > 0,
                TALOS_ERR_SHAPE, "block cfg: sizes must be positive");
  TALOS_REQUIRE(c.attention == TALOS_ATTN_MHA || c.attention == TALOS_ATTN_MLA, TALOS_ERR_DTYPE,
                "block cfg: unknown attention %d", c.attention);
  if (c.attention == TALOS_ATTN_MHA) {
    TALOS_REQUIRE(c.n_heads * c.head_dim == c.d_model, TALOS_ERR_SHAPE,
                  "block cfg: n_heads * head_dim (%d * %d) != d_model %d", c.n_heads, c.head_dim, c.d_model);
    TALOS_REQUIRE(c.head_dim % 2 == 0, TALOS_ERR_SHAPE, "block cfg: head_dim must be even for RoPE pairs");
    TALOS_REQUIRE(c.head_dim <= 128, TALOS_ERR_UNSUPPORTED, "block cfg: head_dim %d > 128", c.head_dim);
  } else {
    TALOS_REQUIRE(c.kv_latent > 0 && c.rope_dim > 0 && c.v_dim > 0, TALOS_ERR_SHAPE,
                  "block cfg: kv_latent, rope_dim and v_dim must be positive for MLA attention");
    TALOS_REQUIRE(c.rope_dim % 2 == 0, TALOS_ERR_SHAPE, "block cfg: rope_dim must be even");
    TALOS_REQUIRE(c.head_dim + c.rope_dim <= 128 && c.v_dim <= 128, TALOS_ERR_UNSUPPORTED,
                  "block cfg: head_dim + rope_dim and v_dim must be <= 128");
    TALOS_REQUIRE(c.kv_latent % 4 == 0 && c.head_dim % 4 == 0 && c.rope_dim % 4 == 0 && c.v_dim % 4 == 0,
                  TALOS_ERR_UNSUPPORTED, "block cfg: MLA widths must be multiples of 4");
    TALOS_REQUIRE((long long)c.batch * c.seq * c.n_heads * (c.head_dim + c.rope_dim) < (1LL << 31),
                  TALOS_ERR_UNSUPPORTED, "block cfg: too many elements for 32-bit indexing");
  }
  TALOS_REQUIRE(c.causal == 0 || c.causal == 1, TALOS_ERR_DTYPE, "block cfg: causal must be 0 or 1");
  TALOS_REQUIRE(c.activation == TALOS_ACT_GELU || c.activation == TALOS_ACT_RELU, TALOS_ERR_DTYPE,
                "block cfg: unknown activation %d", c.activation);
  TALOS_REQUIRE(c.d_model % 4 == 0 && c.ffn_dim % 4 == 0, TALOS_ERR_UNSUPPORTED,
                "block cfg: d_model and ffn_dim must be multiples of 4");
  TALOS_REQUIRE(c.eps >= 0.f && c.rope_base > 0.f, TALOS_ERR_SHAPE, "block cfg: eps >= 0 and rope_base > 0 required");
  TALOS_REQUIRE((long long)c.batch * c.seq * (3LL * c.d_model) < (1LL << 31), TALOS_ERR_UNSUPPORTED,
                "block cfg: batch*seq*3*d_model must stay below 2^31 elements");
  return TALOS_OK;
}

// Whether the environment variable is set to 1 (read when a plan is created).
static bool env_flag(const char* name) {
  const char* v = std::getenv(name);
  return v && v[0] == '1' && v[1] == 0;
}

static int plan_alloc(talos_plan_s* p, float** out, size_t n) {
  void* ptr = nullptr;
  if (n == 0) n = 1;
  hipError_t e = hipMalloc(&ptr, n * sizeof(float));
  if (e != hipSuccess) {
    set_error("plan allocation of %zu floats failed: %s", n, hipGetErrorString(e));
    return TALOS_ERR_ALLOC;
  }
  p->allocs.push_back(ptr);
  *out = static_cast<float*>(ptr);
  return TALOS_OK;
}

static void plan_free(talos_plan_s* p) {
  if (p->side) {
    (void)hipStreamSynchronize(p->side);
    (void)hipStreamDestroy(p->side);
    p->side = nullptr;
  }
  for (hipEvent_t e : {p->ev_fork, p->ev_join})
    if (e) (void)hipEventDestroy(e);
  for (auto& r : p->readers) (void)hipEventDestroy(r.ev);
  p->readers.clear();
  for (void* a : p->allocs) (void)hipFree(a);
  p->allocs.clear();
  profiler_delete(p->prof);
  p->prof = nullptr;
}

// Makes the plan's profiler current on this thread for the duration of an entry point.
struct PlanCall {
  explicit PlanCall(talos_plan_s* p) { profiler_set_current(p->prof); }
  ~PlanCall() { profiler_set_current(nullptr); }
};

// Largest split-K workspace among the weight-gradient GEMMs of a configuration.
static size_t align_ws(size_t bytes) { return (bytes + 255) / 256 * 256; }
static size_t wgrad_ws(talos_plan_s* p, int M_tok, int rows, int cols) {
  GemmDesc g;
  g.transA = 1;
  g.M = rows;
  g.N = cols;
  g.K = M_tok;
  g.ksplit = 0;
  float dummy = 0.f;
  g.dbias = &dummy;  // sized with the fused bias-gradient row
  return gemm_plan_split(g, p->num_cu);
}

// A bf16 copy of n floats registered for base (nullptr: a caller's buffer, set per call).
static uint16_t* add_shadow(talos_plan_s* p, const float* base, size_t n, int* rc) {
  float* mem = nullptr;
  *rc |= plan_alloc(p, &mem, (n + 1) / 2);
  if (!mem) return nullptr;
  p->shadows.push_back({base, n, reinterpret_cast<uint16_t*>(mem)});
  return reinterpret_cast<uint16_t*>(mem);
}
static void set_shadow_base(talos_plan_s* p, const uint16_t* copy, const float* base) {
  for (auto& sh : p->shadows)
    if (sh.copy == copy) sh.base = base;
}
// The bf16 copy of the operand at ptr, or nullptr (fp32 plans keep none).
static uint16_t* shadow_of(const talos_plan_s* p, const void* ptr) {
  const float* f = static_cast<const float*>(ptr);
  for (auto& sh : p->shadows)
    if (sh.base && f >= sh.base && f < sh.base + sh.n) return sh.copy + (f - sh.base);
  return nullptr;
}
static void bf16_operands(const talos_plan_s* p, GemmDesc& g) {
  if (!p->bf16) return;
  g.A16 = shadow_of(p, g.A);
  g.B16 = shadow_of(p, g.B);
  g.C16 = shadow_of(p, g.C);
}
// bf16 copies of the registered fp32 tensors starting at each of srcs (their producers just ran)
static int refresh_shadows(talos_plan_s* p, std::initializer_list<const float*> srcs, hipStream_t s) {
  const float* src[8];
  uint16_t* dst[8];
  long long n[8];
  int k = 0;
  for (const float* f : srcs)
    for (auto& sh : p->shadows)
      if (sh.base == f && k < 8) {
        src[k] = f;
        dst[k] = sh.copy;
        n[k] = (long long)sh.n;
        ++k;
      }
  return cvt_bf16_launch(k, src, dst, n, s);
}

// The saved activations of one latent attention (c_kv, v, q, k, o, lse) and, when scratch, the
// buffers every layer shares (projections before concatenation, attention gradients).
static int alloc_mla_layer(talos_plan_s* p, const MlaDims& D, talos_plan_s::Layer& L) {
  const size_t M = (size_t)D.batch * D.seq, H = D.H, td = (size_t)D.hd + D.r;
  int rc = 0;
  rc |= plan_alloc(p, &L.m.ckv, M * D.L);
  rc |= plan_alloc(p, &L.m.v, M * H * D.vd);
  rc |= plan_alloc(p, &L.m.q, M * H * td);
  rc |= plan_alloc(p, &L.m.k, M * H * td);
  rc |= plan_alloc(p, &L.o, M * H * D.vd);
  rc |= plan_alloc(p, &L.lse, M * H);
  return rc ? TALOS_ERR_ALLOC : TALOS_OK;
}
// The largest dS buffer an MLA plan allocates: 4 GiB (B * H * S^2 entries; C5 needs 134 MB in
// fp32, seq 2048 at batch 64 and 8 heads 8.6 GB). TALOS_DS_BUDGET_MB at plan creation overrides
// it (0 turns the dS path off).
static size_t ds_budget_bytes() {
  if (const char* e = std::getenv("TALOS_DS_BUDGET_MB")) return (size_t)std::strtoull(e, nullptr, 10) << 20;
  return size_t(4) << 30;
}
static int alloc_mla_scratch(talos_plan_s* p, const MlaDims& D) {
  const size_t M = (size_t)D.batch * D.seq, H = D.H, td = (size_t)D.hd + D.r;
  auto& m = p->ms;
  int rc = 0;
  for (float** b : {&m.dqc, &m.dkc}) rc |= plan_alloc(p, b, M * H * D.hd);
  for (float** b : {&m.dqr, &m.dkr}) rc |= plan_alloc(p, b, M * H * D.r);
  for (float** b : {&m.dq, &m.dk}) rc |= plan_alloc(p, b, M * H * td);
  rc |= plan_alloc(p, &m.dv, M * H * D.vd);
  rc |= plan_alloc(p, &m.dckv, M * D.L);
  if (rc) return TALOS_ERR_ALLOC;
  {
    // the dS rows of the attention backward (B * H * S^2 entries, 2 bytes each in bf16 plans):
    // taken within ds_budget_bytes() and when the allocation succeeds; otherwise m.ds stays null,
    // and the forward and backward both take the tiled path, whose scratch is O(S)
    AttnDesc ad;
    ad.batch = D.batch;
    ad.seq = D.seq;
    ad.heads = D.H;
    ad.dk = (int)td;
    ad.dv = D.vd;
    ad.bf16 = p->bf16 ? 1 : 0;
    const size_t bytes = attn_bwd_ds_bytes(ad);
    if (!p->unfused && bytes && bytes <= ds_budget_bytes()) {
      void* ptr = nullptr;
      if (hipMalloc(&ptr, bytes) == hipSuccess) {
        p->allocs.push_back(ptr);
        m.ds = static_cast<float*>(ptr);
      } else {
        (void)hipGetLastError();  // clear the failed allocation; the plan runs without dS
      }
    }
  }
  // split-K workspace of the weight-gradient products
  for (auto rc2 : {std::make_pair(D.d, D.H * D.hd), std::make_pair(D.d, D.H * D.r), std::make_pair(D.L, D.H * D.hd),
                   std::make_pair(D.L, D.H * D.vd), std::make_pair(D.d, D.L), std::make_pair(D.H * D.vd, D.d)})
    p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, wgrad_ws(p, (int)M, rc2.first, rc2.second));
  return TALOS_OK;
}
static int upload_rope_table(talos_plan_s* p, int seq, int width, float base) {
  std::vector<float> cs, sn;
  rope_table_host(seq, width, (double)base, cs, sn);
  int rc = plan_alloc(p, &p->rcos, cs.size());
  rc |= plan_alloc(p, &p->rsin, sn.size());
  if (rc) return TALOS_ERR_ALLOC;
  TALOS_HIP(hipMemcpy(p->rcos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  TALOS_HIP(hipMemcpy(p->rsin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  return TALOS_OK;
}

static int alloc_block_buffers(talos_plan_s* p, const talos_block_cfg& c, int n_layers) {
  const size_t M = (size_t)c.batch * c.seq, d = c.d_model, F = c.ffn_dim, ow = attn_width(c);
  const bool mla = c.attention == TALOS_ATTN_MLA;
  p->layers.resize(n_layers);
  for (int l = 0; l < n_layers; ++l) {
    auto& L = p->layers[l];
    int rc = 0;
    L.x = nullptr;  // the block input, set per call (the previous layer's out, or the caller's x)
    rc |= plan_alloc(p, &L.xn1, M * d);
    rc |= plan_alloc(p, &L.rstd1, M);
    if (mla) {
      rc |= alloc_mla_layer(p, mla_dims(c), L);
    } else {
      rc |= plan_alloc(p, &L.qkv, M * 3 * d);
      rc |= plan_alloc(p, &L.o, M * d);
      rc |= plan_alloc(p, &L.lse, M * c.n_heads);
    }
    rc |= plan_alloc(p, &L.h2, M * d);
    rc |= plan_alloc(p, &L.xn2, M * d);
    rc |= plan_alloc(p, &L.rstd2, M);
    rc |= plan_alloc(p, &L.u, M * F);
    rc |= plan_alloc(p, &L.a, M * F);
    rc |= plan_alloc(p, &L.out, M * d);
    if (rc) return TALOS_ERR_ALLOC;
  }
  int rc = 0;
  rc |= plan_alloc(p, &p->g_out, M * d);
  rc |= plan_alloc(p, &p->g_h2, M * d);
  rc |= plan_alloc(p, &p->g_u, M * F);
  rc |= plan_alloc(p, &p->g_xn, M * d);
  rc |= plan_alloc(p, &p->g_o, M * ow);
  rc |= plan_alloc(p, &p->g_x, M * d);
  rc |= plan_alloc(p, &p->attn_ws, M * c.n_heads);
  if (mla)
    rc |= alloc_mla_scratch(p, mla_dims(c));
  else
    rc |= plan_alloc(p, &p->g_qkv, M * 3 * d);
  if (rc) return TALOS_ERR_ALLOC;
  size_t ws = 0;
  if (!mla)  // the Wqkv and Wo weight gradients run as one launch
    ws = std::max(ws, align_ws(wgrad_ws(p, (int)M, (int)d, 3 * (int)d)) + wgrad_ws(p, (int)M, (int)d, (int)d));
  // the MLP's two weight gradients run as one launch, each in its own part of the workspace
  ws = std::max(ws, align_ws(wgrad_ws(p, (int)M, (int)F, (int)d)) + wgrad_ws(p, (int)M, (int)d, (int)F));
  p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, ws);
  size_t red = std::max(colsum_workspace_bytes((int)M, (int)F), rmsnorm_bwd_workspace_bytes((int)M, (int)d));
  // the dgain partials of a dX product with the norm backward in its epilogue, one per 64-row tile
  red = std::max(red, reduce_parts_workspace_bytes(((int)M + 63) / 64, (int)d));
  p->red_ws_bytes = std::max(p->red_ws_bytes, red);
  return upload_rope_table(p, c.seq, rope_width(c), c.rope_base);
}

static int alloc_workspaces(talos_plan_s* p) {
  int rc = 0;
  rc |= plan_alloc(p, &p->gemm_ws, (p->gemm_ws_bytes + 3) / 4);
  float* red = nullptr;
  rc |= plan_alloc(p, &red, (p->red_ws_bytes + 3) / 4 + 2);
  p->red_ws = reinterpret_cast<double*>(red);
  if ((p->kind == 1 || p->kind == 2) && !p->unfused) {
    // two norm gains a layer (and the PPO plans' tail pair and embedding), one slot each
    p->hold_slots = p->kind == 1 ? 2 : 2 * p->ppo.n_layers + 2;
    float* hold = nullptr;
    rc |= plan_alloc(p, &hold, (size_t)p->hold_slots * ((p->red_ws_bytes + 7) / 8) * 2);
    p->hold_ws = reinterpret_cast<double*>(hold);
  }
  if ((p->kind == 1 || p->kind == 3) && !p->unfused && p->gemm_ws_bytes > 0) {
    // the block's four weight-gradient products (two launches when paired), the MLA block's seven
    p->hold_gslots = p->kind == 1 ? 4 : 8;
    rc |= plan_alloc(p, &p->hold_gws, (size_t)p->hold_gslots * (align_ws(p->gemm_ws_bytes) / sizeof(float)));
  }
  if (rc) return TALOS_ERR_ALLOC;
  // The backward's side stream, when TALOS_BWD_SIDE_STREAM=1 at plan creation. Off by default:
  // overlapping the two streams gains about 1 % of the C4 step, but then the duration of a
  // kernel (events, rocprofv3) includes the time it shares the GPU with the other stream, and
  // per-kernel rooflines stop meaning anything.
  const char* two = std::getenv("TALOS_BWD_SIDE_STREAM");
  if (!(two && two[0] == '1')) return TALOS_OK;
  if (plan_alloc(p, &p->gemm_ws2, (p->gemm_ws_bytes + 3) / 4)) return TALOS_ERR_ALLOC;
  TALOS_HIP(hipStreamCreateWithFlags(&p->side, hipStreamNonBlocking));
  TALOS_HIP(hipEventCreateWithFlags(&p->ev_fork, hipEventDisableTiming));
  TALOS_HIP(hipEventCreateWithFlags(&p->ev_join, hipEventDisableTiming));
  return TALOS_OK;
}

// The embedding gradient kernel's workgroups and input width (embed_wgrad_kernel). 512
// workgroups (two a CU, 256 rows each at C4's 131072): 16.2 us and 7.0 us for the batched
// combination, against 17.2 and 7.3 with 1024 and 17.7 and 8.2 with 2048.
constexpr int kEmbedBlocks = 512;
constexpr int kEmbedIn = 8;

// The next free slot of hold_ws while the PPO backward holds its reductions back, else nullptr.
static double* hold_slot(talos_plan_s* p) {
  if (!p->holding || !p->hold_ws || p->hold_next >= p->hold_slots) return nullptr;
  return p->hold_ws + (size_t)(p->hold_next++) * ((p->red_ws_bytes + 7) / 8);
}
// The next free split-K workspace slot while the backward holds combinations back (one stream
// only: a side stream's products would not be ordered before the flush), else nullptr.
static float* hold_gslot(talos_plan_s* p) {
  if (!p->holding || !p->hold_gws || p->side || p->hold_gnext >= p->hold_gslots) return nullptr;
  return p->hold_gws + (size_t)(p->hold_gnext++) * (align_ws(p->gemm_ws_bytes) / sizeof(float));
}
// Ends the holding when the backward returns, also on an early error return.
struct HoldScope {
  talos_plan_s* p;
  explicit HoldScope(talos_plan_s* q) : p(q) {
    p->held.clear();
    p->held_split.clear();
    p->hold_next = p->hold_gnext = 0;
    p->holding = p->hold_ws != nullptr || p->hold_gws != nullptr;
  }
  ~HoldScope() { p->holding = false; }
};
// The held-back combinations, in batches of kPartsJobsMax / kSplitJobsMax.
static int hold_flush(talos_plan_s* p, hipStream_t s) {
  int rc = TALOS_OK;
  for (size_t i = 0; i < p->held.size() && rc == TALOS_OK; i += kPartsJobsMax)
    rc = reduce_parts_batch_launch((int)std::min<size_t>(kPartsJobsMax, p->held.size() - i), p->held.data() + i, s);
  for (size_t i = 0; i < p->held_split.size() && rc == TALOS_OK; i += kSplitJobsMax)
    rc = gemm_splitk_batch_launch((int)std::min<size_t>(kSplitJobsMax, p->held_split.size() - i),
                                  p->held_split.data() + i, s);
  p->held.clear();
  p->held_split.clear();
  p->hold_next = p->hold_gnext = 0;
  return rc;
}

// GEMM helpers ---------------------------------------------------------------
static int mm_ws(talos_plan_s* p, hipStream_t s, float* wsp, int tA, int tB, int M, int N, int K, const float* A,
                 long long lda, const float* B, long long ldb, float* C, long long ldc, float beta = 0.f,
                 const float* bias = nullptr, const float* resid = nullptr, long long ldr = 0,
                 float* dbias = nullptr) {
  GemmDesc g;
  g.transA = tA;
  g.transB = tB;
  g.M = M;
  g.N = N;
  g.K = K;
  g.A = A;
  g.lda = lda;
  g.B = B;
  g.ldb = ldb;
  g.C = C;
  g.ldc = ldc;
  g.beta = beta;
  g.bias = bias;
  g.resid = resid;
  g.ldr = ldr;
  g.dbias = dbias;
  g.bf16 = p->bf16;
  bf16_operands(p, g);
  g.ksplit = 0;
  const size_t ws = gemm_plan_split(g, p->num_cu);
  // the plan sizes its split-K workspace for the weight-gradient products; any other product
  // whose split would not fit runs unsplit
  if (ws > p->gemm_ws_bytes) g.ksplit = 1;
  g.workspace = wsp;
  // a split product's combination held back where the backward collects them
  float* slot = g.ksplit > 1 && wsp == p->gemm_ws ? hold_gslot(p) : nullptr;
  SplitJob job;
  if (slot) {
    g.workspace = slot;
    g.split_defer = &job;
  }
  const int rc = gemm_launch(g, s);
  if (rc == TALOS_OK && job.part) p->held_split.push_back(job);
  return rc;
}
static int mm(talos_plan_s* p, hipStream_t s, int tA, int tB, int M, int N, int K, const float* A, long long lda,
              const float* B, long long ldb, float* C, long long ldc, float beta = 0.f, const float* bias = nullptr,
              const float* resid = nullptr, long long ldr = 0, float* dbias = nullptr) {
  return mm_ws(p, s, p->gemm_ws, tA, tB, M, N, K, A, lda, B, ldb, C, ldc, beta, bias, resid, ldr, dbias);
}

// The event recorded after the side-stream products that read buf (created on first use).
static int reader_event(talos_plan_s* p, const void* buf, hipEvent_t* ev) {
  for (auto& r : p->readers)
    if (r.buf == buf) {
      *ev = r.ev;
      return TALOS_OK;
    }
  hipEvent_t e = nullptr;
  TALOS_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  p->readers.push_back({buf, e});
  *ev = e;
  return TALOS_OK;
}

// A weight-gradient product C = A^T B (+ the bias gradient) on the side stream, ordered after
// everything issued so far on s; `reads` names the gradient buffer it reads (B, or the buffer B
// points into), which the main stream must not overwrite before the product has run.
static int wgrad(talos_plan_s* p, hipStream_t s, const void* reads, int M, int N, int K, const float* A, long long lda,
                 const float* B, long long ldb, float* C, long long ldc, float* dbias = nullptr) {
  if (!p->side) return mm(p, s, 1, 0, M, N, K, A, lda, B, ldb, C, ldc, 0.f, nullptr, nullptr, 0, dbias);
  TALOS_HIP(hipEventRecord(p->ev_fork, s));
  TALOS_HIP(hipStreamWaitEvent(p->side, p->ev_fork, 0));
  int rc = mm_ws(p, p->side, p->gemm_ws2, 1, 0, M, N, K, A, lda, B, ldb, C, ldc, 0.f, nullptr, nullptr, 0, dbias);
  if (rc) return rc;
  hipEvent_t e = nullptr;
  if ((rc = reader_event(p, reads, &e))) return rc;
  TALOS_HIP(hipEventRecord(e, p->side));
  return TALOS_OK;
}

// One weight-gradient product C = A^T B (+ the bias gradient into dbias); `reads` names the
// gradient buffer it reads (B, or the buffer B points into).
struct WgradOp {
  const void* reads;
  int M, N, K;
  const float* A;
  long long lda;
  const float* B;
  long long ldb;
  float* C;
  long long ldc;
  float* dbias;
};

// Its GemmDesc with the split-K count planned for a workspace of ws_bytes at wsp (unsplit when
// the split would not fit); *used = the workspace bytes the split takes.
static GemmDesc wgrad_desc(const talos_plan_s* p, const WgradOp& w, float* wsp, size_t ws_bytes, size_t* used) {
  GemmDesc g;
  g.transA = 1;
  g.M = w.M;
  g.N = w.N;
  g.K = w.K;
  g.A = w.A;
  g.lda = w.lda;
  g.B = w.B;
  g.ldb = w.ldb;
  g.C = w.C;
  g.ldc = w.ldc;
  g.dbias = w.dbias;
  g.bf16 = p->bf16;
  bf16_operands(p, g);
  g.ksplit = 0;
  size_t ws = gemm_plan_split(g, p->num_cu);
  if (ws > ws_bytes) {
    g.ksplit = 1;
    ws = 0;
  }
  g.workspace = wsp;
  *used = ws;
  return g;
}

// The two weight-gradient products of a block's MLP (W2 and W1, both over all tokens) as one
// launch (gemm_launch_pair: four workgroups per CU where each alone gives two), on the side stream
// when there is one; the first takes the front of the workspace, the second what follows.
// The pair's descriptors: the first at the front of the workspace base, the second after it.
static void pair_descs(const talos_plan_s* p, float* base, const WgradOp& w0, const WgradOp& w1, GemmDesc* g0,
                       GemmDesc* g1) {
  size_t u0 = 0, u1 = 0;
  *g0 = wgrad_desc(p, w0, base, p->gemm_ws_bytes, &u0);
  const size_t off = align_ws(u0);
  *g1 = wgrad_desc(p, w1, base + off / sizeof(float), off < p->gemm_ws_bytes ? p->gemm_ws_bytes - off : 0, &u1);
}

// Whether wgrad_pair would run w0 and w1 as one grid.
static bool wgrad_pairable(const talos_plan_s* p, const WgradOp& w0, const WgradOp& w1) {
  GemmDesc g0, g1;
  pair_descs(p, p->gemm_ws, w0, w1, &g0, &g1);
  return gemm_pairable(g0, g1);
}

static int wgrad_pair(talos_plan_s* p, hipStream_t s, const WgradOp& w0, const WgradOp& w1) {
  hipStream_t ls = s;
  float* base = p->gemm_ws;
  if (p->side) {
    TALOS_HIP(hipEventRecord(p->ev_fork, s));
    TALOS_HIP(hipStreamWaitEvent(p->side, p->ev_fork, 0));
    ls = p->side;
    base = p->gemm_ws2;
  }
  // (one stream: the pair's combinations held back where the backward collects them, its
  // partials in a slot of their own)
  float* slot = p->side ? nullptr : hold_gslot(p);
  if (slot) base = slot;
  GemmDesc g0, g1;
  pair_descs(p, base, w0, w1, &g0, &g1);
  SplitJob j0, j1;
  if (slot) {
    g0.split_defer = &j0;
    g1.split_defer = &j1;
  }
  int rc = gemm_launch_pair(g0, g1, ls);
  if (rc == TALOS_OK && j0.part) p->held_split.push_back(j0);
  if (rc == TALOS_OK && j1.part) p->held_split.push_back(j1);
  if (rc || !p->side) return rc;
  for (const void* buf : {w0.reads, w1.reads}) {
    hipEvent_t e = nullptr;
    if ((rc = reader_event(p, buf, &e))) return rc;
    TALOS_HIP(hipEventRecord(e, p->side));
  }
  return TALOS_OK;
}

// The main stream s waits for the side-stream products that read buf before it overwrites buf.
static int before_write(talos_plan_s* p, hipStream_t s, const void* buf) {
  for (auto& r : p->readers)
    if (r.buf == buf) TALOS_HIP(hipStreamWaitEvent(s, r.ev, 0));
  return TALOS_OK;
}

// dx = RMSNorm backward of dy = g.W^T ([M, K] x [d, K]^T, d = 128 fits one tile row) with the
// norm's input x, gain and rstd; the product's epilogue computes it (C = dy is then not written,
// else C is the scratch the separate kernels use). add: the residual gradient on every row;
// add_last / dy_last: [batch, d] added to dx / dy on the last row of each sample; pre_p / pre_u:
// dy += sum_h pre_p[row][h] pre_u[sample][h] on every row (four terms); the gain's gradient goes
// to dw.
static int norm_bwd_mm(talos_plan_s* p, hipStream_t s, int M, int d, int K, const float* g, long long ldg,
                       const float* W, long long ldw, float* C, const float* x, const float* gain, const float* rstd,
                       const float* add, const float* add_last, const float* dy_last, int seq, float* dx,
                       float* dw, const float* pre_p = nullptr, const float* pre_u = nullptr) {
  GemmDesc gd;
  gd.transB = 1;
  gd.M = M;
  gd.N = d;
  gd.K = K;
  gd.A = g;
  gd.lda = ldg;
  gd.B = W;
  gd.ldb = ldw;
  gd.C = C;
  gd.ldc = d;
  gd.ksplit = 1;
  gd.normb_x = x;
  gd.normb_gain = gain;
  gd.normb_rstd = rstd;
  gd.normb_add = add;
  gd.normb_add_last = add_last;
  gd.normb_dy_last = dy_last;
  gd.normb_pre_p = pre_p;
  gd.normb_pre_u = pre_u;
  gd.normb_seq = seq;
  gd.normb_lens = p->lens;
  gd.normb_dx = dx;
  gd.normb_dw = dw;
  // the gain gradient's combination held back where the PPO backward collects them
  double* slot = dw ? hold_slot(p) : nullptr;
  PartsJob job;
  gd.normb_ws = slot ? slot : p->red_ws;
  gd.normb_ws_bytes = p->red_ws_bytes;
  gd.normb_defer = slot ? &job : nullptr;
  gd.fuse_norm = !p->unfused;
  const int rc = gemm_launch(gd, s);
  if (rc == TALOS_OK && job.cols > 0) p->held.push_back(job);
  return rc;
}

// Everything issued on the side stream completes before anything issued later on s.
static int join_side(talos_plan_s* p, hipStream_t s) {
  if (!p->side) return TALOS_OK;
  TALOS_HIP(hipEventRecord(p->ev_join, p->side));
  TALOS_HIP(hipStreamWaitEvent(s, p->ev_join, 0));
  return TALOS_OK;
}

// Latent attention (MultiHeadLatentAttention::forward, src/transformer.rs:478-557) --------------
static AttnDesc mla_attn_desc(talos_plan_s* p, const MlaDims& D, const talos_plan_s::Layer& L) {
  const int td = D.hd + D.r;
  AttnDesc a;
  a.batch = D.batch;
  a.seq = D.seq;
  a.heads = D.H;
  a.dk = td;
  a.dv = D.vd;
  a.scale = (float)(1.0 / std::sqrt((double)td));  // src/transformer.rs:542
  a.causal = D.causal;
  a.q = L.m.q;
  a.ldq = (long long)D.H * td;
  a.k = L.m.k;
  a.ldk = (long long)D.H * td;
  a.v = L.m.v;
  a.ldv = (long long)D.H * D.vd;
  a.o = L.o;
  a.ldo = (long long)D.H * D.vd;
  a.lse = L.lse;
  a.dq = p->ms.dq;
  a.lddq = (long long)D.H * td;
  a.dk_out = p->ms.dk;
  a.lddk = (long long)D.H * td;
  a.dv_out = p->ms.dv;
  a.lddv = (long long)D.H * D.vd;
  a.rope_cos = p->rcos;
  a.rope_sin = p->rsin;
  a.rope_off = D.hd;  // the decoupled RoPE dims follow the content dims in each head
  a.rope_dim = D.r;
  a.lens = p->lens;
  a.ds = p->ms.ds;
  a.bf16 = p->bf16 ? 1 : 0;
  return a;
}

// xn -> L.o (and L.lse): the projections, RoPE on q_r / k_r, per-head concatenation, attention.
static int mla_attn_forward(talos_plan_s* p, const MlaDims& D, const float* P, const MlaW& w, const float* xn,
                            talos_plan_s::Layer& L, hipStream_t s) {
  const int M = D.batch * D.seq, d = D.d, H = D.H, Lt = D.L, r = D.r, hd = D.hd, vd = D.vd;
  int rc;
  AttnDesc a = mla_attn_desc(p, D, L);
  // the projections write each head's content and rope columns straight into the head-interleaved
  // rows of L.m.q / L.m.k ([M][H*(hd+r)], an output column map in their epilogue). (Reading the
  // content and rope parts from two buffers instead takes the attention kernels' split twins,
  // which spill 8-48 VGPRs at C5's head dims: bf16 C5 0.825 against 0.832 ms.)
  const int td = hd + r;
  // A[M][K] . B[K][N] into C, columns mapped (width cw at offset co of each td block)
  auto proj = [&](int N, int K, const float* A, const float* B, float* C, int cw, int co, bool rope) {
    GemmDesc g;
    g.M = M;
    g.N = N;
    g.K = K;
    g.A = A;
    g.lda = K;
    g.B = B;
    g.ldb = N;
    g.C = C;
    g.ldc = (long long)H * td;
    g.cmap_w = cw;
    g.cmap_pitch = td;
    g.cmap_off = co;
    if (rope) {
      g.rope_cos = p->rcos;
      g.rope_sin = p->rsin;
      g.rope_cols = N;
      g.rope_dim = r;
      g.rope_seq = D.seq;
    }
    g.ksplit = 1;
    g.bf16 = p->bf16;
    bf16_operands(p, g);
    return gemm_launch(g, s);
  };
  if ((rc = mm(p, s, 0, 0, M, Lt, d, xn, d, P + w.wdkv, Lt, L.m.ckv, Lt))) return rc;
  if ((rc = proj(H * hd, Lt, L.m.ckv, P + w.wuk, L.m.k, hd, 0, false))) return rc;
  if ((rc = mm(p, s, 0, 0, M, H * vd, Lt, L.m.ckv, Lt, P + w.wuv, H * vd, L.m.v, H * vd))) return rc;
  if ((rc = proj(H * hd, d, xn, P + w.wq, L.m.q, hd, 0, false))) return rc;
  if ((rc = proj(H * r, d, xn, P + w.wqr, L.m.q, r, hd, true))) return rc;
  if ((rc = proj(H * r, d, xn, P + w.wkr, L.m.k, r, hd, true))) return rc;
  return attn_fwd_launch(a, s);
}

// From g_o = dL/d(L.o) [tokens, H*vd]: the gradients of the six projection weights (written to
// G) and dxn = dL/dxn (overwritten).
static int mla_attn_backward(talos_plan_s* p, const MlaDims& D, const float* P, float* G, const MlaW& w,
                             const float* xn, const talos_plan_s::Layer& L, const float* g_o, float* dxn,
                             hipStream_t s, bool d_ready = false) {
  const int M = D.batch * D.seq, d = D.d, H = D.H, Lt = D.L, r = D.r, hd = D.hd, vd = D.vd;
  const size_t MH = (size_t)M * H;
  auto& m = p->ms;
  AttnDesc a = mla_attn_desc(p, D, L);
  a.dout = g_o;
  a.lddo = (long long)H * vd;
  int rc;
  bool out16 = false;
  if (attn_ds_path(a)) {
    a.d_ready = d_ready ? 1 : 0;
    // the content and rope parts of dq / dk to their own buffers
    a.dq = m.dqc;
    a.lddq = (long long)H * hd;
    a.dq2 = m.dqr;
    a.lddq2 = (long long)H * r;
    a.dk_out = m.dkc;
    a.lddk = (long long)H * hd;
    a.dk2 = m.dkr;
    a.lddk2 = (long long)H * r;
    a.dsplit = hd;
    // bf16 plans with copies: the products below read only the gradients' bf16 copies, so the
    // bf16 kernels write those instead of the fp32 tensors (the same roundings the conversion
    // launch would make)
    uint16_t* c16[5] = {shadow_of(p, m.dqc), shadow_of(p, m.dqr), shadow_of(p, m.dkc), shadow_of(p, m.dkr),
                        shadow_of(p, m.dv)};
    out16 = a.bf16 && c16[0] && c16[1] && c16[2] && c16[3] && c16[4];
    if (out16) {
      a.dq = reinterpret_cast<float*>(c16[0]);
      a.dq2 = reinterpret_cast<float*>(c16[1]);
      a.dk_out = reinterpret_cast<float*>(c16[2]);
      a.dk2 = reinterpret_cast<float*>(c16[3]);
      a.dv_out = reinterpret_cast<float*>(c16[4]);
      a.out_bf16 = 1;
    }
    if ((rc = attn_bwd_launch(a, p->attn_ws, s))) return rc;
  } else {
    if ((rc = attn_bwd_launch(a, p->attn_ws, s))) return rc;
    if ((rc = split_launch(MH, hd, r, m.dq, m.dqc, m.dqr, false, s))) return rc;
    if ((rc = split_launch(MH, hd, r, m.dk, m.dkc, m.dkr, false, s))) return rc;
  }
  // bf16 plans: the products below read the attention gradients in bf16
  if (!out16 && (rc = refresh_shadows(p, {m.dqc, m.dqr, m.dkc, m.dkr, m.dv}, s))) return rc;
  // q / rope-k projections of xn
  if ((rc = mm(p, s, 1, 0, d, H * hd, M, xn, d, m.dqc, H * hd, G + w.wq, H * hd))) return rc;
  if ((rc = mm(p, s, 1, 0, d, H * r, M, xn, d, m.dqr, H * r, G + w.wqr, H * r))) return rc;
  if ((rc = mm(p, s, 1, 0, d, H * r, M, xn, d, m.dkr, H * r, G + w.wkr, H * r))) return rc;
  if ((rc = mm(p, s, 0, 1, M, d, H * hd, m.dqc, H * hd, P + w.wq, H * hd, dxn, d))) return rc;
  if ((rc = mm(p, s, 0, 1, M, d, H * r, m.dqr, H * r, P + w.wqr, H * r, dxn, d, 1.f))) return rc;
  if ((rc = mm(p, s, 0, 1, M, d, H * r, m.dkr, H * r, P + w.wkr, H * r, dxn, d, 1.f))) return rc;
  // up projections of the latent
  if ((rc = mm(p, s, 1, 0, Lt, H * hd, M, L.m.ckv, Lt, m.dkc, H * hd, G + w.wuk, H * hd))) return rc;
  if ((rc = mm(p, s, 1, 0, Lt, H * vd, M, L.m.ckv, Lt, m.dv, H * vd, G + w.wuv, H * vd))) return rc;
  if ((rc = mm(p, s, 0, 1, M, Lt, H * hd, m.dkc, H * hd, P + w.wuk, H * hd, m.dckv, Lt))) return rc;
  if ((rc = mm(p, s, 0, 1, M, Lt, H * vd, m.dv, H * vd, P + w.wuv, H * vd, m.dckv, Lt, 1.f))) return rc;
  // down projection
  if ((rc = mm(p, s, 1, 0, d, Lt, M, xn, d, m.dckv, Lt, G + w.wdkv, Lt))) return rc;
  return mm(p, s, 0, 1, M, d, Lt, m.dckv, Lt, P + w.wdkv, Lt, dxn, d, 1.f);
}

// The block's attention over its qkv buffer (q, k, v column blocks of one [tokens, 3d] buffer).
static AttnDesc block_attn_desc(talos_plan_s* p, const talos_block_cfg& c, talos_plan_s::Layer& L) {
  const int d = c.d_model;
  AttnDesc a;
  a.batch = c.batch;
  a.seq = c.seq;
  a.heads = c.n_heads;
  a.dk = a.dv = c.head_dim;
  a.scale = (float)(1.0 / std::sqrt((double)c.head_dim));
  a.causal = c.causal;
  a.q = L.qkv;
  a.k = L.qkv + d;
  a.v = L.qkv + 2 * d;
  a.ldq = a.ldk = a.ldv = 3 * d;
  a.o = L.o;
  a.ldo = d;
  a.lse = L.lse;
  a.dq = p->g_qkv;
  a.dk_out = p->g_qkv + d;
  a.dv_out = p->g_qkv + 2 * d;
  a.lddq = a.lddk = a.lddv = 3 * d;
  a.rope_cos = p->rcos;
  a.rope_sin = p->rsin;
  a.rope_off = 0;
  a.rope_dim = c.head_dim;
  a.lens = p->lens;
  return a;
}

// A row norm to fuse into the epilogue of the product that makes its input (the next layer's
// RMSNorm1 after the MLP's output product, or layer 0's after the embedding).
struct RowNorm {
  const float* gain = nullptr;
  float* out = nullptr;
  float* rstd = nullptr;
};
static void set_norm(const talos_plan_s* p, GemmDesc& g, const RowNorm& n, float eps) {
  g.fuse_norm = !p->unfused;
  g.norm_gain = n.gain;
  g.norm_out = n.out;
  g.ldn = g.N;
  g.norm_rstd = n.rstd;
  g.norm_eps = eps;
}

// xn1 = rmsnorm(x) (unless the product that made x already wrote L.xn1: normed), qkv = xn1.Wqkv
// (RoPE in the epilogue). L.x must be set.
static int block_qkv_forward(talos_plan_s* p, const talos_block_cfg& c, const float* P, const BlockOff& o,
                             talos_plan_s::Layer& L, hipStream_t s, bool normed) {
  const int M = c.batch * c.seq, d = c.d_model;
  GemmDesc g;
  g.M = M;
  g.N = 3 * d;
  g.K = d;
  g.A = L.xn1;
  g.lda = d;
  g.B = P + o.wqkv;
  g.ldb = 3 * d;
  g.C = L.qkv;
  g.ldc = 3 * d;
  g.rope_cos = p->rcos;
  g.rope_sin = p->rsin;
  g.rope_cols = 2 * d;
  g.rope_dim = c.head_dim;
  g.rope_seq = c.seq;
  g.ksplit = 1;
  if (!normed) {
    // the product normalises x's rows itself (and writes xn1 and rstd1) where it can
    GemmDesc gn = g;
    gn.A = L.x;
    gn.nin_gain = P + o.g1;
    gn.nin_out = L.xn1;
    gn.nin_rstd = L.rstd1;
    gn.nin_eps = c.eps;
    if (!p->unfused && !p->bf16 && gemm_normin_supported(gn)) return gemm_launch(gn, s);
    if (int rc = rmsnorm_fwd_launch(M, d, c.eps, L.x, P + o.g1, L.xn1, L.rstd1, s)) return rc;
  }
  return gemm_launch(g, s);
}

// Attention half of a block's forward: o = attention(rmsnorm(x)) with lse saved.
static int block_attn_forward(talos_plan_s* p, const talos_block_cfg& c, const float* P, const BlockOff& o,
                              talos_plan_s::Layer& L, hipStream_t s, bool normed) {
  if (c.attention == TALOS_ATTN_MLA) {
    if (!normed)
      if (int rc = rmsnorm_fwd_launch(c.batch * c.seq, c.d_model, c.eps, L.x, P + o.g1, L.xn1, L.rstd1, s)) return rc;
    return mla_attn_forward(p, mla_dims(c), P, o.mla, L.xn1, L, s);
  }
  int rc = block_qkv_forward(p, c, P, o, L, s, normed);
  if (rc) return rc;
  return attn_fwd_launch(block_attn_desc(p, c, L), s);
}

// Second half over R rows (all tokens, or only the last token of each sample): h2 = x + o.Wo,
// xn2 = rmsnorm(h2) (fused into the Wo product's epilogue), u = xn2.W1 + b1, a = act(u),
// out = h2 + a.W2 + b2, followed by the next row norm when next is set.
static int block_mlp_forward(talos_plan_s* p, const talos_block_cfg& c, const float* P, const BlockOff& o, int R,
                             const float* x, const float* ob, float* h2, float* xn2, float* rstd2, float* u, float* a,
                             float* out, hipStream_t s, const RowNorm& next = RowNorm{}, bool wo_done = false) {
  const int d = c.d_model, F = c.ffn_dim, ow = attn_width(c);
  int rc;
  if (!wo_done) {  // (wo_done: the attention kernel already wrote h2, xn2 and rstd2)
    GemmDesc g;
    g.M = R;
    g.N = d;
    g.K = ow;
    g.A = ob;
    g.lda = ow;
    g.B = P + o.wo;
    g.ldb = d;
    g.C = h2;
    g.ldc = d;
    g.resid = x;
    g.ldr = d;
    g.ksplit = 1;
    set_norm(p, g, RowNorm{P + o.g2, xn2, rstd2}, c.eps);
    if ((rc = gemm_launch(g, s))) return rc;
  }
  {
    GemmDesc g;
    g.M = R;
    g.N = F;
    g.K = d;
    g.A = xn2;
    g.lda = d;
    g.B = P + o.w1;
    g.ldb = F;
    g.C = a;
    g.ldc = F;
    g.bias = P + o.b1;
    g.act = c.activation == TALOS_ACT_GELU ? GEMM_ACT_GELU : GEMM_ACT_RELU;
    g.aux = u;
    g.ldaux = F;
    g.ksplit = 1;
    rc = gemm_launch(g, s);
    if (rc) return rc;
  }
  GemmDesc g;
  g.M = R;
  g.N = d;
  g.K = F;
  g.A = a;
  g.lda = F;
  g.B = P + o.w2;
  g.ldb = d;
  g.C = out;
  g.ldc = d;
  g.bias = P + o.b2;
  g.resid = h2;
  g.ldr = d;
  g.ksplit = 1;
  if (next.out) set_norm(p, g, next, c.eps);
  return gemm_launch(g, s);
}

// Forward of one block; L.x must be set (and L.xn1 / L.rstd1 when normed). Writes L.out, and the
// next row norm of L.out when next is set.
constexpr int kWoFuseD = 128;  // the model width attn_fwd_wo_launch takes

// At S <= 64 with four 32-wide heads and d = 128 (the C3 / C4 blocks) the attention kernel also forms
// h2 = x + o.Wo and its RMSNorm (attn_fwd_wo_launch), and the MLP half starts at W1.
static int block_forward(talos_plan_s* p, const talos_block_cfg& c, const float* P, const BlockOff& o,
                         talos_plan_s::Layer& L, hipStream_t s, bool normed = false,
                         const RowNorm& next = RowNorm{}) {
  bool wo_done = false;
  int rc;
  if (c.attention == TALOS_ATTN_MHA && !p->unfused && !p->bf16 && c.d_model == kWoFuseD && attn_width(c) == kWoFuseD) {
    const AttnWoDesc wd{P + o.wo, L.x, L.h2, P + o.g2, L.xn2, L.rstd2, c.eps};
    const AttnDesc ad = block_attn_desc(p, c, L);
    if (attn_fwd_wo_supported(ad, wd)) {
      if ((rc = block_qkv_forward(p, c, P, o, L, s, normed))) return rc;
      if ((rc = attn_fwd_wo_launch(ad, wd, s))) return rc;
      wo_done = true;
    }
  }
  if (!wo_done && (rc = block_attn_forward(p, c, P, o, L, s, normed))) return rc;
  return block_mlp_forward(p, c, P, o, c.batch * c.seq, L.x, L.o, L.h2, L.xn2, L.rstd2, L.u, L.a, L.out, s, next,
                           wo_done);
}

// MLP half backward over R rows: gout = dL/dout; writes the W2 / W1 / gain2 gradients, the
// gradient of h2 (g_h2, residual included) and of o (g_o), and uses g_u, g_xn as scratch.
static int block_mlp_backward(talos_plan_s* p, const talos_block_cfg& c, const float* P, float* G, const BlockOff& o,
                              int R, const float* ob, const float* h2, const float* xn2, const float* rstd2,
                              const float* u, const float* a, const float* gout, float* g_u, float* g_xn, float* g_h2,
                              float* g_o, hipStream_t s, bool skip_go = false, bool defer_wo = false) {
  const int d = c.d_model, F = c.ffn_dim, ow = attn_width(c);
  int rc = before_write(p, s, g_u);
  if (rc) return rc;
  {
    GemmDesc g;
    g.transB = 1;
    g.M = R;
    g.N = F;
    g.K = d;
    g.A = gout;
    g.lda = d;
    g.B = P + o.w2;
    g.ldb = d;
    g.C = g_u;
    g.ldc = F;
    g.dact = c.activation == TALOS_ACT_GELU ? GEMM_DACT_GELU : GEMM_DACT_RELU;
    g.aux = const_cast<float*>(u);  // read only: the derivative epilogue
    g.ldaux = F;
    g.ksplit = 1;
    rc = gemm_launch(g, s);
    if (rc) return rc;
  }
  // the weight gradients of out = h2 + a.W2 + b2 and of u = xn2.W1 + b1, in one launch
  rc = wgrad_pair(p, s, WgradOp{gout, F, d, R, a, F, gout, d, G + o.w2, d, G + o.b2},
                  WgradOp{g_u, d, F, R, xn2, d, g_u, F, G + o.w1, F, G + o.b1});
  if (rc) return rc;
  // xn2 = rmsnorm2(h2): g_h2 = its backward of g_u.W1^T, plus the residual gradient gout
  if ((rc = before_write(p, s, g_h2))) return rc;
  rc = norm_bwd_mm(p, s, R, d, F, g_u, F, P + o.w1, F, g_xn, h2, P + o.g2, rstd2, gout, nullptr, nullptr, 1, g_h2,
                   G + o.g2);
  if (rc) return rc;
  // h2 = x + o.Wo (defer_wo: the caller launches this weight gradient together with Wqkv's)
  if (!defer_wo && (rc = wgrad(p, s, g_h2, ow, d, R, ob, ow, g_h2, d, G + o.wo, d))) return rc;
  if (skip_go) return TALOS_OK;  // the attention backward forms g_o = g_h2.Wo^T itself
  return mm(p, s, 0, 1, R, ow, d, g_h2, d, P + o.wo, d, g_o, ow);
}

// rmsnorm1's backward from p->g_xn = dL/dxn1: the gain1 gradient and dx, which also receives the
// residual gradient reaching x through h2, given on every row (g_h2) or on the last token of each
// sample only (g_h2_last, [batch, d]). dx is overwritten: the residual arrives through g_h2 or
// g_h2_last, never through dx's old contents.
static int block_norm1_backward(talos_plan_s* p, const talos_block_cfg& c, const float* P, float* G,
                                const BlockOff& o, const talos_plan_s::Layer& L, const float* g_h2,
                                const float* g_h2_last, float* dx, hipStream_t s) {
  if (int rc = before_write(p, s, dx)) return rc;
  return rmsnorm_bwd_launch(c.batch * c.seq, c.d_model, L.x, P + o.g1, L.rstd1, p->g_xn, 0.f, dx, 0.f, G + o.g1,
                            p->red_ws, s, g_h2, g_h2_last, c.seq, p->lens);
}

// Standard attention, from the qkv gradient (p->g_qkv) back to x: the Wqkv gradient, dxn1 and
// rmsnorm1's backward (block_norm1_backward).
static int block_qkv_backward(talos_plan_s* p, const talos_block_cfg& c, const float* P, float* G, const BlockOff& o,
                              talos_plan_s::Layer& L, const float* g_h2, const float* g_h2_last, float* dx,
                              hipStream_t s, const WgradOp* with = nullptr) {
  const int M = c.batch * c.seq, d = c.d_model;
  // qkv = xn1.Wqkv (with: another weight gradient over the same tokens, launched together where
  // their splits are alike, else one after the other)
  const WgradOp wqkv{p->g_qkv, d, 3 * d, M, L.xn1, d, p->g_qkv, 3 * d, G + o.wqkv, 3 * d, nullptr};
  int rc = with ? wgrad_pair(p, s, wqkv, *with)
                : wgrad(p, s, wqkv.reads, wqkv.M, wqkv.N, wqkv.K, wqkv.A, wqkv.lda, wqkv.B, wqkv.ldb, wqkv.C, wqkv.ldc);
  if (rc) return rc;
  // xn1 = rmsnorm1(x): dx = its backward of g_qkv.Wqkv^T, plus the residual gradient through h2
  if ((rc = before_write(p, s, dx))) return rc;
  return norm_bwd_mm(p, s, M, d, 3 * d, p->g_qkv, 3 * d, P + o.wqkv, 3 * d, p->g_xn, L.x, P + o.g1, L.rstd1, g_h2,
                     g_h2_last, nullptr, c.seq, dx, G + o.g1);
}

// Attention half backward over all rows: g_o = dL/do [tokens, attn_width], the residual gradient
// reaching x through h2 (g_h2 on every row, or g_h2_last on the last-token rows); writes the
// attention weights' and gain1's gradients and dx.
static int block_attn_backward(talos_plan_s* p, const talos_block_cfg& c, const float* P, float* G, const BlockOff& o,
                               talos_plan_s::Layer& L, const float* g_o, const float* g_h2, const float* g_h2_last,
                               float* dx, hipStream_t s, const WgradOp* with = nullptr) {
  if (c.attention == TALOS_ATTN_MLA) {
    int rc = mla_attn_backward(p, mla_dims(c), P, G, o.mla, L.xn1, L, g_o, p->g_xn, s);
    if (rc) return rc;
    return block_norm1_backward(p, c, P, G, o, L, g_h2, g_h2_last, dx, s);
  }
  AttnDesc a = block_attn_desc(p, c, L);
  a.dout = g_o;
  a.lddo = c.d_model;
  int rc = before_write(p, s, p->g_qkv);
  if (rc == TALOS_OK) rc = attn_bwd_launch(a, p->attn_ws, s);
  if (rc) return rc;
  return block_qkv_backward(p, c, P, G, o, L, g_h2, g_h2_last, dx, s, with);
}

// Backward of one block: gout = dL/dout (read), writes dparams slots and dx. At S <= 32 with
// four 32-wide heads and d = 128 the backward folds the input gradient of o.Wo, g_o = g_h2.Wo^T,
// into the attention backward (attn_bwd_wo_launch) instead of storing g_o and reading it back.
static int block_backward(talos_plan_s* p, const talos_block_cfg& c, const float* P, float* G, const BlockOff& o,
                          talos_plan_s::Layer& L, const float* gout, float* dx, hipStream_t s) {
  const int M = c.batch * c.seq;
  AttnDesc ad = block_attn_desc(p, c, L);
  const bool mha = c.attention == TALOS_ATTN_MHA;
  const bool fold = mha && !p->unfused && !p->bf16 && c.d_model == kWoFuseD && attn_width(c) == kWoFuseD &&
                    attn_bwd_wo_supported(ad, P + o.wo, p->g_h2);
  // standard attention: where their splits are alike (C3's 32K tokens), the Wo weight gradient
  // waits for Wqkv's and launches with it; otherwise (C4's, 771 against 512 tokens a split) it
  // runs as soon as g_h2 is ready
  const int d = c.d_model, ow = attn_width(c);
  const WgradOp wo{p->g_h2, ow, d, M, L.o, ow, p->g_h2, d, G + o.wo, d, nullptr};
  const WgradOp wqkv{p->g_qkv, d, 3 * d, M, L.xn1, d, p->g_qkv, 3 * d, G + o.wqkv, 3 * d, nullptr};
  const bool pair = mha && wgrad_pairable(p, wqkv, wo);
  int rc = block_mlp_backward(p, c, P, G, o, M, L.o, L.h2, L.xn2, L.rstd2, L.u, L.a, gout, p->g_u, p->g_xn, p->g_h2,
                              p->g_o, s, fold, pair);
  if (rc) return rc;
  if (!fold) return block_attn_backward(p, c, P, G, o, L, p->g_o, p->g_h2, nullptr, dx, s, pair ? &wo : nullptr);
  if ((rc = before_write(p, s, p->g_qkv))) return rc;
  if ((rc = attn_bwd_wo_launch(ad, P + o.wo, p->g_h2, s))) return rc;
  return block_qkv_backward(p, c, P, G, o, L, p->g_h2, nullptr, dx, s, pair ? &wo : nullptr);
}

// Whether the PPO plan's last layer runs the attention of the last query only (standard
// attention with the head shapes of the last-query kernels); otherwise it runs full attention
// and gathers the last rows.
static bool ppo_lastq(talos_plan_s* p, const talos_block_cfg& c, talos_plan_s::Layer& L) {
  return c.attention == TALOS_ATTN_MHA && attn_lastq_supported(block_attn_desc(p, c, L));
}

// Whether the last layer's last-query attention absorbs its value projection (v_j = xn1_j . Wv,
// which carries no rotation): o_h = (sum_j p_j xn1_j) . Wv_h, so the values are never formed on
// every row, their weight gradient is a product over the samples (sum_b z_bh^T dO_bh) and their
// share of dL/dxn1 rows (sum_h p_j^h Wv_h dO_h) is formed in the dX product's epilogue from the
// rows' weights p_j^h and u_h = Wv_h dO_h, added to the keys' share there.
// Four 32-wide heads, d = 128 (the kernels' shapes); the plan's buffers exist (p->wpre).
static bool ppo_vabs(talos_plan_s* p, const talos_block_cfg& c, talos_plan_s::Layer& L) {
  if (!p->wpre || !ppo_lastq(p, c, L)) return false;
  AttnDesc ad = block_attn_desc(p, c, L);
  ad.q_last = p->lr.q;
  ad.ldq_last = c.d_model;
  ad.dq_last = p->lr.dq;
  ad.lddq_last = c.d_model;
  return attn_lastq_vabs_supported(ad, L.xn1, c.d_model) != 0;
}

// o[:, h] = z[:, h] . Wv_h for the H heads of hd (one batched product; Wv_h the columns
// 2d + h hd of Wqkv) and its transpose u[:, h] = dO[:, h] . Wv_h^T.
static int vabs_out(talos_plan_s* p, int B, int d, int H, int hd, const float* z, const float* wv, long long ldw,
                    float* o, hipStream_t s) {
  GemmDesc g;
  g.M = B;
  g.N = hd;
  g.K = d;
  g.A = z;
  g.lda = (long long)H * d;
  g.sA = d;
  g.B = wv;
  g.ldb = ldw;
  g.sB = hd;
  g.C = o;
  g.ldc = (long long)H * hd;
  g.sC = hd;
  g.batch = H;
  g.ksplit = 1;
  return gemm_launch(g, s);
}
static int vabs_u(talos_plan_s* p, int B, int d, int H, int hd, const float* g_o, const float* wv, long long ldw,
                  float* u, hipStream_t s) {
  GemmDesc g;
  g.transB = 1;
  g.M = B;
  g.N = d;
  g.K = hd;
  g.A = g_o;
  g.lda = (long long)H * hd;
  g.sA = hd;
  g.B = wv;
  g.ldb = ldw;
  g.sB = hd;
  g.C = u;
  g.ldc = (long long)H * d;
  g.sC = d;
  g.batch = H;
  g.ksplit = 1;
  return gemm_launch(g, s);
}

// Last-token gather / scatter (last_row: common.hpp) -------------------------
__global__ void gather_last_kernel(int B, int S, int d, const int32_t* __restrict__ lens,
                                   const float* __restrict__ h, float* __restrict__ out) {
  const long long n = (long long)B * d;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const long long b = i / d;
    const int e = (int)(i % d);
    out[i] = h[(b * S + last_row(lens, (int)b, S)) * d + e];
  }
}
// g[M, d] = 0 except the last-token rows, which receive gl[b]
__global__ void scatter_last_kernel(int B, int S, int d, const int32_t* __restrict__ lens,
                                    const float* __restrict__ gl, float* __restrict__ g) {
  const long long n = (long long)B * S * d;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    const long long row = i / d;
    const int e = (int)(i % d);
    const int b = (int)(row / S), t = (int)(row % S);
    g[i] = t == last_row(lens, b, S) ? gl[(long long)b * d + e] : 0.f;
  }
}

// Clipped PPO loss over the minibatch (closed form of the per-sample graph of
// src/ppo.rs:702-749, mean over the batch as src/ppo.rs:754-755). One workgroup; f64 math.
// Per sample: lp = z - lse(z); ratio = exp(lp[a] - old); surr1 = ratio*adv;
// surr2 = clip(ratio, 1-eps, 1+eps)*adv; the smaller by value is kept (ties take surr2, whose
// gradient passes only inside the clip range); v = (value - ret)^2; ent = -sum p*lp;
// loss = -pol + cv*v - ce*ent. One thread per sample; each workgroup writes its sums of the loss,
// approx_kl = (ratio - 1) - log_ratio (src/ppo.rs:726-729), pol, v and ent to one partial row,
// which ppo_loss_final_kernel adds up in a fixed order.
constexpr int kLossParts = 5;
__global__ __launch_bounds__(256) void ppo_loss_kernel(int B, int A, float clip_eps, float cv, float ce,
                                                       const float* __restrict__ logits,
                                                       const float* __restrict__ values,
                                                       const int32_t* __restrict__ actions,
                                                       const float* __restrict__ adv, const float* __restrict__ ret,
                                                       const float* __restrict__ old_logp,
                                                       float* __restrict__ dlogits, float* __restrict__ dvalues,
                                                       int with_grad, double* __restrict__ part) {
  __shared__ double red[4];
  double total = 0.0, s_kl = 0.0, s_pol = 0.0, s_v = 0.0, s_ent = 0.0;
  const double invB = 1.0 / (double)B;
  for (int b = blockIdx.x * blockDim.x + threadIdx.x; b < B; b += gridDim.x * blockDim.x) {
    const float* z = logits + (long long)b * A;
    double mx = -INFINITY;
    for (int j = 0; j < A; ++j) mx = fmax(mx, (double)z[j]);
    double se = 0.0;
    for (int j = 0; j < A; ++j) se += exp((double)z[j] - mx);
    const double lse = log(se) + mx;
    double ent = 0.0;
    for (int j = 0; j < A; ++j) {
      const double lp = (double)z[j] - lse;
      ent -= exp(lp) * lp;
    }
    const int a = actions[b];
    if (a < 0 || a >= A) {
      // the reference panics on an out-of-range action (mask[action], src/ppo.rs:714-720); here
      // the loss becomes NaN and the sample contributes no gradient
      total = NAN;
      if (with_grad) {
        for (int k = 0; k < A; ++k) dlogits[(long long)b * A + k] = 0.f;
        dvalues[b] = 0.f;
      }
      continue;
    }
    const double log_ratio = ((double)z[a] - lse) - (double)old_logp[b];
    const double ratio = exp(log_ratio);
    const double ad = adv[b];
    const double lo = 1.0 - (double)clip_eps, hi = 1.0 + (double)clip_eps;
    const double s1 = ratio * ad;
    const double rc = fmin(fmax(ratio, lo), hi);
    const double s2 = rc * ad;
    double pol, gr;
    if (s1 < s2) {
      pol = s1;
      gr = ad;
    } else {
      pol = s2;
      gr = (ratio >= lo && ratio <= hi) ? ad : 0.0;
    }
    const double vd = (double)values[b] - (double)ret[b];
    total += -pol + (double)cv * vd * vd - (double)ce * ent;
    s_kl += (ratio - 1.0) - log_ratio;
    s_pol += pol;
    s_v += vd * vd;
    s_ent += ent;
    if (with_grad) {
      for (int k = 0; k < A; ++k) {
        const double lp = (double)z[k] - lse;
        const double pk = exp(lp);
        const double dk = (k == a ? 1.0 : 0.0) - pk;
        dlogits[(long long)b * A + k] = (float)((-gr * ratio * dk + (double)ce * pk * (lp + ent)) * invB);
      }
      dvalues[b] = (float)(2.0 * (double)cv * vd * invB);
    }
  }
  const double sums[kLossParts] = {block_sum(total, red), block_sum(s_kl, red), block_sum(s_pol, red),
                                   block_sum(s_v, red), block_sum(s_ent, red)};
  if (threadIdx.x == 0)
    for (int i = 0; i < kLossParts; ++i) part[(long long)blockIdx.x * kLossParts + i] = sums[i];
}

// The actor / critic heads, the clipped PPO loss and their backward in one kernel, from the
// out_proj rows pout [B, d] (the closed form above, per sample). One wave per sample at a time:
// lane k < A holds logit k = pout . Wa[:, k] + ba[k] (fp32 dot products reduced over the wave),
// the loss terms run in f64 on those lanes, and the wave then writes the out_proj row gradient
// g_pout = dz . Wa^T + dvalue . Wc^T and adds pout^T dz, dz, pout dvalue, dvalue to its share of
// the head gradients (LDS, fp32 over its samples). Each workgroup writes its partial sums (f64) of
// the loss statistics and of the head gradients, laid out as the parameters Wa | ba | Wc | bc;
// ppo_heads_final_kernel adds the workgroups up in a fixed order.
constexpr int kHeadWaves = 16;
constexpr int kHeadSamples = 16;  // samples per workgroup (1 per wave) of the fused heads kernel
// d * (A + 1) + A + 1 of the fused path: the per-wave sums of 16 waves stay within 64 KB of LDS
constexpr int kHeadMaxRow = 1008;
__global__ __launch_bounds__(64 * kHeadWaves) void ppo_heads_kernel(int B, int d, int A, float clip_eps, float cv, float ce,
                                                        const float* __restrict__ pout, const float* __restrict__ Wa,
                                                        const float* __restrict__ ba, const float* __restrict__ Wc,
                                                        const float* __restrict__ bc,
                                                        const int32_t* __restrict__ actions,
                                                        const float* __restrict__ adv, const float* __restrict__ ret,
                                                        const float* __restrict__ old_logp, float* __restrict__ g_pout,
                                                        double* __restrict__ part) {
  extern __shared__ float sh[];  // per wave: dWa [d*A] | dba [A] | dWc [d] | dbc [1]
  __shared__ double sl[kHeadWaves][kLossParts];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int R = d * (A + 1) + A + 1;
  float* acc = sh + wv * R;
  for (int i = lane; i < R; i += 64) acc[i] = 0.f;
  __syncthreads();  // zeroed by other lanes than the ones that add to each entry
  double total = 0.0, s_kl = 0.0, s_pol = 0.0, s_v = 0.0, s_ent = 0.0;
  const double invB = 1.0 / (double)B;
  const bool own = lane < A;
  const int b_end = min(B, (int)(blockIdx.x + 1) * kHeadSamples);
  for (int b = blockIdx.x * kHeadSamples + wv; b < b_end; b += kHeadWaves) {
    const float* pr = pout + (long long)b * d;
    float zk = 0.f;
    for (int k = 0; k < A; ++k) {
      float t = 0.f;
      for (int i = lane; i < d; i += 64) t += pr[i] * Wa[(long long)i * A + k];
      t = wave_sum(t);
      if (lane == k) zk = t + ba[k];
    }
    float tv = 0.f;
    for (int i = lane; i < d; i += 64) tv += pr[i] * Wc[i];
    const double value = (double)(wave_sum(tv) + bc[0]);
    // log-softmax over the A lanes, f64
    double mx = own ? (double)zk : -INFINITY;
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
    const double se = wave_sum(own ? exp((double)zk - mx) : 0.0);
    const double lse = log(se) + mx;
    const double lpk = (double)zk - lse, pk = own ? exp(lpk) : 0.0;
    const double ent = -wave_sum(own ? pk * lpk : 0.0);
    const int a = actions[b];
    double dzk = 0.0, dv = 0.0;
    if (a < 0 || a >= A) {
      // the reference panics on an out-of-range action (mask[action], src/ppo.rs:714-720); here
      // the loss becomes NaN and the sample contributes no gradient
      total = NAN;
    } else {
      const double za = __shfl(lpk, a, 64);
      const double log_ratio = za - (double)old_logp[b];
      const double ratio = exp(log_ratio);
      const double ad = adv[b];
      const double lo = 1.0 - (double)clip_eps, hi = 1.0 + (double)clip_eps;
      const double s1 = ratio * ad;
      const double s2 = fmin(fmax(ratio, lo), hi) * ad;
      double pol, gr;
      if (s1 < s2) {
        pol = s1;
        gr = ad;
      } else {
        pol = s2;
        gr = (ratio >= lo && ratio <= hi) ? ad : 0.0;
      }
      const double vd = value - (double)ret[b];
      total += -pol + (double)cv * vd * vd - (double)ce * ent;
      s_kl += (ratio - 1.0) - log_ratio;
      s_pol += pol;
      s_v += vd * vd;
      s_ent += ent;
      if (own) dzk = (-gr * ratio * ((lane == a ? 1.0 : 0.0) - pk) + (double)ce * pk * (lpk + ent)) * invB;
      dv = 2.0 * (double)cv * vd * invB;
    }
    const float dzf = (float)dzk, dvf = (float)dv;
    // g_pout and this wave's share of the head gradients
    for (int i = lane; i < d; i += 64) {
      const float x = pr[i];
      float g = dvf * Wc[i];
      for (int k = 0; k < A; ++k) {
        const float dz = __shfl(dzf, k, 64);
        g += dz * Wa[(long long)i * A + k];
        acc[i * A + k] += x * dz;
      }
      acc[d * A + A + i] += x * dvf;
      g_pout[(long long)b * d + i] = g;
    }
    if (own) acc[d * A + lane] += dzf;
    if (lane == 0) acc[R - 1] += dvf;
  }
  if (lane == 0) {
    sl[wv][0] = total;
    sl[wv][1] = s_kl;
    sl[wv][2] = s_pol;
    sl[wv][3] = s_v;
    sl[wv][4] = s_ent;
  }
  __syncthreads();
  double* P = part + (long long)blockIdx.x * (kLossParts + R);
  if (threadIdx.x < kLossParts) {
    double t = 0.0;
    for (int w = 0; w < kHeadWaves; ++w) t += sl[w][threadIdx.x];
    P[threadIdx.x] = t;
  }
  for (int i = threadIdx.x; i < R; i += blockDim.x) {
    double t = 0.0;
    for (int w = 0; w < kHeadWaves; ++w) t += (double)sh[w * R + i];
    P[kLossParts + i] = t;
  }
}

// loss[0] = mean loss, stats (optional) = (or +=) the sums of kl, pol, v, ent and the count, and
// the head gradients G[0, R) = Wa | ba | Wc | bc: each the fixed-order sum of the workgroups'
// partials. 1024 threads per workgroup: lane <-> one of 64 consecutive elements, wave w <->
// partials w, w + 16, ..., combined in LDS in wave order.
__global__ __launch_bounds__(1024) void ppo_heads_final_kernel(int nblk, int B, int R, const double* __restrict__ part,
                                                               float* __restrict__ loss, double* __restrict__ stats,
                                                               int stats_acc, float* __restrict__ G) {
  // 16 columns per workgroup: lane (column lane % 16, q = lane / 16) of wave w adds the partial
  // rows k = 4w + q + 64i into four accumulators (i % 4), then 16 threads add a column's 64 sums
  // in a fixed order
  __shared__ double red[64][16];
  const int W = kLossParts + R;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, cl = lane & 15;
  const int e = blockIdx.x * 16 + cl;
  double t0 = 0.0, t1 = 0.0, t2 = 0.0, t3 = 0.0;
  if (e < W) {
    const long long step = 64LL * W;
    int k = 4 * w + (lane >> 4);
    for (; k + 192 < nblk; k += 256) {
      const double* q = part + (long long)k * W + e;
      const double a0 = q[0], a1 = q[step], a2 = q[2 * step], a3 = q[3 * step];
      t0 += a0;
      t1 += a1;
      t2 += a2;
      t3 += a3;
    }
    for (; k < nblk; k += 64) t0 += part[(long long)k * W + e];
  }
  red[4 * w + (lane >> 4)][cl] = (t0 + t1) + (t2 + t3);
  __syncthreads();
  if (threadIdx.x >= 16 || e >= W) return;
  double sum = 0.0;
  for (int i = 0; i < 64; ++i) sum += red[i][cl];
  if (e >= kLossParts) {
    G[e - kLossParts] = (float)sum;
  } else if (e == 0) {
    if (loss) loss[0] = (float)(sum / (double)B);
    if (stats) stats[4] = (stats_acc ? stats[4] : 0.0) + (double)B;
  } else if (stats) {
    stats[e - 1] = (stats_acc ? stats[e - 1] : 0.0) + sum;
  }
}

// loss[0] = mean loss; stats (optional) = (or +=) the sums of kl, pol, v, ent and the count.
__global__ __launch_bounds__(64) void ppo_loss_final_kernel(int nblk, int B, const double* __restrict__ part,
                                                            float* __restrict__ loss, double* __restrict__ stats,
                                                            int stats_acc) {
  if (threadIdx.x != 0) return;
  double sums[kLossParts] = {0.0, 0.0, 0.0, 0.0, 0.0};
  for (int k = 0; k < nblk; ++k)
    for (int i = 0; i < kLossParts; ++i) sums[i] += part[(long long)k * kLossParts + i];
  if (loss) loss[0] = (float)(sums[0] / (double)B);
  if (stats) {
    for (int i = 0; i < 4; ++i) stats[i] = (stats_acc ? stats[i] : 0.0) + sums[i + 1];
    stats[4] = (stats_acc ? stats[4] : 0.0) + (double)B;
  }
}

int check_ppo_cfg(const talos_ppo_cfg& c) {
  TALOS_REQUIRE(c.in_dim > 0 && c.n_layers >= 0 && c.n_actions > 0, TALOS_ERR_SHAPE,
                "ppo cfg: in_dim, n_actions must be positive and n_layers >= 0");
  TALOS_REQUIRE(c.n_actions <= 64, TALOS_ERR_UNSUPPORTED, "ppo cfg: n_actions %d > 64", c.n_actions);
  TALOS_REQUIRE(c.clip_eps >= 0.f, TALOS_ERR_SHAPE, "ppo cfg: clip_eps must be >= 0");
  return check_block_cfg(block_cfg_of(c));
}

// Policy forward up to logits / values for c.batch samples (at most the plan's batch); the
// per-sample lengths of the call are p->lens.
// ---- The last layer's MLP half and the heads' inputs on the last-token rows -------------------
// With B last-token rows (one per sample) the tail of the forward (h2 = x + o.Wo, RMSNorm2,
// act(.W1 + b1), .W2 + b2 + h2, the final RMSNorm, out_proj) and the matching chain of the
// backward (out_proj's dX, the final norm's backward, dGELU / dReLU, W1's dX, RMSNorm2's backward,
// Wo's dX) are row-local: one kernel each keeps 16 rows in LDS and runs every product on the
// matrix cores (rowtile.hpp) with the weights streamed from L2, instead of a dozen launches of
// 4096-row GEMMs and row kernels that are each a few microseconds of latency. The saved
// activations and the row gradients the weight-gradient products read are written as before.
constexpr int kTailWaves = 8;
constexpr int kTailThreads = 64 * kTailWaves;

struct TailFwdArgs {
  int B, relu, seq;
  float eps;
  const int32_t* lens;
  const float* x;  // [B * seq][D]: the last layer's input, whose last-token rows are the residual
  const float* o;  // [B][D]: the attention output on the last-token rows (attention width D)
  const float *wo, *g2, *w1, *b1, *w2, *b2, *gf, *wout, *bout;
  float *h2, *xn2, *rstd2, *u, *a, *last, *lastn, *rstdf, *pout;
};

// rows of [16][LD] LDS from global [rows][D] (zeros past n rows); with seq > 0, row b is the
// last-token row b * seq + last_row(lens, b, seq) of a [B * seq][D] buffer
template <int D, int LD>
__device__ __forceinline__ void tail_rows_in(float* dst, const float* __restrict__ src, int r0, int n,
                                             const int32_t* lens = nullptr, int seq = 0) {
  for (int i = threadIdx.x; i < kRowTileRows * (D / 4); i += kTailThreads) {
    const int e = i / (D / 4), c = 4 * (i % (D / 4));
    long long row = r0 + e;
    if (seq > 0 && e < n) row = row * seq + last_row(lens, r0 + e, seq);
    const float4 v = e < n ? *reinterpret_cast<const float4*>(src + row * D + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    *reinterpret_cast<float4*>(dst + e * LD + c) = v;
  }
}
// the first n rows of [16][LD] LDS to global [rows][D]
template <int D, int LD>
__device__ __forceinline__ void tail_rows_out(float* __restrict__ dst, const float* src, int r0, int n) {
  for (int i = threadIdx.x; i < kRowTileRows * (D / 4); i += kTailThreads) {
    const int e = i / (D / 4), c = 4 * (i % (D / 4));
    if (e < n)
      *reinterpret_cast<float4*>(dst + (long long)(r0 + e) * D + c) = *reinterpret_cast<const float4*>(src + e * LD + c);
  }
}

template <int D, int F>
__global__ __launch_bounds__(kTailThreads) void ppo_tail_fwd_kernel(TailFwdArgs a) {
  constexpr int E = kRowTileRows, W = kTailWaves, LDD = D + 4, LDF = F + 4;
  __shared__ __align__(16) float sx[E * LDD], sh[E * LDD], sn[E * LDD], sa[E * LDF];
  __shared__ float srs[E];
  const int r0 = blockIdx.x * E, nr = min(E, a.B - r0);
  tail_rows_in<D, LDD>(sx, a.x, r0, nr, a.lens, a.seq);
  tail_rows_in<D, LDD>(sn, a.o, r0, nr);
  RowGain<D> gn;
  gn.load(a.g2);
  lds_barrier();
  // h2 = x + o.Wo
  rowtile_mm_stream<D, D, LDD, D, W, D, false>(sn, a.wo, nullptr, [&](int e, int n, float v) {
    sh[e * LDD + n] = v + sx[e * LDD + n];
  });
  lds_barrier();
  tail_rows_out<D, LDD>(a.h2, sh, r0, nr);
  row_norm<D, LDD>(sh, sn, a.eps, gn, srs);  // xn2
  RowGain<D> gf;
  gf.load(a.gf);
  lds_barrier();
  tail_rows_out<D, LDD>(a.xn2, sn, r0, nr);
  if (threadIdx.x < nr) a.rstd2[r0 + threadIdx.x] = srs[threadIdx.x];
  // a = act(xn2.W1 + b1); u = gelu'(.) for GELU, the pre-activation for ReLU
  const bool relu = a.relu;
  float* ga = a.a;
  float* gu = a.u;
  rowtile_mm_stream<D, F, LDD, F, W, D, false>(sn, a.w1, a.b1, [&](int e, int n, float v) {
    float act, aux;
    if (relu) {
      aux = v;
      act = fmaxf(v, 0.f);
    } else {
      act = gelu_fd(v, &aux);
    }
    sa[e * LDF + n] = act;
    if (e < nr) {
      ga[(long long)(r0 + e) * F + n] = act;
      gu[(long long)(r0 + e) * F + n] = aux;
    }
  });
  lds_barrier();
  // last = h2 + a.W2 + b2
  rowtile_mm_stream<F, D, LDF, D, W, 128, false>(sa, a.w2, a.b2, [&](int e, int n, float v) {
    sx[e * LDD + n] = v + sh[e * LDD + n];
  });
  lds_barrier();
  tail_rows_out<D, LDD>(a.last, sx, r0, nr);
  row_norm<D, LDD>(sx, sn, a.eps, gf, srs);  // the final norm
  lds_barrier();
  tail_rows_out<D, LDD>(a.lastn, sn, r0, nr);
  if (threadIdx.x < nr) a.rstdf[r0 + threadIdx.x] = srs[threadIdx.x];
  // pout = lastn.Wout + bout
  float* po = a.pout;
  rowtile_mm_stream<D, D, LDD, D, W, D, false>(sn, a.wout, a.bout, [&](int e, int n, float v) {
    if (e < nr) po[(long long)(r0 + e) * D + n] = v;
  });
}

struct TailBwdArgs {
  int B, relu;
  const float *g_pout;                 // [B][D] dL/dpout
  const float *wout, *gf, *last, *rstdf;
  const float *w2, *u, *w1, *g2, *h2, *rstd2, *wo;
  float *g_last, *g_u, *g_h2, *g_o;  // row gradients
  double* part;                      // [blocks][2D] f64 partial dgains: the final norm's, then norm2's
};

// RMSNorm backward of the 16 rows in LDS (16 lanes per row, threads 0..255): dx = rstd * (dy *
// gain - x_hat * mean(dy * gain * x_hat)) (+ add), x_hat = x * rstd; the lane's dgain terms
// dy * x_hat are summed over rows into part[c] (f64, in a fixed order) by the caller through dwl.
template <int D, int LD>
__device__ __forceinline__ void tail_norm_bwd(const float* x, const float* rstd, const RowGain<D>& gn,
                                              const float* dy, const float* add, float* dx, float* dwl, int nr) {
  constexpr int LPR = 16, PER = RowGain<D>::PER;
  if (threadIdx.x >= kRowTileRows * LPR) return;  // whole waves
  const int row = threadIdx.x / LPR, l = threadIdx.x % LPR;
  const bool on = row < nr;
  const float r = on ? rstd[row] : 0.f;
  float xh[PER], gg[PER];
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = l + j * LPR;
    xh[j] = on ? x[row * LD + c] * r : 0.f;
    gg[j] = on ? dy[row * LD + c] : 0.f;
    dot += gg[j] * gn.g[j] * xh[j];
  }
  dot = group_sum<LPR>(dot);
  const float md = dot * (1.0f / (float)D);
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = l + j * LPR;
    float v = r * (gg[j] * gn.g[j] - xh[j] * md);
    if (add) v += add[row * LD + c];
    dx[row * LD + c] = v;
    dwl[row * LD + c] = gg[j] * xh[j];
  }
}
// part[c] = sum over the 16 rows of dwl[row][c], in row order, in f64
template <int D, int LD>
__device__ __forceinline__ void tail_dgain_part(const float* dwl, double* part) {
  for (int c = threadIdx.x; c < D; c += kTailThreads) {
    double s = 0.0;
#pragma unroll
    for (int e = 0; e < kRowTileRows; ++e) s += (double)dwl[e * LD + c];
    part[c] = s;
  }
}

template <int D, int F>
__global__ __launch_bounds__(kTailThreads) void ppo_tail_bwd_kernel(TailBwdArgs a) {
  constexpr int E = kRowTileRows, W = kTailWaves, LDD = D + 4, LDF = F + 4;
  __shared__ __align__(16) float sg[E * LDD], sx[E * LDD], sy[E * LDD], sw[E * LDD], su[E * LDF];
  __shared__ float srs[E];
  const int r0 = blockIdx.x * E, nr = min(E, a.B - r0);
  tail_rows_in<D, LDD>(sg, a.g_pout, r0, nr);
  tail_rows_in<D, LDD>(sx, a.last, r0, nr);
  // u (gelu' or the pre-activation) staged in LDS now: read in the dGELU / dReLU phase from LDS
  // instead of by loads that would each wait behind the previous element's store of g_u
  tail_rows_in<F, LDF>(su, a.u, r0, nr);
  if (threadIdx.x < E) srs[threadIdx.x] = threadIdx.x < nr ? a.rstdf[r0 + threadIdx.x] : 0.f;
  RowGain<D> gf;
  gf.load(a.gf);
  lds_barrier();
  // dL/dlastn = g_pout.Wout^T
  rowtile_mm_stream<D, D, LDD, D, W, D, true>(sg, a.wout, nullptr, [&](int e, int n, float v) { sy[e * LDD + n] = v; });
  lds_barrier();
  // the final norm's backward: g_last
  tail_norm_bwd<D, LDD>(sx, srs, gf, sy, nullptr, sg, sw, nr);
  lds_barrier();
  tail_dgain_part<D, LDD>(sw, a.part + (long long)blockIdx.x * 2 * D);
  tail_rows_out<D, LDD>(a.g_last, sg, r0, nr);
  tail_rows_in<D, LDD>(sx, a.h2, r0, nr);
  if (threadIdx.x < E) srs[threadIdx.x] = threadIdx.x < nr ? a.rstd2[r0 + threadIdx.x] : 0.f;
  // g_u = (g_last.W2^T) * gelu'(u), or masked by u > 0 for ReLU
  const bool relu = a.relu;
  float* gu = a.g_u;
  rowtile_mm_stream<D, F, LDD, D, W, D, true>(sg, a.w2, nullptr, [&](int e, int n, float v) {
    const float uu = su[e * LDF + n];  // zero on rows past nr
    const float g = relu ? (uu > 0.f ? v : 0.f) : v * uu;
    if (e < nr) gu[(long long)(r0 + e) * F + n] = g;
    su[e * LDF + n] = g;
  });
  RowGain<D> g2;
  g2.load(a.g2);
  lds_barrier();
  // dL/dxn2 = g_u.W1^T
  rowtile_mm_stream<F, D, LDF, F, W, 128, true>(su, a.w1, nullptr, [&](int e, int n, float v) { sy[e * LDD + n] = v; });
  lds_barrier();
  // RMSNorm2's backward with the residual gradient g_last: g_h2
  tail_norm_bwd<D, LDD>(sx, srs, g2, sy, sg, sx, sw, nr);
  lds_barrier();
  tail_dgain_part<D, LDD>(sw, a.part + (long long)blockIdx.x * 2 * D + D);
  tail_rows_out<D, LDD>(a.g_h2, sx, r0, nr);
  // g_o = g_h2.Wo^T
  float* go = a.g_o;
  rowtile_mm_stream<D, D, LDD, D, W, D, true>(sx, a.wo, nullptr, [&](int e, int n, float v) {
    if (e < nr) go[(long long)(r0 + e) * D + n] = v;
  });
}

// Whether the last-row tail runs as the two kernels above: a standard or latent block whose
// attention width is d, and an instantiated (d, ffn) shape.
static bool tail_fused(const talos_plan_s* p, const talos_ppo_cfg& c) {
  if (p->unfused || c.n_layers < 1 || c.batch < 1) return false;
  const talos_block_cfg bc = block_cfg_of(c);
  if (attn_width(bc) != c.d_model) return false;
  return (c.d_model == 128 && c.ffn_dim == 512) || (c.d_model == 64 && c.ffn_dim == 128);
}

// ---- Weight gradients over the last-token rows: dW = X^T G for several products in one launch ----
// The products of the last layer's tail (out_proj, W2, W1, Wo) and its query projection reduce
// over only B rows, too few for the big GEMM tiles: as split-K GEMMs each was a launch and a
// reduction of mostly latency. Here every 64x64 output tile of every product, times row chunks
// of kRowsChunk, is one 256-thread workgroup (wave = one 32x32 quadrant as 2x2
// v_mfma_f32_16x16x4_f32 tiles, lane l feeding X[row + l / 16][m + l % 16] and
// G[row + l / 16][n + l % 16] from LDS); the f32 chunk partials (and the bias column sums) are
// then added in a fixed order in f64 by one reduction launch.
constexpr int kRowsWgradMax = 6;
constexpr int kRowsChunk = 256;
struct RowsWgradProblem {
  const float* X;  // [rows][kx]
  const float* G;  // [rows][ng]
  float* dW;       // [kx][ng]
  float* dbias;    // [ng] = sum of G over the rows, or null
  long long ldx, ldg, ldw;
  int kx, ng, tiles_n, tile0, bias0;
};
struct RowsWgradArgs {
  int rows, nprob, chunks, ntiles, nbias;
  float* part;  // [chunks][ntiles][64 * 64], then [chunks][nbias]
  RowsWgradProblem pr[kRowsWgradMax];
};

__global__ __launch_bounds__(256) void rows_wgrad_kernel(RowsWgradArgs a) {
  const int t = blockIdx.x % a.ntiles, chunk = blockIdx.x / a.ntiles;
  int pi = 0;
  while (pi + 1 < a.nprob && t >= a.pr[pi + 1].tile0) ++pi;
  const RowsWgradProblem& P = a.pr[pi];
  const int lt = t - P.tile0;
  const int m0 = (lt / P.tiles_n) * 64, n0 = (lt % P.tiles_n) * 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1, i = lane & 15, kq = lane >> 4;
  const int na = n0 + 32 * wn + i;
  const bool bn0 = na < P.ng, bn1 = na + 16 < P.ng;
  const int r0 = chunk * kRowsChunk, r1 = min(a.rows, r0 + kRowsChunk);
  rt_floatx4 acc[2][2];
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = rt_floatx4{0.f, 0.f, 0.f, 0.f};
  float bs0 = 0.f, bs1 = 0.f;  // bias column sums over this lane's rows
  // Steps of 32 rows: the X and G pieces [32][64] are read as float4 (2 + 2 per thread) into
  // registers one step ahead, then stored to one of two LDS buffers, from which each lane reads
  // its operand columns.
  constexpr int SR = 32, LDT = 80;  // row pitch: the four row groups of a read fall in distinct banks
  __shared__ __align__(16) float sX[2][SR * LDT], sG[2][SR * LDT];
  const int lr = threadIdx.x >> 4, lc = 4 * (threadIdx.x & 15);  // rows lr and lr + 16, columns lc..lc+3
  const bool vx = P.kx % 4 == 0 && P.ldx % 4 == 0 && ((uintptr_t)P.X & 15) == 0;
  const bool vg = P.ng % 4 == 0 && P.ldg % 4 == 0 && ((uintptr_t)P.G & 15) == 0;
  auto ld4 = [&](const float* base, long long ld, int row, int col, int lim, bool vec) {
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < r1) {
      const float* q = base + (long long)row * ld + col;
      if (vec) {
        if (col < lim) v = *reinterpret_cast<const float4*>(q);
      } else {
        if (col < lim) v.x = q[0];
        if (col + 1 < lim) v.y = q[1];
        if (col + 2 < lim) v.z = q[2];
        if (col + 3 < lim) v.w = q[3];
      }
    }
    return v;
  };
  float4 px[2], pg[2];
  auto fetch = [&](int r) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      px[h] = ld4(P.X, P.ldx, r + lr + 16 * h, m0 + lc, P.kx, vx);
      pg[h] = ld4(P.G, P.ldg, r + lr + 16 * h, n0 + lc, P.ng, vg);
    }
  };
  fetch(r0);
  int buf = 0;
  for (int r = r0; r < r1; r += SR, buf ^= 1) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      *reinterpret_cast<float4*>(&sX[buf][(lr + 16 * h) * LDT + lc]) = px[h];
      *reinterpret_cast<float4*>(&sG[buf][(lr + 16 * h) * LDT + lc]) = pg[h];
    }
    __syncthreads();
    if (r + SR < r1) fetch(r + SR);
    const float* xs = sX[buf];
    const float* gs = sG[buf];
#pragma unroll
    for (int s = 0; s < SR / 4; ++s) {
      const int row = 4 * s + kq;
      const float x0 = xs[row * LDT + 32 * wm + i], x1 = xs[row * LDT + 32 * wm + 16 + i];
      const float g0 = gs[row * LDT + 32 * wn + i], g1 = gs[row * LDT + 32 * wn + 16 + i];
      acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, g0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, g1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, g0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, g1, acc[1][1], 0, 0, 0);
      bs0 += g0;
      bs1 += g1;
    }
  }
  float* tp = a.part + ((long long)chunk * a.ntiles + t) * 4096;
#pragma unroll
  for (int x = 0; x < 2; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 32 * wm + 16 * x + 4 * kq + q, n = 32 * wn + 16 * y + i;
        tp[m * 64 + n] = acc[x][y][q];
      }
  if (P.dbias && m0 == 0 && wm == 0) {
    // the four row groups (kq) of a column, added in kq order
    bs0 += __shfl_xor(bs0, 16);
    bs1 += __shfl_xor(bs1, 16);
    bs0 += __shfl_xor(bs0, 32);
    bs1 += __shfl_xor(bs1, 32);
    if (kq == 0) {
      float* bp = a.part + (long long)a.chunks * a.ntiles * 4096 + (long long)chunk * a.nbias + P.bias0;
      if (bn0) bp[na] = bs0;
      if (bn1) bp[na + 16] = bs1;
    }
  }
}

// dW[k][n] (and dbias[n]) = the chunk partials added in a fixed order in f64 (chunk c into
// accumulator c % 4); thread per output.
__global__ __launch_bounds__(256) void rows_wgrad_reduce_kernel(RowsWgradArgs a, long long nw) {
  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
  if (o >= nw + a.nbias) return;
  if (o < nw) {
    long long off = o;
    int pi = 0;
    while (off >= (long long)a.pr[pi].kx * a.pr[pi].ng) {
      off -= (long long)a.pr[pi].kx * a.pr[pi].ng;
      ++pi;
    }
    const RowsWgradProblem& P = a.pr[pi];
    const int k = (int)(off / P.ng), n = (int)(off % P.ng);
    const long long e = (long long)(P.tile0 + (k / 64) * P.tiles_n + n / 64) * 4096 + (k % 64) * 64 + n % 64;
    const long long step = (long long)a.ntiles * 4096;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    int c = 0;
    for (; c + 3 < a.chunks; c += 4) {
      const float* q = a.part + c * step + e;
      const float v0 = q[0], v1 = q[step], v2 = q[2 * step], v3 = q[3 * step];
      s0 += v0;
      s1 += v1;
      s2 += v2;
      s3 += v3;
    }
    for (; c < a.chunks; ++c) s0 += (double)a.part[c * step + e];
    P.dW[(long long)k * P.ldw + n] = (float)((s0 + s1) + (s2 + s3));
  } else {
    const int b = (int)(o - nw);
    int pi = a.nprob - 1;
    while (pi > 0 && (a.pr[pi].dbias == nullptr || b < a.pr[pi].bias0)) --pi;
    const RowsWgradProblem& P = a.pr[pi];
    const float* bp = a.part + (long long)a.chunks * a.ntiles * 4096 + b;
    double s = 0.0;
    for (int c = 0; c < a.chunks; ++c) s += (double)bp[(long long)c * a.nbias];
    P.dbias[b - P.bias0] = (float)s;
  }
}

// Host side: collect up to kRowsWgradMax products over the same rows, then launch both kernels.
struct RowsWgrad {
  RowsWgradArgs a{};
  void add(const float* X, long long ldx, int kx, const float* G, long long ldg, int ng, float* dW, long long ldw,
           float* dbias = nullptr) {
    RowsWgradProblem& P = a.pr[a.nprob++];
    P.X = X;
    P.ldx = ldx;
    P.kx = kx;
    P.G = G;
    P.ldg = ldg;
    P.ng = ng;
    P.dW = dW;
    P.ldw = ldw;
    P.dbias = dbias;
    P.tiles_n = (int)ceil_div((size_t)ng, 64);
    P.tile0 = a.ntiles;
    a.ntiles += (int)ceil_div((size_t)kx, 64) * P.tiles_n;
    P.bias0 = a.nbias;
    if (dbias) a.nbias += ng;
  }
  static size_t ws_floats(int rows, int ntiles, int nbias) {
    const size_t chunks = std::max<size_t>(1, ceil_div((size_t)rows, kRowsChunk));
    return chunks * ((size_t)ntiles * 4096 + nbias);
  }
  int launch(int rows, float* ws, size_t ws_floats_avail, hipStream_t s) {
    a.rows = rows;
    a.chunks = std::max(1, (int)ceil_div((size_t)rows, kRowsChunk));
    a.part = ws;
    TALOS_REQUIRE(ws_floats(rows, a.ntiles, a.nbias) <= ws_floats_avail, TALOS_ERR_SHAPE,
                  "row weight gradients: workspace too small");
    long long nw = 0;
    double flops = 0.0, bytes = 0.0;
    for (int i = 0; i < a.nprob; ++i) {
      nw += (long long)a.pr[i].kx * a.pr[i].ng;
      flops += 2.0 * rows * a.pr[i].kx * a.pr[i].ng;
      bytes += 4.0 * ((double)rows * (a.pr[i].kx + a.pr[i].ng) + (double)a.pr[i].kx * a.pr[i].ng);
    }
    {
      ProfScope ps(s, "rows_wgrad_kernel", flops, bytes + 4.0 * a.chunks * ((double)a.ntiles * 4096 + a.nbias));
      hipLaunchKernelGGL(rows_wgrad_kernel, dim3((unsigned)(a.ntiles * a.chunks)), dim3(256), 0, s, a);
      TALOS_LAUNCHED("rows_wgrad_kernel");
    }
    ProfScope ps(s, "rows_wgrad_reduce_kernel", 0.0, 4.0 * (a.chunks + 1.0) * ((double)a.ntiles * 4096 + a.nbias));
    hipLaunchKernelGGL(rows_wgrad_reduce_kernel, dim3((unsigned)ceil_div((size_t)(nw + a.nbias), 256)), dim3(256), 0, s,
                       a, nw);
    TALOS_LAUNCHED("rows_wgrad_reduce_kernel");
    return TALOS_OK;
  }
};

// Workspace floats of the tail's row weight gradients (out_proj, W2, W1 with biases; Wo) and of
// the last-query layer's dW_q, over B rows.
static size_t rows_wgrad_ws_floats(int B, int d, int F) {
  auto tl = [](int k, int n) { return (int)(ceil_div((size_t)k, 64) * ceil_div((size_t)n, 64)); };
  return std::max(RowsWgrad::ws_floats(B, 2 * tl(d, d) + tl(F, d) + tl(d, F), 2 * d + F),
                  RowsWgrad::ws_floats(B, tl(d, d), 0));
}

// The forward tail on the c.batch last-token rows: x the last layer's input on every row, p->lr.o
// the attention output on the last rows. Writes p->lr (h2, xn2, rstd2, u, a), p->last,
// p->lastn, p->rstdf and p->pout.
static int tail_fwd_launch(talos_plan_s* p, const talos_ppo_cfg& c, const talos_block_cfg& bc, const float* P,
                           const BlockOff& bo, const PpoOff& po, const float* x, hipStream_t s) {
  auto& R = p->lr;
  const int B = c.batch, D = c.d_model, F = c.ffn_dim;
  TailFwdArgs a{};
  a.B = B;
  a.relu = bc.activation != TALOS_ACT_GELU;
  a.seq = c.seq;
  a.eps = c.eps;
  a.lens = p->lens;
  a.x = x;
  a.o = R.o;
  a.wo = P + bo.wo;
  a.g2 = P + bo.g2;
  a.w1 = P + bo.w1;
  a.b1 = P + bo.b1;
  a.w2 = P + bo.w2;
  a.b2 = P + bo.b2;
  a.gf = P + po.gf;
  a.wout = P + po.wout;
  a.bout = P + po.bout;
  a.h2 = R.h2;
  a.xn2 = R.xn2;
  a.rstd2 = R.rstd2;
  a.u = R.u;
  a.a = R.a;
  a.last = p->last;
  a.lastn = p->lastn;
  a.rstdf = p->rstdf;
  a.pout = p->pout;
  const double flops = 2.0 * B * (2.0 * D * D + 2.0 * D * F);
  const double bytes = 4.0 * (2.0 * D * D + 2.0 * D * F + F + 5.0 * D) + 4.0 * B * (2.0 * D + 5.0 * D + 2.0 * F + 2.0);
  ProfScope ps(s, "ppo_tail_fwd_kernel", flops, bytes);
  const dim3 grid((unsigned)ceil_div((size_t)B, kRowTileRows));
  if (D == 128)
    hipLaunchKernelGGL((ppo_tail_fwd_kernel<128, 512>), grid, dim3(kTailThreads), 0, s, a);
  else
    hipLaunchKernelGGL((ppo_tail_fwd_kernel<64, 128>), grid, dim3(kTailThreads), 0, s, a);
  return launch_status("ppo_tail_fwd_kernel");
}

// Workspace of the backward tail: the partial dgains of both norms, reduced in one launch.
static size_t tail_bwd_ws_bytes(int B, int D) {
  return reduce_parts_workspace_bytes((int)ceil_div((size_t)B, kRowTileRows), 2 * D);
}

// The backward tail on the B last-token rows from p->g_pout: the row gradients p->g_last,
// p->lr.g_u, p->lr.g_h2 and p->lr.g_o, the final gain's and gain2's gradients, and the weight
// gradients of out_proj, W2, W1 and Wo.
static int tail_bwd_launch(talos_plan_s* p, const talos_ppo_cfg& c, const talos_block_cfg& bc, const float* P,
                           float* G, const BlockOff& bo, const PpoOff& po, hipStream_t s) {
  auto& R = p->lr;
  const int B = c.batch, D = c.d_model, F = c.ffn_dim;
  const int nblk = (int)ceil_div((size_t)B, kRowTileRows);
  TALOS_REQUIRE(tail_bwd_ws_bytes(B, D) <= p->red_ws_bytes, TALOS_ERR_SHAPE, "tail backward: workspace too small");
  int rc;
  for (float* b : {p->g_last, R.g_u, R.g_h2, R.g_o})
    if ((rc = before_write(p, s, b))) return rc;
  TailBwdArgs a{};
  a.B = B;
  a.relu = bc.activation != TALOS_ACT_GELU;
  a.g_pout = p->g_pout;
  a.wout = P + po.wout;
  a.gf = P + po.gf;
  a.last = p->last;
  a.rstdf = p->rstdf;
  a.w2 = P + bo.w2;
  a.u = R.u;
  a.w1 = P + bo.w1;
  a.g2 = P + bo.g2;
  a.h2 = R.h2;
  a.rstd2 = R.rstd2;
  a.wo = P + bo.wo;
  a.g_last = p->g_last;
  a.g_u = R.g_u;
  a.g_h2 = R.g_h2;
  a.g_o = R.g_o;
  double* slot = hold_slot(p);  // (held back where the PPO backward collects them)
  a.part = slot ? slot : p->red_ws;
  {
    const double flops = 2.0 * B * (2.0 * D * D + 2.0 * D * F);
    const double bytes = 4.0 * (2.0 * D * D + 2.0 * D * F + 2.0 * D) + 4.0 * B * (3.0 * D + 2.0 + F + 3.0 * D + F) +
                         16.0 * nblk * D;
    ProfScope ps(s, "ppo_tail_bwd_kernel", flops, bytes);
    const dim3 grid((unsigned)nblk);
    if (D == 128)
      hipLaunchKernelGGL((ppo_tail_bwd_kernel<128, 512>), grid, dim3(kTailThreads), 0, s, a);
    else
      hipLaunchKernelGGL((ppo_tail_bwd_kernel<64, 128>), grid, dim3(kTailThreads), 0, s, a);
    if ((rc = launch_status("ppo_tail_bwd_kernel"))) return rc;
  }
  if (slot && nblk <= kPartsOnePass) {
    PartsJob job;
    job.cols = 2 * D;
    job.nparts = nblk;
    job.part = a.part;
    job.out = G + po.gf;
    job.split = D;
    job.out2 = G + bo.g2;
    p->held.push_back(job);
  } else if ((rc = reduce_parts_launch(2 * D, nblk, a.part, 0.f, G + po.gf, s, D, G + bo.g2))) {
    return rc;
  }
  // out_proj, W2, W1 and Wo from the row gradients
  RowsWgrad rw;
  rw.add(p->lastn, D, D, p->g_pout, D, D, G + po.wout, D, G + po.bout);
  rw.add(R.a, F, F, p->g_last, D, D, G + bo.w2, D, G + bo.b2);
  rw.add(R.xn2, D, D, R.g_u, F, F, G + bo.w1, F, G + bo.b1);
  rw.add(R.o, D, D, R.g_h2, D, D, G + bo.wo, D);
  return rw.launch(B, p->gemm_ws, p->gemm_ws_bytes / sizeof(float), s);
}

// ---- Products over the last-token rows: Y = X W (or X W^T), 16 rows per workgroup ------------
// The last layer's query projection (with the gather of its input rows, which the dW_q product
// also reads) and its transpose in the backward: one row-tile launch each, instead of a gather
// and a 64x64-tile GEMM.
constexpr int kRowsMmWaves = 4;
template <int D, int LDW, bool TRANS>
__global__ __launch_bounds__(64 * kRowsMmWaves) void rows_mm_kernel(int B, int seq, const int32_t* lens,
                                                                    const float* __restrict__ X, long long ldx,
                                                                    float* __restrict__ xcopy, const float* W,
                                                                    float* __restrict__ Y) {
  constexpr int E = kRowTileRows, LD = D + 4;
  __shared__ __align__(16) float sx[E * LD];
  const int r0 = blockIdx.x * E, nr = min(E, B - r0);
  for (int i = threadIdx.x; i < E * (D / 4); i += 64 * kRowsMmWaves) {
    const int e = i / (D / 4), c = 4 * (i % (D / 4));
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e < nr) {
      long long row = r0 + e;
      if (seq > 0) row = row * seq + last_row(lens, r0 + e, seq);
      v = *reinterpret_cast<const float4*>(X + row * ldx + c);
      if (xcopy) *reinterpret_cast<float4*>(xcopy + (long long)(r0 + e) * D + c) = v;
    }
    *reinterpret_cast<float4*>(sx + e * LD + c) = v;
  }
  __syncthreads();
  rowtile_mm_stream<D, D, LD, LDW, kRowsMmWaves, D, TRANS>(sx, W, nullptr, [&](int e, int n, float v) {
    if (e < nr) Y[(long long)(r0 + e) * D + n] = v;
  });
}
// Y[B][d] = rows of X (the last-token rows of a [B * seq][ldx] buffer when seq > 0; copied to
// xcopy when given) times the d x d block of W (row pitch ldw = 3d: the query columns of Wqkv;
// W^T when trans). d = 128, 16-byte aligned rows.
static bool rows_mm_applies(int d, const float* X, long long ldx, long long ldw, const float* Y, const float* xcopy) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(Y) | reinterpret_cast<uintptr_t>(xcopy);
  return d == 128 && ldw == 3 * d && ldx % 4 == 0 && (al & 15) == 0;
}
static int rows_mm_launch(int B, int seq, const int32_t* lens, const float* X, long long ldx, float* xcopy,
                          const float* W, bool trans, float* Y, hipStream_t s) {
  constexpr int D = 128;
  ProfScope ps(s, "rows_mm_kernel", 2.0 * B * D * D, 4.0 * (D * D + (2.0 + (xcopy != nullptr)) * B * D));
  const dim3 grid((unsigned)ceil_div((size_t)B, kRowTileRows));
  if (trans)
    hipLaunchKernelGGL((rows_mm_kernel<D, 3 * D, true>), grid, dim3(64 * kRowsMmWaves), 0, s, B, seq, lens, X, ldx,
                       xcopy, W, Y);
  else
    hipLaunchKernelGGL((rows_mm_kernel<D, 3 * D, false>), grid, dim3(64 * kRowsMmWaves), 0, s, B, seq, lens, X, ldx,
                       xcopy, W, Y);
  return launch_status("rows_mm_kernel");
}

// ---- Embedding with the first RMSNorm: h0 = states . We + be, xn1 = rmsnorm(h0; g1) ----------
// K = 8 leaves the product nothing to do on the matrix cores; the launch is the 2 x 64 MB of row
// writes. Half a wave per row: lane q of the 32 holds columns 4q..4q+3 of We (8 x 4 floats), be
// and g1 in registers, reads the row's 8 states (one 32-byte piece shared by the 32 lanes), and
// writes h0, xn1 as float4; the sum of squares is a 32-lane DPP / swizzle reduction.
constexpr int kEmbedNormThreads = 256;
__global__ __launch_bounds__(kEmbedNormThreads) void embed_norm_kernel(int rows, float eps,
                                                                      const float* __restrict__ states,
                                                                      const float* __restrict__ we,
                                                                      const float* __restrict__ be,
                                                                      const float* __restrict__ gain, float* __restrict__ h,
                                                                      float* __restrict__ xn, float* __restrict__ rstd) {
  constexpr int D = 128, IN = kEmbedIn;
  const int q = threadIdx.x & 31, c = 4 * q;
  float4 w[IN];
#pragma unroll
  for (int k = 0; k < IN; ++k) w[k] = *reinterpret_cast<const float4*>(we + k * D + c);
  const float4 b = *reinterpret_cast<const float4*>(be + c), g = *reinterpret_cast<const float4*>(gain + c);
  const int half = (blockIdx.x * kEmbedNormThreads + threadIdx.x) >> 5, halves = gridDim.x * kEmbedNormThreads / 32;
  for (int r = half; r < rows; r += halves) {
    const float4 s0 = *reinterpret_cast<const float4*>(states + (long long)r * IN);
    const float4 s1 = *reinterpret_cast<const float4*>(states + (long long)r * IN + 4);
    const float sv[IN] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float4 o = b;
#pragma unroll
    for (int k = 0; k < IN; ++k) {
      o.x = fmaf(sv[k], w[k].x, o.x);
      o.y = fmaf(sv[k], w[k].y, o.y);
      o.z = fmaf(sv[k], w[k].z, o.z);
      o.w = fmaf(sv[k], w[k].w, o.w);
    }
    float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
    ss = group_sum<16>(ss);
    ss += __shfl_xor(ss, 16);  // the two 16-lane halves of the row
    const float rs = 1.0f / sqrtf(ss / (float)D + eps);
    const long long base = (long long)r * D + c;
    *reinterpret_cast<float4*>(h + base) = o;
    *reinterpret_cast<float4*>(xn + base) = make_float4(o.x * rs * g.x, o.y * rs * g.y, o.z * rs * g.z, o.w * rs * g.w);
    if (q == 0) rstd[r] = rs;
  }
}
static bool embed_norm_applies(const talos_ppo_cfg& c, const PpoOff& po, const float* P, const float* states,
                               const float* h, const RowNorm& n) {
  const uintptr_t al = reinterpret_cast<uintptr_t>(states) | reinterpret_cast<uintptr_t>(P + po.we) |
                       reinterpret_cast<uintptr_t>(P + po.be) | reinterpret_cast<uintptr_t>(n.gain) |
                       reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(n.out);
  return c.in_dim == kEmbedIn && c.d_model == 128 && n.out != nullptr && (al & 15) == 0;
}

static int ppo_forward(talos_plan_s* p, const talos_ppo_cfg& c, const float* P, const float* states,
                       hipStream_t s, bool heads = true) {
  const talos_block_cfg bc = block_cfg_of(c);
  const PpoOff po = ppo_offsets(c);
  const int M = c.batch * c.seq, d = c.d_model, A = c.n_actions, ow = attn_width(bc);
  const bool tail = tail_fused(p, c);
  // each layer's RMSNorm1 runs in the epilogue of the product that makes its input
  auto norm1_of = [&](int l) {
    const BlockOff bo = block_offsets(bc, po.blocks + (size_t)l * block_params(bc));
    return RowNorm{P + bo.g1, p->layers[l].xn1, p->layers[l].rstd1};
  };
  int rc;
  {
    GemmDesc g;
    g.M = M;
    g.N = d;
    g.K = c.in_dim;
    g.A = states;
    g.lda = c.in_dim;
    g.B = P + po.we;
    g.ldb = d;
    g.C = p->h0;
    g.ldc = d;
    g.bias = P + po.be;
    g.ksplit = 1;
    const RowNorm n1 = c.n_layers > 0 ? norm1_of(0) : RowNorm{};
    if (!p->unfused && embed_norm_applies(c, po, P, states, p->h0, n1)) {
      ProfScope ps_e(s, "embed_norm_kernel", 2.0 * M * kEmbedIn * d, 4.0 * M * (kEmbedIn + 2.0 * d + 1.0));
      const unsigned blocks = std::min<unsigned>(ceil_div((size_t)M, kEmbedNormThreads / 32), 8192);
      hipLaunchKernelGGL(embed_norm_kernel, dim3(blocks), dim3(kEmbedNormThreads), 0, s, M, c.eps, states, P + po.we,
                         P + po.be, n1.gain, p->h0, n1.out, n1.rstd);
      if ((rc = launch_status("embed_norm_kernel"))) return rc;
    } else {
      if (c.n_layers > 0) set_norm(p, g, n1, c.eps);
      if ((rc = gemm_launch(g, s))) return rc;
    }
  }
  const float* h = p->h0;
  size_t base = po.blocks;
  // the last-token rows of a [M, w] buffer into [batch, w]
  auto gather = [&](const float* src, float* dst, int w) {
    ProfScope ps_g(s, "gather_last_kernel", 0.0, 8.0 * c.batch * w);
    hipLaunchKernelGGL(gather_last_kernel, dim3(ceil_div((size_t)c.batch * w, 256)), dim3(256), 0, s, c.batch, c.seq,
                       w, p->lens, src, dst);
    return launch_status("gather_last_kernel");
  };
  for (int l = 0; l < c.n_layers; ++l) {
    BlockOff bo = block_offsets(bc, base);
    auto& L = p->layers[l];
    L.x = const_cast<float*>(h);
    if (l + 1 < c.n_layers) {
      rc = block_forward(p, bc, P, bo, L, s, true, norm1_of(l + 1));
      if (rc) return rc;
      h = L.out;
    } else {
      // Only the last token of each sample reaches the heads, and everything after attention is
      // per row: the last layer runs its MLP half on those B rows and writes p->last directly.
      const bool vabs = ppo_vabs(p, bc, L);
      if (ppo_lastq(p, bc, L)) {
        // attention of the last query only: keys (and values, unless absorbed) on every row, the
        // query on the last rows (rotated inside the attention kernel)
        auto& R = p->lr;
        {
          GemmDesc g;
          g.M = M;
          g.N = vabs ? d : 2 * d;
          g.K = d;
          g.A = L.xn1;
          g.lda = d;
          g.B = P + bo.wqkv + d;
          g.ldb = 3 * d;
          g.C = L.qkv + d;
          g.ldc = 3 * d;
          g.rope_cos = p->rcos;
          g.rope_sin = p->rsin;
          g.rope_cols = d;  // the k columns
          g.rope_dim = bc.head_dim;
          g.rope_seq = c.seq;
          g.ksplit = 1;
          if ((rc = gemm_launch(g, s))) return rc;
        }
        if (rows_mm_applies(d, L.xn1, d, 3 * d, R.q, R.xn1)) {
          if ((rc = rows_mm_launch(c.batch, c.seq, p->lens, L.xn1, d, R.xn1, P + bo.wqkv, false, R.q, s))) return rc;
        } else {
          if ((rc = gather(L.xn1, R.xn1, d))) return rc;
          if ((rc = mm(p, s, 0, 0, c.batch, d, d, R.xn1, d, P + bo.wqkv, 3 * d, R.q, d))) return rc;
        }
        AttnDesc ad = block_attn_desc(p, bc, L);
        ad.q_last = R.q;
        ad.ldq_last = d;
        if (vabs) {
          ad.dq_last = R.dq;  // (only checked for alignment here)
          ad.lddq_last = d;
          rc = attn_fwd_lastq_z_launch(ad, L.xn1, d, R.z, R.lse, s);
          if (rc == TALOS_OK) rc = vabs_out(p, c.batch, d, bc.n_heads, bc.head_dim, R.z, P + bo.wqkv + 2 * d, 3 * d, R.o, s);
        } else {
          rc = attn_fwd_lastq_launch(ad, R.o, d, R.lse, s);
        }
      } else {
        rc = block_attn_forward(p, bc, P, bo, L, s, true);
        if (rc == TALOS_OK) rc = gather(L.o, p->lr.o, ow);
      }
      if (rc) return rc;
      if (tail) {  // through out_proj in one kernel
        if ((rc = tail_fwd_launch(p, c, bc, P, bo, po, L.x, s))) return rc;
      } else {
        if ((rc = gather(L.x, p->lr.x, d))) return rc;
        rc = block_mlp_forward(p, bc, P, bo, c.batch, p->lr.x, p->lr.o, p->lr.h2, p->lr.xn2, p->lr.rstd2, p->lr.u,
                               p->lr.a, p->last, s);
        if (rc) return rc;
      }
    }
    base = bo.end;
  }
  if (c.n_layers == 0) {
    rc = gather(h, p->last, d);
    if (rc) return rc;
  }
  if (!tail) {
    rc = rmsnorm_fwd_launch(c.batch, d, c.eps, p->last, P + po.gf, p->lastn, p->rstdf, s);
    if (rc) return rc;
    rc = mm(p, s, 0, 0, c.batch, d, d, p->lastn, d, P + po.wout, d, p->pout, d, 0.f, P + po.bout);
    if (rc) return rc;
  }
  if (!heads) return TALOS_OK;  // the minibatch runs the heads inside ppo_heads_kernel
  rc = mm(p, s, 0, 0, c.batch, A, d, p->pout, d, P + po.wa, A, p->logits, A, 0.f, P + po.ba);
  if (rc) return rc;
  return mm(p, s, 0, 0, c.batch, 1, d, p->pout, d, P + po.wc, 1, p->values, 1, 0.f, P + po.bc);
}


// ---------------------------------------------------------------------------
// MLA block (talos_mla_cfg): out = x + MLA(rmsnorm(x; g)), the graph of
// MultiHeadLatentAttention::forward (src/transformer.rs:478-557) with the position of RoPE the
// sequence index. Parameters: g[d] | W_dkv[d,L] | W_uk[L,H*hd] | W_uv[L,H*vd] | W_q[d,H*hd] |
// W_kr[d,H*r] | W_qr[d,H*r] | W_o[H*vd,d].
// ---------------------------------------------------------------------------
struct MlaOff {
  size_t g;
  MlaW w;
  size_t end;
};
static MlaOff mla_offsets(const talos_mla_cfg& c) {
  MlaOff o;
  o.g = 0;
  o.w = mla_weights(mla_dims(c), o.g + (size_t)c.d_model);
  o.end = o.w.end;
  return o;
}

static int check_mla_cfg(const talos_mla_cfg& c) {
  TALOS_REQUIRE(c.batch > 0 && c.seq > 0 && c.d_model > 0 && c.n_heads > 0 && c.kv_latent > 0 && c.rope_dim > 0 &&
                    c.head_dim > 0 && c.v_dim > 0,
                TALOS_ERR_SHAPE, "mla cfg: sizes must be positive");
  TALOS_REQUIRE(c.rope_dim % 2 == 0, TALOS_ERR_SHAPE, "mla cfg: rope_dim must be even");
  TALOS_REQUIRE(c.head_dim + c.rope_dim <= 128 && c.v_dim <= 128, TALOS_ERR_UNSUPPORTED,
                "mla cfg: head_dim + rope_dim and v_dim must be <= 128");
  TALOS_REQUIRE(c.d_model % 4 == 0 && c.kv_latent % 4 == 0 && c.head_dim % 4 == 0 && c.rope_dim % 4 == 0 &&
                    c.v_dim % 4 == 0,
                TALOS_ERR_UNSUPPORTED, "mla cfg: all widths must be multiples of 4");
  TALOS_REQUIRE(c.causal == 0 || c.causal == 1, TALOS_ERR_DTYPE, "mla cfg: causal must be 0 or 1");
  TALOS_REQUIRE(c.precision == TALOS_PREC_FP32 || c.precision == TALOS_PREC_BF16, TALOS_ERR_DTYPE,
                "mla cfg: unknown precision %d", c.precision);
  TALOS_REQUIRE(c.eps >= 0.f && c.rope_base > 0.f, TALOS_ERR_SHAPE, "mla cfg: eps >= 0 and rope_base > 0 required");
  TALOS_REQUIRE((long long)c.batch * c.seq * c.n_heads * (c.head_dim + c.rope_dim) < (1LL << 31),
                TALOS_ERR_UNSUPPORTED, "mla cfg: too many elements for 32-bit indexing");
  return TALOS_OK;
}

// Forward + backward of the MLA block for loss = sum(out * gout).
static int mla_fwd_bwd(talos_plan_s* p, const float* P, const float* x, const float* gout, float* out, float* G,
                       float* dx, hipStream_t s) {
  const talos_mla_cfg& c = p->mla;
  const MlaOff o = mla_offsets(c);
  const MlaDims D = mla_dims(c);
  auto& L = p->layers[0];
  const int M = c.batch * c.seq, d = c.d_model, ow = c.n_heads * c.v_dim;
  int rc;
  // bf16 plans: this call's weights and output gradient have bf16 copies (one conversion launch
  // each, the output gradient's with the attention's output); the norm writes its output's copy
  set_shadow_base(p, p->p16, p->p16 ? P : nullptr);
  set_shadow_base(p, p->g16, p->g16 ? gout : nullptr);
  // ---- forward
  if ((rc = rmsnorm_fwd_launch(M, d, c.eps, x, P + o.g, L.xn1, L.rstd1, s, shadow_of(p, L.xn1)))) return rc;
  if ((rc = refresh_shadows(p, {P}, s))) return rc;
  if ((rc = mla_attn_forward(p, D, P, o.w, L.xn1, L, s))) return rc;
  if ((rc = refresh_shadows(p, {L.o, gout}, s))) return rc;
  if ((rc = mm(p, s, 0, 0, M, d, ow, L.o, ow, P + o.w.wo, d, out, d, 0.f, nullptr, x, d))) return rc;
  // ---- backward (its split-K weight gradients' combinations held back to one launch at the end)
  HoldScope hold(p);
  if ((rc = mm(p, s, 1, 0, ow, d, M, L.o, ow, gout, d, G + o.w.wo, d))) return rc;
  // dO = gout . Wo^T; where the attention backward takes the dS path, the product's epilogue also
  // forms that backward's D = rowsum(dO . O) into its workspace (no row-dot launch)
  const bool d_ready =
      p->rowdot && attn_ds_path(mla_attn_desc(p, D, L)) && (c.v_dim == 32 || c.v_dim == 64) && ow % 128 == 0;
  if (d_ready) {
    GemmDesc g;
    g.transB = 1;
    g.M = M;
    g.N = ow;
    g.K = d;
    g.A = gout;
    g.lda = d;
    g.B = P + o.w.wo;
    g.ldb = d;
    g.C = p->g_o;
    g.ldc = ow;
    g.rd_o = L.o;
    g.rd_ldo = ow;
    g.rd_D = p->attn_ws;
    g.rd_w = c.v_dim;
    g.rd_seq = c.seq;
    g.rd_heads = c.n_heads;
    g.ksplit = 1;
    g.bf16 = p->bf16;
    bf16_operands(p, g);
    if ((rc = gemm_launch(g, s))) return rc;
  } else if ((rc = mm(p, s, 0, 1, M, ow, d, gout, d, P + o.w.wo, d, p->g_o, ow))) {
    return rc;
  }
  if ((rc = mla_attn_backward(p, D, P, G, o.w, L.xn1, L, p->g_o, p->g_xn, s, d_ready))) return rc;
  // residual + rmsnorm
  if ((rc = rmsnorm_bwd_launch(M, d, x, P + o.g, L.rstd1, p->g_xn, 1.f, dx, 0.f, G + o.g, p->red_ws, s, gout)))
    return rc;
  p->holding = false;
  return hold_flush(p, s);
}

const talos_ppo_cfg* ppo_plan_cfg(talos_plan plan) {
  return (plan != nullptr && plan->kind == 2) ? &plan->ppo : nullptr;
}

}  // namespace talos

using namespace talos;

extern "C" {

size_t talos_block_param_count(const talos_block_cfg* cfg) { return cfg ? block_params(*cfg) : 0; }

size_t talos_ppo_param_count(const talos_ppo_cfg* cfg) { return cfg ? ppo_params(*cfg) : 0; }

int talos_block_plan_create(const talos_block_cfg* cfg, talos_plan* plan) {
  TALOS_NONNULL(cfg);
  TALOS_NONNULL(plan);
  *plan = nullptr;
  int rc = check_block_cfg(*cfg);
  if (rc) return rc;
  TALOS_DEVICE();
  auto* p = new talos_plan_s();
  p->kind = 1;
  p->prof = profiler_new();
  p->unfused = env_flag("TALOS_PLAN_UNFUSED");
  p->blk = *cfg;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess) p->num_cu = prop.multiProcessorCount;
  rc = alloc_block_buffers(p, *cfg, 1);
  if (rc == TALOS_OK) rc = alloc_workspaces(p);
  if (rc) {
    plan_free(p);
    delete p;
    return rc;
  }
  *plan = p;
  return TALOS_OK;
}

int talos_block_fwd_bwd_f32(talos_plan plan, const float* params, const float* x, const float* gout, float* out,
                            float* dparams, float* dx, talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 1, TALOS_ERR_HANDLE, "%s: not a block plan", __func__);
  TALOS_NONNULL(params);
  TALOS_NONNULL(x);
  TALOS_NONNULL(gout);
  TALOS_NONNULL(dparams);
  TALOS_NONNULL(dx);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  PlanCall pc(plan);
  const talos_block_cfg& c = plan->blk;
  const size_t M = (size_t)c.batch * c.seq, d = c.d_model;
  BlockOff bo = block_offsets(c, 0);
  auto& L = plan->layers[0];
  L.x = const_cast<float*>(x);
  // the forward's last product writes the caller's out itself (the backward does not read it)
  float* const own_out = L.out;
  const bool direct = out && out != x;
  if (direct) L.out = out;
  int rc = block_forward(plan, c, params, bo, L, s);
  L.out = own_out;
  if (rc) return rc;
  if (out && !direct) TALOS_HIP(hipMemcpyAsync(out, L.out, M * d * 4, hipMemcpyDeviceToDevice, s));
  {
    // the two gain gradients' combinations held back and run as one launch after the backward
    HoldScope hold(plan);
    rc = block_backward(plan, c, params, dparams, bo, L, gout, dx, s);
    plan->holding = false;
    if (rc == TALOS_OK) rc = hold_flush(plan, s);
  }
  if (rc) return rc;
  return entry_done(join_side(plan, s), as_stream(stream));
}

int talos_ppo_plan_create(const talos_ppo_cfg* cfg, talos_plan* plan) {
  TALOS_NONNULL(cfg);
  TALOS_NONNULL(plan);
  *plan = nullptr;
  int rc = check_ppo_cfg(*cfg);
  if (rc) return rc;
  TALOS_DEVICE();
  auto* p = new talos_plan_s();
  p->kind = 2;
  p->prof = profiler_new();
  p->unfused = env_flag("TALOS_PLAN_UNFUSED");
  p->ppo = *cfg;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess) p->num_cu = prop.multiProcessorCount;
  const talos_block_cfg bc = block_cfg_of(*cfg);
  const size_t M = (size_t)cfg->batch * cfg->seq, d = cfg->d_model, B = cfg->batch, A = cfg->n_actions;
  rc = alloc_block_buffers(p, bc, cfg->n_layers);
  rc |= plan_alloc(p, &p->h0, M * d);
  rc |= plan_alloc(p, &p->last, B * d);
  rc |= plan_alloc(p, &p->lastn, B * d);
  rc |= plan_alloc(p, &p->rstdf, B);
  rc |= plan_alloc(p, &p->pout, B * d);
  rc |= plan_alloc(p, &p->logits, B * A);
  rc |= plan_alloc(p, &p->values, B);
  rc |= plan_alloc(p, &p->g_logits, B * A);
  rc |= plan_alloc(p, &p->g_values, B);
  rc |= plan_alloc(p, &p->g_pout, B * d);
  rc |= plan_alloc(p, &p->g_lastn, B * d);
  rc |= plan_alloc(p, &p->g_last, B * d);
  {  // the last layer's last-token rows
    const size_t F = cfg->ffn_dim, ow = attn_width(bc);
    auto& R = p->lr;
    for (float** b : {&R.x, &R.h2, &R.xn2, &R.g_xn, &R.g_h2, &R.xn1, &R.q, &R.dq, &R.g_xnq}) rc |= plan_alloc(p, b, B * d);
    for (float** b : {&R.o, &R.g_o}) rc |= plan_alloc(p, b, B * ow);
    for (float** b : {&R.u, &R.a, &R.g_u}) rc |= plan_alloc(p, b, B * F);
    rc |= plan_alloc(p, &R.rstd2, B);
    rc |= plan_alloc(p, &R.lse, B * cfg->n_heads);
    // the absorbed-value path (four 32-wide heads, d = 128: the kernels' shapes)
    if (!p->unfused && bc.attention == TALOS_ATTN_MHA && d == 128 && cfg->n_heads == 4 && bc.head_dim == 32 &&
        cfg->seq <= 256 && cfg->n_layers > 0) {
      for (float** b : {&R.z, &R.uv}) rc |= plan_alloc(p, b, B * cfg->n_heads * d);
      rc |= plan_alloc(p, &p->wpre, M * 4);
    }
  }
  {  // per-workgroup loss partials (doubles)
    float* lw = nullptr;
    const size_t R = (size_t)cfg->d_model * (A + 1) + A + 1;
    const size_t heads = (size_t)ceil_div(B, kHeadSamples) * (kLossParts + R);
    rc |= plan_alloc(p, &lw, 2 * std::max((size_t)kLossParts * ceil_div(B, 256), heads));
    p->loss_ws = reinterpret_cast<double*>(lw);
  }
  if (rc == TALOS_OK) {
    p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, wgrad_ws(p, (int)M, cfg->in_dim, (int)d));
    p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, wgrad_ws(p, (int)B, (int)d, (int)d));
    p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, wgrad_ws(p, (int)B, (int)d, (int)A));
    p->red_ws_bytes = std::max(p->red_ws_bytes, colsum_workspace_bytes((int)M, (int)d));
    p->red_ws_bytes = std::max(p->red_ws_bytes, reduce_parts_workspace_bytes(kEmbedBlocks, (kEmbedIn + 1) * (int)d));
    p->red_ws_bytes = std::max(p->red_ws_bytes, tail_bwd_ws_bytes((int)B, (int)d));
    p->gemm_ws_bytes = std::max(p->gemm_ws_bytes, sizeof(float) * rows_wgrad_ws_floats((int)B, (int)d, cfg->ffn_dim));
    rc = alloc_workspaces(p);
  }
  if (rc) {
    plan_free(p);
    delete p;
    return rc ? rc : TALOS_ERR_ALLOC;
  }
  *plan = p;
  return TALOS_OK;
}

// Lengths of the PPO call in progress, visible to the block kernels through the plan.
struct LensScope {
  talos_plan_s* p;
  LensScope(talos_plan_s* p_, const int32_t* lens) : p(p_) { p->lens = lens; }
  ~LensScope() { p->lens = nullptr; }
};

static int ppo_check_n(const talos_plan_s* p, int n, const char* fn) {
  TALOS_REQUIRE(n >= 1 && n <= p->ppo.batch, TALOS_ERR_SHAPE, "%s: n=%d outside [1, %d] (the plan's batch)", fn, n,
                p->ppo.batch);
  return TALOS_OK;
}

int talos_ppo_forward_n_f32(talos_plan plan, int n, const float* params, const float* states, const int32_t* lengths,
                            float* logits, float* values, talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 2, TALOS_ERR_HANDLE, "%s: not a ppo plan", __func__);
  TALOS_NONNULL(params);
  TALOS_NONNULL(states);
  if (int rc = ppo_check_n(plan, n, __func__)) return rc;
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  PlanCall pc(plan);
  LensScope ls(plan, lengths);
  talos_ppo_cfg c = plan->ppo;
  c.batch = n;
  int rc = ppo_forward(plan, c, params, states, s);
  if (rc) return rc;
  if (logits)
    TALOS_HIP(hipMemcpyAsync(logits, plan->logits, (size_t)n * c.n_actions * 4, hipMemcpyDeviceToDevice, s));
  if (values) TALOS_HIP(hipMemcpyAsync(values, plan->values, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_ppo_forward_f32(talos_plan plan, const float* params, const float* states, float* logits, float* values,
                          talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 2, TALOS_ERR_HANDLE, "%s: not a ppo plan", __func__);
  return talos_ppo_forward_n_f32(plan, plan->ppo.batch, params, states, nullptr, logits, values, stream);
}

// One minibatch of n samples: forward, loss (and its statistics), backward into dparams.
// The embedding's weight and bias gradients, [I + 1][128] (W_e rows, then b_e): dW[i][c] =
// sum_r states[r][i] g[r][c] and db[c] = sum_r g[r][c], for I = in_dim = 8 and d = 128. A
// product of 8 rows would leave most of a 64x64 MFMA tile empty and write kEmbedBlocks-fold
// split-K partials; here each workgroup sums a contiguous chunk of rows (32 float4 column groups
// x 8 row lanes, f32 over the lane's rows, f64 across lanes) into one partial row, and
// reduce_parts_launch adds the partials in a fixed order.
__global__ __launch_bounds__(256) void embed_wgrad_kernel(int rows, const float* __restrict__ states,
                                                          const float* __restrict__ g, double* __restrict__ part) {
  constexpr int I = kEmbedIn, N = 128;
  __shared__ float red[8][(I + 1) * N];
  const int cg = threadIdx.x & 31, rl = threadIdx.x >> 5;
  const int chunk = (rows + gridDim.x - 1) / gridDim.x, r0 = blockIdx.x * chunk, r1 = min(rows, r0 + chunk);
  float4 acc[I + 1];
#pragma unroll
  for (int i = 0; i <= I; ++i) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
  for (int r = r0 + rl; r < r1; r += 8) {
    const float4 gv = *reinterpret_cast<const float4*>(g + (long long)r * N + 4 * cg);
    const float4 a0 = *reinterpret_cast<const float4*>(states + (long long)r * I);
    const float4 a1 = *reinterpret_cast<const float4*>(states + (long long)r * I + 4);
    const float av[I] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
    for (int i = 0; i < I; ++i) {
      acc[i].x = fmaf(av[i], gv.x, acc[i].x);
      acc[i].y = fmaf(av[i], gv.y, acc[i].y);
      acc[i].z = fmaf(av[i], gv.z, acc[i].z);
      acc[i].w = fmaf(av[i], gv.w, acc[i].w);
    }
    acc[I].x += gv.x;
    acc[I].y += gv.y;
    acc[I].z += gv.z;
    acc[I].w += gv.w;
  }
#pragma unroll
  for (int i = 0; i <= I; ++i) *reinterpret_cast<float4*>(&red[rl][i * N + 4 * cg]) = acc[i];
  __syncthreads();
  for (int c = threadIdx.x; c < (I + 1) * N; c += 256) {
    double sum = 0.0;
#pragma unroll
    for (int l = 0; l < 8; ++l) sum += (double)red[l][c];
    part[(long long)blockIdx.x * (I + 1) * N + c] = sum;
  }
}

// Whether the embedding gradient takes embed_wgrad_kernel: in_dim 8, d 128, b_e right after W_e,
// 16-byte rows.
static bool embed_wgrad_applies(const talos_ppo_cfg& c, const PpoOff& po, const float* states, const float* g) {
  return c.in_dim == kEmbedIn && c.d_model == 128 && po.be == po.we + (size_t)kEmbedIn * 128 &&
         ((reinterpret_cast<uintptr_t>(states) | reinterpret_cast<uintptr_t>(g)) & 15) == 0;
}

static int ppo_minibatch(talos_plan_s* p, int n, const float* params, const float* states, const int32_t* actions,
                         const float* adv, const float* ret, const float* old_logp, float* loss_out, float* dparams,
                         double* stats, int stats_acc, hipStream_t s) {
  talos_ppo_cfg c = p->ppo;
  c.batch = n;
  const talos_block_cfg bc = block_cfg_of(c);
  const PpoOff po = ppo_offsets(c);
  const int M = c.batch * c.seq, d = c.d_model, A = c.n_actions, B = c.batch;
  // the heads, loss and their backward in one kernel when the per-wave head gradients fit in LDS
  const int R = d * (A + 1) + A + 1;
  const bool fused_heads = R <= kHeadMaxRow && !p->unfused;
  int rc = ppo_forward(p, c, params, states, s, !fused_heads);
  if (rc) return rc;
  float* G = dparams;
  if (fused_heads) {
    const int nblk = (int)ceil_div((size_t)B, kHeadSamples);
    {
      ProfScope ps_h(s, "ppo_heads_kernel", 4.0 * B * (double)d * (A + 1),
                     4.0 * (2.0 * B * d + 5.0 * B) + 8.0 * nblk * (kLossParts + R));
      hipLaunchKernelGGL(ppo_heads_kernel, dim3(nblk), dim3(64 * kHeadWaves), (size_t)kHeadWaves * R * sizeof(float),
                         s, B, d, A, c.clip_eps, c.value_coef, c.entropy_coef, p->pout, params + po.wa,
                         params + po.ba, params + po.wc, params + po.bc, actions, adv, ret, old_logp, p->g_pout,
                         p->loss_ws);
      TALOS_LAUNCHED("ppo_heads_kernel");
    }
    ProfScope ps_f(s, "ppo_heads_final_kernel", 0.0, 8.0 * nblk * (kLossParts + R) + 4.0 * R);
    hipLaunchKernelGGL(ppo_heads_final_kernel, dim3(ceil_div((size_t)kLossParts + R, 16)), dim3(1024), 0, s, nblk, B,
                       R, p->loss_ws, loss_out, stats, stats_acc, G + po.wa);
    TALOS_LAUNCHED("ppo_heads_final_kernel");
  } else {
    const int nblk = (int)ceil_div((size_t)B, 256);
    {
      ProfScope ps_l(s, "ppo_loss_kernel", 0.0, 4.0 * B * (2.0 * A + 5.0));
      hipLaunchKernelGGL(ppo_loss_kernel, dim3(nblk), dim3(256), 0, s, B, A, c.clip_eps, c.value_coef,
                         c.entropy_coef, p->logits, p->values, actions, adv, ret, old_logp, p->g_logits, p->g_values,
                         1, p->loss_ws);
      TALOS_LAUNCHED("ppo_loss_kernel");
    }
    {
      ProfScope ps_f(s, "ppo_loss_final_kernel", 0.0, 8.0 * nblk * kLossParts);
      hipLaunchKernelGGL(ppo_loss_final_kernel, dim3(1), dim3(64), 0, s, nblk, B, p->loss_ws, loss_out, stats,
                         stats_acc);
      TALOS_LAUNCHED("ppo_loss_final_kernel");
    }
    // heads
    rc = mm(p, s, 1, 0, d, A, B, p->pout, d, p->g_logits, A, G + po.wa, A, 0.f, nullptr, nullptr, 0, G + po.ba);
    if (rc) return rc;
    rc = mm(p, s, 1, 0, d, 1, B, p->pout, d, p->g_values, 1, G + po.wc, 1, 0.f, nullptr, nullptr, 0, G + po.bc);
    if (rc) return rc;
    rc = mm(p, s, 0, 1, B, d, A, p->g_logits, A, params + po.wa, A, p->g_pout, d);
    if (rc) return rc;
    rc = mm(p, s, 0, 1, B, d, 1, p->g_values, 1, params + po.wc, 1, p->g_pout, d, 1.f);
    if (rc) return rc;
  }
  std::vector<BlockOff> offs;
  size_t base = po.blocks;
  for (int l = 0; l < c.n_layers; ++l) {
    offs.push_back(block_offsets(bc, base));
    base = offs.back().end;
  }
  // from here the gain and embedding gradients' combinations are held back (hold_flush below)
  HoldScope hold(p);
  const bool tail = tail_fused(p, c);
  if (tail) {  // out_proj through the last layer's MLP half: the row gradients in one kernel
    if ((rc = tail_bwd_launch(p, c, bc, params, G, offs.back(), po, s))) return rc;
  } else {
    // out_proj
    rc = wgrad(p, s, p->g_pout, d, d, B, p->lastn, d, p->g_pout, d, G + po.wout, d, G + po.bout);
    if (rc) return rc;
    rc = mm(p, s, 0, 1, B, d, d, p->g_pout, d, params + po.wout, d, p->g_lastn, d);
    if (rc) return rc;
    // final rmsnorm on the last-token rows
    rc = rmsnorm_bwd_launch(B, d, p->last, params + po.gf, p->rstdf, p->g_lastn, 0.f, p->g_last, 0.f, G + po.gf,
                            p->red_ws, s);
    if (rc) return rc;
  }
  // rows of a [B, w] last-token gradient into a full [M, w] one, zero elsewhere
  auto scatter = [&](const float* src, float* dst, int w) {
    ProfScope ps_s(s, "scatter_last_kernel", 0.0, 4.0 * ((double)M * w + (double)B * w));
    const size_t blocks = ceil_div((size_t)M * w, 256);
    hipLaunchKernelGGL(scatter_last_kernel, dim3(blocks > 65536 ? 65536 : blocks), dim3(256), 0, s, B, c.seq, w,
                       p->lens, src, dst);
    return launch_status("scatter_last_kernel");
  };
  // blocks, last to first; the gradient ping-pongs between g_out and g_x
  float* gcur = p->g_out;
  float* gnext = p->g_x;
  if (c.n_layers == 0) {
    rc = scatter(p->g_last, p->g_out, d);
    if (rc) return rc;
  } else {
    // the last layer: MLP half on the last-token rows (the forward's p->lr), then the attention
    // half from the last rows' gradients
    const int l = c.n_layers - 1;
    auto& R = p->lr;
    auto& L = p->layers[l];
    if (!tail) {
      rc = block_mlp_backward(p, bc, params, G, offs[l], B, R.o, R.h2, R.xn2, R.rstd2, R.u, R.a, p->g_last, R.g_u,
                              R.g_xn, R.g_h2, R.g_o, s);
      if (rc) return rc;
    }
    if (ppo_lastq(p, bc, L)) {
      // keys / values on every row, the query on the last rows (its gradient in R.dq)
      const BlockOff& o = offs[l];
      AttnDesc ad = block_attn_desc(p, bc, L);
      ad.q_last = R.q;
      ad.ldq_last = d;
      ad.dq_last = R.dq;
      ad.lddq_last = d;
      if ((rc = before_write(p, s, p->g_qkv))) return rc;
      if ((rc = before_write(p, s, R.dq))) return rc;
      const bool vabs = ppo_vabs(p, bc, L);
      const int H = bc.n_heads, hd = bc.head_dim;
      if (vabs) {
        if ((rc = vabs_u(p, B, d, H, hd, R.g_o, params + o.wqkv + 2 * d, 3 * d, R.uv, s))) return rc;
        if ((rc = before_write(p, s, p->wpre))) return rc;
        rc = attn_bwd_lastq_z_launch(ad, L.xn1, d, R.uv, R.o, d, R.lse, R.g_o, d, p->wpre, s);
      } else {
        rc = attn_bwd_lastq_launch(ad, R.o, d, R.lse, R.g_o, d, s);
      }
      if (rc) return rc;
      float* g_kv = p->g_qkv + d;
      // the key (and value) weight gradients over every row
      if ((rc = wgrad(p, s, p->g_qkv, d, vabs ? d : 2 * d, M, L.xn1, d, g_kv, 3 * d, G + o.wqkv + d, 3 * d))) return rc;
      {
        RowsWgrad rw;  // dW_q over the last rows; absorbed values: dWv_h = sum_b z_bh^T dO_bh
        rw.add(R.xn1, d, d, R.dq, d, d, G + o.wqkv, 3 * d);
        if (vabs)
          for (int h = 0; h < H; ++h)
            rw.add(R.z + (size_t)h * d, (long long)H * d, d, R.g_o + (size_t)h * hd, d, hd, G + o.wqkv + 2 * d + h * hd,
                   3 * d);
        if ((rc = rw.launch(B, p->gemm_ws, p->gemm_ws_bytes / sizeof(float), s))) return rc;
      }
      // dxn1 = g_kv.Wkv^T on every row, plus dq.Wq^T on the last rows; then rmsnorm1's backward
      // with the residual gradient R.g_h2 on the last rows
      if (rows_mm_applies(d, R.dq, d, 3 * d, R.g_xnq, nullptr))
        rc = rows_mm_launch(B, 0, nullptr, R.dq, d, nullptr, params + o.wqkv, true, R.g_xnq, s);
      else
        rc = mm(p, s, 0, 1, B, d, d, R.dq, d, params + o.wqkv, 3 * d, R.g_xnq, d);
      if (rc) return rc;
      if ((rc = before_write(p, s, p->g_out))) return rc;
      rc = norm_bwd_mm(p, s, M, d, vabs ? d : 2 * d, g_kv, 3 * d, params + o.wqkv + d, 3 * d, p->g_xn, L.x,
                       params + o.g1, L.rstd1, nullptr, R.g_h2, R.g_xnq, c.seq, p->g_out, G + o.g1,
                       vabs ? p->wpre : nullptr, vabs ? R.uv : nullptr);
    } else {
      // the row gradients spread over the full token grid
      const int ow = attn_width(bc);
      rc = scatter(R.g_o, p->g_o, ow);
      if (rc == TALOS_OK) rc = block_attn_backward(p, bc, params, G, offs[l], L, p->g_o, nullptr, R.g_h2, p->g_out, s);
    }
    if (rc) return rc;
  }
  for (int l = c.n_layers - 2; l >= 0; --l) {
    rc = block_backward(p, bc, params, G, offs[l], p->layers[l], gcur, gnext, s);
    if (rc) return rc;
    std::swap(gcur, gnext);
  }
  // embed
  if (embed_wgrad_applies(c, po, states, gcur)) {
    double* slot = kEmbedBlocks <= kPartsOnePass ? hold_slot(p) : nullptr;
    double* part = slot ? slot : p->red_ws;
    {
      ProfScope ps_e(s, "embed_wgrad_kernel", 2.0 * M * (kEmbedIn + 1) * d,
                     4.0 * M * (kEmbedIn + d) + 8.0 * kEmbedBlocks * (kEmbedIn + 1) * d);
      hipLaunchKernelGGL(embed_wgrad_kernel, dim3(kEmbedBlocks), dim3(256), 0, s, M, states, gcur, part);
      TALOS_LAUNCHED("embed_wgrad_kernel");
    }
    if (slot) {
      PartsJob job;
      job.cols = (kEmbedIn + 1) * d;
      job.nparts = kEmbedBlocks;
      job.part = part;
      job.out = G + po.we;
      p->held.push_back(job);
    } else {
      rc = reduce_parts_launch((kEmbedIn + 1) * d, kEmbedBlocks, part, 0.f, G + po.we, s);
    }
  } else {
    rc = wgrad(p, s, gcur, c.in_dim, d, M, states, c.in_dim, gcur, d, G + po.we, d, G + po.be);
  }
  if (rc) return rc;
  // the held-back gain and embedding gradient combinations, in one launch
  p->holding = false;
  if ((rc = hold_flush(p, s))) return rc;
  return join_side(p, s);
}

int talos_ppo_minibatch_f32(talos_plan plan, int n, const float* params, const float* states, const int32_t* lengths,
                            const int32_t* actions, const float* adv, const float* ret, const float* old_logp,
                            float* loss, float* dparams, double* stats, int stats_accumulate, talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 2, TALOS_ERR_HANDLE, "%s: not a ppo plan", __func__);
  TALOS_NONNULL(params);
  TALOS_NONNULL(states);
  TALOS_NONNULL(actions);
  TALOS_NONNULL(adv);
  TALOS_NONNULL(ret);
  TALOS_NONNULL(old_logp);
  TALOS_NONNULL(dparams);
  if (int rc = ppo_check_n(plan, n, __func__)) return rc;
  TALOS_DEVICE();
  PlanCall pc(plan);
  LensScope ls(plan, lengths);
  const int rc = ppo_minibatch(plan, n, params, states, actions, adv, ret, old_logp, loss, dparams, stats,
                               stats_accumulate, as_stream(stream));
  return entry_done(rc, as_stream(stream));
}

int talos_ppo_fwd_bwd_f32(talos_plan plan, const float* params, const float* states, const int32_t* actions,
                          const float* adv, const float* ret, const float* old_logp, float* loss_out, float* dparams,
                          talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 2, TALOS_ERR_HANDLE, "%s: not a ppo plan", __func__);
  return talos_ppo_minibatch_f32(plan, plan->ppo.batch, params, states, nullptr, actions, adv, ret, old_logp,
                                 loss_out, dparams, nullptr, 0, stream);
}

static int ppo_head_loss(const char* fn, int n, int A, float clip_eps, float cv, float ce, const float* logits,
                         const float* values, const int32_t* actions, const float* adv, const float* ret,
                         const float* old_logp, float* loss, double* stats, int stats_acc, float* dlogits,
                         float* dvalues, talos_stream_t stream) {
  TALOS_REQUIRE(n >= 0 && A > 0, TALOS_ERR_SHAPE, "%s: bad shape n=%d n_actions=%d", fn, n, A);
  TALOS_REQUIRE(clip_eps >= 0.f, TALOS_ERR_SHAPE, "%s: clip_eps must be >= 0", fn);
  TALOS_REQUIRE(stats_acc == 0 || stats_acc == 1, TALOS_ERR_SHAPE, "%s: stats_accumulate must be 0 or 1", fn);
  TALOS_REQUIRE(n == 0 || (logits && values && actions && adv && ret && old_logp), TALOS_ERR_NULL,
                "%s: null input", fn);
  TALOS_DEVICE();
  const hipStream_t s = as_stream(stream);
  // an empty minibatch: the mean over no samples (NaN, as 0.0 / 0 in the reference's f64), no gradient
  const int nblk = (int)std::max<size_t>(1, ceil_div((size_t)n, 256));
  EntryScratch ws;
  int rc = ws.acquire((size_t)nblk * kLossParts * sizeof(double), s);
  if (rc) return rc;
  double* part = static_cast<double*>(ws.ptr);
  const int with_grad = dlogits != nullptr;
  hipLaunchKernelGGL(ppo_loss_kernel, dim3(nblk), dim3(256), 0, s, n, A, clip_eps, cv, ce, logits, values, actions,
                     adv, ret, old_logp, dlogits, dvalues, with_grad, part);
  rc = launch_status("ppo_loss_kernel");
  if (!rc && (loss || stats)) {
    hipLaunchKernelGGL(ppo_loss_final_kernel, dim3(1), dim3(64), 0, s, nblk, n, part, loss, stats, stats_acc);
    rc = launch_status("ppo_loss_final_kernel");
  }
  const int rel = ws.release();
  return entry_done(rc ? rc : rel, s);
}

int talos_ppo_head_loss_fwd_f32(int n, int n_actions, float clip_eps, float value_coef, float entropy_coef,
                                const float* logits, const float* values, const int32_t* actions, const float* adv,
                                const float* ret, const float* old_logp, float* loss, double* stats,
                                int stats_accumulate, talos_stream_t stream) {
  TALOS_REQUIRE(loss || stats, TALOS_ERR_NULL, "%s: loss and stats are both null", __func__);
  return ppo_head_loss(__func__, n, n_actions, clip_eps, value_coef, entropy_coef, logits, values, actions, adv, ret,
                       old_logp, loss, stats, stats_accumulate, nullptr, nullptr, stream);
}

int talos_ppo_head_loss_bwd_f32(int n, int n_actions, float clip_eps, float value_coef, float entropy_coef,
                                const float* logits, const float* values, const int32_t* actions, const float* adv,
                                const float* ret, const float* old_logp, float* dlogits, float* dvalues, float* loss,
                                talos_stream_t stream) {
  TALOS_NONNULL(dlogits);
  TALOS_NONNULL(dvalues);
  return ppo_head_loss(__func__, n, n_actions, clip_eps, value_coef, entropy_coef, logits, values, actions, adv, ret,
                       old_logp, loss, nullptr, 0, dlogits, dvalues, stream);
}

size_t talos_mla_param_count(const talos_mla_cfg* cfg) { return cfg ? mla_offsets(*cfg).end : 0; }

int talos_mla_plan_create(const talos_mla_cfg* cfg, talos_plan* plan) {
  TALOS_NONNULL(cfg);
  TALOS_NONNULL(plan);
  *plan = nullptr;
  int rc = check_mla_cfg(*cfg);
  if (rc) return rc;
  TALOS_DEVICE();
  auto* p = new talos_plan_s();
  p->kind = 3;
  p->prof = profiler_new();
  p->unfused = env_flag("TALOS_PLAN_UNFUSED");
  p->mla = *cfg;
  p->bf16 = cfg->precision == TALOS_PREC_BF16;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, 0) == hipSuccess) p->num_cu = prop.multiProcessorCount;
  const talos_mla_cfg& c = *cfg;
  const MlaDims D = mla_dims(c);
  const size_t M = (size_t)c.batch * c.seq, d = c.d_model, H = c.n_heads;
  p->layers.resize(1);
  auto& L = p->layers[0];
  rc = 0;
  rc |= plan_alloc(p, &L.xn1, M * d);
  rc |= plan_alloc(p, &L.rstd1, M);
  rc |= alloc_mla_layer(p, D, L);
  rc |= plan_alloc(p, &p->g_o, M * H * c.v_dim);
  rc |= plan_alloc(p, &p->g_xn, M * d);
  rc |= plan_alloc(p, &p->attn_ws, M * H);
  if (rc == TALOS_OK) rc = alloc_mla_scratch(p, D);
  // TALOS_MLA_ROWDOT=0 at plan creation: the attention backward forms D itself (attn_rowdot_kernel)
  const char* rowdot_env = std::getenv("TALOS_MLA_ROWDOT");
  p->rowdot = !(rowdot_env && rowdot_env[0] == '0');
  // TALOS_BF16_COPIES=0 at plan creation: no bf16 copies (every bf16-in product reads its fp32
  // operands and rounds them at staging; the same roundings, so the same results)
  const char* copies_env = std::getenv("TALOS_BF16_COPIES");
  const bool copies = !(copies_env && copies_env[0] == '0');
  if (rc == TALOS_OK && p->bf16 && !p->unfused && copies) {
    // the bf16 copies of every tensor a bf16-in product reads (the activations, the attention's
    // output and gradients, the latent's gradient, the weights and the output gradient)
    const size_t Hh = H * c.head_dim, Hr = H * c.rope_dim, Hv = H * c.v_dim, Lt = c.kv_latent;
    auto& m = p->ms;
    add_shadow(p, L.xn1, M * d, &rc);
    add_shadow(p, L.m.ckv, M * Lt, &rc);
    add_shadow(p, L.o, M * Hv, &rc);
    add_shadow(p, m.dqc, M * Hh, &rc);
    add_shadow(p, m.dqr, M * Hr, &rc);
    add_shadow(p, m.dkc, M * Hh, &rc);
    add_shadow(p, m.dkr, M * Hr, &rc);
    add_shadow(p, m.dv, M * Hv, &rc);
    add_shadow(p, m.dckv, M * Lt, &rc);
    p->p16 = add_shadow(p, nullptr, mla_offsets(c).end, &rc);
    p->g16 = add_shadow(p, nullptr, M * d, &rc);
    rc = rc ? TALOS_ERR_ALLOC : TALOS_OK;
  }
  if (rc == TALOS_OK) rc = upload_rope_table(p, c.seq, c.rope_dim, c.rope_base);
  if (rc == TALOS_OK) {
    p->red_ws_bytes = std::max(p->red_ws_bytes, rmsnorm_bwd_workspace_bytes((int)M, (int)d));
    rc = alloc_workspaces(p);
  }
  if (rc) {
    plan_free(p);
    delete p;
    return rc;
  }
  *plan = p;
  return TALOS_OK;
}

int talos_mla_fwd_bwd_f32(talos_plan plan, const float* params, const float* x, const float* gout, float* out,
                          float* dparams, float* dx, talos_stream_t stream) {
  TALOS_REQUIRE(plan != nullptr && plan->kind == 3, TALOS_ERR_HANDLE, "%s: not an mla plan", __func__);
  TALOS_NONNULL(params);
  TALOS_NONNULL(x);
  TALOS_NONNULL(gout);
  TALOS_NONNULL(out);
  TALOS_NONNULL(dparams);
  TALOS_NONNULL(dx);
  TALOS_DEVICE();
  PlanCall pc(plan);
  return entry_done(mla_fwd_bwd(plan, params, x, gout, out, dparams, dx, as_stream(stream)), as_stream(stream));
}

int talos_plan_profiler(talos_plan plan, talos_profiler* prof) {
  TALOS_REQUIRE(plan != nullptr && plan->prof != nullptr, TALOS_ERR_HANDLE, "%s: invalid plan", __func__);
  TALOS_NONNULL(prof);
  *prof = reinterpret_cast<talos_profiler>(plan->prof);
  return TALOS_OK;
}

int talos_plan_destroy(talos_plan plan) {
  if (plan == nullptr) return TALOS_OK;
  TALOS_DEVICE();
  (void)hipDeviceSynchronize();
  plan_free(plan);
  delete plan;
  return TALOS_OK;
}

}  // extern "C"
