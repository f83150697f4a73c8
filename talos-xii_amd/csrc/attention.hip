// attention.hip -- fused scaled-dot-product attention forward and backward for gfx950.
//
// Replaces the reference chain transpose -> batched_matmul_qt_k -> scale_tensor -> softmax ->
// batched_matmul_probs_v -> transpose (src/transformer.rs:519-557, 877-1121) and its backward
// closures (src/transformer.rs:920-955, 1010-1047, 1098-1117). q/k/v/o stay in the token-major
// projection layout [batch, seq, heads, dim] (row stride ld), so no transpose or reshape copy is
// ever made; the S x S score matrix never leaves registers.
//
// The sequences of the policy configurations are short (32..256 tokens, head dims 32..96), so
// one lane owns one query (forward, dQ) or one key (dK, dV) and keeps its rows in registers;
// key/value (or query/dO) tiles of all the (batch, head) pairs of a workgroup are staged in LDS
// and read as wave-wide broadcasts. The forward keeps an online (running max) softmax and saves
// lse = max + log(sum) per query; the backward recomputes P = exp(s - lse) and uses
// D_i = dO_i . O_i, so neither pass stores an S x S matrix. Causal masking (key j <= query i)
// is applied by loop bounds, so masked probabilities are exactly 0 and cost nothing.
#include "attention.hpp"

namespace talos {

struct AttnArgs {
  int B, S, H, dk, dv;
  float scale;
  int causal;
  const float* q;
  long long ldq;
  const float* k;
  long long ldk;
  const float* v;
  long long ldv;
  float* o;
  long long ldo;
  float* lse;
  const float* dout;
  long long lddo;
  float* dq;
  long long lddq;
  float* dk_out;
  long long lddk;
  float* dv_out;
  long long lddv;
  float* D;
  const float* rcos;
  const float* rsin;
  int rope_off, rope_dim;
  int P, QB, KT;
};

// Applies R^T (rotation by -theta at position pos) to dims [off, off + rdim) of a register row.
template <int DKM>
__device__ __forceinline__ void rope_transpose_row(float (&g)[DKM], const AttnArgs& a, int pos) {
  if (a.rcos == nullptr) return;
  const int half = a.rope_dim >> 1;
#pragma unroll
  for (int e = 0; e < DKM; e += 2) {
    if (e >= a.rope_off && e < a.rope_off + a.rope_dim) {
      const int pi = (e - a.rope_off) >> 1;
      const float c = a.rcos[pos * half + pi], s = a.rsin[pos * half + pi];
      const float g0 = g[e], g1 = g[e + 1];
      g[e] = g0 * c + g1 * s;
      g[e + 1] = -g0 * s + g1 * c;
    }
  }
}

// Dot product of a register row with an LDS row, as four independent FMA chains.
template <int D>
__device__ __forceinline__ float dot_row(const float (&r)[D], const float* __restrict__ t) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
  for (int e = 0; e < D; e += 4) {
    s0 = fmaf(r[e], t[e], s0);
    s1 = fmaf(r[e + 1], t[e + 1], s1);
    s2 = fmaf(r[e + 2], t[e + 2], s2);
    s3 = fmaf(r[e + 3], t[e + 3], s3);
  }
  return (s0 + s1) + (s2 + s3);
}

// Cooperative copy of rows [r0, r0 + nr) of each of the workgroup's P pairs into an LDS tile
// [P][nr][DM] (dims >= dim are zero-filled).
template <int DM>
__device__ __forceinline__ void stage_rows(float* tile, const float* __restrict__ src, long long ld, int dim,
                                           const AttnArgs& a, int pair0, int r0, int nr) {
  const int n = a.P * nr * DM;
  for (int idx = threadIdx.x; idx < n; idx += blockDim.x) {
    const int e = idx % DM;
    const int r = (idx / DM) % nr;
    const int pp = idx / (DM * nr);
    const int pair = pair0 + pp;
    const int row = r0 + r;
    float val = 0.f;
    if (e < dim && row < a.S && pair < a.B * a.H) {
      const int b = pair / a.H, h = pair % a.H;
      val = src[((long long)b * a.S + row) * ld + (long long)h * dim + e];
    }
    tile[idx] = val;
  }
}

template <int DKM, int DVM>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  float* Ks = smem;
  float* Vs = smem + a.P * a.KT * DKM;
  const int t = threadIdx.x;
  const int pl = t / a.QB;
  const int qi = blockIdx.y * a.QB + t % a.QB;
  const int pair0 = blockIdx.x * a.P;
  const int pair = pair0 + pl;
  const bool active = pl < a.P && pair < a.B * a.H && qi < a.S;
  const int b = pair / a.H, h = pair % a.H;

  float q[DKM], o[DVM];
#pragma unroll
  for (int e = 0; e < DKM; ++e) q[e] = 0.f;
#pragma unroll
  for (int e = 0; e < DVM; ++e) o[e] = 0.f;
  if (active) {
    const float* qr = a.q + ((long long)b * a.S + qi) * a.ldq + (long long)h * a.dk;
#pragma unroll
    for (int e = 0; e < DKM; ++e) q[e] = e < a.dk ? qr[e] * a.scale : 0.f;
  }
  float m = -INFINITY, l = 0.f;
  const int qmax = min(a.S, (int)(blockIdx.y + 1) * a.QB);  // exclusive bound of this block's queries
  const int kend = a.causal ? qmax : a.S;
  for (int k0 = 0; k0 < kend; k0 += a.KT) {
    const int nk = min(a.KT, kend - k0);
    __syncthreads();
    stage_rows<DKM>(Ks, a.k, a.ldk, a.dk, a, pair0, k0, a.KT);
    stage_rows<DVM>(Vs, a.v, a.ldv, a.dv, a, pair0, k0, a.KT);
    __syncthreads();
    if (!active) continue;
    const int jn = a.causal ? min(nk, qi - k0 + 1) : nk;
    const float* kt = Ks + pl * a.KT * DKM;
    const float* vt = Vs + pl * a.KT * DVM;
    for (int j = 0; j < jn; ++j) {
      const float s = dot_row<DKM>(q, kt + j * DKM);
      if (s > m) {
        const float corr = expf(m - s);
        l *= corr;
#pragma unroll
        for (int e = 0; e < DVM; ++e) o[e] *= corr;
        m = s;
      }
      const float p = expf(s - m);
      l += p;
#pragma unroll
      for (int e = 0; e < DVM; ++e) o[e] = fmaf(p, vt[j * DVM + e], o[e]);
    }
  }
  if (!active) return;
  const float inv = 1.0f / l;
  float* orow = a.o + ((long long)b * a.S + qi) * a.ldo + (long long)h * a.dv;
#pragma unroll
  for (int e = 0; e < DVM; ++e)
    if (e < a.dv) orow[e] = o[e] * inv;
  a.lse[(long long)pair * a.S + qi] = m + logf(l);
}

// dQ (and D = dO . O) with one lane per query.
template <int DKM, int DVM>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  float* Ks = smem;
  float* Vs = smem + a.P * a.KT * DKM;
  const int t = threadIdx.x;
  const int pl = t / a.QB;
  const int qi = blockIdx.y * a.QB + t % a.QB;
  const int pair0 = blockIdx.x * a.P;
  const int pair = pair0 + pl;
  const bool active = pl < a.P && pair < a.B * a.H && qi < a.S;
  const int b = pair / a.H, h = pair % a.H;

  float q[DKM], g[DVM], dq[DKM];
  float D = 0.f, lse = 0.f;
#pragma unroll
  for (int e = 0; e < DKM; ++e) q[e] = dq[e] = 0.f;
#pragma unroll
  for (int e = 0; e < DVM; ++e) g[e] = 0.f;
  if (active) {
    const long long tok = (long long)b * a.S + qi;
    const float* qr = a.q + tok * a.ldq + (long long)h * a.dk;
    const float* gr = a.dout + tok * a.lddo + (long long)h * a.dv;
    const float* orow = a.o + tok * a.ldo + (long long)h * a.dv;
#pragma unroll
    for (int e = 0; e < DKM; ++e) q[e] = e < a.dk ? qr[e] * a.scale : 0.f;
#pragma unroll
    for (int e = 0; e < DVM; ++e) {
      g[e] = e < a.dv ? gr[e] : 0.f;
      D = fmaf(g[e], e < a.dv ? orow[e] : 0.f, D);
    }
    lse = a.lse[(long long)pair * a.S + qi];
    a.D[(long long)pair * a.S + qi] = D;
  }
  const int qmax = min(a.S, (int)(blockIdx.y + 1) * a.QB);
  const int kend = a.causal ? qmax : a.S;
  for (int k0 = 0; k0 < kend; k0 += a.KT) {
    const int nk = min(a.KT, kend - k0);
    __syncthreads();
    stage_rows<DKM>(Ks, a.k, a.ldk, a.dk, a, pair0, k0, a.KT);
    stage_rows<DVM>(Vs, a.v, a.ldv, a.dv, a, pair0, k0, a.KT);
    __syncthreads();
    if (!active) continue;
    const int jn = a.causal ? min(nk, qi - k0 + 1) : nk;
    const float* kt = Ks + pl * a.KT * DKM;
    const float* vt = Vs + pl * a.KT * DVM;
    for (int j = 0; j < jn; ++j) {
      const float s = dot_row<DKM>(q, kt + j * DKM);
      const float dp = dot_row<DVM>(g, vt + j * DVM);
      const float p = expf(s - lse);
      const float ds = p * (dp - D);
#pragma unroll
      for (int e = 0; e < DKM; ++e) dq[e] = fmaf(ds, kt[j * DKM + e], dq[e]);
    }
  }
  if (!active) return;
#pragma unroll
  for (int e = 0; e < DKM; ++e) dq[e] *= a.scale;
  rope_transpose_row<DKM>(dq, a, qi);
  float* dqr = a.dq + ((long long)b * a.S + qi) * a.lddq + (long long)h * a.dk;
#pragma unroll
  for (int e = 0; e < DKM; ++e)
    if (e < a.dk) dqr[e] = dq[e];
}

// dK and/or dV with one lane per key; query-side rows (Q, dO, lse, D) staged in LDS.
template <int DKM, int DVM, bool DO_DK, bool DO_DV>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  float* Qs = smem;
  float* Gs = Qs + a.P * a.KT * DKM;
  float* Ls = Gs + a.P * a.KT * DVM;
  float* Ds = Ls + a.P * a.KT;
  const int t = threadIdx.x;
  const int pl = t / a.QB;
  const int kj = blockIdx.y * a.QB + t % a.QB;
  const int pair0 = blockIdx.x * a.P;
  const int pair = pair0 + pl;
  const bool active = pl < a.P && pair < a.B * a.H && kj < a.S;
  const int b = pair / a.H, h = pair % a.H;

  float k[DKM], v[DVM], dk[DKM], dv[DVM];
#pragma unroll
  for (int e = 0; e < DKM; ++e) k[e] = dk[e] = 0.f;
#pragma unroll
  for (int e = 0; e < DVM; ++e) v[e] = dv[e] = 0.f;
  if (active) {
    const long long tok = (long long)b * a.S + kj;
    const float* kr = a.k + tok * a.ldk + (long long)h * a.dk;
    const float* vr = a.v + tok * a.ldv + (long long)h * a.dv;
#pragma unroll
    for (int e = 0; e < DKM; ++e) k[e] = e < a.dk ? kr[e] * a.scale : 0.f;
    if (DO_DK) {
#pragma unroll
      for (int e = 0; e < DVM; ++e) v[e] = e < a.dv ? vr[e] : 0.f;
    }
  }
  // queries i >= the smallest key of this block contribute when causal
  const int qstart = a.causal ? (int)blockIdx.y * a.QB : 0;
  for (int i0 = qstart - (qstart % a.KT); i0 < a.S; i0 += a.KT) {
    const int ni = min(a.KT, a.S - i0);
    __syncthreads();
    stage_rows<DKM>(Qs, a.q, a.ldq, a.dk, a, pair0, i0, a.KT);
    stage_rows<DVM>(Gs, a.dout, a.lddo, a.dv, a, pair0, i0, a.KT);
    for (int idx = threadIdx.x; idx < a.P * a.KT; idx += blockDim.x) {
      const int pp = idx / a.KT, r = idx % a.KT;
      const int pr = pair0 + pp, row = i0 + r;
      const bool ok = pr < a.B * a.H && row < a.S;
      Ls[idx] = ok ? a.lse[(long long)pr * a.S + row] : 0.f;
      Ds[idx] = ok ? a.D[(long long)pr * a.S + row] : 0.f;
    }
    __syncthreads();
    if (!active) continue;
    const int ibeg = a.causal ? max(0, kj - i0) : 0;
    const float* qt = Qs + pl * a.KT * DKM;
    const float* gt = Gs + pl * a.KT * DVM;
    const float* lt = Ls + pl * a.KT;
    const float* dt = Ds + pl * a.KT;
    for (int i = ibeg; i < ni; ++i) {
      const float s = dot_row<DKM>(k, qt + i * DKM);
      const float p = expf(s - lt[i]);
      if (DO_DV) {
#pragma unroll
        for (int e = 0; e < DVM; ++e) dv[e] = fmaf(p, gt[i * DVM + e], dv[e]);
      }
      if (DO_DK) {
        const float dp = dot_row<DVM>(v, gt + i * DVM);
        const float ds = p * (dp - dt[i]);
#pragma unroll
        for (int e = 0; e < DKM; ++e) dk[e] = fmaf(ds, qt[i * DKM + e], dk[e]);
      }
    }
  }
  if (!active) return;
  const long long tok = (long long)b * a.S + kj;
  if (DO_DK) {
#pragma unroll
    for (int e = 0; e < DKM; ++e) dk[e] *= a.scale;
    rope_transpose_row<DKM>(dk, a, kj);
    float* dkr = a.dk_out + tok * a.lddk + (long long)h * a.dk;
#pragma unroll
    for (int e = 0; e < DKM; ++e)
      if (e < a.dk) dkr[e] = dk[e];
  }
  if (DO_DV) {
    float* dvr = a.dv_out + tok * a.lddv + (long long)h * a.dv;
#pragma unroll
    for (int e = 0; e < DVM; ++e)
      if (e < a.dv) dvr[e] = dv[e];
  }
}

// Workgroup geometry: P pairs x QB queries (QB = min(S, 256)), tile of KT rows such that the
// staged tiles stay within 48 KB of LDS.
static void geometry(AttnArgs& a, int dkm, int dvm, int extra_per_row) {
  a.QB = a.S < 256 ? a.S : 256;
  a.P = a.S < 256 ? 256 / a.S : 1;
  const int budget = 48 * 1024 / 4;
  int kt = budget / (a.P * (dkm + dvm + extra_per_row));
  kt = kt >= 64 ? 64 : (kt >= 32 ? 32 : (kt >= 16 ? 16 : 8));
  a.KT = kt;
}

static bool pick_dims(int dk, int dv, int* dkm, int* dvm) {
  if (dk <= 32 && dv <= 32) { *dkm = 32; *dvm = 32; return true; }
  if (dk <= 64 && dv <= 64) { *dkm = 64; *dvm = 64; return true; }
  if (dk <= 96 && dv <= 64) { *dkm = 96; *dvm = 64; return true; }
  if (dk <= 128 && dv <= 128) { *dkm = 128; *dvm = 128; return true; }
  return false;
}

// Algorithmic work of one pass over all (batch, head) pairs: `per_pair_flops` flops per
// (query, key) pair that the mask keeps, `bytes` of HBM traffic.
static double kept_pairs(const AttnArgs& a) {
  const double S = a.S;
  return (double)a.B * a.H * (a.causal ? S * (S + 1) / 2 : S * S);
}

#define ATTN_DISPATCH(DK, DV, KERNEL, ...)                                                          \
  if (dkm == DK && dvm == DV) {                                                                     \
    ProfScope ps(s, #KERNEL "<" #DK ", " #DV ">", flops, bytes);                                    \
    hipLaunchKernelGGL((KERNEL<DK, DV, ##__VA_ARGS__>), grid, dim3(256), lds, s, a);               \
    return launch_status(#KERNEL);                                                                  \
  }

int attn_fwd_launch(const AttnDesc& d, hipStream_t s) {
  int dkm, dvm;
  if (!pick_dims(d.dk, d.dv, &dkm, &dvm)) {
    set_error("attention: head dims (%d, %d) exceed the supported (128, 128)", d.dk, d.dv);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a{};
  a.B = d.batch; a.S = d.seq; a.H = d.heads; a.dk = d.dk; a.dv = d.dv; a.scale = d.scale; a.causal = d.causal;
  a.q = d.q; a.ldq = d.ldq; a.k = d.k; a.ldk = d.ldk; a.v = d.v; a.ldv = d.ldv;
  a.o = d.o; a.ldo = d.ldo; a.lse = d.lse;
  if ((long long)a.B * a.H * a.S == 0) return TALOS_OK;
  geometry(a, dkm, dvm, 0);
  const size_t lds = (size_t)a.P * a.KT * (dkm + dvm) * sizeof(float);
  dim3 grid(ceil_div((size_t)a.B * a.H, a.P), ceil_div(a.S, a.QB));
  const double rows = (double)a.B * a.S * a.H;  // (token, head) rows
  // QK^T and PV over the kept pairs; q, k, v read, o and lse written
  const double flops = kept_pairs(a) * (2.0 * a.dk + 2.0 * a.dv);
  const double bytes = 4.0 * rows * (2.0 * a.dk + a.dv) + 4.0 * rows * (a.dv + 1.0);
  ATTN_DISPATCH(32, 32, attn_fwd_kernel)
  ATTN_DISPATCH(64, 64, attn_fwd_kernel)
  ATTN_DISPATCH(96, 64, attn_fwd_kernel)
  ATTN_DISPATCH(128, 128, attn_fwd_kernel)
  return TALOS_ERR_UNSUPPORTED;
}

size_t attn_bwd_workspace_bytes(const AttnDesc& d) {
  return (size_t)d.batch * d.heads * d.seq * sizeof(float);
}

int attn_bwd_launch(const AttnDesc& d, float* ws, hipStream_t s) {
  int dkm, dvm;
  if (!pick_dims(d.dk, d.dv, &dkm, &dvm)) {
    set_error("attention: head dims (%d, %d) exceed the supported (128, 128)", d.dk, d.dv);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a{};
  a.B = d.batch; a.S = d.seq; a.H = d.heads; a.dk = d.dk; a.dv = d.dv; a.scale = d.scale; a.causal = d.causal;
  a.q = d.q; a.ldq = d.ldq; a.k = d.k; a.ldk = d.ldk; a.v = d.v; a.ldv = d.ldv;
  a.o = d.o; a.ldo = d.ldo; a.lse = d.lse;
  a.dout = d.dout; a.lddo = d.lddo;
  a.dq = d.dq; a.lddq = d.lddq; a.dk_out = d.dk_out; a.lddk = d.lddk; a.dv_out = d.dv_out; a.lddv = d.lddv;
  a.D = ws;
  a.rcos = d.rope_cos; a.rsin = d.rope_sin; a.rope_off = d.rope_off; a.rope_dim = d.rope_dim;
  if ((long long)a.B * a.H * a.S == 0) return TALOS_OK;
  const double rows = (double)a.B * a.S * a.H;
  int rc;
  {
    geometry(a, dkm, dvm, 0);
    const size_t lds = (size_t)a.P * a.KT * (dkm + dvm) * sizeof(float);
    dim3 grid(ceil_div((size_t)a.B * a.H, a.P), ceil_div(a.S, a.QB));
    // s = q.k, dp = dO.v, dq += ds k; reads q k v o dO lse, writes dq and D
    const double flops = kept_pairs(a) * (4.0 * a.dk + 2.0 * a.dv);
    const double bytes = 4.0 * rows * (3.0 * a.dk + 3.0 * a.dv + 2.0);
    rc = [&]() -> int {
      ATTN_DISPATCH(32, 32, attn_bwd_dq_kernel)
      ATTN_DISPATCH(64, 64, attn_bwd_dq_kernel)
      ATTN_DISPATCH(96, 64, attn_bwd_dq_kernel)
      ATTN_DISPATCH(128, 128, attn_bwd_dq_kernel)
      return TALOS_ERR_UNSUPPORTED;
    }();
    if (rc) return rc;
  }
  geometry(a, dkm, dvm, 2);
  const size_t lds = (size_t)a.P * a.KT * (dkm + dvm + 2) * sizeof(float);
  dim3 grid(ceil_div((size_t)a.B * a.H, a.P), ceil_div(a.S, a.QB));
  if (dkm + dvm <= 64) {
    // small heads: one pass computes both dK and dV; reads q dO lse D k v, writes dk dv
    const double flops = kept_pairs(a) * (4.0 * a.dk + 4.0 * a.dv);
    const double bytes = 4.0 * rows * (3.0 * a.dk + 3.0 * a.dv + 2.0);
    ATTN_DISPATCH(32, 32, attn_bwd_dkv_kernel, true, true)
  }
  rc = [&]() -> int {
    const double flops = kept_pairs(a) * (4.0 * a.dk + 2.0 * a.dv);
    const double bytes = 4.0 * rows * (3.0 * a.dk + 2.0 * a.dv + 2.0);
    ATTN_DISPATCH(64, 64, attn_bwd_dkv_kernel, true, false)
    ATTN_DISPATCH(96, 64, attn_bwd_dkv_kernel, true, false)
    ATTN_DISPATCH(128, 128, attn_bwd_dkv_kernel, true, false)
    return TALOS_ERR_UNSUPPORTED;
  }();
  if (rc) return rc;
  const double flops = kept_pairs(a) * (2.0 * a.dk + 2.0 * a.dv);
  const double bytes = 4.0 * rows * (2.0 * a.dk + 2.0 * a.dv + 1.0);
  ATTN_DISPATCH(64, 64, attn_bwd_dkv_kernel, false, true)
  ATTN_DISPATCH(96, 64, attn_bwd_dkv_kernel, false, true)
  ATTN_DISPATCH(128, 128, attn_bwd_dkv_kernel, false, true)
  return TALOS_ERR_UNSUPPORTED;
}

static int check_attn(const char* fn, int batch, int seq, int heads, int qk_dim, int v_dim, int causal, int ld_q,
                      int ld_k, int ld_v, int ld_o) {
  TALOS_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0 && qk_dim > 0 && v_dim > 0, TALOS_ERR_SHAPE,
                "%s: bad shape (batch=%d seq=%d heads=%d qk_dim=%d v_dim=%d)", fn, batch, seq, heads, qk_dim, v_dim);
  TALOS_REQUIRE(qk_dim <= 128 && v_dim <= 128, TALOS_ERR_UNSUPPORTED, "%s: head dims (%d, %d) exceed 128", fn, qk_dim,
                v_dim);
  TALOS_REQUIRE(causal == 0 || causal == 1, TALOS_ERR_DTYPE, "%s: causal must be 0 or 1", fn);
  TALOS_REQUIRE(ld_q >= heads * qk_dim && ld_k >= heads * qk_dim && ld_v >= heads * v_dim && ld_o >= heads * v_dim,
                TALOS_ERR_SHAPE, "%s: a row stride is smaller than heads * dim", fn);
  return TALOS_OK;
}

}  // namespace talos

using namespace talos;

extern "C" {

int talos_attn_fwd_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal, const float* q,
                       int ld_q, const float* k, int ld_k, const float* v, int ld_v, float* o, int ld_o, float* lse,
                       talos_stream_t stream) {
  TALOS_NONNULL(q);
  TALOS_NONNULL(k);
  TALOS_NONNULL(v);
  TALOS_NONNULL(o);
  TALOS_NONNULL(lse);
  int rc = check_attn(__func__, batch, seq, heads, qk_dim, v_dim, causal, ld_q, ld_k, ld_v, ld_o);
  if (rc) return rc;
  TALOS_DEVICE();
  AttnDesc d;
  d.batch = batch; d.seq = seq; d.heads = heads; d.dk = qk_dim; d.dv = v_dim; d.scale = scale; d.causal = causal;
  d.q = q; d.ldq = ld_q; d.k = k; d.ldk = ld_k; d.v = v; d.ldv = ld_v; d.o = o; d.ldo = ld_o; d.lse = lse;
  return attn_fwd_launch(d, as_stream(stream));
}

int talos_attn_bwd_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal, const float* q,
                       int ld_q, const float* k, int ld_k, const float* v, int ld_v, const float* o, int ld_o,
                       const float* lse, const float* dout, int ld_do, float* dq, int ld_dq, float* dk, int ld_dk,
                       float* dv, int ld_dv, talos_stream_t stream) {
  TALOS_NONNULL(q);
  TALOS_NONNULL(k);
  TALOS_NONNULL(v);
  TALOS_NONNULL(o);
  TALOS_NONNULL(lse);
  TALOS_NONNULL(dout);
  TALOS_NONNULL(dq);
  TALOS_NONNULL(dk);
  TALOS_NONNULL(dv);
  int rc = check_attn(__func__, batch, seq, heads, qk_dim, v_dim, causal, ld_q, ld_k, ld_v, ld_o);
  if (rc) return rc;
  TALOS_REQUIRE(ld_do >= heads * v_dim && ld_dq >= heads * qk_dim && ld_dk >= heads * qk_dim && ld_dv >= heads * v_dim,
                TALOS_ERR_SHAPE, "%s: a gradient row stride is smaller than heads * dim", __func__);
  TALOS_DEVICE();
  AttnDesc d;
  d.batch = batch; d.seq = seq; d.heads = heads; d.dk = qk_dim; d.dv = v_dim; d.scale = scale; d.causal = causal;
  d.q = q; d.ldq = ld_q; d.k = k; d.ldk = ld_k; d.v = v; d.ldv = ld_v;
  d.o = const_cast<float*>(o); d.ldo = ld_o; d.lse = const_cast<float*>(lse);
  d.dout = dout; d.lddo = ld_do; d.dq = dq; d.lddq = ld_dq; d.dk_out = dk; d.lddk = ld_dk; d.dv_out = dv; d.lddv = ld_dv;
  hipStream_t s = as_stream(stream);
  float* ws = nullptr;
  const size_t bytes = attn_bwd_workspace_bytes(d);
  if (bytes) TALOS_HIP(hipMallocAsync(reinterpret_cast<void**>(&ws), bytes, s));
  rc = attn_bwd_launch(d, ws, s);
  if (ws) TALOS_HIP(hipFreeAsync(ws, s));
  return rc;
}

}  // extern "C"
