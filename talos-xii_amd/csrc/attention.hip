// attention.hip -- fused scaled-dot-product attention forward and backward on CDNA4 matrix cores.
//
// Replaces the reference chain transpose -> batched_matmul_qt_k -> scale_tensor -> softmax ->
// batched_matmul_probs_v -> transpose (src/transformer.rs:519-557, 877-1121) and its backward
// closures (src/transformer.rs:920-955, 1010-1047, 1098-1117). q/k/v/o stay in the token-major
// projection layout [batch, seq, heads, dim] (row stride ld), so no transpose or reshape copy is
// ever made, and no S x S matrix is ever stored.
//
// Work unit: one wave64 per 32-row block of one (batch, head) pair -- a query block for the
// forward and dQ, a key block for dK / dV. Every product is a chain of v_mfma_f32_32x32x2_f32
// over the head dimension or over a 32-key / 32-query block:
//   forward   S^T[key, q] = K . Q^T        O[q, e]  += P . V
//   dQ pass   S^T, dP^T[key, q] = V . dO^T, dS^T = P^T (dP^T - D)     dQ[q, e] += dS . K
//   dK/dV     S[q, key] = Q . K^T, dP = dO . V^T, dS = P (dP - D)     dV += P^T . dO, dK += dS^T . Q
// The 32x32 accumulator layout of the score MFMA (lane <-> column, register r <-> row
// 8*(r/4) + 4*(lane/32) + r%4) is exactly the A-operand layout of the next MFMA when the
// contraction over the block's 32 rows visits them in that order, so probabilities feed the
// second product straight from registers. Operand rows are read from global memory by the lane
// that owns them (each lane holds half of a row: elements [D/2 * (lane/32), D/2 * (lane/32 + 1))).
// The forward makes two passes over the key blocks when there are several (row max / sum, then
// normalised P . V) and saves lse = max + log(sum); the backward recomputes P = exp(s - lse)
// and uses D_q = dO_q . O_q. Causal masking (key <= query) and the sequence end are applied to
// the scores, so masked probabilities are exactly 0; key blocks past the diagonal are skipped.
#include <cstdlib>
#include <mutex>

#include "attention.hpp"

namespace talos {

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct AttnArgs {
  int B, S, H, dk, dv;
  float scale;
  int causal;
  float* ds;  // the tiled backward's dS rows ([B*H][S][S]) when it forms dQ from them, else null
  // with ds: dq / dk columns [dsplit, dk) of each head go to dq2 / dk2 (head width dk - dsplit) and
  // columns [0, dsplit) to dq / dk_out at head width dsplit (null: one buffer, head width dk)
  float *dq2, *dk2;
  long long lddq2, lddk2;
  int dsplit;
  int out16;  // the bf16 dS kernels: dq / dq2 / dk_out / dk2 / dv_out are bf16 buffers (AttnDesc::out_bf16)
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
  int vec;  // every row half is 16-byte aligned and the head dims equal the template dims
  const int32_t* lens;  // per-batch key count (nullptr: all S keys)
  const float* q_last;  // last-query kernels: unrotated query rows [B, H*dk] (nullptr: q's rows)
  long long ldq_last;
  float* dq_last;       // last-query backward: the query gradient rows [B, H*dk] (nullptr: dq)
  long long lddq_last;
};

// Keys of batch entry b that take part: lens[b] clamped to [0, S] (rows past it are padding).
__device__ __forceinline__ int key_len(const AttnArgs& a, int b) {
  if (a.lens == nullptr) return a.S;
  const int L = a.lens[b];
  return L < 0 ? 0 : (L > a.S ? a.S : L);
}

constexpr float kNegInf = -INFINITY;
// Every exponential here is of a softmax argument s - max or s - lse (<= 0, -inf for a masked
// key): __expf, the hardware exp2 of the scaled argument (relative error about |x| 2^-24, and
// exactly 0 at -inf), instead of expf's range-reduced sequence of a dozen instructions.

// Load style per kernel (SEL of load_half) and minimum waves per SIMD the register allocation
// must allow (compile-time tuning knobs).
#ifndef TALOS_ATTN_FWD_SEL
#define TALOS_ATTN_FWD_SEL 0
#endif
#ifndef TALOS_ATTN_BWD_SEL
#define TALOS_ATTN_BWD_SEL 0
#endif
#ifndef TALOS_ATTN_FUSED_SEL
#define TALOS_ATTN_FUSED_SEL 1
#endif
constexpr bool kFwdSel = TALOS_ATTN_FWD_SEL, kBwdSel = TALOS_ATTN_BWD_SEL, kFusedSel = TALOS_ATTN_FUSED_SEL;
#ifndef TALOS_ATTN_FWD_WAVES
#define TALOS_ATTN_FWD_WAVES 1
#endif
#ifndef TALOS_ATTN_BWD_WAVES
#define TALOS_ATTN_BWD_WAVES 1
#endif

// Zeros that out-of-range rows and columns read instead of memory: selecting the address (not the
// loaded value) keeps every load unconditional, so a lane's loads issue back to back with no
// branch around them, and the values are exactly 0.
__device__ __align__(16) float kAttnZeros[128] = {};  // global (not constant) memory: selecting between it and a row keeps global loads

// Loads half of row `row` (elements [HALF*h, HALF*h + HALF) of the head's `dim` values starting
// at column col0) times `scale`; rows >= S and elements >= dim read as 0. SEL = true selects the
// address (kAttnZeros for the out-of-range rows / columns), so the loads are unconditional and
// issue back to back at the cost of registers; SEL = false branches around them (fewer registers,
// more waves per SIMD).
template <int HALF, bool SEL>
__device__ __forceinline__ void load_half(float (&r)[HALF], const float* __restrict__ base, long long ld,
                                          long long tok0, int row, int S, int col0, int dim, int h, float scale,
                                          bool vec) {
  if (!SEL && row >= S) {
#pragma unroll
    for (int i = 0; i < HALF; ++i) r[i] = 0.f;
    return;
  }
  const float* src = (!SEL || row < S) ? base + (tok0 + row) * ld + col0 : kAttnZeros;
  if (vec) {
#pragma unroll
    for (int i = 0; i < HALF; i += 4) {
      const float4 v = *reinterpret_cast<const float4*>(src + HALF * h + i);
      r[i] = v.x * scale;
      r[i + 1] = v.y * scale;
      r[i + 2] = v.z * scale;
      r[i + 3] = v.w * scale;
    }
  } else {
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
      const int e = HALF * h + i;
      if (SEL)
        r[i] = *(e < dim ? src + e : kAttnZeros + e) * scale;
      else
        r[i] = e < dim ? src[e] * scale : 0.f;
    }
  }
}

// Row index within a 32-row block held by accumulator register r of this lane.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// acc += X_block . Y_block^T over the head dimension: lane rows x (A operand, rows of the result)
// and y (B operand, columns of the result), both given as this lane's row halves.
template <int HALF>
__device__ __forceinline__ floatx16 mfma_rows(const float (&x)[HALF], const float (&y)[HALF], floatx16 acc) {
#pragma unroll
  for (int s = 0; s < HALF; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(x[s], y[s], acc, 0, 0, 0);
  return acc;
}

// acc[eb] += P_block . M[rows of the block, eb*32 + lane%32] for each 32-column block eb of the
// head: P is given in accumulator layout (register s <-> block row acc_row(s, h)), M is read
// from global memory row by row (rows >= S and columns >= dim read as 0).
template <int NB, bool SEL>
__device__ __forceinline__ void mfma_p_rows(const float (&P)[16], const float* __restrict__ base, long long ld,
                                            long long tok0, int row0, int S, int col0, int dim, int l32, int h,
                                            floatx16 (&acc)[NB]) {
  // out-of-range rows / columns read as 0 (SEL: see load_half)
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const int row = row0 + acc_row(s, h);
    const float* src = base + (tok0 + row) * ld + col0;
#pragma unroll
    for (int eb = 0; eb < NB; ++eb) {
      const int e = eb * 32 + l32;
      float m;
      if (SEL)
        m = *((row < S && e < dim) ? src + e : kAttnZeros + e);
      else
        m = (row < S && e < dim) ? src[e] : 0.f;
      acc[eb] = __builtin_amdgcn_mfma_f32_32x32x2f32(P[s], m, acc[eb], 0, 0, 0);
    }
  }
}

// Applies R^T (rotation by -theta at position pos) to an output element of column e whose
// pair partner (column e ^ 1) sits in the neighbouring lane. All lanes must call it.
// Branch-free: the table (kAttnZeros when there is none) is read at a clamped index and the
// result selected, so the loads of consecutive elements issue back to back.
__device__ __forceinline__ float rope_t(float g, int e, int pos, const AttnArgs& a, bool active) {
  const float partner = __shfl_xor(g, 1, 64);
  const bool table = a.rcos != nullptr;
  const int half = a.rope_dim >> 1;
  const bool in = table && active && e >= a.rope_off && e < a.rope_off + a.rope_dim;
  const int idx = in ? pos * half + ((e - a.rope_off) >> 1) : 0;
  const float c = (table ? a.rcos : kAttnZeros)[idx], s = (table ? a.rsin : kAttnZeros)[idx];
  // (g0, g1) -> (g0 c + g1 s, -g0 s + g1 c)
  const float rot = (e & 1) ? fmaf(-partner, s, g * c) : fmaf(g, c, partner * s);
  return in ? rot : g;
}

// ---------------------------------------------------------------------------
// Forward: wave per (pair, query block)
// ---------------------------------------------------------------------------
template <int DKM, int DVM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_FWD_WAVES))) void attn_fwd_kernel(
    AttnArgs a) {
  constexpr int KH = DKM / 2, OB = DVM / 32;
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int nqb = (a.S + 31) >> 5;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.B * a.H * nqb) return;  // uniform per wave
  const int pair = item / nqb, qb = item % nqb;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int q = qb * 32 + l32;  // this lane's query (score columns)
  const int Sk = key_len(a, b);

  float qv[KH];
  load_half<KH, kFwdSel>(qv, a.q, a.ldq, tok0, q, a.S, hd * a.dk, a.dk, h, a.scale, a.vec);
  const int kb_last = a.causal ? min(qb, (Sk - 1) >> 5) : (Sk - 1) >> 5;

  // scores of key block kb in S^T layout, masked
  auto scores = [&](int kb, float (&sv)[16]) {
    float kv[KH];
    load_half<KH, kFwdSel>(kv, a.k, a.ldk, tok0, kb * 32 + l32, a.S, hd * a.dk, a.dk, h, 1.f, a.vec);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    acc = mfma_rows<KH>(kv, qv, acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb * 32 + acc_row(r, h);
      const bool ok = key < Sk && (!a.causal || key <= q);
      sv[r] = ok ? acc[r] : kNegInf;
    }
  };

  float m = kNegInf, l = 0.f;
  float sv[16];
  for (int kb = 0; kb <= kb_last; ++kb) {
    scores(kb, sv);
    float bm = kNegInf;
#pragma unroll
    for (int r = 0; r < 16; ++r) bm = fmaxf(bm, sv[r]);
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    float bs = 0.f;
    if (mn != kNegInf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) bs += __expf(sv[r] - mn);
    }
    bs += __shfl_xor(bs, 32, 64);
    l = (m == kNegInf ? 0.f : l * __expf(m - mn)) + bs;
    m = mn;
  }
  const float inv_l = l > 0.f ? 1.f / l : 0.f;

  floatx16 oacc[OB];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[ob][r] = 0.f;
  for (int kb = 0; kb <= kb_last; ++kb) {
    if (kb_last > 0) scores(kb, sv);  // one key block: the scores of pass 1 are still in sv
    float P[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) P[r] = (m == kNegInf) ? 0.f : __expf(sv[r] - m) * inv_l;
    mfma_p_rows<OB, kFwdSel>(P, a.v, a.ldv, tok0, kb * 32, a.S, hd * a.dv, a.dv, l32, h, oacc);
  }
  // O in accumulator layout: register r <-> query qb*32 + acc_row(r, h), lane <-> column
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = ob * 32 + l32;
      if (qr < a.S && e < a.dv) a.o[(tok0 + qr) * a.ldo + hd * a.dv + e] = oacc[ob][r];
    }
  if (h == 0 && q < a.S) a.lse[(long long)pair * a.S + q] = (l > 0.f) ? m + logf(l) : kNegInf;
}

// Forward for S <= 32 at head dims 32 / 32 with 16-byte rows: one key block, so a wave's q, k and
// v rows are all in flight before the first product and the softmax needs no running rescale.
// Same arithmetic as attn_fwd_kernel's single-block pass. s32_pair is one wave's (batch, head)
// pair: it stores O and the row logsumexp and returns O in accumulator layout (register r <->
// query acc_row(r, h), lane <-> column l32).
__device__ __forceinline__ floatx16 s32_pair(const AttnArgs& a, int pair, int l32, int h) {
  constexpr int KH = 16;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int q = l32;
  const int Sk = key_len(a, b);
  float qv[KH], kv[KH], vm[16];
  load_half<KH, true>(qv, a.q, a.ldq, tok0, q, a.S, hd * a.dk, 32, h, a.scale, true);
  load_half<KH, true>(kv, a.k, a.ldk, tok0, l32, a.S, hd * a.dk, 32, h, 1.f, true);
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const int row = acc_row(s, h);
    vm[s] = *(row < a.S ? a.v + (tok0 + row) * a.ldv + hd * a.dv + l32 : kAttnZeros + l32);
  }
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  acc = mfma_rows<KH>(kv, qv, acc);  // S^T: register r <-> key acc_row(r, h), lane <-> query
  float sv[16], m = kNegInf;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = acc_row(r, h);
    const bool ok = key < Sk && (!a.causal || key <= q);
    sv[r] = ok ? acc[r] : kNegInf;
    m = fmaxf(m, sv[r]);
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.f;
  if (m != kNegInf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) l += __expf(sv[r] - m);
  }
  l += __shfl_xor(l, 32, 64);
  const float inv_l = l > 0.f ? 1.f / l : 0.f;
  floatx16 oacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) oacc[r] = 0.f;
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float p = (m == kNegInf) ? 0.f : __expf(sv[s] - m) * inv_l;
    oacc = __builtin_amdgcn_mfma_f32_32x32x2f32(p, vm[s], oacc, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int qr = acc_row(r, h);
    if (qr < a.S) a.o[(tok0 + qr) * a.ldo + hd * a.dv + l32] = oacc[r];
  }
  if (h == 0 && q < a.S) a.lse[(long long)pair * a.S + q] = (l > 0.f) ? m + logf(l) : kNegInf;
  return oacc;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_FWD_WAVES))) void
attn_fwd_s32_kernel(AttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= a.B * a.H) return;  // uniform per wave
  (void)s32_pair(a, pair, lane & 31, lane >> 5);
}

// The attention output projection, its residual and the next RMSNorm fused behind the S <= 32
// attention of four 32-wide heads (d = 128): h2 = x + O.Wo, xn = rmsnorm(h2) * gain, rstd (the
// first product of the block's MLP half and its norm epilogue, in the order the GEMM epilogue
// adds them). A workgroup is one batch entry: its four waves are the entry's four heads, whose O
// blocks meet in LDS as the entry's [32, 128] attention output; wave w then forms the columns
// [32 w, 32 w + 32) of O.Wo with v_mfma_f32_32x32x2f32 (A = O rows from LDS, B = Wo rows from
// memory, both walking k in the same order 8j + 4h + q), and after a second pass through LDS each
// wave takes eight whole token rows for the residual, the row norm and the coalesced stores.
constexpr int kWoD = 128, kWoP = kWoD + 4;
struct WoArgs {
  const float* wo;     // [128, 128], row k = input feature
  const float* resid;  // x, rows of 128
  float* h2;
  const float* gain;
  float* xn;
  float* rstd;
  float eps;
};
// The tail both fused kernels share, once the entry's attention output rows [0, 32 RB) are in T
// (pitch kWoP): wave wv (of 4 RB) forms the 32 x 32 block (rows 32 (wv / 4).., columns
// 32 (wv % 4)..) of O.Wo with v_mfma_f32_32x32x2f32 (A = O rows from T, B = Wo rows from memory,
// both walking k in the order 8j + 4h + q), the blocks pass through T again, and wave wv takes
// the eight token rows 8 wv .. 8 wv + 7 for the residual, the row norm and the stores (lane <->
// columns 2 lane, 2 lane + 1). Rows >= nrows are neither read nor written.
template <int RB>
__device__ __forceinline__ void wo_resid_norm(const WoArgs& w, float* T, long long tok0, int nrows, int lane,
                                              int wv) {
  const int l32 = lane & 31, h = lane >> 5;
  const int r0 = 32 * (wv >> 2), n = 32 * (wv & 3) + l32;
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll 4
  for (int j = 0; j < kWoD / 8; ++j) {
    const float4 o4 = *reinterpret_cast<const float4*>(T + (r0 + l32) * kWoP + 8 * j + 4 * h);
    const float* wr = w.wo + (long long)(8 * j + 4 * h) * kWoD + n;
    const float w0 = wr[0], w1 = wr[kWoD], w2 = wr[2 * kWoD], w3 = wr[3 * kWoD];
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(o4.x, w0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(o4.y, w1, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(o4.z, w2, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(o4.w, w3, acc, 0, 0, 0);
  }
  __syncthreads();  // every wave has read the O rows
#pragma unroll
  for (int r = 0; r < 16; ++r) T[(r0 + acc_row(r, h)) * kWoP + n] = acc[r];
  __syncthreads();
  float2 res[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = wv * 8 + i;
    res[i] = t < nrows ? *reinterpret_cast<const float2*>(w.resid + (tok0 + t) * kWoD + 2 * lane)
                       : make_float2(0.f, 0.f);
  }
  const float2 g = *reinterpret_cast<const float2*>(w.gain + 2 * lane);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int t = wv * 8 + i;
    if (t >= nrows) break;  // uniform per wave
    const float2 pv = *reinterpret_cast<const float2*>(T + t * kWoP + 2 * lane);
    const float2 v = make_float2(pv.x + res[i].x, pv.y + res[i].y);
    const long long row = tok0 + t;
    *reinterpret_cast<float2*>(w.h2 + row * kWoD + 2 * lane) = v;
    const float ss = wave_sum(v.x * v.x + v.y * v.y);
    const float r = 1.0f / sqrtf(ss / (float)kWoD + w.eps);
    *reinterpret_cast<float2*>(w.xn + row * kWoD + 2 * lane) = make_float2(v.x * r * g.x, v.y * r * g.y);
    if (lane == 0 && w.rstd) w.rstd[row] = r;
  }
}

// compiled with a four-wave occupancy hint (the compiler then schedules it into 96 VGPRs instead
// of 100; both allow five waves a SIMD): 122.7 -> 115.6 us at C4, measured
#ifndef TALOS_ATTN_FWD_WO_WAVES
#define TALOS_ATTN_FWD_WO_WAVES 4
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_FWD_WO_WAVES))) void
attn_fwd_s32_wo_kernel(AttnArgs a, WoArgs w) {
  __shared__ __align__(16) float T[32 * kWoP];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int b = blockIdx.x;
  const floatx16 oacc = s32_pair(a, b * 4 + wv, l32, h);
#pragma unroll
  for (int r = 0; r < 16; ++r) T[acc_row(r, h) * kWoP + wv * 32 + l32] = oacc[r];
  __syncthreads();
  wo_resid_norm<1>(w, T, (long long)b * a.S, a.S, lane, wv);
}

// The same for 32 < S <= 64: a workgroup of eight waves per batch entry. The entry's V rows [64,
// 128] are staged in LDS first (coalesced float4 loads; the P.V products read their B operand
// there, which keeps the kernel within 128 VGPRs, two workgroups per CU). Wave wv takes the
// query block qb = wv / 4 of head wv % 4 (so each SIMD holds one wave of each query block, and
// the causal first block, which has one key block, pairs with the second, which has two): the
// scores of its one or two key blocks in S^T layout, one softmax over both, O = P.V as in
// s32_pair, O and lse stored, and O's block into T. Then O.Wo and the rows as above, over the
// entry's 64 token rows.
constexpr int kVP = kWoD + 8;  // V tile pitch: rows 4 apart start 32 banks apart
__global__ __launch_bounds__(512) void attn_fwd_s64_wo_kernel(AttnArgs a, WoArgs w) {
  constexpr int KH = 16;
  __shared__ __align__(16) float T[64 * kWoP];
  __shared__ __align__(16) float Vs[64 * kVP];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int b = blockIdx.x, hd = wv & 3, qb = wv >> 2, pair = b * 4 + hd;
  const long long tok0 = (long long)b * a.S;
  const int q = 32 * qb + l32;
  const int Sk = key_len(a, b);
  const bool two = (!a.causal || qb == 1) && Sk > 32;  // the second key block takes part (uniform)
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // V rows: 64 x 32 float4s, rows >= S as zeros
    const int idx = threadIdx.x + 512 * i, row = idx >> 5, c = 4 * (idx & 31);
    const float* src = row < a.S ? a.v + (tok0 + row) * a.ldv + c : kAttnZeros + c;
    *reinterpret_cast<float4*>(Vs + row * kVP + c) = *reinterpret_cast<const float4*>(src);
  }
  float qv[KH], kv[2][KH];
  load_half<KH, true>(qv, a.q, a.ldq, tok0, q, a.S, hd * a.dk, 32, h, a.scale, true);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (kb == 1 && !two) break;
    load_half<KH, true>(kv[kb], a.k, a.ldk, tok0, 32 * kb + l32, a.S, hd * a.dk, 32, h, 1.f, true);
  }
  float sv[2][16], m = kNegInf;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (kb == 1 && !two) break;
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    acc = mfma_rows<KH>(kv[kb], qv, acc);  // S^T: register r <-> key 32 kb + acc_row(r, h), lane <-> query
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = 32 * kb + acc_row(r, h);
      const bool ok = key < Sk && (!a.causal || key <= q);
      sv[kb][r] = ok ? acc[r] : kNegInf;
      m = fmaxf(m, sv[kb][r]);
    }
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  float l = 0.f;
  if (m != kNegInf) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      if (kb == 1 && !two) break;
#pragma unroll
      for (int r = 0; r < 16; ++r) l += __expf(sv[kb][r] - m);
    }
  }
  l += __shfl_xor(l, 32, 64);
  const float inv_l = l > 0.f ? 1.f / l : 0.f;
  __syncthreads();  // the V tile is staged
  floatx16 oacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) oacc[r] = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    if (kb == 1 && !two) break;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const float p = (m == kNegInf) ? 0.f : __expf(sv[kb][s] - m) * inv_l;
      const float vm = Vs[(32 * kb + acc_row(s, h)) * kVP + hd * 32 + l32];
      oacc = __builtin_amdgcn_mfma_f32_32x32x2f32(p, vm, oacc, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int qr = 32 * qb + acc_row(r, h);
    if (qr < a.S) a.o[(tok0 + qr) * a.ldo + hd * a.dv + l32] = oacc[r];
    T[qr * kWoP + hd * 32 + l32] = oacc[r];
  }
  if (h == 0 && q < a.S) a.lse[(long long)pair * a.S + q] = (l > 0.f) ? m + logf(l) : kNegInf;
  __syncthreads();
  wo_resid_norm<2>(w, T, tok0, a.S, lane, wv);
}

// ---------------------------------------------------------------------------
// Forward for seq > 32: a workgroup per (pair, tile of 128 queries), one wave per 32-query block.
// K and V stream through LDS in blocks of 32 keys, one copy serving the four waves, the next
// block fetched into registers while the current one is in use. One pass with the running
// softmax: a block's scores raise the row maximum, and the O accumulators and the row sum are
// rescaled by exp(m_old - m_new) before the block's P.V is added. S^T layout as
// attn_fwd_kernel (register r <-> key acc_row(r, h), lane <-> query), so the probabilities are
// the A operand of P.V straight from registers; the per-query factors reach O's layout
// (register r <-> query acc_row(r, h)) through a 32-float LDS slice per wave.
// ---------------------------------------------------------------------------
constexpr int kQTile = 128;  // queries per workgroup (4 waves x 32)

// Element group g (4 consecutive floats) of a [32 rows, DM] block starting at row0: row 4g / DM,
// column 4g % DM; rows >= nrows and columns >= dim read as 0.
template <int DM>
__device__ __forceinline__ float4 block_ld4(const float* __restrict__ base, long long ld, long long tok0, int row0,
                                            int nrows, int col0, int dim, int g, bool vec) {
  const int idx = 4 * g, row = idx / DM, col = idx % DM;
  const int r = row0 + row;
  if (r >= nrows) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float* src = base + (tok0 + r) * ld + col0 + col;
  if (vec) return *reinterpret_cast<const float4*>(src);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = col + j < dim ? src[j] : 0.f;
  return make_float4(v[0], v[1], v[2], v[3]);
}
// block_ld4's element group g as an offset from the block's first element (row0's, at col0): where
// every row of a block is below nrows and dim == DM (16-byte rows), a tiled kernel's loop loads
// it from the block's wave-uniform start plus this loop-invariant offset, one unconditional
// float4 load each (rows * ld < 2^31: the plans' 32-bit indexing bound)
template <int DM>
__device__ __forceinline__ int block_off(long long ld, int g) {
  const int idx = 4 * g;
  return (int)((idx / DM) * ld) + idx % DM;
}
// ... and its place in an LDS block of pitch P
template <int DM, int P>
__device__ __forceinline__ void block_st4(float* tile, int g, float4 v) {
  const int idx = 4 * g;
  *reinterpret_cast<float4*>(tile + (idx / DM) * P + idx % DM) = v;
}

// q / k rows of head hd (a kernel's AttnArgs a and tok0 in scope)
#define ATTN_LD_Q_HALF(HALF, SEL, r, row, h, scale) \
  load_half<HALF, SEL>(r, a.q, a.ldq, tok0, row, a.S, hd * a.dk, a.dk, h, scale, a.vec)
#define ATTN_LD_K_HALF(HALF, SEL, r, row, h, scale) \
  load_half<HALF, SEL>(r, a.k, a.ldk, tok0, row, a.S, hd * a.dk, a.dk, h, scale, a.vec)
#define ATTN_BLK_Q(DM, row0, g) block_ld4<DM>(a.q, a.ldq, tok0, row0, a.S, hd * a.dk, a.dk, g, a.vec)
#define ATTN_BLK_K(DM, row0, g) block_ld4<DM>(a.k, a.ldk, tok0, row0, a.S, hd * a.dk, a.dk, g, a.vec)

// Orders the wave's own LDS writes before its later reads (no workgroup barrier).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-query factors of this wave (lane l32 holds query l32's; h == 0 writes) into O's layout:
// f[r] is the factor of query acc_row(r, h).
__device__ __forceinline__ void bcast_rows(float* slice, float v, int l32, int h, float (&f)[16]);

#ifndef TALOS_ATTN_TILED_WAVES
#define TALOS_ATTN_TILED_WAVES 3
#endif
template <int DKM, int DVM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DKM > 64 ? 2 : TALOS_ATTN_TILED_WAVES))) void
attn_fwd_tiled_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, OB = DVM / 32;
  constexpr int PK = DKM + 4, PV = DVM + 4;  // 16-byte rows; eight consecutive rows on distinct bank groups
  constexpr int KL = DKM / 32, VL = DVM / 32;  // float4 groups per thread per block
  __shared__ __align__(16) float Ks[32 * PK];
  __shared__ __align__(16) float Vs[32 * PV];
  __shared__ __align__(16) float Wr[4][32];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b);
  const int qb = tile * 4 + wv;
  const int q = qb * 32 + l32;
  const bool wave_on = qb * 32 < a.S;
  const int q_hi = min(a.S, (tile + 1) * kQTile) - 1;
  const int kb_end = Sk == 0 ? -1 : (a.causal ? min(q_hi, Sk - 1) : Sk - 1) >> 5;  // uniform per workgroup
  const int wave_kb_end = a.causal ? min(kb_end, qb) : kb_end;

  float qv[KH];
  ATTN_LD_Q_HALF(KH, kFwdSel, qv, q, h, a.scale);
  float4 rk[KL], rv[VL];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rk[i] = ATTN_BLK_K(DKM, kb * 32, i * 256 + (int)threadIdx.x);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      rv[i] = block_ld4<DVM>(a.v, a.ldv, tok0, kb * 32, a.S, hd * a.dv, a.dv, i * 256 + (int)threadIdx.x, a.vec);
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4<DKM, PK>(Ks, i * 256 + (int)threadIdx.x, rk[i]);
#pragma unroll
    for (int i = 0; i < VL; ++i) block_st4<DVM, PV>(Vs, i * 256 + (int)threadIdx.x, rv[i]);
  };

  float m = kNegInf, l = 0.f;
  floatx16 oacc[OB];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[ob][r] = 0.f;
  if (kb_end >= 0) {
    fetch(0);
    stash();
  }
  __syncthreads();
  for (int kb = 0; kb <= kb_end; ++kb) {
    const bool more = kb < kb_end;
    if (more) fetch(kb + 1);
    if (wave_on && kb <= wave_kb_end) {
      floatx16 acc;  // S^T, this lane's half of key row l32 read from LDS four values at a time
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int i = 0; i < KH; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(Ks + l32 * PK + KH * h + i);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, qv[i], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, qv[i + 1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, qv[i + 2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, qv[i + 3], acc, 0, 0, 0);
      }
      float sv[16], bm = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * 32 + acc_row(r, h);
        const bool ok = key < Sk && (!a.causal || key <= q);
        sv[r] = ok ? acc[r] : kNegInf;
        bm = fmaxf(bm, sv[r]);
      }
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m, bm);
      const float alpha = (m == kNegInf) ? 0.f : __expf(m - mn);
      float P[16], bs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        P[r] = (mn == kNegInf) ? 0.f : __expf(sv[r] - mn);  // exp(-inf) = 0 for the masked keys
        bs += P[r];
      }
      bs += __shfl_xor(bs, 32, 64);
      l = l * alpha + bs;
      m = mn;
      float al[16];
      bcast_rows(Wr[wv], alpha, l32, h, al);
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[ob][r] *= al[r];
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {
        const float* vrow = Vs + acc_row(s2, h) * PV + l32;
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
          oacc[ob] = __builtin_amdgcn_mfma_f32_32x32x2f32(P[s2], vrow[ob * 32], oacc[ob], 0, 0, 0);
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
  float il[16];
  bcast_rows(Wr[wv], l > 0.f ? 1.f / l : 0.f, l32, h, il);
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = ob * 32 + l32;
      if (qr < a.S && e < a.dv) a.o[(tok0 + qr) * a.ldo + hd * a.dv + e] = oacc[ob][r] * il[r];
    }
  if (h == 0 && q < a.S) a.lse[(long long)pair * a.S + q] = (l > 0.f) ? m + logf(l) : kNegInf;
}

// ---------------------------------------------------------------------------
// dQ (and D = dO . O): wave per (pair, query block), S^T layout
// ---------------------------------------------------------------------------
template <int DKM, int DVM>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2, QB = DKM / 32;
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int nqb = (a.S + 31) >> 5;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.B * a.H * nqb) return;
  const int pair = item / nqb, qb = item % nqb;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int q = qb * 32 + l32;

  float qv[KH], gv[VH];
  load_half<KH, kBwdSel>(qv, a.q, a.ldq, tok0, q, a.S, hd * a.dk, a.dk, h, a.scale, a.vec);
  load_half<VH, kBwdSel>(gv, a.dout, a.lddo, tok0, q, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
  float D;
  {
    float ov[VH];
    load_half<VH, kBwdSel>(ov, a.o, a.ldo, tok0, q, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < VH; i += 2) {
      d0 = fmaf(gv[i], ov[i], d0);
      d1 = fmaf(gv[i + 1], ov[i + 1], d1);
    }
    D = d0 + d1;
    D += __shfl_xor(D, 32, 64);
  }
  const bool qok = q < a.S;
  const float lse = a.lse[(long long)pair * a.S + (qok ? q : 0)];
  if (h == 0 && qok) a.D[(long long)pair * a.S + q] = D;

  floatx16 dq[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  const int Sk = key_len(a, b);
  const int kb_last = a.causal ? min(qb, (Sk - 1) >> 5) : (Sk - 1) >> 5;
  for (int kb = 0; kb <= kb_last; ++kb) {
    floatx16 sacc, pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
    {
      float kv[KH];
      load_half<KH, kBwdSel>(kv, a.k, a.ldk, tok0, kb * 32 + l32, a.S, hd * a.dk, a.dk, h, 1.f, a.vec);
      sacc = mfma_rows<KH>(kv, qv, sacc);
    }
    {
      float vv[VH];
      load_half<VH, kBwdSel>(vv, a.v, a.ldv, tok0, kb * 32 + l32, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
      pacc = mfma_rows<VH>(vv, gv, pacc);
    }
    float dS[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb * 32 + acc_row(r, h);
      const bool ok = qok && key < Sk && (!a.causal || key <= q);
      const float p = __expf(ok ? sacc[r] - lse : kNegInf);
      dS[r] = p * (pacc[r] - D);
    }
    mfma_p_rows<QB, kBwdSel>(dS, a.k, a.ldk, tok0, kb * 32, a.S, hd * a.dk, a.dk, l32, h, dq);
  }
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dq[i][r] * a.scale, e, qr, a, qr < a.S);
      if (qr < a.S && e < a.dk) a.dq[(tok0 + qr) * a.lddq + hd * a.dk + e] = g;
    }
}

// ---------------------------------------------------------------------------
// dK / dV: wave per (pair, key block), S layout (lane <-> key)
// ---------------------------------------------------------------------------
template <int DKM, int DVM>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2, KB = DKM / 32, VB = DVM / 32;
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
  const int nkb = (a.S + 31) >> 5;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= a.B * a.H * nkb) return;
  const int pair = item / nkb, kb = item % nkb;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int key = kb * 32 + l32;

  float kv[KH], vv[VH];
  load_half<KH, kBwdSel>(kv, a.k, a.ldk, tok0, key, a.S, hd * a.dk, a.dk, h, a.scale, a.vec);
  load_half<VH, kBwdSel>(vv, a.v, a.ldv, tok0, key, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
  floatx16 dk[KB], dv[VB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[i][r] = 0.f;
  const bool kok = key < key_len(a, b);
  const int nqb = (a.S + 31) >> 5;
  for (int qb = a.causal ? kb : 0; qb < nqb; ++qb) {
    floatx16 sacc, pacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
    {
      float qv[KH];
      load_half<KH, kBwdSel>(qv, a.q, a.ldq, tok0, qb * 32 + l32, a.S, hd * a.dk, a.dk, h, 1.f, a.vec);
      sacc = mfma_rows<KH>(qv, kv, sacc);  // S[q, key]
    }
    {
      float gq[VH];
      load_half<VH, kBwdSel>(gq, a.dout, a.lddo, tok0, qb * 32 + l32, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
      pacc = mfma_rows<VH>(gq, vv, pacc);  // dP[q, key]
    }
    float P[16], dS[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const bool ok = kok && qr < a.S && (!a.causal || key <= qr);
      const long long li = (long long)pair * a.S + (qr < a.S ? qr : 0);
      const float lse_r = a.lse[li], d_r = a.D[li];  // unconditional loads (clamped index)
      const float p = __expf(ok ? sacc[r] - lse_r : kNegInf);
      P[r] = p;
      dS[r] = p * (pacc[r] - d_r);
    }
    mfma_p_rows<VB, kBwdSel>(P, a.dout, a.lddo, tok0, qb * 32, a.S, hd * a.dv, a.dv, l32, h, dv);
    mfma_p_rows<KB, kBwdSel>(dS, a.q, a.ldq, tok0, qb * 32, a.S, hd * a.dk, a.dk, l32, h, dk);
  }
  // dK / dV in accumulator layout: register r <-> key kb*32 + acc_row(r, h), lane <-> column
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dk[i][r] * a.scale, e, kr, a, kr < a.S);
      if (kr < a.S && e < a.dk) a.dk_out[(tok0 + kr) * a.lddk + hd * a.dk + e] = g;
    }
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      if (kr < a.S && e < a.dv) a.dv_out[(tok0 + kr) * a.lddv + hd * a.dv + e] = dv[i][r];
    }
}

// ---------------------------------------------------------------------------
// Backward for seq > 32, LDS-tiled like attn_fwd_tiled_kernel (FlashAttention-2's split):
//  * dQ (and D = dO . O): a workgroup per (pair, 128-query tile), one wave per 32-query block,
//    K and V streaming through LDS in 32-key blocks. S^T = K.Q^T and dP^T = V.dO^T in the S^T
//    layout, P = exp(S - lse), dS = P (dP - D); dQ += dS . K with dS the A operand in registers
//    and K's columns read from the staged block.
//  * dK / dV: a workgroup per (pair, 128-key tile), one wave per 32-key block, Q, dO, lse and D
//    streaming through LDS in 32-query blocks. S = Q.K^T and dP = dO.V^T in the S layout
//    (register r <-> query acc_row(r, h), lane <-> key); dV += P^T . dO and dK += dS^T . Q.
// ---------------------------------------------------------------------------
template <int DKM, int DVM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DKM > 32 ? 2 : TALOS_ATTN_TILED_WAVES))) void
attn_bwd_dq_tiled_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2, QB = DKM / 32;
  constexpr int PK = DKM + 4, PV = DVM + 4;
  constexpr int KL = DKM / 32, VL = DVM / 32;
  __shared__ __align__(16) float Ks[32 * PK];
  __shared__ __align__(16) float Vs[32 * PV];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b);
  const int qb = tile * 4 + wv;
  const int q = qb * 32 + l32;
  const bool wave_on = qb * 32 < a.S;
  const bool qok = q < a.S;
  const int q_hi = min(a.S, (tile + 1) * kQTile) - 1;
  const int kb_end = Sk == 0 ? -1 : (a.causal ? min(q_hi, Sk - 1) : Sk - 1) >> 5;
  const int wave_kb_end = a.causal ? min(kb_end, qb) : kb_end;

  float qv[KH], gv[VH];
  load_half<KH, kBwdSel>(qv, a.q, a.ldq, tok0, q, a.S, hd * a.dk, a.dk, h, a.scale, a.vec);
  load_half<VH, kBwdSel>(gv, a.dout, a.lddo, tok0, q, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
  float D;
  {
    float ov[VH];
    load_half<VH, kBwdSel>(ov, a.o, a.ldo, tok0, q, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < VH; i += 2) {
      d0 = fmaf(gv[i], ov[i], d0);
      d1 = fmaf(gv[i + 1], ov[i + 1], d1);
    }
    D = d0 + d1;
    D += __shfl_xor(D, 32, 64);
  }
  const float lse = a.lse[(long long)pair * a.S + (qok ? q : 0)];
  if (h == 0 && qok) a.D[(long long)pair * a.S + q] = D;

  // PF: the next block is fetched into registers during the current one; at head dims past 96
  // those registers would spill, so the block is loaded after the barrier instead and the other
  // workgroup on the CU covers the latency
  constexpr bool PF = DKM + DVM <= 160;
  float4 rk[KL], rv[VL];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rk[i] = block_ld4<DKM>(a.k, a.ldk, tok0, kb * 32, a.S, hd * a.dk, a.dk, i * 256 + (int)threadIdx.x, a.vec);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      rv[i] = block_ld4<DVM>(a.v, a.ldv, tok0, kb * 32, a.S, hd * a.dv, a.dv, i * 256 + (int)threadIdx.x, a.vec);
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4<DKM, PK>(Ks, i * 256 + (int)threadIdx.x, rk[i]);
#pragma unroll
    for (int i = 0; i < VL; ++i) block_st4<DVM, PV>(Vs, i * 256 + (int)threadIdx.x, rv[i]);
  };
  floatx16 dq[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  if (kb_end >= 0) {
    fetch(0);
    stash();
  }
  __syncthreads();
  for (int kb = 0; kb <= kb_end; ++kb) {
    const bool more = kb < kb_end;
    if (PF && more) fetch(kb + 1);
    if (wave_on && kb <= wave_kb_end) {
      floatx16 sacc, pacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
      for (int i = 0; i < KH; i += 4) {  // S^T = K . (scale Q)^T
        const float4 v = *reinterpret_cast<const float4*>(Ks + l32 * PK + KH * h + i);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, qv[i], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, qv[i + 1], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, qv[i + 2], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, qv[i + 3], sacc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < VH; i += 4) {  // dP^T = V . dO^T
        const float4 v = *reinterpret_cast<const float4*>(Vs + l32 * PV + VH * h + i);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, gv[i], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, gv[i + 1], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, gv[i + 2], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, gv[i + 3], pacc, 0, 0, 0);
      }
      float dS[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * 32 + acc_row(r, h);
        const bool ok = qok && key < Sk && (!a.causal || key <= q);
        const float p = __expf(ok ? sacc[r] - lse : kNegInf);
        dS[r] = p * (pacc[r] - D);
      }
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {  // dQ += dS . K
        const float* krow = Ks + acc_row(s2, h) * PK + l32;
#pragma unroll
        for (int i = 0; i < QB; ++i) dq[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(dS[s2], krow[i * 32], dq[i], 0, 0, 0);
      }
    }
    __syncthreads();
    if (more) {
      if (!PF) fetch(kb + 1);
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dq[i][r] * a.scale, e, qr, a, qr < a.S);
      if (qr < a.S && e < a.dk) a.dq[(tok0 + qr) * a.lddq + hd * a.dk + e] = g;
    }
}

// Column e of head hd of a dq / dk row: into dst (head width dk), or split at `split` between dst
// (head width split) and dst2 (head width dk - split) when dst2 is given.
__device__ __forceinline__ void store_head_col(float* dst, long long ld, float* dst2, long long ld2, int split,
                                               long long row, int hd, int dk, int e, float g) {
  if (dst2 == nullptr) dst[row * ld + (long long)hd * dk + e] = g;
  else if (e < split) dst[row * ld + (long long)hd * split + e] = g;
  else dst2[row * ld2 + (long long)hd * (dk - split) + (e - split)] = g;
}

// DS: every dS value of the wave's key blocks is also stored to a.ds (row of query q, column of
// key), through a per-wave LDS tile so the global stores are 16-byte pieces of rows, for
// attn_bwd_dq_ds_kernel; D comes from attn_rowdot_kernel. (Two waves a SIMD at every head dim: at
// three, head dims 32 spilled 2 VGPRs, 28 with DS.)
template <int DKM, int DVM, bool DS = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void
attn_bwd_dkv_tiled_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2, KB = DKM / 32, VB = DVM / 32;
  constexpr int PK = DKM + 4, PV = DVM + 4;
  constexpr int KL = DKM / 32, VL = DVM / 32;
  __shared__ __align__(16) float Qs[32 * PK];
  __shared__ __align__(16) float Gs[32 * PV];
  __shared__ __align__(16) float LD[2][32];  // lse, D of the staged query block
  __shared__ float Ts[DS ? 4 : 1][DS ? 32 * 33 : 1];  // DS: each wave's dS tile on its way out
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int kb = tile * 4 + wv;  // this wave's key block
  const int key = kb * 32 + l32;
  const bool wave_on = kb * 32 < a.S;
  const bool kok = key < key_len(a, b);
  const int nqb = (a.S + 31) >> 5;
  const int qb_beg = a.causal ? tile * 4 : 0;  // the tile's first key block can see no earlier query
  if (key_len(a, b) <= tile * kQTile) {
    // no key of this tile takes part: dK = dV = 0
    if (!wave_on) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      if (kr >= a.S) continue;
      for (int e = l32; e < a.dk; e += 32) {
        if constexpr (DS)
          store_head_col(a.dk_out, a.lddk, a.dk2, a.lddk2, a.dsplit, tok0 + kr, hd, a.dk, e, 0.f);
        else
          a.dk_out[(tok0 + kr) * a.lddk + hd * a.dk + e] = 0.f;
      }
      for (int e = l32; e < a.dv; e += 32) a.dv_out[(tok0 + kr) * a.lddv + hd * a.dv + e] = 0.f;
    }
    return;
  }

  float kv[KH], vv[VH];
  ATTN_LD_K_HALF(KH, kBwdSel, kv, key, h, a.scale);
  load_half<VH, kBwdSel>(vv, a.v, a.ldv, tok0, key, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
  floatx16 dk[KB], dv[VB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[i][r] = 0.f;

  constexpr bool PF = DKM + DVM <= 128;  // as in attn_bwd_dq_tiled_kernel (K, V rows, dK, dV live)
  float4 rq[KL], rg[VL];
  float rl = 0.f;
  auto fetch = [&](int qb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rq[i] = ATTN_BLK_Q(DKM, qb * 32, i * 256 + t);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      rg[i] = block_ld4<DVM>(a.dout, a.lddo, tok0, qb * 32, a.S, hd * a.dv, a.dv, i * 256 + t, a.vec);
    if (t < 64) {  // lse (t < 32) and D (32 <= t < 64) of the block's queries
      const int qr = qb * 32 + (t & 31);
      const long long li = (long long)pair * a.S + (qr < a.S ? qr : 0);
      rl = (t < 32 ? a.lse : a.D)[li];
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4<DKM, PK>(Qs, i * 256 + t, rq[i]);
#pragma unroll
    for (int i = 0; i < VL; ++i) block_st4<DVM, PV>(Gs, i * 256 + t, rg[i]);
    if (t < 64) LD[t >> 5][t & 31] = rl;
  };
  fetch(qb_beg);
  stash();
  __syncthreads();
  for (int qb = qb_beg; qb < nqb; ++qb) {
    const bool more = qb + 1 < nqb;
    if (PF && more) fetch(qb + 1);
    if (wave_on && (!a.causal || qb >= kb)) {
      floatx16 sacc, pacc;
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
      for (int i = 0; i < KH; i += 4) {  // S = Q . (scale K)^T
        const float4 v = *reinterpret_cast<const float4*>(Qs + l32 * PK + KH * h + i);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, kv[i], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, kv[i + 1], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, kv[i + 2], sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, kv[i + 3], sacc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < VH; i += 4) {  // dP = dO . V^T
        const float4 v = *reinterpret_cast<const float4*>(Gs + l32 * PV + VH * h + i);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.x, vv[i], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.y, vv[i + 1], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.z, vv[i + 2], pacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x2f32(v.w, vv[i + 3], pacc, 0, 0, 0);
      }
      float P[16], dS[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // queries 8j + 4h + 0..3 of the block
        const float4 l4 = *reinterpret_cast<const float4*>(&LD[0][8 * j + 4 * h]);
        const float4 d4 = *reinterpret_cast<const float4*>(&LD[1][8 * j + 4 * h]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * j + u;
          const int qr = qb * 32 + acc_row(r, h);
          const bool ok = kok && qr < a.S && (!a.causal || key <= qr);
          const float p = __expf(ok ? sacc[r] - lv[u] : kNegInf);
          P[r] = p;
          dS[r] = p * (pacc[r] - dv4[u]);
          if constexpr (DS) Ts[wv][acc_row(r, h) * 33 + l32] = dS[r];  // row: query, column: key
        }
      }
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {  // dV += P^T . dO, dK += dS^T . Q
        const float* grow = Gs + acc_row(s2, h) * PV + l32;
        const float* qrow = Qs + acc_row(s2, h) * PK + l32;
#pragma unroll
        for (int i = 0; i < VB; ++i) dv[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(P[s2], grow[i * 32], dv[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < KB; ++i) dk[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(dS[s2], qrow[i * 32], dk[i], 0, 0, 0);
      }
      if constexpr (DS) {  // the block's dS tile [32 queries][32 keys] to a.ds, 16-byte row pieces
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = i * 64 + lane, row = g >> 3, c = 4 * (g & 7);
          const int qr = qb * 32 + row, k0 = kb * 32 + c;
          const float* tr = Ts[wv] + row * 33 + c;
          if (qr < a.S && k0 < a.S)
            *reinterpret_cast<float4*>(a.ds + ((long long)pair * a.S + qr) * a.S + k0) =
                make_float4(tr[0], tr[1], tr[2], tr[3]);
        }
      }
    }
    __syncthreads();
    if (more) {
      if (!PF) fetch(qb + 1);
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dk[i][r] * a.scale, e, kr, a, kr < a.S);
      if (kr < a.S && e < a.dk) {
        if constexpr (DS)
          store_head_col(a.dk_out, a.lddk, a.dk2, a.lddk2, a.dsplit, tok0 + kr, hd, a.dk, e, g);
        else
          a.dk_out[(tok0 + kr) * a.lddk + hd * a.dk + e] = g;
      }
    }
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      if (kr < a.S && e < a.dv) a.dv_out[(tok0 + kr) * a.lddv + hd * a.dv + e] = dv[i][r];
    }
}

// D[pair * S + q] = sum_e dO[q][e] O[q][e] over the head's dv columns: 16 lanes a row (float4s of
// columns 4 lane + 64 j on 16-byte rows, else elements lane + 16 j), 16 rows a workgroup.
__global__ __launch_bounds__(256) void attn_rowdot_kernel(AttnArgs a) {
  const long long r = (long long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  const long long rows = (long long)a.B * a.H * a.S;
  float d = 0.f;
  if (r < rows) {
    const int pair = (int)(r / a.S), q = (int)(r % a.S), b = pair / a.H, hd = pair % a.H;
    const long long row = (long long)b * a.S + q;
    const float* g = a.dout + row * a.lddo + (long long)hd * a.dv;
    const float* o = a.o + row * a.ldo + (long long)hd * a.dv;
    if (a.vec) {  // 16-byte rows: a float4 a lane, 64 columns a pass
      for (int e = 4 * c; e < a.dv; e += 64) {
        const float4 g4 = *reinterpret_cast<const float4*>(g + e), o4 = *reinterpret_cast<const float4*>(o + e);
        d = fmaf(g4.x, o4.x, fmaf(g4.y, o4.y, fmaf(g4.z, o4.z, fmaf(g4.w, o4.w, d))));
      }
    } else {
      for (int e = c; e < a.dv; e += 16) d = fmaf(g[e], o[e], d);
    }
  }
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) d += __shfl_xor(d, off, 64);
  if (r < rows && c == 0) a.D[r] = d;
}

// dQ = dS . K from the dS rows attn_bwd_dkv_tiled_kernel<.., .., true> stored (a.ds), instead of
// forming S, P and dP again: a workgroup is 128 queries of one (batch, head) pair as in
// attn_bwd_dq_tiled_kernel (wave = 32 queries), and for each 32-key block the K rows and the
// tile's [128 x 32] dS block are staged in LDS (loaded one block ahead into registers); the dS
// block is read transposed there (pitch 33), one value a product step. seq % 4 == 0.
template <int DKM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_TILED_WAVES))) void
attn_bwd_dq_ds_kernel(AttnArgs a) {
  constexpr int QB = DKM / 32, PK = DKM + 4, KL = DKM / 32, PD = 33;
  __shared__ __align__(16) float Ks[32 * PK];
  __shared__ float Ds[kQTile * PD];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b);
  const int qb = tile * 4 + wv;
  const bool wave_on = qb * 32 < a.S;
  const int q_hi = min(a.S, (tile + 1) * kQTile) - 1;
  const int kb_end = Sk == 0 ? -1 : (a.causal ? min(q_hi, Sk - 1) : Sk - 1) >> 5;
  const int wave_kb_end = a.causal ? min(kb_end, qb) : kb_end;
  const float* dsp = a.ds + (long long)pair * a.S * a.S;
  float4 rk[KL], rd[4];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rk[i] = ATTN_BLK_K(DKM, kb * 32, i * 256 + t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // float4 i * 256 + t of the block: query row / 8, keys 4 (t % 8) ..
      const int g = i * 256 + t, qr = tile * kQTile + (g >> 3), key = kb * 32 + 4 * (g & 7);
      rd[i] = qr < a.S && key < a.S ? *reinterpret_cast<const float4*>(dsp + (long long)qr * a.S + key)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4<DKM, PK>(Ks, i * 256 + t, rk[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = i * 256 + t;
      float* d = Ds + (g >> 3) * PD + 4 * (g & 7);
      d[0] = rd[i].x;
      d[1] = rd[i].y;
      d[2] = rd[i].z;
      d[3] = rd[i].w;
    }
  };
  floatx16 dq[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  if (kb_end >= 0) {
    fetch(0);
    stash();
  }
  __syncthreads();
  for (int kb = 0; kb <= kb_end; ++kb) {
    const bool more = kb < kb_end;
    if (more) fetch(kb + 1);
    if (wave_on && kb <= wave_kb_end) {
      const float* drow = Ds + (wv * 32 + l32) * PD;
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {  // dQ += dS . K
        const float dsv = drow[acc_row(s2, h)];
        const float* krow = Ks + acc_row(s2, h) * PK + l32;
#pragma unroll
        for (int i = 0; i < QB; ++i) dq[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(dsv, krow[i * 32], dq[i], 0, 0, 0);
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dq[i][r] * a.scale, e, qr, a, qr < a.S);
      if (qr < a.S && e < a.dk) store_head_col(a.dq, a.lddq, a.dq2, a.lddq2, a.dsplit, tok0 + qr, hd, a.dk, e, g);
    }
}

// ---------------------------------------------------------------------------
// bf16-in / fp32-accumulate variants of the tiled forward and the dS backward (plans whose
// products take bf16 operands): the same workgroup layout, online softmax and dS round trip, with
// every contraction on v_mfma_f32_32x32x16_bf16 (eight head or key values a lane per product
// instead of one). Operands are rounded to bf16 (nearest even, v_cvt_pk_bf16_f32) as they are
// staged; softmax, the scores, P, lse, D and all accumulators stay fp32. The dS rows go out as
// bf16 (the dQ product rounds them to bf16 as its operand either way), half the fp32 bytes.
//
// Operand maps. A product's k-slots 8h + j (j < 8) of lane (l32, h) must name the same head
// dimension or key in A and B:
//  * row products (S^T = K Q^T, S = Q K^T, dP = dO V^T): slot 8h + j of product s is head column
//    HALF*h + 8s + j, the lane's A fragment one 16-byte read of a row-major bf16 tile, its B
//    fragment the lane's own row half converted once;
//  * accumulator products (O += P V, dV += P^T dO, dK += dS^T Q): A is P / dS straight from the
//    accumulator registers, so slot 8h + j of product t is block row acc_row(8t + j, h) =
//    16t + 8(j / 4) + 4h + j % 4, and B reads those rows of one column from the row-major bf16
//    tile (V, dO, scale Q) by two transposing reads (lds_frag_tr);
//  * dQ += dS K: slot 8h + j of product t is key 16t + 8h + j, one 16-byte read from the bf16 dS
//    rows and two transposing reads of the row-major K tile.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  const floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ bf16x8 frag8(const float* f) {
  const uint4 u = {pk_bf16(f[0], f[1]), pk_bf16(f[2], f[3]), pk_bf16(f[4], f[5]), pk_bf16(f[6], f[7])};
  return __builtin_bit_cast(bf16x8, u);
}
__device__ __forceinline__ bf16x8 lds_frag16(const uint16_t* p) {  // 16-byte aligned
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}
// A B fragment over rows of a row-major bf16 tile (pitch P, a multiple of 4): lane (l32, h) gets
// column c0 + l32 of rows r0 + HS h + 0..3, then of rows r0 + HS h + D2 + 0..3, by two
// ds_read_b64_tr_b16. That instruction works on groups of 16 lanes: lane 4a + j of a group gives
// the address of four consecutive values (row a of a 4 x 16 block, columns 4j .. 4j + 3) and lane
// l receives column l of the block's four rows. Group g = lane / 16 covers columns 16 (g % 2) ..
// of its rows (h = g / 2), so each lane reads one 8-byte piece and no tile is stored transposed.
typedef short shortx4 __attribute__((ext_vector_type(4)));
template <int HS, int D2>
__device__ __forceinline__ bf16x8 lds_frag_tr(const uint16_t* tile, int P, int r0, int c0, int lane) {
  typedef __attribute__((address_space(3))) shortx4* lds_x4;
  const int g = lane >> 4, a = (lane >> 2) & 3, j = lane & 3;
  const uint16_t* p = tile + (r0 + HS * (g >> 1) + a) * P + c0 + 16 * (g & 1) + 4 * j;
  const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4)(p));
  const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4)(p + D2 * P));
  const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
  const uint4 u = {l2.x, l2.y, h2.x, h2.y};
  return __builtin_bit_cast(bf16x8, u);
}
// Element group g of a [32, DM] block (as block_st4), times sc, into a row-major bf16 tile of
// pitch RP ...
template <int DM, int RP>
__device__ __forceinline__ void block_st4_bf(uint16_t* tile, int g, float4 v, float sc = 1.f) {
  const int idx = 4 * g;
  *reinterpret_cast<uint2*>(tile + (idx / DM) * RP + idx % DM) =
      make_uint2(pk_bf16(v.x * sc, v.y * sc), pk_bf16(v.z * sc, v.w * sc));
}
// A gradient element g of a bf16 kernel's output: fp32, or with out16 its bf16 (nearest even, as
// the plans' conversion launch rounds) in a uint16_t buffer; store_head_col's layouts.
__device__ __forceinline__ void put_out(float* dst, long long idx, float g, bool out16) {
  if (out16)
    reinterpret_cast<uint16_t*>(dst)[idx] = (uint16_t)pk_bf16(g, 0.f);
  else
    dst[idx] = g;
}
__device__ __forceinline__ void store_head_col_o(float* dst, long long ld, float* dst2, long long ld2, int split,
                                                 long long row, int hd, int dk, int e, float g, bool out16) {
  if (dst2 == nullptr) put_out(dst, row * ld + (long long)hd * dk + e, g, out16);
  else if (e < split) put_out(dst, row * ld + (long long)hd * split + e, g, out16);
  else put_out(dst2, row * ld2 + (long long)hd * (dk - split) + (e - split), g, out16);
}
// Pitches (bf16 elements): row-major tiles DM + 8 (rows 16 bytes apart in bank offset, so the 16
// lanes of a 16-byte read hit distinct banks); the dQ kernel's dS rows 32 + 8.
constexpr int kDsP = 40;
// waves per SIMD the bf16 kernels are compiled for (forward, dK / dV, dQ); C5: four waves for dQ
// (8 VGPRs spill in its split twin) 0.883-0.892 -> 0.878-0.881 ms, two for the forward no better,
// three for dK / dV or four for the forward spill 43-376 VGPRs
#ifndef TALOS_ATTN_BF_FWD_WAVES
#define TALOS_ATTN_BF_FWD_WAVES 3
#endif
#ifndef TALOS_ATTN_BF_DKV_WAVES
#define TALOS_ATTN_BF_DKV_WAVES 2
#endif
#ifndef TALOS_ATTN_BF_DQ_WAVES
#define TALOS_ATTN_BF_DQ_WAVES 4
#endif

template <int DKM, int DVM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BF_FWD_WAVES))) void
attn_fwd_tiled_bf16_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, OB = DVM / 32, KS = KH / 8;
  constexpr int RK = DKM + 8, RV = DVM + 8;
  constexpr int KL = DKM / 32, VL = DVM / 32;
  __shared__ __align__(16) uint16_t Kb[32 * RK];
  __shared__ __align__(16) uint16_t Vb[32 * RV];
  __shared__ __align__(16) float Wr[4][32];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b);
  const int qb = tile * 4 + wv;
  const int q = qb * 32 + l32;
  const bool wave_on = qb * 32 < a.S;
  const int q_hi = min(a.S, (tile + 1) * kQTile) - 1;
  const int kb_end = Sk == 0 ? -1 : (a.causal ? min(q_hi, Sk - 1) : Sk - 1) >> 5;
  const int wave_kb_end = a.causal ? min(kb_end, qb) : kb_end;

  bf16x8 qf[KS];
  {
    float qv[KH];
    ATTN_LD_Q_HALF(KH, kFwdSel, qv, q, h, a.scale);
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = frag8(qv + 8 * s);
  }
  float4 rk[KL], rv[VL];
  auto fetch = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rk[i] = ATTN_BLK_K(DKM, kb * 32, i * 256 + t);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      rv[i] = block_ld4<DVM>(a.v, a.ldv, tok0, kb * 32, a.S, hd * a.dv, a.dv, i * 256 + t, a.vec);
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4_bf<DKM, RK>(Kb, i * 256 + t, rk[i]);
#pragma unroll
    for (int i = 0; i < VL; ++i) block_st4_bf<DVM, RV>(Vb, i * 256 + t, rv[i]);
  };

  float m = kNegInf, l = 0.f;
  floatx16 oacc[OB];
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[ob][r] = 0.f;
  if (kb_end >= 0) {
    fetch(0);
    stash();
  }
  __syncthreads();
  for (int kb = 0; kb <= kb_end; ++kb) {
    const bool more = kb < kb_end;
    if (more) fetch(kb + 1);
    if (wave_on && kb <= wave_kb_end) {
      floatx16 acc;  // S^T: rows keys, columns queries
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_frag16(Kb + l32 * RK + KH * h + 8 * s), qf[s], acc, 0, 0, 0);
      float sv[16], bm = kNegInf;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * 32 + acc_row(r, h);
        const bool ok = key < Sk && (!a.causal || key <= q);
        sv[r] = ok ? acc[r] : kNegInf;
        bm = fmaxf(bm, sv[r]);
      }
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mn = fmaxf(m, bm);
      const float alpha = (m == kNegInf) ? 0.f : __expf(m - mn);
      float P[16], bs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        P[r] = (mn == kNegInf) ? 0.f : __expf(sv[r] - mn);
        bs += P[r];
      }
      bs += __shfl_xor(bs, 32, 64);
      l = l * alpha + bs;
      m = mn;
      float al[16];
      bcast_rows(Wr[wv], alpha, l32, h, al);
#pragma unroll
      for (int ob = 0; ob < OB; ++ob)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[ob][r] *= al[r];
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {  // O += P V over the block's keys, 16 a product
        const bf16x8 pf = frag8(P + 8 * t2);
#pragma unroll
        for (int ob = 0; ob < OB; ++ob)
          oacc[ob] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, lds_frag_tr<4, 8>(Vb, RV, 16 * t2, ob * 32, lane),
                                                             oacc[ob], 0, 0, 0);
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
  float il[16];
  bcast_rows(Wr[wv], l > 0.f ? 1.f / l : 0.f, l32, h, il);
#pragma unroll
  for (int ob = 0; ob < OB; ++ob)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = ob * 32 + l32;
      if (qr < a.S && e < a.dv) a.o[(tok0 + qr) * a.ldo + hd * a.dv + e] = oacc[ob][r] * il[r];
    }
  if (h == 0 && q < a.S) a.lse[(long long)pair * a.S + q] = (l > 0.f) ? m + logf(l) : kNegInf;
}

template <int DKM, int DVM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BF_DKV_WAVES))) void
attn_bwd_dkv_bf16_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2, KB = DKM / 32, VB = DVM / 32, KS = KH / 8, VS = VH / 8;
  constexpr int RK = DKM + 8, RV = DVM + 8;
  constexpr int KL = DKM / 32, VL = DVM / 32;
  __shared__ __align__(16) uint16_t Qb[32 * RK];  // bf16(scale q) rows: S and, transposed, dK
  __shared__ __align__(16) uint16_t Gb[32 * RV];  // bf16(dO) rows: dP and, transposed, dV
  __shared__ __align__(16) float LD[2][32];
  __shared__ float Ts[4][32 * 33];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int kb = tile * 4 + wv;
  const int key = kb * 32 + l32;
  const bool wave_on = kb * 32 < a.S;
  const bool kok = key < key_len(a, b);
  const int nqb = (a.S + 31) >> 5;
  const int qb_beg = a.causal ? tile * 4 : 0;
  if (key_len(a, b) <= tile * kQTile) {
    if (!wave_on) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      if (kr >= a.S) continue;
      for (int e = l32; e < a.dk; e += 32)
        store_head_col_o(a.dk_out, a.lddk, a.dk2, a.lddk2, a.dsplit, tok0 + kr, hd, a.dk, e, 0.f, a.out16);
      for (int e = l32; e < a.dv; e += 32) put_out(a.dv_out, (tok0 + kr) * a.lddv + hd * a.dv + e, 0.f, a.out16);
    }
    return;
  }

  bf16x8 kf[KS], vf[VS];
  {
    float kv[KH], vv[VH];
    // the scale goes on the staged Q rows (as the forward's on q), so S = bf16(scale q) bf16(k)^T
    // is the forward's product and exp(S - lse) its P
    ATTN_LD_K_HALF(KH, kBwdSel, kv, key, h, 1.f);
    load_half<VH, kBwdSel>(vv, a.v, a.ldv, tok0, key, a.S, hd * a.dv, a.dv, h, 1.f, a.vec);
#pragma unroll
    for (int s = 0; s < KS; ++s) kf[s] = frag8(kv + 8 * s);
#pragma unroll
    for (int s = 0; s < VS; ++s) vf[s] = frag8(vv + 8 * s);
  }
  floatx16 dk[KB], dv[VB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[i][r] = 0.f;

  float4 rq[KL], rg[VL];
  float rl = 0.f;
  auto fetch = [&](int qb) {
#pragma unroll
    for (int i = 0; i < KL; ++i)
      rq[i] = ATTN_BLK_Q(DKM, qb * 32, i * 256 + t);
#pragma unroll
    for (int i = 0; i < VL; ++i)
      rg[i] = block_ld4<DVM>(a.dout, a.lddo, tok0, qb * 32, a.S, hd * a.dv, a.dv, i * 256 + t, a.vec);
    if (t < 64) {
      const int qr = qb * 32 + (t & 31);
      const long long li = (long long)pair * a.S + (qr < a.S ? qr : 0);
      rl = (t < 32 ? a.lse : a.D)[li];
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4_bf<DKM, RK>(Qb, i * 256 + t, rq[i], a.scale);
#pragma unroll
    for (int i = 0; i < VL; ++i) block_st4_bf<DVM, RV>(Gb, i * 256 + t, rg[i]);
    if (t < 64) LD[t >> 5][t & 31] = rl;
  };
  fetch(qb_beg);
  stash();
  __syncthreads();
  for (int qb = qb_beg; qb < nqb; ++qb) {
    const bool more = qb + 1 < nqb;
    if (more) fetch(qb + 1);
    if (wave_on && (!a.causal || qb >= kb)) {
      floatx16 sacc, pacc;  // rows queries, columns keys
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_frag16(Qb + l32 * RK + KH * h + 8 * s), kf[s], sacc, 0, 0, 0);
#pragma unroll
      for (int s = 0; s < VS; ++s)
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_frag16(Gb + l32 * RV + VH * h + 8 * s), vf[s], pacc, 0, 0, 0);
      float P[16], dS[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 l4 = *reinterpret_cast<const float4*>(&LD[0][8 * j + 4 * h]);
        const float4 d4 = *reinterpret_cast<const float4*>(&LD[1][8 * j + 4 * h]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int r = 4 * j + u;
          const int qr = qb * 32 + acc_row(r, h);
          const bool ok = kok && qr < a.S && (!a.causal || key <= qr);
          const float p = __expf(ok ? sacc[r] - lv[u] : kNegInf);
          P[r] = p;
          dS[r] = p * (pacc[r] - dv4[u]);
          Ts[wv][acc_row(r, h) * 33 + l32] = dS[r];
        }
      }
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {  // dV += P^T dO, dK += dS^T Q over the block's queries
        const bf16x8 pf = frag8(P + 8 * t2), sf = frag8(dS + 8 * t2);
#pragma unroll
        for (int i = 0; i < VB; ++i)
          dv[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, lds_frag_tr<4, 8>(Gb, RV, 16 * t2, i * 32, lane), dv[i],
                                                          0, 0, 0);
#pragma unroll
        for (int i = 0; i < KB; ++i)
          dk[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(sf, lds_frag_tr<4, 8>(Qb, RK, 16 * t2, i * 32, lane), dk[i],
                                                          0, 0, 0);
      }
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // the block's dS tile [32 queries][32 keys] to a.ds as bf16
        const int g = i * 64 + lane, row = g >> 3, c = 4 * (g & 7);
        const int qr = qb * 32 + row, k0 = kb * 32 + c;
        const float* tr = Ts[wv] + row * 33 + c;
        if (qr < a.S && k0 < a.S)
          *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.ds) + ((long long)pair * a.S + qr) * a.S + k0) =
              make_uint2(pk_bf16(tr[0], tr[1]), pk_bf16(tr[2], tr[3]));
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dk[i][r], e, kr, a, kr < a.S);  // the staged Q rows carry the scale
      if (kr < a.S && e < a.dk)
        store_head_col_o(a.dk_out, a.lddk, a.dk2, a.lddk2, a.dsplit, tok0 + kr, hd, a.dk, e, g, a.out16);
    }
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kr = kb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      if (kr < a.S && e < a.dv) put_out(a.dv_out, (tok0 + kr) * a.lddv + hd * a.dv + e, dv[i][r], a.out16);
    }
}

template <int DKM>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BF_DQ_WAVES))) void
attn_bwd_dq_ds_bf16_kernel(AttnArgs a) {
  constexpr int QB = DKM / 32, KL = DKM / 32;
  constexpr int RK = DKM + 8;
  __shared__ __align__(16) uint16_t Kb[32 * RK];         // bf16(k) rows, read transposed
  __shared__ __align__(16) uint16_t Db[kQTile * kDsP];  // dS rows of the tile's queries, bf16
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int t = threadIdx.x;
  const int ntile = (a.S + kQTile - 1) / kQTile;
  const int pair = blockIdx.x / ntile, tile = blockIdx.x % ntile;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b);
  const int qb = tile * 4 + wv;
  const bool wave_on = qb * 32 < a.S;
  const int q_hi = min(a.S, (tile + 1) * kQTile) - 1;
  const int kb_end = Sk == 0 ? -1 : (a.causal ? min(q_hi, Sk - 1) : Sk - 1) >> 5;
  const int wave_kb_end = a.causal ? min(kb_end, qb) : kb_end;
  const uint16_t* dsp = reinterpret_cast<const uint16_t*>(a.ds) + (long long)pair * a.S * a.S;  // bf16 rows
  float4 rk[KL];
  uint2 rd[4];
  // whole 32-row blocks with 16-byte rows and no head padding: loop-invariant addresses
  const bool fast = a.vec && a.dk == DKM;
  int kbo[KL];
#pragma unroll
  for (int i = 0; i < KL; ++i) kbo[i] = block_off<DKM>(a.ldk, i * 256 + t);
  auto fetch = [&](int kb) {
    if (fast && (kb + 1) * 32 <= a.S) {
      const float* kblk = a.k + (tok0 + kb * 32) * a.ldk + hd * a.dk;
#pragma unroll
      for (int i = 0; i < KL; ++i) rk[i] = *reinterpret_cast<const float4*>(kblk + kbo[i]);
    } else {
#pragma unroll
      for (int i = 0; i < KL; ++i)
        rk[i] = ATTN_BLK_K(DKM, kb * 32, i * 256 + t);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // query row g / 8 of the tile, keys 4 (g % 8) .. + 3
      const int g = i * 256 + t, qr = tile * kQTile + (g >> 3), k = kb * 32 + 4 * (g & 7);
      rd[i] = qr < a.S && k < a.S ? *reinterpret_cast<const uint2*>(dsp + (long long)qr * a.S + k) : make_uint2(0u, 0u);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) block_st4_bf<DKM, RK>(Kb, i * 256 + t, rk[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = i * 256 + t;
      *reinterpret_cast<uint2*>(Db + (g >> 3) * kDsP + 4 * (g & 7)) = rd[i];
    }
  };
  floatx16 dq[QB];
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  if (kb_end >= 0) {
    fetch(0);
    stash();
  }
  __syncthreads();
  for (int kb = 0; kb <= kb_end; ++kb) {
    const bool more = kb < kb_end;
    if (more) fetch(kb + 1);
    if (wave_on && kb <= wave_kb_end) {
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {  // dQ += dS K over keys 16 t2 + 8 h + 0..7
        const bf16x8 df = lds_frag16(Db + (wv * 32 + l32) * kDsP + 16 * t2 + 8 * h);
#pragma unroll
        for (int i = 0; i < QB; ++i)
          dq[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df, lds_frag_tr<8, 4>(Kb, RK, 16 * t2, i * 32, lane),
                                                          dq[i], 0, 0, 0);
      }
    }
    __syncthreads();
    if (more) {
      stash();
      __syncthreads();
    }
  }
  if (!wave_on) return;
#pragma unroll
  for (int i = 0; i < QB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = qb * 32 + acc_row(r, h);
      const int e = i * 32 + l32;
      const float g = rope_t(dq[i][r] * a.scale, e, qr, a, qr < a.S);
      if (qr < a.S && e < a.dk) store_head_col_o(a.dq, a.lddq, a.dq2, a.lddq2, a.dsplit, tok0 + qr, hd, a.dk, e, g, a.out16);
    }
}

// ---------------------------------------------------------------------------
// Single-block backward (seq <= 32): one wave per (batch, head) pair computes dQ, dK and dV from
// one read of q, k, v, o and dO (D = dO . O is formed in the wave). S layout (lane <-> key,
// register r <-> query acc_row(r, h)); dS is transposed through the wave's LDS slice for dQ.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void bcast_rows(float* slice, float v, int l32, int h, float (&f)[16]) {
  if (h == 0) slice[l32] = v;
  wave_lds_sync();
#pragma unroll
  for (int j = 0; j < 4; ++j) {  // queries 8j + 4h + 0..3: one 16-byte read each
    const float4 x = *reinterpret_cast<const float4*>(slice + 8 * j + 4 * h);
    f[4 * j] = x.x; f[4 * j + 1] = x.y; f[4 * j + 2] = x.z; f[4 * j + 3] = x.w;
  }
  wave_lds_sync();  // every lane has read before the slice is written again
}

constexpr int kTS = 33;  // pitch of the transposed dS tile: a column read touches 32 banks

// Offset of element (row, col) in a staged tile of pitch TP. At TP = 32 a row is 128 bytes, so
// the 16-byte accesses of 16 lanes to 16 consecutive rows would share two groups of banks (eight
// lanes on each); the row's 16-byte column groups are therefore permuted by (row / 2) % 8, which
// puts those 16 accesses on 16 distinct groups of four banks. A float4 at a column that is a
// multiple of 4 stays contiguous.
template <int TP>
__device__ __forceinline__ int stg(int row, int col) {
  if constexpr (TP == 32) return row * 32 + ((((col >> 2) ^ (row >> 1)) & 7) << 2) + (col & 3);
  return row * TP + col;
}

// The element (acc_row(s, h), l32) of a swizzled 32-pitch tile: row acc_row = 8 (s / 4) + 4 h +
// s % 4 puts bits 1 and 3 of s into the permutation, so the lane needs four base offsets (one per
// value of those bits, h and l32 folded in), and the rest, (8 (s / 4) + s % 4) * 32, is a constant
// of the unrolled loop.
struct AccRowBases {
  int o[4];
  __device__ __forceinline__ AccRowBases(int l32, int h) {
    const int v = (l32 >> 2) ^ (h << 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = 128 * h + ((((k & 1) | ((k >> 1) << 2)) ^ v) << 2) + (l32 & 3);
  }
  __device__ __forceinline__ int at(int s) const {
    return o[((s >> 1) & 1) | (((s >> 2) & 1) << 1)] + (8 * (s >> 2) + (s & 3)) * 32;
  }
};

// Stores this lane's half row (the load_half layout) into row l32 of an LDS tile of pitch TP.
template <int HALF, int TP>
__device__ __forceinline__ void stage_half(float* tile, const float (&r)[HALF], int l32, int h) {
#pragma unroll
  for (int i = 0; i < HALF; i += 4)
    *reinterpret_cast<float4*>(tile + stg<TP>(l32, HALF * h + i)) = make_float4(r[i], r[i + 1], r[i + 2], r[i + 3]);
}

// mfma_p_rows with the operand rows read from an LDS tile of pitch TP (rows >= S hold zeros).
template <int NB, int TP>
__device__ __forceinline__ void mfma_p_lds(const float (&P)[16], const float* tile, int l32, int h,
                                           floatx16 (&acc)[NB]) {
  static_assert(TP != 32 || NB == 1, "a swizzled tile is one 32-column block");
  const AccRowBases ab(l32, h);
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float* src = tile + (TP == 32 ? ab.at(s) : acc_row(s, h) * TP + l32);
#pragma unroll
    for (int eb = 0; eb < NB; ++eb)
      acc[eb] = __builtin_amdgcn_mfma_f32_32x32x2f32(P[s], src[eb * 32], acc[eb], 0, 0, 0);
  }
}

#ifndef TALOS_ATTN_STAGE
#define TALOS_ATTN_STAGE 1
#endif

// The per-wave LDS slice of the fused backward. STAGE (head dims 32): the dO, Q and K rows the
// wave loads are also written to its slice, and the three P-products read them there instead of
// re-reading global memory; the dS^T tile then reuses the dO tile. Staged tile pitch: 16-byte
// rows; the dS^T tile (pitch kTS) spills from the dO tile into the Q tile, which is dead by then;
// 12.5 KB per wave keeps three workgroups on a CU.
template <int DKM, int DVM>
struct BwdSlice {
  static constexpr bool STAGE = TALOS_ATTN_STAGE && DKM == 32 && DVM == 32;
  static constexpr int TP = 32;
  static constexpr int WSZ = STAGE ? 3 * 32 * TP + 64 : 32 * kTS + 64;
  static_assert(!STAGE || 32 * kTS <= 64 * TP, "the dS^T tile must end before the K tile");
};

// The fused backward of one (batch, head) pair once its rows are in registers (load_half layout:
// gv = dO, ov = O, qv = scale * Q, kv = K, vv = V) with the query row's lse; W is the wave's LDS
// slice. GS_STAGED: the dO tile already holds gv (the kernel that forms dO itself put it there).
// BLOCK (head dims 32): the wave's rows are the 32 queries from q0 and the 32 keys from k0 of a
// longer sequence, and the block's dQ (unscaled), dK and dV accumulators are returned in out[0..2]
// instead of stored, for the caller to add to the other blocks' before the store.
template <int DKM, int DVM, bool GS_STAGED, bool BLOCK = false>
__device__ __forceinline__ void bwd_fused_core(const AttnArgs& a, float* W, int pair, int l32, int h,
                                               const float (&gv)[DVM / 2], const float (&ov)[DVM / 2],
                                               const float (&qv)[DKM / 2], const float (&kv)[DKM / 2],
                                               const float (&vv)[DVM / 2], float lse, int q0 = 0, int k0 = 0,
                                               floatx16* out = nullptr) {
  constexpr int KH = DKM / 2, VH = DVM / 2, KB = DKM / 32, VB = DVM / 32;
  constexpr bool STAGE = BwdSlice<DKM, DVM>::STAGE;
  static_assert(!BLOCK || (STAGE && KB == 1 && VB == 1), "the block form is for staged head dims 32");
  constexpr int TP = BwdSlice<DKM, DVM>::TP;
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  float* const Gs = W;             // staged dO [query][e]
  float* const Qs = W + 32 * TP;   // staged scale * Q [query][e]
  float* const Ks = W + 64 * TP;   // staged K [key][e]
  float* const T = W;              // dS^T [query][key] (pitch kTS)
  float* const Dl = W + (STAGE ? 96 * TP : 32 * kTS);  // D[query]
  float* const Ll = Dl + 32;                            // lse[query]
  const bool rok = q0 + l32 < a.S;             // this lane's row (query q0 + l32 of q / dO / O)
  const bool kok = k0 + l32 < key_len(a, b);   // ... and its key k0 + l32 of k / v takes part
  if constexpr (STAGE && !GS_STAGED) stage_half<VH, TP>(Gs, gv, l32, h);
  {
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < VH; i += 2) {
      d0 = fmaf(gv[i], ov[i], d0);
      d1 = fmaf(gv[i + 1], ov[i + 1], d1);
    }
    float D = d0 + d1;
    D += __shfl_xor(D, 32, 64);
    if (h == 0) {
      Dl[l32] = rok ? D : 0.f;
      Ll[l32] = rok ? lse : 0.f;
    }
  }
  floatx16 sacc, pacc;
#pragma unroll
  for (int r = 0; r < 16; ++r) sacc[r] = pacc[r] = 0.f;
  if constexpr (STAGE) {
    stage_half<KH, TP>(Qs, qv, l32, h);
    stage_half<KH, TP>(Ks, kv, l32, h);
  }
  sacc = mfma_rows<KH>(qv, kv, sacc);  // S[q, key]
  pacc = mfma_rows<VH>(gv, vv, pacc);  // dP[q, key]
  wave_lds_sync();
  // lse / D of the queries acc_row(4j .. 4j+3, h) = 8j + 4h + 0..3: one 16-byte read each
  float lq[16], dq_[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float4 l4 = *reinterpret_cast<const float4*>(Ll + 8 * j + 4 * h);
    const float4 d4 = *reinterpret_cast<const float4*>(Dl + 8 * j + 4 * h);
    lq[4 * j] = l4.x; lq[4 * j + 1] = l4.y; lq[4 * j + 2] = l4.z; lq[4 * j + 3] = l4.w;
    dq_[4 * j] = d4.x; dq_[4 * j + 1] = d4.y; dq_[4 * j + 2] = d4.z; dq_[4 * j + 3] = d4.w;
  }
  float P[16], dS[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int qr = acc_row(r, h);
    const bool ok = kok && q0 + qr < a.S && (!a.causal || k0 + l32 <= q0 + qr);
    const float p = __expf(ok ? sacc[r] - lq[r] : kNegInf);  // exp(-inf) = 0: no branch
    P[r] = p;
    dS[r] = p * (pacc[r] - dq_[r]);
    if constexpr (!STAGE) T[qr * kTS + l32] = dS[r];
  }
  floatx16 dk[KB], dv[VB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dk[i][r] = 0.f;
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dv[i][r] = 0.f;
  if constexpr (STAGE) {
    mfma_p_lds<VB, TP>(P, Gs, l32, h, dv);   // dV = P^T . dO
    mfma_p_lds<KB, TP>(dS, Qs, l32, h, dk);  // dK = dS^T . (scale Q)
    wave_lds_sync();                         // the dO tile is free: dS^T goes there
#pragma unroll
    for (int r = 0; r < 16; ++r) T[acc_row(r, h) * kTS + l32] = dS[r];
  } else {
    mfma_p_rows<VB, kFusedSel>(P, a.dout, a.lddo, tok0, 0, a.S, hd * a.dv, a.dv, l32, h, dv);  // dV = P^T . dO
    mfma_p_rows<KB, kFusedSel>(dS, a.q, a.ldq, tok0, 0, a.S, hd * a.dk, a.dk, l32, h, dk);     // dK = dS^T . Q
  }
  wave_lds_sync();
  float dST[16];  // lane <-> query l32, register r <-> key acc_row(r, h)
#pragma unroll
  for (int r = 0; r < 16; ++r) dST[r] = T[l32 * kTS + acc_row(r, h)];
  floatx16 dq[KB];
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) dq[i][r] = 0.f;
  if constexpr (STAGE)
    mfma_p_lds<KB, TP>(dST, Ks, l32, h, dq);  // dQ = dS . K
  else
    mfma_p_rows<KB, kFusedSel>(dST, a.k, a.ldk, tok0, 0, a.S, hd * a.dk, a.dk, l32, h, dq);  // dQ = dS . K
  if constexpr (BLOCK) {
    out[0] = dq[0];
    out[1] = dk[0];
    out[2] = dv[0];
    return;
  }
  const float dk_scale = STAGE ? 1.f : a.scale;  // the staged Q already carries the scale
  // row acc_row(r, h) of each result: a query for dQ, a key for dK / dV; lane <-> column
#pragma unroll
  for (int i = 0; i < KB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, h);
      const int e = i * 32 + l32;
      const bool ok = row < a.S;
      const float gq = rope_t(dq[i][r] * a.scale, e, row, a, ok);
      const float gk = rope_t(dk[i][r] * dk_scale, e, row, a, ok);
      if (ok && e < a.dk) {
        a.dq[(tok0 + row) * a.lddq + hd * a.dk + e] = gq;
        a.dk_out[(tok0 + row) * a.lddk + hd * a.dk + e] = gk;
      }
    }
#pragma unroll
  for (int i = 0; i < VB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, h);
      const int e = i * 32 + l32;
      if (row < a.S && e < a.dv) a.dv_out[(tok0 + row) * a.lddv + hd * a.dv + e] = dv[i][r];
    }
}


// VEC: every row is known 16-byte aligned (a.vec), so the row loads take no branch and the five
// operands' loads are all in flight before the first use.
template <int DKM, int DVM, bool VEC = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BWD_WAVES))) void
attn_bwd_fused_kernel(AttnArgs a) {
  constexpr int KH = DKM / 2, VH = DVM / 2;
  __shared__ __align__(16) float lds[4][BwdSlice<DKM, DVM>::WSZ];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int pair = blockIdx.x * 4 + wv;
  if (pair >= a.B * a.H) return;  // uniform per wave; the kernel has no workgroup barrier
  const int b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const bool rok = l32 < a.S;
  // every row this wave reads, issued before the first use: one memory latency, not five
  float gv[VH], ov[VH], qv[KH], kv[KH], vv[VH];
  const bool vec = VEC || a.vec;
  load_half<VH, kFusedSel>(gv, a.dout, a.lddo, tok0, l32, a.S, hd * a.dv, a.dv, h, 1.f, vec);
  load_half<VH, kFusedSel>(ov, a.o, a.ldo, tok0, l32, a.S, hd * a.dv, a.dv, h, 1.f, vec);
  load_half<KH, kFusedSel>(qv, a.q, a.ldq, tok0, l32, a.S, hd * a.dk, a.dk, h, a.scale, vec);
  load_half<KH, kFusedSel>(kv, a.k, a.ldk, tok0, l32, a.S, hd * a.dk, a.dk, h, 1.f, vec);
  load_half<VH, kFusedSel>(vv, a.v, a.ldv, tok0, l32, a.S, hd * a.dv, a.dv, h, 1.f, vec);
  const float lse = a.lse[(long long)pair * a.S + (rok ? l32 : 0)];
  bwd_fused_core<DKM, DVM, false>(a, lds[wv], pair, l32, h, gv, ov, qv, kv, vv, lse);
}

// The S <= 32 backward of four 32-wide heads (d = 128) with the output projection's input
// gradient folded in: dO = dh2 . Wo^T is formed here instead of read (h2 = x + O.Wo, Wo [128,
// 128] with row j = O's column j). A workgroup is one batch entry, its waves the entry's heads:
// the waves load the entry's dh2 rows [32, 128] into the dO tiles of their four LDS slices
// (wave w: columns [32 w, 32 w + 32)); after a barrier wave w forms its head's dO[t][e] =
// sum_n dh2[t][n] Wo[32 w + e][n] with v_mfma_f32_32x32x2f32 (A = dh2 rows from the slices, B =
// Wo rows read as float4s along n, both walking n in the order 8j + 4h + q), and after a second
// barrier writes dO into its own dO tile and reads it back in load_half layout; from there the
// pair's backward is attn_bwd_fused_kernel's.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BWD_WAVES))) void
attn_bwd_s32_wo_kernel(AttnArgs a, const float* __restrict__ wo, const float* __restrict__ gh2) {
  constexpr int TP = BwdSlice<32, 32>::TP;
  static_assert(BwdSlice<32, 32>::STAGE, "the folded dO lives in the staged dO tile");
  __shared__ __align__(16) float lds[4][BwdSlice<32, 32>::WSZ];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int b = blockIdx.x, pair = b * 4 + wv;
  const long long tok0 = (long long)b * a.S;
  const bool rok = l32 < a.S;
  float gv[16], ov[16], qv[16], kv[16], vv[16];
  // this wave's quarter of the dh2 rows (token l32, columns 32 wv + 16 h ..), zero past S
  load_half<16, true>(gv, gh2, kWoD, tok0, l32, a.S, wv * 32, 32, h, 1.f, true);
  load_half<16, true>(ov, a.o, a.ldo, tok0, l32, a.S, wv * a.dv, a.dv, h, 1.f, true);
  load_half<16, true>(qv, a.q, a.ldq, tok0, l32, a.S, wv * a.dk, a.dk, h, a.scale, true);
  load_half<16, true>(kv, a.k, a.ldk, tok0, l32, a.S, wv * a.dk, a.dk, h, 1.f, true);
  load_half<16, true>(vv, a.v, a.ldv, tok0, l32, a.S, wv * a.dv, a.dv, h, 1.f, true);
  const float lse = a.lse[(long long)pair * a.S + (rok ? l32 : 0)];
  stage_half<16, TP>(lds[wv], gv, l32, h);
  __syncthreads();
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  const float* wrow = wo + (long long)(wv * 32 + l32) * kWoD;
#pragma unroll 4
  for (int j = 0; j < kWoD / 8; ++j) {
    const int n0 = 8 * j + 4 * h;  // columns n0 .. n0 + 3 of dh2 and of Wo's row
    const float4 g4 = *reinterpret_cast<const float4*>(lds[n0 >> 5] + stg<TP>(l32, n0 & 31));
    const float4 w4 = *reinterpret_cast<const float4*>(wrow + n0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.x, w4.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.y, w4.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.z, w4.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(g4.w, w4.w, acc, 0, 0, 0);
  }
  __syncthreads();  // every wave has read the dh2 quarters
  // dO in accumulator layout (register r <-> token acc_row(r, h), lane <-> e) into the dO tile
  float* const Gs = lds[wv];
  {
    const AccRowBases ab(l32, h);
#pragma unroll
    for (int r = 0; r < 16; ++r) Gs[ab.at(r)] = acc[r];
  }
  wave_lds_sync();
#pragma unroll
  for (int i = 0; i < 16; i += 4) {
    const float4 g4 = *reinterpret_cast<const float4*>(Gs + stg<TP>(l32, 16 * h + i));
    gv[i] = g4.x;
    gv[i + 1] = g4.y;
    gv[i + 2] = g4.z;
    gv[i + 3] = g4.w;
  }
  bwd_fused_core<32, 32, true>(a, lds[wv], pair, l32, h, gv, ov, qv, kv, vv, lse);
}

// The backward for 32 < S <= 64 at head dims 32: a workgroup per (batch, head) pair, each wave a
// 32 x 32 block of queries [32 qb, 32 qb + 32) and keys [32 kb, 32 kb + 32). NW = 4: all four
// blocks, wave w = (qb, kb) = (w / 2, w % 2); NW = 3 (causal): the three blocks on or below the
// diagonal, w = 0, 1, 2 -> (0, 0), (1, 0), (1, 1), since block (0, 1) has every key masked (three
// LDS slices also fit four workgroups on a CU where four fit three). Each wave runs the fused
// single-block backward on its block (its q / dO / O rows and its k / v rows loaded before the
// first product, dO, Q and K staged in its LDS slice) and keeps the block's dQ, dK and dV
// accumulators; then the blocks meet in LDS: dQ of queries qb = block (qb, 0) + block (qb, 1),
// dK and dV of keys kb = block (0, kb) + block (1, kb), added in that order and stored by the
// first of the two waves (a block with no partner stores its own). A block whose keys are all
// past the entry's length adds zeros. Replaces the split dQ / dK-dV kernels (and their D
// workspace) at these lengths.
template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(TALOS_ATTN_BWD_WAVES))) void
attn_bwd_s64_kernel(AttnArgs a) {
  static_assert(NW == 3 || NW == 4, "three (causal) or four blocks");
  constexpr bool TRI = NW == 3;
  constexpr int WSZ = BwdSlice<32, 32>::WSZ;
  static_assert(4 * 16 * 64 <= NW * WSZ, "the partial blocks fit the slices");
  __shared__ __align__(16) float lds[NW][WSZ];
  const int lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5, wv = threadIdx.x >> 6;
  const int qb = TRI ? (wv + 1) >> 1 : wv >> 1, kb = TRI ? wv >> 1 : wv & 1, q0 = 32 * qb, k0 = 32 * kb;
  const int pair = blockIdx.x, b = pair / a.H, hd = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  float gv[16], ov[16], qv[16], kv[16], vv[16];
  load_half<16, true>(gv, a.dout, a.lddo, tok0, q0 + l32, a.S, hd * a.dv, 32, h, 1.f, true);
  load_half<16, true>(ov, a.o, a.ldo, tok0, q0 + l32, a.S, hd * a.dv, 32, h, 1.f, true);
  load_half<16, true>(qv, a.q, a.ldq, tok0, q0 + l32, a.S, hd * a.dk, 32, h, a.scale, true);
  load_half<16, true>(kv, a.k, a.ldk, tok0, k0 + l32, a.S, hd * a.dk, 32, h, 1.f, true);
  load_half<16, true>(vv, a.v, a.ldv, tok0, k0 + l32, a.S, hd * a.dv, 32, h, 1.f, true);
  const float lse = a.lse[(long long)pair * a.S + min(q0 + l32, a.S - 1)];
  floatx16 res[3];  // dQ (unscaled), dK, dV of this block
  if ((a.causal && k0 > q0 + 31) || k0 >= key_len(a, b)) {  // every key masked (uniform per wave)
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) res[i][r] = 0.f;
  } else {
    bwd_fused_core<32, 32, false, true>(a, lds[wv], pair, l32, h, gv, ov, qv, kv, vv, lse, q0, k0, res);
  }
  __syncthreads();  // every wave is done with its slice
  // which sums this wave takes part in: dQ of qb pairs (qb, 0) with (qb, 1), dK / dV of kb pairs
  // (0, kb) with (1, kb); under TRI, block (0, 0) stores dQ alone and block (1, 1) dK / dV alone
  const bool dq_pair = !(TRI && qb == 0), dkv_pair = !(TRI && kb == 1);
  // partial blocks in accumulator layout (register r of lane l at [r][l]): dQ of qb at X[qb],
  // dK / dV of kb at X[2 + 2 kb] / X[3 + 2 kb]
  float* const X = &lds[0][0];
  if (kb == 1 && dq_pair) {
#pragma unroll
    for (int r = 0; r < 16; ++r) X[(qb * 16 + r) * 64 + lane] = res[0][r];
  }
  if (qb == 1 && dkv_pair) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      X[((2 + 2 * kb) * 16 + r) * 64 + lane] = res[1][r];
      X[((3 + 2 * kb) * 16 + r) * 64 + lane] = res[2][r];
    }
  }
  __syncthreads();
  if (kb == 0) {  // dQ rows q0 + acc_row(r, h)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = q0 + acc_row(r, h);
      const bool ok = row < a.S;
      const float sum = dq_pair ? res[0][r] + X[(qb * 16 + r) * 64 + lane] : res[0][r];
      const float g = rope_t(sum * a.scale, l32, row, a, ok);
      if (ok) a.dq[(tok0 + row) * a.lddq + hd * a.dk + l32] = g;
    }
  }
  if (qb == 0 || !dkv_pair) {  // dK, dV rows k0 + acc_row(r, h); the staged Q carried the scale
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = k0 + acc_row(r, h);
      const bool ok = row < a.S;
      const float sk = dkv_pair ? res[1][r] + X[((2 + 2 * kb) * 16 + r) * 64 + lane] : res[1][r];
      const float sv = dkv_pair ? res[2][r] + X[((3 + 2 * kb) * 16 + r) * 64 + lane] : res[2][r];
      const float gk = rope_t(sk, l32, row, a, ok);
      if (ok) {
        a.dk_out[(tok0 + row) * a.lddk + hd * a.dk + l32] = gk;
        a.dv_out[(tok0 + row) * a.lddv + hd * a.dv + l32] = sv;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Launch
// ---------------------------------------------------------------------------
// TALOS_ATTN_LEGACY=1 (read once): the per-wave kernels for seq > 32 instead of the LDS-tiled
// ones (a debugging switch: the two differ by fp32 rounding).
static bool attn_legacy() {
  static const bool v = [] {
    const char* e = std::getenv("TALOS_ATTN_LEGACY");
    return e && e[0] == '1';
  }();
  return v;
}

static bool pick_dims(int dk, int dv, int* dkm, int* dvm) {
  if (dk <= 32 && dv <= 32) { *dkm = 32; *dvm = 32; return true; }
  if (dk <= 64 && dv <= 64) { *dkm = 64; *dvm = 64; return true; }
  if (dk <= 96 && dv <= 64) { *dkm = 96; *dvm = 64; return true; }
  if (dk <= 128 && dv <= 128) { *dkm = 128; *dvm = 128; return true; }
  return false;
}

static AttnArgs make_args(const AttnDesc& d, int dkm, int dvm) {
  AttnArgs a{};
  a.B = d.batch; a.S = d.seq; a.H = d.heads; a.dk = d.dk; a.dv = d.dv; a.scale = d.scale; a.causal = d.causal;
  a.q = d.q; a.ldq = d.ldq; a.k = d.k; a.ldk = d.ldk; a.v = d.v; a.ldv = d.ldv;
  a.o = d.o; a.ldo = d.ldo; a.lse = d.lse;
  a.dout = d.dout; a.lddo = d.lddo;
  a.dq = d.dq; a.lddq = d.lddq; a.dk_out = d.dk_out; a.lddk = d.lddk; a.dv_out = d.dv_out; a.lddv = d.lddv;
  a.rcos = d.rope_cos; a.rsin = d.rope_sin; a.rope_off = d.rope_off; a.rope_dim = d.rope_dim;
  a.lens = d.lens;
  a.q_last = d.q_last; a.ldq_last = d.ldq_last; a.dq_last = d.dq_last; a.lddq_last = d.lddq_last;
  a.dq2 = d.dq2; a.lddq2 = d.lddq2; a.dk2 = d.dk2; a.lddk2 = d.lddk2; a.dsplit = d.dsplit;
  a.out16 = d.out_bf16;
  // row halves start at (token * ld + head * dim + half * dim/2): 16-byte aligned when all of
  // ld, dim and dim/2 are multiples of 4 and the bases are aligned
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  bool vec = d.dk == dkm && d.dv == dvm && (dkm / 2) % 4 == 0 && (dvm / 2) % 4 == 0;
  for (long long ld : {d.ldq, d.ldk, d.ldv, d.ldo}) vec = vec && ld % 4 == 0;
  vec = vec && al(d.q) && al(d.k) && al(d.v) && al(d.o);
  if (d.dout) vec = vec && d.lddo % 4 == 0 && al(d.dout);
  a.vec = vec ? 1 : 0;
  return a;
}

// Algorithmic work: flops per kept (query, key) pair, bytes of HBM traffic.
static double kept_pairs(const AttnArgs& a) {
  const double S = a.S;
  return (double)a.B * a.H * (a.causal ? S * (S + 1) / 2 : S * S);
}

#define ATTN_DISPATCH(DK, DV, KERNEL)                                                     \
  if (dkm == DK && dvm == DV) {                                                           \
    ProfScope ps(s, #KERNEL "<" #DK ", " #DV ">", flops, bytes);                          \
    hipLaunchKernelGGL((KERNEL<DK, DV>), grid, dim3(256), 0, s, a);                       \
    return launch_status(#KERNEL);                                                        \
  }
#define ATTN_ALL(KERNEL)           \
  ATTN_DISPATCH(32, 32, KERNEL)    \
  ATTN_DISPATCH(64, 64, KERNEL)    \
  ATTN_DISPATCH(96, 64, KERNEL)    \
  ATTN_DISPATCH(128, 128, KERNEL)  \
  set_error("attention: no kernel for head dims (%d, %d)", dkm, dvm); \
  return TALOS_ERR_UNSUPPORTED;

int attn_fwd_launch(const AttnDesc& d, hipStream_t s) {
  int dkm, dvm;
  if (!pick_dims(d.dk, d.dv, &dkm, &dvm)) {
    set_error("attention: head dims (%d, %d) exceed the supported (128, 128)", d.dk, d.dv);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, dkm, dvm);
  if ((long long)a.B * a.H * a.S == 0) return TALOS_OK;
  const long long items = (long long)a.B * a.H * ((a.S + 31) / 32);
  dim3 grid(ceil_div((size_t)items, 4));
  const double rows = (double)a.B * a.S * a.H;  // (token, head) rows
  // QK^T and PV over the kept pairs; q, k, v read, o and lse written
  const double flops = kept_pairs(a) * (2.0 * a.dk + 2.0 * a.dv);
  const double bytes = 4.0 * rows * (2.0 * a.dk + a.dv) + 4.0 * rows * (a.dv + 1.0);
  if (d.dk == 32 && d.dv == 32 && a.S <= 32 && a.vec) {
    ProfScope ps(s, "attn_fwd_s32_kernel", flops, bytes);
    hipLaunchKernelGGL(attn_fwd_s32_kernel, dim3(ceil_div((size_t)a.B * a.H, 4)), dim3(256), 0, s, a);
    return launch_status("attn_fwd_s32_kernel");
  }
  if (a.S > 32 && !attn_legacy()) {
    // K / V rows are read once per 128-query tile (the queries' rows and the outputs once)
    const double tiles = (a.S + kQTile - 1) / kQTile;
    const double tbytes = 4.0 * rows * (a.dk + 2.0 * a.dv + 1.0) + 4.0 * a.B * a.H * tiles * a.S * (a.dk + a.dv);
    grid = dim3((unsigned)((long long)a.B * a.H * (long long)tiles));
    // bf16 only where the backward is the bf16 dS path, so both form P from the same products
    const bool bf16 = d.bf16 && attn_ds_path(d);
#define TILED_BF(DK, DV)                                                                    \
    if (dkm == DK && dvm == DV && bf16) {                                                   \
      ProfScope ps(s, "attn_fwd_tiled_bf16_kernel<" #DK ", " #DV ">", flops, tbytes);       \
      hipLaunchKernelGGL((attn_fwd_tiled_bf16_kernel<DK, DV>), grid, dim3(256), 0, s, a);   \
      return launch_status("attn_fwd_tiled_bf16_kernel");                                   \
    }
    TILED_BF(32, 32)
    TILED_BF(64, 64)
    TILED_BF(96, 64)
#undef TILED_BF
#define TILED(DK, DV)                                                                       \
    if (dkm == DK && dvm == DV) {                                                           \
      ProfScope ps(s, "attn_fwd_tiled_kernel<" #DK ", " #DV ">", flops, tbytes);            \
      hipLaunchKernelGGL((attn_fwd_tiled_kernel<DK, DV>), grid, dim3(256), 0, s, a);        \
      return launch_status("attn_fwd_tiled_kernel");                                        \
    }
    TILED(32, 32)
    TILED(64, 64)
    TILED(96, 64)
    TILED(128, 128)
#undef TILED
    set_error("attention forward: no tiled kernel for head dims (%d, %d)", dkm, dvm);
    return TALOS_ERR_UNSUPPORTED;
  }
  ATTN_ALL(attn_fwd_kernel)
}

int attn_fwd_wo_supported(const AttnDesc& d, const AttnWoDesc& w) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return d.dk == 32 && d.dv == 32 && d.heads == 4 && d.seq >= 1 && d.seq <= 64 && d.ldo == kWoD &&
         w.wo != nullptr && w.resid != nullptr && w.h2 != nullptr && w.gain != nullptr && w.xn != nullptr &&
         al(w.wo) && al(w.resid) && al(w.h2) && al(w.gain) && al(w.xn) && make_args(d, 32, 32).vec;
}

int attn_fwd_wo_launch(const AttnDesc& d, const AttnWoDesc& wd, hipStream_t s) {
  if (!attn_fwd_wo_supported(d, wd)) {
    set_error("attention + Wo: the fused kernels take S <= 64, four 32-wide heads, d = 128 and aligned rows");
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, 32, 32);
  if (a.B == 0) return TALOS_OK;
  WoArgs w{wd.wo, wd.resid, wd.h2, wd.gain, wd.xn, wd.rstd, wd.eps};
  const double rows = (double)a.B * a.S * a.H, tok = (double)a.B * a.S;
  const double flops = kept_pairs(a) * (2.0 * a.dk + 2.0 * a.dv) + 2.0 * tok * kWoD * kWoD;
  // q, k, v, x read; o, lse, h2, xn, rstd written (Wo from cache)
  const double bytes = 4.0 * rows * (2.0 * a.dk + a.dv) + 4.0 * rows * (a.dv + 1.0) + 4.0 * tok * (3.0 * kWoD + 1.0);
  if (a.S > 32) {
    ProfScope ps(s, "attn_fwd_s64_wo_kernel", flops, bytes);
    hipLaunchKernelGGL(attn_fwd_s64_wo_kernel, dim3(a.B), dim3(512), 0, s, a, w);
    return launch_status("attn_fwd_s64_wo_kernel");
  }
  ProfScope ps(s, "attn_fwd_s32_wo_kernel", flops, bytes);
  hipLaunchKernelGGL(attn_fwd_s32_wo_kernel, dim3(a.B), dim3(256), 0, s, a, w);
  return launch_status("attn_fwd_s32_wo_kernel");
}

int attn_bwd_wo_supported(const AttnDesc& d, const float* wo, const float* gh2) {
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return d.dk == 32 && d.dv == 32 && d.heads == 4 && d.seq >= 1 && d.seq <= 32 && d.ldo == kWoD && wo && gh2 &&
         al(wo) && al(gh2) && d.dq && d.dk_out && d.dv_out && make_args(d, 32, 32).vec;
}

int attn_bwd_wo_launch(const AttnDesc& d, const float* wo, const float* gh2, hipStream_t s) {
  if (!attn_bwd_wo_supported(d, wo, gh2)) {
    set_error("attention backward + Wo: the fused kernel takes S <= 32, four 32-wide heads, d = 128 and aligned "
              "rows");
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, 32, 32);
  if (a.B == 0) return TALOS_OK;
  const double rows = (double)a.B * a.S * a.H, tok = (double)a.B * a.S;
  // S = QK^T, dP = dO V^T, dV = P^T dO, dK = dS^T Q, dQ = dS K over the kept pairs, plus dO = dh2 Wo^T;
  // dh2, O, Q, K, V, lse read, dQ, dK, dV written (Wo from cache)
  const double flops = kept_pairs(a) * (4.0 * a.dk + 6.0 * a.dv) + 2.0 * tok * kWoD * kWoD;
  const double bytes = 4.0 * tok * kWoD + 4.0 * rows * (2.0 * a.dk + 2.0 * a.dv + 1.0) + 4.0 * rows * (2.0 * a.dk + a.dv);
  ProfScope ps(s, "attn_bwd_s32_wo_kernel", flops, bytes);
  hipLaunchKernelGGL(attn_bwd_s32_wo_kernel, dim3(a.B), dim3(256), 0, s, a, wo, gh2);
  return launch_status("attn_bwd_s32_wo_kernel");
}

size_t attn_bwd_workspace_bytes(const AttnDesc& d) {
  return (size_t)d.batch * d.heads * d.seq * sizeof(float);
}

static int attn_bwd_dq(const AttnArgs& a, int dkm, int dvm, hipStream_t s) {
  const long long items = (long long)a.B * a.H * ((a.S + 31) / 32);
  dim3 grid(ceil_div((size_t)items, 4));
  const double rows = (double)a.B * a.S * a.H;
  // s = q.k, dp = dO.v, dq += ds k; reads q k v o dO lse, writes dq and D
  const double flops = kept_pairs(a) * (4.0 * a.dk + 2.0 * a.dv);
  const double bytes = 4.0 * rows * (3.0 * a.dk + 3.0 * a.dv + 2.0);
  // up to 64 queries a 128-query tile leaves half its waves idle: the per-wave kernel is faster
  if (!attn_legacy() && a.S > 64) {
    // q, dO, O rows read and dq, D written once; K / V rows once per 128-query tile
    const double tiles = (a.S + kQTile - 1) / kQTile;
    const double tbytes = 4.0 * rows * (2.0 * a.dk + 2.0 * a.dv + 2.0) + 4.0 * a.B * a.H * tiles * a.S * (a.dk + a.dv);
    grid = dim3((unsigned)((long long)a.B * a.H * (long long)tiles));
#define TILED(DK, DV)                                                                        \
    if (dkm == DK && dvm == DV) {                                                            \
      ProfScope ps(s, "attn_bwd_dq_tiled_kernel<" #DK ", " #DV ">", flops, tbytes);          \
      hipLaunchKernelGGL((attn_bwd_dq_tiled_kernel<DK, DV>), grid, dim3(256), 0, s, a);      \
      return launch_status("attn_bwd_dq_tiled_kernel");                                      \
    }
    TILED(32, 32)
    TILED(64, 64)
    TILED(96, 64)
#undef TILED
    // head dims 128: the tiled kernel's operands and accumulators exceed the register file
  }
  ATTN_ALL(attn_bwd_dq_kernel)
}

static int attn_bwd_dkv(const AttnArgs& a, int dkm, int dvm, hipStream_t s) {
  const long long items = (long long)a.B * a.H * ((a.S + 31) / 32);
  dim3 grid(ceil_div((size_t)items, 4));
  const double rows = (double)a.B * a.S * a.H;
  // s = q.k, dp = dO.v, dv += p dO, dk += ds q; reads q dO lse D k v, writes dk dv
  const double flops = kept_pairs(a) * (4.0 * a.dk + 4.0 * a.dv);
  const double bytes = 4.0 * rows * (3.0 * a.dk + 3.0 * a.dv + 2.0);
  if (!attn_legacy()) {
    // k, v rows read and dk, dv written once; Q / dO rows and lse / D once per 128-key tile
    const double tiles = (a.S + kQTile - 1) / kQTile;
    const double tbytes = 4.0 * rows * (2.0 * a.dk + 2.0 * a.dv) + 4.0 * a.B * a.H * tiles * a.S * (a.dk + a.dv + 2.0);
    grid = dim3((unsigned)((long long)a.B * a.H * (long long)tiles));
#define TILED(DK, DV)                                                                        \
    if (dkm == DK && dvm == DV) {                                                            \
      ProfScope ps(s, "attn_bwd_dkv_tiled_kernel<" #DK ", " #DV ">", flops, tbytes);         \
      hipLaunchKernelGGL((attn_bwd_dkv_tiled_kernel<DK, DV>), grid, dim3(256), 0, s, a);     \
      return launch_status("attn_bwd_dkv_tiled_kernel");                                     \
    }
    TILED(32, 32)
    TILED(64, 64)
    TILED(96, 64)
#undef TILED
    // head dims 128: as in attn_bwd_dq
  }
  ATTN_ALL(attn_bwd_dkv_kernel)
}

static int attn_bwd_fused(const AttnArgs& a, int dkm, int dvm, hipStream_t s) {
  dim3 grid(ceil_div((size_t)a.B * a.H, 4));
  const double rows = (double)a.B * a.S * a.H;
  // s = q.k, dp = dO.v, dv = p^T dO, dk = ds^T q, dq = ds k; reads q k v o dO lse, writes dq dk dv
  const double flops = kept_pairs(a) * (6.0 * a.dk + 4.0 * a.dv);
  const double bytes = 4.0 * rows * (4.0 * a.dk + 4.0 * a.dv + 1.0);
  if (dkm == 32 && dvm == 32 && a.vec) {
    ProfScope ps(s, "attn_bwd_fused_kernel<32, 32, true>", flops, bytes);
    hipLaunchKernelGGL((attn_bwd_fused_kernel<32, 32, true>), grid, dim3(256), 0, s, a);
    return launch_status("attn_bwd_fused_kernel");
  }
  ATTN_ALL(attn_bwd_fused_kernel)
}

// The tiled backward with dQ formed from stored dS rows (d.ds): seq > 64 on the tiled kernels'
// head dims, rows of whole float4s.
bool attn_bwd_ds_supported(const AttnDesc& d) {
  int dkm, dvm;
  if (attn_legacy() || d.seq <= 64 || d.seq % 4 != 0 || !pick_dims(d.dk, d.dv, &dkm, &dvm)) return false;
  return (dkm == 32 && dvm == 32) || (dkm == 64 && dvm == 64) || (dkm == 96 && dvm == 64);
}

bool attn_ds_path(const AttnDesc& d) {
  return d.ds && (reinterpret_cast<uintptr_t>(d.ds) & 15) == 0 && attn_bwd_ds_supported(d);
}

size_t attn_bwd_ds_bytes(const AttnDesc& d) {
  const size_t entry = d.bf16 ? 2 : 4;  // bf16 plans keep dS as bf16 rows
  return attn_bwd_ds_supported(d) ? entry * (size_t)d.batch * d.heads * d.seq * d.seq : 0;
}

static int attn_bwd_with_ds(AttnArgs a, int dkm, int dvm, float* ds, bool bf16, bool d_ready, hipStream_t s) {
  a.ds = ds;
  const double rows = (double)a.B * a.S * a.H, tiles = (a.S + kQTile - 1) / kQTile, pairs = kept_pairs(a);
  if (!d_ready) {  // D = rowsum(dO * O)
    ProfScope ps(s, "attn_rowdot_kernel", 2.0 * rows * a.dv, 4.0 * rows * (2.0 * a.dv + 1.0));
    hipLaunchKernelGGL(attn_rowdot_kernel, dim3(ceil_div((size_t)rows, 16)), dim3(256), 0, s, a);
    if (int rc = launch_status("attn_rowdot_kernel")) return rc;
  }
  // dK / dV: s = q.k, dp = dO.v, dv += p dO, dk += ds q; k, v rows once, q / dO / O rows and lse
  // once per 128-key tile; dS written
  {
    const double bytes = 4.0 * rows * (2.0 * a.dk + 2.0 * a.dv) +
                         4.0 * a.B * a.H * tiles * a.S * (a.dk + a.dv + 2.0) + (bf16 ? 2.0 : 4.0) * pairs;
    dim3 grid((unsigned)((long long)a.B * a.H * (long long)tiles));
#define TILED(DK, DV)                                                                              \
    if (dkm == DK && dvm == DV && bf16) {                                                          \
      ProfScope ps(s, "attn_bwd_dkv_bf16_kernel<" #DK ", " #DV ">", pairs * (4.0 * a.dk + 4.0 * a.dv), bytes); \
      hipLaunchKernelGGL((attn_bwd_dkv_bf16_kernel<DK, DV>), grid, dim3(256), 0, s, a);           \
      if (int rc = launch_status("attn_bwd_dkv_bf16_kernel")) return rc;                           \
    } else if (dkm == DK && dvm == DV) {                                                           \
      ProfScope ps(s, "attn_bwd_dkv_tiled_kernel<" #DK ", " #DV ", true>", pairs * (4.0 * a.dk + 4.0 * a.dv), bytes); \
      hipLaunchKernelGGL((attn_bwd_dkv_tiled_kernel<DK, DV, true>), grid, dim3(256), 0, s, a);    \
      if (int rc = launch_status("attn_bwd_dkv_tiled_kernel")) return rc;                          \
    }
    TILED(32, 32)
    TILED(64, 64)
    TILED(96, 64)
#undef TILED
  }
  // dQ = dS . K: dS read, K rows once per 128-query tile, dq written
  const double bytes = (bf16 ? 2.0 : 4.0) * pairs + 4.0 * a.B * a.H * tiles * a.S * a.dk + 4.0 * rows * a.dk;
  dim3 grid((unsigned)((long long)a.B * a.H * (long long)tiles));
#define TILED(DK)                                                                                  \
  if (dkm == DK && bf16) {                                                                         \
    ProfScope ps(s, "attn_bwd_dq_ds_bf16_kernel<" #DK ">", pairs * 2.0 * a.dk, bytes);            \
    hipLaunchKernelGGL((attn_bwd_dq_ds_bf16_kernel<DK>), grid, dim3(256), 0, s, a);               \
    return launch_status("attn_bwd_dq_ds_bf16_kernel");                                            \
  }                                                                                                \
  if (dkm == DK) {                                                                                 \
    ProfScope ps(s, "attn_bwd_dq_ds_kernel<" #DK ">", pairs * 2.0 * a.dk, bytes);                 \
    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<DK>), grid, dim3(256), 0, s, a);                    \
    return launch_status("attn_bwd_dq_ds_kernel");                                                 \
  }
  TILED(32)
  TILED(64)
  TILED(96)
#undef TILED
  set_error("attention backward: no dS kernel for head dims (%d, %d)", dkm, dvm);
  return TALOS_ERR_UNSUPPORTED;
}

bool attn_bwd_uses_workspace(const AttnDesc& d) {
  return (long long)d.batch * d.heads * d.seq > 0 && d.seq > 32;
}

int attn_bwd_launch(const AttnDesc& d, float* ws, hipStream_t s) {
  int dkm, dvm;
  if (!pick_dims(d.dk, d.dv, &dkm, &dvm)) {
    set_error("attention: head dims (%d, %d) exceed the supported (128, 128)", d.dk, d.dv);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, dkm, dvm);
  a.D = ws;
  if ((long long)a.B * a.H * a.S == 0) return TALOS_OK;
  if (a.S <= 32) return attn_bwd_fused(a, dkm, dvm, s);
  if (a.S <= 64 && d.dk == 32 && d.dv == 32 && a.vec && !attn_legacy()) {
    const double rows = (double)a.B * a.S * a.H;
    ProfScope ps(s, a.causal ? "attn_bwd_s64_kernel<3>" : "attn_bwd_s64_kernel<4>", kept_pairs(a) * (6.0 * a.dk + 4.0 * a.dv),
                 4.0 * rows * (4.0 * a.dk + 4.0 * a.dv + 1.0));
    if (a.causal)
      hipLaunchKernelGGL(attn_bwd_s64_kernel<3>, dim3((unsigned)((long long)a.B * a.H)), dim3(192), 0, s, a);
    else
      hipLaunchKernelGGL(attn_bwd_s64_kernel<4>, dim3((unsigned)((long long)a.B * a.H)), dim3(256), 0, s, a);
    return launch_status("attn_bwd_s64_kernel");
  }
  if (d.out_bf16 && !(d.bf16 && attn_ds_path(d))) {
    set_error("attention backward: bf16 gradient outputs need the bf16 dS path (bf16, attn_ds_path)");
    return TALOS_ERR_UNSUPPORTED;
  }
  if (attn_ds_path(d)) {
    // the forward decided on the same predicate (its bf16 kernel, split inputs): the backward
    // must not fall back to another path here
    if (!ws) {
      set_error("attention backward: the dS path needs the workspace (attn_bwd_workspace_bytes)");
      return TALOS_ERR_NULL;
    }
    return attn_bwd_with_ds(a, dkm, dvm, d.ds, d.bf16 != 0, d.d_ready != 0, s);
  }
  if (d.dq2 || d.dk2) {
    set_error("attention backward: split dq / dk outputs need the dS path (attn_ds_path)");
    return TALOS_ERR_UNSUPPORTED;
  }
  int rc = attn_bwd_dq(a, dkm, dvm, s);
  if (rc) return rc;
  return attn_bwd_dkv(a, dkm, dvm, s);
}

// ---------------------------------------------------------------------------
// Last query only: attention for the one query row per sample a caller reads (the last token,
// row key_len - 1), over all of that sample's keys. Row-parallel layout: a wave covers 64 / C
// key rows per pass with C = D / 4 lanes per row, each lane holding 4 consecutive elements
// (16-byte loads and stores, a row's C lanes read or write its D floats contiguously). Dot
// products reduce over a row's C lanes, per-element sums over the wave's rows.
// ---------------------------------------------------------------------------
template <int C>
__device__ __forceinline__ float row_sum(float v) {  // over the C lanes of a row
#pragma unroll
  for (int o = 1; o < C; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int C>
__device__ __forceinline__ float col_sum(float v) {  // over the rows of a pass (lanes c, c + C, ...)
#pragma unroll
  for (int o = C; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int C>
__device__ __forceinline__ float col_max(float v) {
#pragma unroll
  for (int o = C; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void st4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ float dot4(float4 a, float4 b) { return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w; }
// R^T at position pos on the two interleaved pairs of elements e0 .. e0 + 3 (e0 even)
__device__ __forceinline__ float4 rope_t4(float4 g, int e0, int pos, const AttnArgs& a) {
  if (a.rcos == nullptr) return g;
  const int half = a.rope_dim >> 1;
  float r[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const int e = e0 + i;
    if (e >= a.rope_off && e < a.rope_off + a.rope_dim) {
      const int idx = pos * half + ((e - a.rope_off) >> 1);
      const float c = a.rcos[idx], sn = a.rsin[idx];
      const float g0 = r[i], g1 = r[i + 1];
      r[i] = fmaf(g0, c, g1 * sn);
      r[i + 1] = fmaf(-g0, sn, g1 * c);
    }
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}

// R at position pos on the two interleaved pairs of elements e0 .. e0 + 3 (e0 even):
// (x0, x1) -> (x0 c - x1 s, x0 s + x1 c), the rotation of src/transformer.rs:276-292
__device__ __forceinline__ float4 rope4(float4 x, int e0, int pos, const AttnArgs& a) {
  if (a.rcos == nullptr) return x;
  const int half = a.rope_dim >> 1;
  float r[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const int e = e0 + i;
    if (e >= a.rope_off && e < a.rope_off + a.rope_dim) {
      const int idx = pos * half + ((e - a.rope_off) >> 1);
      const float c = a.rcos[idx], sn = a.rsin[idx];
      const float x0 = r[i], x1 = r[i + 1];
      r[i] = fmaf(x0, c, -x1 * sn);
      r[i + 1] = fmaf(x0, sn, x1 * c);
    }
  }
  return make_float4(r[0], r[1], r[2], r[3]);
}
// The last query of batch entry b (row t), rotated: from q's row, or from q_last's row b.
__device__ __forceinline__ float4 last_query(const AttnArgs& a, int b, long long tok0, int t, int hh, int D, int c) {
  if (a.q_last) return rope4(ld4(a.q_last + (long long)b * a.ldq_last + hh * D + 4 * c), 4 * c, t, a);
  return ld4(a.q + (tok0 + t) * a.ldq + hh * D + 4 * c);
}

// o_last[b, h] = softmax(scale q_t . K^T) V over keys j < L (t = L - 1); lse_last[b*H + h].
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_lastq_kernel(AttnArgs a, float* __restrict__ o_last, long long ldol,
                                                             float* __restrict__ lse_last) {
  constexpr int C = D / 4, RPP = 64 / C;  // lanes per row, rows per pass
  const int lane = threadIdx.x & 63, c = lane % C, r = lane / C;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= a.B * a.H) return;  // uniform per wave
  const int b = pair / a.H, hh = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b), t = Sk - 1;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float m = kNegInf, l = 0.f;
  if (Sk > 0) {
    float4 q = last_query(a, b, tok0, t, hh, D, c);
    q = make_float4(q.x * a.scale, q.y * a.scale, q.z * a.scale, q.w * a.scale);
    for (int j0 = 0; j0 < Sk; j0 += RPP) {
      const int j = j0 + r;
      const bool ok = j < Sk;
      const int jj = ok ? j : t;  // in-range row for the (discarded) loads of padding lanes
      const float4 k = ld4(a.k + (tok0 + jj) * a.ldk + hh * D + 4 * c);
      const float4 v = ld4(a.v + (tok0 + jj) * a.ldv + hh * D + 4 * c);
      const float sc = row_sum<C>(dot4(q, k));
      const float s = ok ? sc : kNegInf;
      const float mn = fmaxf(m, col_max<C>(s));
      const float p = ok ? __expf(s - mn) : 0.f;
      const float corr = m == kNegInf ? 0.f : __expf(m - mn);
      l = l * corr + col_sum<C>(p);  // p is the same on a row's C lanes: the sum over the pass's rows
      acc = make_float4(acc.x * corr + p * v.x, acc.y * corr + p * v.y, acc.z * corr + p * v.z,
                        acc.w * corr + p * v.w);
      m = mn;
    }
  }
  acc = make_float4(col_sum<C>(acc.x), col_sum<C>(acc.y), col_sum<C>(acc.z), col_sum<C>(acc.w));
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (r == 0) st4(o_last + (long long)b * ldol + hh * D + 4 * c, make_float4(acc.x * inv, acc.y * inv, acc.z * inv,
                                                                          acc.w * inv));
  if (lane == 0) lse_last[pair] = l > 0.f ? m + logf(l) : kNegInf;
}

// Backward with dO non-zero on the last query only: dv_j = p_j dO, dk_j = R^T(dS_j scale q_t),
// dq_t = R^T(scale sum_j dS_j k_j), every other dq row 0; rows j >= L get dk = dv = 0.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_lastq_kernel(AttnArgs a, const float* __restrict__ o_last,
                                                             long long ldol, const float* __restrict__ lse_last,
                                                             const float* __restrict__ do_last, long long lddol) {
  constexpr int C = D / 4, RPP = 64 / C;
  const int lane = threadIdx.x & 63, c = lane % C, r = lane / C;
  const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= a.B * a.H) return;
  const int b = pair / a.H, hh = pair % a.H;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b), t = Sk > 0 ? Sk - 1 : 0;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 qs = z4, g = z4;
  float Dd = 0.f, lse = 0.f;
  if (Sk > 0) {
    const float4 q = last_query(a, b, tok0, t, hh, D, c);
    qs = make_float4(q.x * a.scale, q.y * a.scale, q.z * a.scale, q.w * a.scale);
    g = ld4(do_last + (long long)b * lddol + hh * D + 4 * c);
    Dd = row_sum<C>(dot4(g, ld4(o_last + (long long)b * ldol + hh * D + 4 * c)));
    lse = lse_last[pair];
  }
  float4 dq = z4;
  for (int j0 = 0; j0 < a.S; j0 += RPP) {
    const int j = j0 + r;
    const bool in = j < a.S, ok = j < Sk;
    const int jj = ok ? j : 0;
    const float4 k = ld4(a.k + (tok0 + jj) * a.ldk + hh * D + 4 * c);
    const float4 v = ld4(a.v + (tok0 + jj) * a.ldv + hh * D + 4 * c);
    const float s = row_sum<C>(dot4(qs, k));
    const float p = ok ? __expf(s - lse) : 0.f;
    const float dp = row_sum<C>(dot4(g, v));
    const float dS = p * (dp - Dd);
    dq = make_float4(dq.x + dS * k.x, dq.y + dS * k.y, dq.z + dS * k.z, dq.w + dS * k.w);
    if (in) {
      const long long row = tok0 + j;
      st4(a.dv_out + row * a.lddv + hh * D + 4 * c, make_float4(p * g.x, p * g.y, p * g.z, p * g.w));
      st4(a.dk_out + row * a.lddk + hh * D + 4 * c,
          rope_t4(make_float4(dS * qs.x, dS * qs.y, dS * qs.z, dS * qs.w), 4 * c, j, a));
      if (a.dq_last == nullptr && (j != t || Sk == 0)) st4(a.dq + row * a.lddq + hh * D + 4 * c, z4);
    }
  }
  dq = make_float4(col_sum<C>(dq.x) * a.scale, col_sum<C>(dq.y) * a.scale, col_sum<C>(dq.z) * a.scale,
                   col_sum<C>(dq.w) * a.scale);
  if (a.dq_last) {
    if (r == 0) st4(a.dq_last + (long long)b * a.lddq_last + hh * D + 4 * c, Sk > 0 ? rope_t4(dq, 4 * c, t, a) : z4);
  } else if (r == 0 && Sk > 0) {
    st4(a.dq + (tok0 + t) * a.lddq + hh * D + 4 * c, rope_t4(dq, 4 * c, t, a));
  }
}

// ---------------------------------------------------------------------------
// Last query with the value projection absorbed (the policy's last layer): v_j = xn_j . Wv per
// head, and V carries no rotation, so o_h = sum_j p_j v_j = (sum_j p_j xn_j) . Wv_h. The forward
// forms z_h = sum_j p_j xn_j over the sample's normalised input rows xn (width W = 128) instead
// of reading value rows, and the caller multiplies z_h by Wv_h (a small batched product); the
// backward takes u_h = Wv_h dO_h from the caller, forms dP_j = xn_j . u_h, and writes, besides dK
// and the last query's dq, the weights p_j^h of every row, from which the product that forms the
// rest of dL/dxn adds the value path's share, sum_h p_j^h u_h, in its epilogue. No value rows are
// ever formed.
// ---------------------------------------------------------------------------
constexpr int kVabsW = 128, kVabsH = 4, kVabsMaxS = 256;

// A workgroup per sample, wave h its head h: z[b, h] = sum_j p_j xn_j ([B][H][W]) and
// lse_last[b*H + h]. Each wave first scores its head over the sample's keys (row layout, the
// scores kept in LDS, exact maximum and sum); then wave w takes the keys j = w, w + H, ..., loads
// each such xn row once (two columns a lane) and accumulates p_j^h xn_j for all H heads; the H
// waves' partial sums are added in wave order.
template <int D>
__global__ __launch_bounds__(64 * kVabsH) void attn_fwd_lastq_z_kernel(AttnArgs a, const float* __restrict__ xn,
                                                                       long long ldx, float* __restrict__ z,
                                                                       float* __restrict__ lse_last) {
  constexpr int C = D / 4, RPP = 64 / C;
  __shared__ float ps[kVabsH][kVabsMaxS];
  __shared__ float mh[kVabsH], ilh[kVabsH];
  __shared__ __align__(16) float zp[kVabsH][kVabsH][kVabsW];  // [wave][head][column]
  const int lane = threadIdx.x & 63, c = lane % C, r = lane / C, hh = threadIdx.x >> 6;
  const int b = blockIdx.x, pair = b * a.H + hh;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b), t = Sk - 1;
  float m = kNegInf;
  if (Sk > 0) {
    float4 q = last_query(a, b, tok0, t, hh, D, c);
    q = make_float4(q.x * a.scale, q.y * a.scale, q.z * a.scale, q.w * a.scale);
    for (int j0 = 0; j0 < Sk; j0 += RPP) {
      const int j = j0 + r;
      const bool ok = j < Sk;
      const float4 k = ld4(a.k + (tok0 + (ok ? j : t)) * a.ldk + hh * D + 4 * c);
      const float s = ok ? row_sum<C>(dot4(q, k)) : kNegInf;
      if (ok && c == 0) ps[hh][j] = s;
      m = fmaxf(m, col_max<C>(s));
    }
  }
  wave_lds_sync();
  float l = 0.f;
  for (int j = lane; j < Sk; j += 64) l += __expf(ps[hh][j] - m);
  l = wave_sum(l);
  if (lane == 0) {
    mh[hh] = m;
    ilh[hh] = l > 0.f ? 1.f / l : 0.f;
    lse_last[pair] = l > 0.f ? m + logf(l) : kNegInf;
  }
  __syncthreads();
  float2 acc[kVabsH];
#pragma unroll
  for (int i = 0; i < kVabsH; ++i) acc[i] = make_float2(0.f, 0.f);
  for (int j = hh; j < Sk; j += kVabsH) {
    const float2 x = *reinterpret_cast<const float2*>(xn + (tok0 + j) * ldx + 2 * lane);
#pragma unroll
    for (int i = 0; i < kVabsH; ++i) {
      const float pj = __expf(ps[i][j] - mh[i]) * ilh[i];
      acc[i] = make_float2(fmaf(pj, x.x, acc[i].x), fmaf(pj, x.y, acc[i].y));
    }
  }
#pragma unroll
  for (int i = 0; i < kVabsH; ++i) *reinterpret_cast<float2*>(&zp[hh][i][2 * lane]) = acc[i];
  __syncthreads();
  float2 zs = make_float2(0.f, 0.f);
#pragma unroll
  for (int w = 0; w < kVabsH; ++w) {
    const float2 v = *reinterpret_cast<const float2*>(&zp[w][hh][2 * lane]);
    zs = make_float2(zs.x + v.x, zs.y + v.y);
  }
  *reinterpret_cast<float2*>(z + (long long)pair * kVabsW + 2 * lane) = zs;
}

// A workgroup per sample, wave h its head h (kVabsH heads of D). dk rows j < S (zero past the
// sample's keys), dq_last, and prow[b*S + j][h] = p_j^h (zero past the keys); u = [B][H][W].
template <int D>
__global__ __launch_bounds__(64 * kVabsH) void attn_bwd_lastq_z_kernel(AttnArgs a, const float* __restrict__ xn,
                                                                       long long ldx, const float* __restrict__ u,
                                                                       const float* __restrict__ o_last, long long ldol,
                                                                       const float* __restrict__ lse_last,
                                                                       const float* __restrict__ do_last,
                                                                       long long lddol, float* __restrict__ prow) {
  constexpr int C = D / 4, RPP = 64 / C;
  __shared__ float ps[kVabsH][kVabsMaxS], dss[kVabsH][kVabsMaxS];
  __shared__ __align__(16) float us[kVabsH][kVabsW];
  const int lane = threadIdx.x & 63, c = lane % C, r = lane / C, hh = threadIdx.x >> 6;
  const int b = blockIdx.x, pair = b * a.H + hh;
  const long long tok0 = (long long)b * a.S;
  const int Sk = key_len(a, b), t = Sk > 0 ? Sk - 1 : 0;
  const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 qs = z4;
  float Dd = 0.f, lse = 0.f;
  if (Sk > 0) {
    const float4 q = last_query(a, b, tok0, t, hh, D, c);
    qs = make_float4(q.x * a.scale, q.y * a.scale, q.z * a.scale, q.w * a.scale);
    const float4 g = ld4(do_last + (long long)b * lddol + hh * D + 4 * c);
    Dd = row_sum<C>(dot4(g, ld4(o_last + (long long)b * ldol + hh * D + 4 * c)));
    lse = lse_last[pair];
  }
  const float2 uh = *reinterpret_cast<const float2*>(u + (long long)pair * kVabsW + 2 * lane);
  *reinterpret_cast<float2*>(&us[hh][2 * lane]) = uh;
  __shared__ float Dl[kVabsH];
  if (lane == 0) Dl[hh] = Dd;
  // p_j for every key (row layout)
  for (int j0 = 0; j0 < a.S; j0 += RPP) {
    const int j = j0 + r;
    const bool ok = j < Sk;
    const float4 k = ld4(a.k + (tok0 + (ok ? j : 0)) * a.ldk + hh * D + 4 * c);
    const float s = row_sum<C>(dot4(qs, k));
    if (c == 0 && j < a.S) ps[hh][j] = ok ? __expf(s - lse) : 0.f;
  }
  __syncthreads();
  // dS_j^h = p_j^h (xn_j . u_h - D_h) for every head: wave w takes the key pairs j0 = 2w, 2w + 2H,
  // ... (32 lanes a row, float4 each, two rows a pass), each xn row read once for all H heads
  {
    constexpr int C2 = kVabsW / 4;  // 32 lanes per xn row
    const int c2 = lane % C2, rh = lane / C2;
    float4 u4[kVabsH];
#pragma unroll
    for (int i = 0; i < kVabsH; ++i) u4[i] = *reinterpret_cast<const float4*>(&us[i][4 * c2]);
    for (int j0 = 2 * hh; j0 < Sk; j0 += 2 * kVabsH) {
      const int j = j0 + rh;
      const bool ok = j < Sk;
      const float4 x = ld4(xn + (tok0 + (ok ? j : j0)) * ldx + 4 * c2);
#pragma unroll
      for (int i = 0; i < kVabsH; ++i) {
        const float dp = row_sum<C2>(dot4(x, u4[i]));
        if (ok && c2 == 0) dss[i][j] = ps[i][j] * (dp - Dl[i]);
      }
    }
  }
  __syncthreads();
  // dk_j = R^T(dS_j scale q), dq = R^T(scale sum_j dS_j k_j) (row layout)
  float4 dq = z4;
  for (int j0 = 0; j0 < a.S; j0 += RPP) {
    const int j = j0 + r;
    const bool ok = j < Sk;
    const float dS = ok ? dss[hh][j] : 0.f;
    if (ok) {
      const float4 k = ld4(a.k + (tok0 + j) * a.ldk + hh * D + 4 * c);
      dq = make_float4(dq.x + dS * k.x, dq.y + dS * k.y, dq.z + dS * k.z, dq.w + dS * k.w);
    }
    if (j < a.S)
      st4(a.dk_out + (tok0 + j) * a.lddk + hh * D + 4 * c,
          rope_t4(make_float4(dS * qs.x, dS * qs.y, dS * qs.z, dS * qs.w), 4 * c, j, a));
  }
  dq = make_float4(col_sum<C>(dq.x) * a.scale, col_sum<C>(dq.y) * a.scale, col_sum<C>(dq.z) * a.scale,
                   col_sum<C>(dq.w) * a.scale);
  if (r == 0) st4(a.dq_last + (long long)b * a.lddq_last + hh * D + 4 * c, Sk > 0 ? rope_t4(dq, 4 * c, t, a) : z4);
  // every row's weights p_j^h (the value path's share of dL/dxn is formed from them downstream)
  for (int f = threadIdx.x; f < a.S * kVabsH; f += 64 * kVabsH) prow[tok0 * kVabsH + f] = ps[f % kVabsH][f / kVabsH];
}

int attn_lastq_vabs_supported(const AttnDesc& d, const float* xn, long long ldx) {
  auto al = [](const void* p, long long ld) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0; };
  return d.dk == 32 && d.dv == 32 && d.heads == kVabsH && d.seq >= 1 && d.seq <= kVabsMaxS && xn != nullptr &&
         al(xn, ldx) && al(d.k, d.ldk) && d.q_last != nullptr && al(d.q_last, d.ldq_last) && d.dq_last != nullptr &&
         al(d.dq_last, d.lddq_last) && (d.dk_out == nullptr || al(d.dk_out, d.lddk));
}

int attn_fwd_lastq_z_launch(const AttnDesc& d, const float* xn, long long ldx, float* z, float* lse_last,
                            hipStream_t s) {
  if (!attn_lastq_vabs_supported(d, xn, ldx)) {
    set_error("attention (last query, absorbed values): needs head dims 32, %d heads, seq <= %d, aligned rows",
              kVabsH, kVabsMaxS);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, 32, 32);
  if ((long long)a.B * a.H == 0) return TALOS_OK;
  const double rows = (double)a.B * a.H;
  // q row, k rows and xn rows of the sample read; z and lse written
  ProfScope ps(s, "attn_fwd_lastq_z_kernel<32>", rows * a.S * 2.0 * (d.dk + kVabsW),
               4.0 * (rows * (a.S * d.dk + d.dk + kVabsW + 1.0) + (double)a.B * a.S * kVabsW));
  hipLaunchKernelGGL(attn_fwd_lastq_z_kernel<32>, dim3((unsigned)a.B), dim3(64 * kVabsH), 0, s, a, xn, ldx, z,
                     lse_last);
  return launch_status("attn_fwd_lastq_z_kernel");
}

int attn_bwd_lastq_z_launch(const AttnDesc& d, const float* xn, long long ldx, const float* u, const float* o_last,
                            long long ldol, const float* lse_last, const float* do_last, long long lddol, float* prow,
                            hipStream_t s) {
  if (!attn_lastq_vabs_supported(d, xn, ldx) || d.dk_out == nullptr || prow == nullptr) {
    set_error("attention backward (last query, absorbed values): needs head dims 32, %d heads, seq <= %d, dk and "
              "the value-path rows", kVabsH, kVabsMaxS);
    return TALOS_ERR_UNSUPPORTED;
  }
  AttnArgs a = make_args(d, 32, 32);
  if ((long long)a.B * a.S == 0) return TALOS_OK;
  const double rows = (double)a.B * a.H;
  // k and xn rows read, dk rows and the weights written; q, o, dO, u of the last row read
  ProfScope ps(s, "attn_bwd_lastq_z_kernel<32>", rows * a.S * (6.0 * d.dk + 2.0 * kVabsW),
               4.0 * (rows * a.S * (2.0 * d.dk + 1.0) + (double)a.B * a.S * kVabsW + rows * (4.0 * d.dk + kVabsW)));
  hipLaunchKernelGGL(attn_bwd_lastq_z_kernel<32>, dim3((unsigned)a.B), dim3(64 * kVabsH), 0, s, a, xn, ldx, u, o_last,
                     ldol, lse_last, do_last, lddol, prow);
  return launch_status("attn_bwd_lastq_z_kernel");
}

int attn_lastq_supported(const AttnDesc& d) {
  auto al = [](const void* p, long long ld) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ld % 4 == 0; };
  return (d.dk == d.dv && (d.dk == 32 || d.dk == 64) && al(d.q, d.ldq) && al(d.k, d.ldk) && al(d.v, d.ldv) &&
          (d.q_last == nullptr || al(d.q_last, d.ldq_last)) && (d.dq_last == nullptr || al(d.dq_last, d.lddq_last)))
             ? 1
             : 0;
}

int attn_fwd_lastq_launch(const AttnDesc& d, float* o_last, long long ldol, float* lse_last, hipStream_t s) {
  AttnArgs a = make_args(d, d.dk, d.dv);
  if ((long long)a.B * a.H == 0) return TALOS_OK;
  dim3 grid(ceil_div((size_t)a.B * a.H, 4));
  // q row, k and v over the sample's keys read; o row and lse written
  const double rows = (double)a.B * a.H;
  ProfScope ps(s, d.dk == 32 ? "attn_fwd_lastq_kernel<32>" : "attn_fwd_lastq_kernel<64>",
               rows * a.S * 4.0 * d.dk, 4.0 * rows * ((2.0 * a.S + 2.0) * d.dk + 1.0));
  if (d.dk == 32)
    hipLaunchKernelGGL(attn_fwd_lastq_kernel<32>, grid, dim3(256), 0, s, a, o_last, ldol, lse_last);
  else
    hipLaunchKernelGGL(attn_fwd_lastq_kernel<64>, grid, dim3(256), 0, s, a, o_last, ldol, lse_last);
  return launch_status("attn_fwd_lastq_kernel");
}

int attn_bwd_lastq_launch(const AttnDesc& d, const float* o_last, long long ldol, const float* lse_last,
                          const float* do_last, long long lddol, hipStream_t s) {
  AttnArgs a = make_args(d, d.dk, d.dv);
  if ((long long)a.B * a.H * a.S == 0) return TALOS_OK;
  dim3 grid(ceil_div((size_t)a.B * a.H, 4));
  // k, v read and dq, dk, dv written over every row; q, o, dO of the last row read
  const double rows = (double)a.B * a.H;
  ProfScope ps(s, d.dk == 32 ? "attn_bwd_lastq_kernel<32>" : "attn_bwd_lastq_kernel<64>",
               rows * a.S * 10.0 * d.dk, 4.0 * rows * ((5.0 * a.S + 3.0) * d.dk + 1.0));
  if (d.dk == 32)
    hipLaunchKernelGGL(attn_bwd_lastq_kernel<32>, grid, dim3(256), 0, s, a, o_last, ldol, lse_last, do_last, lddol);
  else
    hipLaunchKernelGGL(attn_bwd_lastq_kernel<64>, grid, dim3(256), 0, s, a, o_last, ldol, lse_last, do_last, lddol);
  return launch_status("attn_bwd_lastq_kernel");
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

// Validates the arguments of the attention backward entry points and fills the descriptor.
static int attn_bwd_desc(const char* fn, int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal,
                         const float* q, int ld_q, const float* k, int ld_k, const float* v, int ld_v, const float* o,
                         int ld_o, const float* lse, const float* dout, int ld_do, float* dq, int ld_dq, float* dk,
                         int ld_dk, float* dv, int ld_dv, AttnDesc* out) {
  TALOS_NONNULL(q);
  TALOS_NONNULL(k);
  TALOS_NONNULL(v);
  TALOS_NONNULL(o);
  TALOS_NONNULL(lse);
  TALOS_NONNULL(dout);
  TALOS_NONNULL(dq);
  TALOS_NONNULL(dk);
  TALOS_NONNULL(dv);
  int rc = check_attn(fn, batch, seq, heads, qk_dim, v_dim, causal, ld_q, ld_k, ld_v, ld_o);
  if (rc) return rc;
  TALOS_REQUIRE(ld_do >= heads * v_dim && ld_dq >= heads * qk_dim && ld_dk >= heads * qk_dim && ld_dv >= heads * v_dim,
                TALOS_ERR_SHAPE, "%s: a gradient row stride is smaller than heads * dim", fn);
  AttnDesc& d = *out;
  d.batch = batch; d.seq = seq; d.heads = heads; d.dk = qk_dim; d.dv = v_dim; d.scale = scale; d.causal = causal;
  d.q = q; d.ldq = ld_q; d.k = k; d.ldk = ld_k; d.v = v; d.ldv = ld_v;
  d.o = const_cast<float*>(o); d.ldo = ld_o; d.lse = const_cast<float*>(lse);
  d.dout = dout; d.lddo = ld_do; d.dq = dq; d.lddq = ld_dq; d.dk_out = dk; d.lddk = ld_dk; d.dv_out = dv; d.lddv = ld_dv;
  return TALOS_OK;
}

// The static scratch of talos_attn_bwd_noalloc_f32: D = rowsum(dO * O) of every (batch, head,
// query) row, written by attn_bwd_dq_kernel and read by attn_bwd_dkv_kernel of the same call (so
// nothing in it needs clearing). Each GPU holds its own copy for the life of the process; its
// device address is looked up once per device (hipGetSymbolAddress) and kept, and only that
// address is ever handed to a kernel. Calls that overlap on one GPU share the array and race.
constexpr size_t kAttnScratchRows = size_t(1) << 20;  // 4 MiB
static __device__ __align__(256) float scratch[kAttnScratchRows];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static float* g_scratch_ptr[kMaxDevices] = {};

static int attn_scratch(float** out) {
  int dev = 0;
  TALOS_HIP(hipGetDevice(&dev));
  TALOS_REQUIRE(dev >= 0 && dev < kMaxDevices, TALOS_ERR_UNSUPPORTED, "attention scratch: device %d >= %d", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    TALOS_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    TALOS_REQUIRE(ptr != nullptr, TALOS_ERR_HIP, "attention scratch: hipGetSymbolAddress gave no address");
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
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
  return entry_done(attn_fwd_launch(d, as_stream(stream)), as_stream(stream));
}

int talos_attn_bwd_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal, const float* q,
                       int ld_q, const float* k, int ld_k, const float* v, int ld_v, const float* o, int ld_o,
                       const float* lse, const float* dout, int ld_do, float* dq, int ld_dq, float* dk, int ld_dk,
                       float* dv, int ld_dv, talos_stream_t stream) {
  AttnDesc d;
  int rc = attn_bwd_desc(__func__, batch, seq, heads, qk_dim, v_dim, scale, causal, q, ld_q, k, ld_k, v, ld_v, o, ld_o,
                         lse, dout, ld_do, dq, ld_dq, dk, ld_dk, dv, ld_dv, &d);
  if (rc) return rc;
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  EntryScratch ws;
  if ((rc = ws.acquire(attn_bwd_uses_workspace(d) ? attn_bwd_workspace_bytes(d) : 0, s))) return rc;
  rc = attn_bwd_launch(d, static_cast<float*>(ws.ptr), s);
  const int rel = ws.release();
  return entry_done(rc ? rc : rel, as_stream(stream));
}

int talos_attn_bwd_noalloc_f32(int batch, int seq, int heads, int qk_dim, int v_dim, float scale, int causal,
                               const float* q, int ld_q, const float* k, int ld_k, const float* v, int ld_v,
                               const float* o, int ld_o, const float* lse, const float* dout, int ld_do, float* dq,
                               int ld_dq, float* dk, int ld_dk, float* dv, int ld_dv, talos_stream_t stream) {
  AttnDesc d;
  int rc = attn_bwd_desc(__func__, batch, seq, heads, qk_dim, v_dim, scale, causal, q, ld_q, k, ld_k, v, ld_v, o, ld_o,
                         lse, dout, ld_do, dq, ld_dq, dk, ld_dk, dv, ld_dv, &d);
  if (rc) return rc;
  const size_t rows = (size_t)batch * heads * seq;
  TALOS_REQUIRE(rows <= kAttnScratchRows, TALOS_ERR_UNSUPPORTED,
                "%s: batch * heads * seq = %zu exceeds the %zu (batch, head, query) rows of the static scratch", __func__,
                rows, kAttnScratchRows);
  TALOS_DEVICE();
  float* ws = nullptr;
  if (attn_bwd_uses_workspace(d))
    if ((rc = attn_scratch(&ws))) return rc;
  return entry_done(attn_bwd_launch(d, ws, as_stream(stream)), as_stream(stream));
}

}  // extern "C"
