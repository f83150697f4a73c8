// gemm.hip -- fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32) for gfx950.
//
// Replaces the row-accumulation matmul of the reference and its backward
// (src/autograd.rs:200-354): forward C = A.B, dA += dC.B^T, dB += A^T.dC, plus the batched
// Q.K^T / P.V products of attention (src/transformer.rs:877-1050).
//
// Tiling: a 256-thread workgroup owns a 128x128 tile of C; each of its four waves owns a
// 64x64 quarter as 2x2 MFMA 32x32 accumulators (64 accumulator registers per lane). K advances
// in chunks of 32 staged through LDS; the next chunk is fetched into registers while the matrix
// cores work on the current one. Each operand panel keeps the layout the operand has in memory:
// k-contiguous operands (A plain, B transposed) as rows of 32 k values (pitch 36), read by the
// MFMA lanes as 16-byte fragments of 4 consecutive k; the others k-major (pitch 136), read one
// value per lane. Global loads and LDS stores are 16 bytes wide in both cases, and the k order
// of the MFMA chain (step s, half h <-> k = 8(s/4) + 4h + s%4) is shared by the two operands.
// Interior tiles take an unchecked load / store path; only edge tiles test bounds per element.
// The epilogue (bias, residual, activation or its derivative, RoPE) is a compile-time set of
// flags, so each instantiation carries only the code it uses.
// Long-K products with a small C (the weight gradients, K = tokens) are split over K; the fp32
// partial tiles are combined in f64 by a second kernel, which keeps the gradient sums over
// 10^5 tokens within the accuracy of an fp32 dot product of length K/ksplit.
#include <algorithm>

#include "gemm.hpp"
#include "rowops.hpp"

namespace talos {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 32;
// k-major panel X[k][r]: the two half-waves read rows k and k + 4, whose offset 4 * 136 = 32
// mod 64 banks keeps them on disjoint banks.
constexpr int LDS_S = 136;
// k-contiguous panel X[r][k]: 16-byte fragments of 16 consecutive rows fall on 16 distinct
// groups of 4 banks (row * 9 mod 16).
constexpr int KP = 36;
constexpr int PANEL = (BK * LDS_S > 128 * KP) ? BK * LDS_S : 128 * KP;  // floats per panel
constexpr int NT = 256;
// Tuning knobs (compile-time): TALOS_GEMM_DBUF = 1 double-buffers the LDS panels (one barrier per
// K chunk); TALOS_GEMM_WAVES = minimum waves per SIMD the register allocation must allow.
#ifndef TALOS_GEMM_DBUF
#define TALOS_GEMM_DBUF 0
#endif
#ifndef TALOS_GEMM_WAVES
#define TALOS_GEMM_WAVES 4
#endif
// Split-K sizing: target workgroups per CU and the minimum K per split (512: at 32768 tokens the
// weight gradients take 64 splits instead of 128, C3 0.614-0.620 -> 0.608-0.609 ms; 768 and 1024
// starve the grid, 128 doubles the partials).
#ifndef TALOS_SPLITK_WG_PER_CU
#define TALOS_SPLITK_WG_PER_CU 2
#endif
#ifndef TALOS_SPLITK_MIN_K
#define TALOS_SPLITK_MIN_K 512
#endif
constexpr int NBUF = TALOS_GEMM_DBUF ? 2 : 1;
// Rows whose operands the 64-row norm-backward epilogue keeps in flight ahead of the row it
// finishes (normb_rows), without and with the last-row addends (8: a thread's eight rows all
// issued before the first, C3 0.587-0.592 -> 0.584-0.587 ms against 4).
#ifndef TALOS_NB_AHEAD
#define TALOS_NB_AHEAD 8
#endif
#ifndef TALOS_NB_AHEAD_LAST
#define TALOS_NB_AHEAD_LAST 1
#endif
// Whether the products with the four-term addend (E_NBPRE) take 64-row tiles at every size (1) or
// only where the 128-row tiles would leave fewer than two workgroups per CU (0).
#ifndef TALOS_NBPRE_M64
#define TALOS_NBPRE_M64 0
#endif
// Wave priority (s_setprio) of the main loop's products, 0..3 (1: C4 2.398 -> 2.388 ms).
#ifndef TALOS_GEMM_PRIO
#define TALOS_GEMM_PRIO 1
#endif

// Epilogue flags (template parameter E).
enum : int {
  E_BETA = 1,    // + beta * C
  E_BIAS = 2,    // + bias[col]
  E_RESID = 4,   // + resid[row, col]
  E_GELU = 8,    // aux = gelu'(v); v = gelu(v)   (the backward then multiplies by aux)
  E_RELU = 16,   // aux = v; v = relu(v)
  E_DGELU = 32,  // v *= aux (aux = gelu' saved by the forward's E_GELU)
  E_DRELU = 64,  // v = aux > 0 ? v : 0
  E_ROPE = 128,  // rotate interleaved pairs of columns [0, rope_cols)
  E_SPLIT = 256,  // write the fp32 partial tile of this K split (no epilogue)
  E_DBIAS = 512,  // also sum the columns of op(B) (bias gradient; transA = 1, transB = 0)
  E_NORM = 1024,  // also RMSNorm each output row (N = 128: the whole row is in the tile)
  E_NORMB = 2048,  // the output rows are dL/d(RMSNorm output): write that norm's backward instead
  E_NORMIN = 4096,  // RMSNorm A's rows first (GemmDesc::nin_*): B rows scaled by the gain, rows by rstd
  E_NBPRE = 8192,   // with E_NORMB: the addend sum_h P[row][h] U[sample][h] (four terms) before the norm backward
  E_CMAP = 16384,   // C's columns through the output column map (GemmArgs::cmap_*)
  E_NBLAST = 32768,  // with E_NORMB: the last-row addends (GemmDesc::normb_add_last / normb_dy_last) may be set
  E_ROWDOT = 65536   // also the row dots by head of C with rd_o (GemmDesc::rd_*)
};

struct GemmArgs {
  int M, N, K;
  const float* A;
  long long lda, sA;
  const float* B;
  long long ldb, sB;
  float* C;
  long long ldc, sC;
  float alpha, beta;
  const float* bias;
  const float* resid;
  long long ldr;
  float* aux;
  long long ldaux;
  const float* rcos;
  const float* rsin;
  int rope_cols, rope_dim, rope_seq;
  int cmap_w, cmap_pitch, cmap_off;  // output column map (GemmDesc::cmap_*; cmap_w 0: none)
  const float* rd_o;  // E_ROWDOT (GemmDesc::rd_*)
  long long rd_ldo;
  float* rd_D;
  int rd_w, rd_seq, rd_heads;
  int ksplit, kper;
  float* part;  // [batch][ksplit][M + (dbias ? 1 : 0)][N]
  float* dbias;
  float beta_dbias;
  const float* norm_gain;  // E_NORM: norm_out = C * rstd * gain, rstd = 1 / sqrt(mean(C^2) + eps)
  float* norm_out;
  long long ldn;
  float* norm_rstd;
  float norm_eps;
  const float* nin_gain;  // E_NORMIN
  float* nin_out;
  float* nin_rstd;
  float nin_eps;
  const float* nb_x;  // E_NORMB (GemmDesc::normb_*); nb_part [row tiles][N] f64 dgain partials
  const float* nb_rstd;
  const float* nb_gain;
  const float* nb_add;
  const float* nb_add_last;
  const float* nb_dy_last;
  const float* nb_pre_p;  // E_NBPRE: [M][4]
  const float* nb_pre_u;  // E_NBPRE: [M / nb_seq][4][N]
  int nb_seq;
  const int32_t* nb_lens;
  float* nb_dx;
  double* nb_part;
  int vecA, vecB;
  const uint16_t* A16;  // bf16 copies of A / B (bf16-in products; GemmDesc::A16 / B16)
  const uint16_t* B16;
  uint16_t* C16;        // bf16 copy of C written by the epilogue
  int vecA16, vecB16, vecC16;  // 16-byte rows of A16 / B16, 8-byte rows of C16
  int nblocks;  // tiles * batch * ksplit (the grid is padded to a multiple of 8)
};

// Loads the op(A) panel [ROWS x BK] of chunk k0 into registers (ROWS / 32 float4s a thread).
// CHECK = false: the whole panel is in bounds and 16-byte aligned.
template <bool TA, bool CHECK, int ROWS = BM>
__device__ __forceinline__ void load_a(const GemmArgs& p, const float* __restrict__ A, int m0, int k0, int kend,
                                       float4 (&r)[ROWS / 32]) {
  static_assert(ROWS == 128 || ROWS == 64, "128- or 64-row panels");
  constexpr int RS = ROWS == 128 ? 7 : 6;  // log2(ROWS)
  const int t = threadIdx.x;
  if (!TA) {
    const int m = m0 + (t & (ROWS - 1));
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      const int k = k0 + 4 * ((t >> RS) + (NT / ROWS) * i);
      const float* src = A + (long long)m * p.lda + k;
      if (!CHECK || (p.vecA && m < p.M && k + 3 < kend)) {
        r[i] = *reinterpret_cast<const float4*>(src);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (m < p.M && k + j < kend) ? src[j] : 0.f;
        r[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    const int m = m0 + 4 * (t & (ROWS / 4 - 1));
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      const int k = k0 + (t >> (RS - 2)) + (NT / (ROWS / 4)) * i;
      const float* src = A + (long long)k * p.lda + m;
      if (!CHECK || (p.vecA && k < kend && m + 3 < p.M)) {
        r[i] = *reinterpret_cast<const float4*>(src);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (k < kend && m + j < p.M) ? src[j] : 0.f;
        r[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

template <bool TA, int ROWS = BM>
__device__ __forceinline__ void store_a(float* As, const float4 (&r)[ROWS / 32]) {
  constexpr int RS = ROWS == 128 ? 7 : 6;  // log2(ROWS)
  const int t = threadIdx.x;
  if (!TA) {  // k-contiguous panel As[m][k]
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      const int kk = 4 * ((t >> RS) + (NT / ROWS) * i);
      *reinterpret_cast<float4*>(As + (t & (ROWS - 1)) * KP + kk) = r[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < ROWS / 32; ++i) {
      const int kk = (t >> (RS - 2)) + (NT / (ROWS / 4)) * i;
      *reinterpret_cast<float4*>(As + kk * LDS_S + 4 * (t & (ROWS / 4 - 1))) = r[i];
    }
  }
}

// op(B) panel [BK x BN]: transB = 0 is the same access pattern as transA = 1 and vice versa.
template <bool TB, bool CHECK>
__device__ __forceinline__ void load_b(const GemmArgs& p, const float* __restrict__ B, int n0, int k0, int kend,
                                       float4 (&r)[4]) {
  const int t = threadIdx.x;
  if (TB) {
    const int n = n0 + (t & 127);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + 4 * ((t >> 7) + 2 * i);
      const float* src = B + (long long)n * p.ldb + k;
      if (!CHECK || (p.vecB && n < p.N && k + 3 < kend)) {
        r[i] = *reinterpret_cast<const float4*>(src);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (n < p.N && k + j < kend) ? src[j] : 0.f;
        r[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  } else {
    const int n = n0 + 4 * (t & 31);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + (t >> 5) + 8 * i;
      const float* src = B + (long long)k * p.ldb + n;
      if (!CHECK || (p.vecB && k < kend && n + 3 < p.N)) {
        r[i] = *reinterpret_cast<const float4*>(src);
      } else {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (k < kend && n + j < p.N) ? src[j] : 0.f;
        r[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

template <bool TB>
__device__ __forceinline__ void store_b(float* Bs, const float4 (&r)[4]) {
  store_a<!TB, BN>(Bs, r);
}

// MFMA operand values of rows r and r + 32 of a panel at k = k0 .. k0 + 3 (k0 = 8j + 4h):
// KC = true, a k-contiguous panel X[r][k] (two 16-byte reads); KC = false, a k-major panel
// X[k][r] (one value per k).
template <bool KC>
__device__ __forceinline__ void frag4(const float* X, int r, int k0, float (&f0)[4], float (&f1)[4]) {
  if (KC) {
    const float4 v0 = *reinterpret_cast<const float4*>(X + r * KP + k0);
    const float4 v1 = *reinterpret_cast<const float4*>(X + (r + 32) * KP + k0);
    f0[0] = v0.x; f0[1] = v0.y; f0[2] = v0.z; f0[3] = v0.w;
    f1[0] = v1.x; f1[1] = v1.y; f1[2] = v1.z; f1[3] = v1.w;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f0[q] = X[(k0 + q) * LDS_S + r];
      f1[q] = X[(k0 + q) * LDS_S + r + 32];
    }
  }
}

// frag4's first row block only (row r at k = k0 .. k0 + 3)
template <bool KC>
__device__ __forceinline__ void frag1(const float* X, int r, int k0, float (&f0)[4]) {
  if (KC) {
    const float4 v0 = *reinterpret_cast<const float4*>(X + r * KP + k0);
    f0[0] = v0.x; f0[1] = v0.y; f0[2] = v0.z; f0[3] = v0.w;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) f0[q] = X[(k0 + q) * LDS_S + r];
  }
}

template <bool TA, bool TB, int ROWS = BM>
__device__ __forceinline__ void load_chunk(const GemmArgs& p, const float* A, const float* B, int m0, int n0, int k0,
                                           int kend, bool interior, float4 (&ra)[ROWS / 32], float4 (&rb)[4]) {
  if (interior && k0 + BK <= kend) {
    load_a<TA, false, ROWS>(p, A, m0, k0, kend, ra);
    load_b<TB, false>(p, B, n0, k0, kend, rb);
  } else {
    load_a<TA, true, ROWS>(p, A, m0, k0, kend, ra);
    load_b<TB, true>(p, B, n0, k0, kend, rb);
  }
}

// Epilogue of one element (everything but RoPE, which needs the neighbouring lane).
template <int E>
__device__ __forceinline__ float epi_value(const GemmArgs& p, float acc, int row, int col, const float* C,
                                           const float* __restrict__ resid) {
  float v = p.alpha * acc;
  if constexpr ((E & E_BETA) != 0) v += p.beta * C[(long long)row * p.ldc + col];
  if constexpr ((E & E_BIAS) != 0) v += p.bias[col];
  if constexpr ((E & E_RESID) != 0) v += resid[(long long)row * p.ldr + col];
  if constexpr ((E & E_DGELU) != 0) v *= p.aux[(long long)row * p.ldaux + col];
  if constexpr ((E & E_DRELU) != 0) v = p.aux[(long long)row * p.ldaux + col] > 0.f ? v : 0.f;
  if constexpr ((E & E_GELU) != 0) {
    float dv;
    v = gelu_fd(v, &dv);
    if (p.aux) p.aux[(long long)row * p.ldaux + col] = dv;
  }
  if constexpr ((E & E_RELU) != 0) {
    if (p.aux) p.aux[(long long)row * p.ldaux + col] = v;
    v = fmaxf(v, 0.f);
  }
  return v;
}

// Index into the [rope_seq, rope_dim / 2] cos / sin table of the interleaved pair that starts at
// column c (even) of row `row`: position row % rope_seq, pair (c % rope_dim) / 2 of its head. Each
// pair is indexed on its own, so a head whose width is not a multiple of 4 (its pairs straddle the
// float4 groups) takes its own pairs, never the next head's. -1 for columns past rope_cols.
__device__ __forceinline__ int rope_index(const GemmArgs& p, int row, int c) {
  if (c >= p.rope_cols) return -1;
  return (row % p.rope_seq) * (p.rope_dim >> 1) + ((c % p.rope_dim) >> 1);
}

// Epilogue of four consecutive columns [col, col + 4) of one row, read from / written to global
// memory as float4 (interior) or per element (edges). RoPE pairs (2i, 2i+1) sit in (x, y) and
// (z, w) because col is a multiple of 4.
// Operands of one row's epilogue loaded by the caller ahead of the stores of earlier rows (C
// may alias them as far as the compiler knows, so a load after a store would wait for it): the
// aux piece the backward's multiply reads (E_DGELU / E_DRELU), the RoPE cos / sin pairs, the bias.
struct EpiPre {
  float4 aux, rope, bias;
};
template <int E>
__device__ __forceinline__ EpiPre epi_preload(const GemmArgs& p, int row, int col, bool full, float4 bias) {
  EpiPre q;
  q.bias = bias;
  q.aux = make_float4(0.f, 0.f, 0.f, 0.f);
  q.rope = make_float4(1.f, 1.f, 0.f, 0.f);
  if constexpr ((E & (E_DGELU | E_DRELU)) != 0)
    if (full) q.aux = *reinterpret_cast<const float4*>(p.aux + (long long)row * p.ldaux + col);
  if constexpr ((E & E_ROPE) != 0) {
    if (row < p.M && col < p.rope_cols) {
      const int i0 = rope_index(p, row, col), i1 = rope_index(p, row, col + 2);
      q.rope = make_float4(p.rcos[i0], i1 >= 0 ? p.rcos[i1] : 1.f, p.rsin[i0], i1 >= 0 ? p.rsin[i1] : 0.f);
    }
  }
  return q;
}
// C's column of product column c (E_CMAP: GemmArgs::cmap_*)
template <int E>
__device__ __forceinline__ int out_col(const GemmArgs& p, int c) {
  if constexpr ((E & E_CMAP) != 0) return (c / p.cmap_w) * p.cmap_pitch + p.cmap_off + c % p.cmap_w;
  return c;
}

template <int E, bool PRE = false>
__device__ __forceinline__ float4 epi_store4(const GemmArgs& p, float4 v, int row, int col, float* C,
                                             const float* __restrict__ resid, bool full, const EpiPre& pre = EpiPre{}) {
  float o[4] = {v.x * p.alpha, v.y * p.alpha, v.z * p.alpha, v.w * p.alpha};
  if constexpr ((E & E_ROPE) != 0) {
    if (col < p.rope_cols && row < p.M) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // the table entry of pair (col + 2j, col + 2j + 1); -1 (identity) past the rotated columns
        const int ij = PRE ? 0 : rope_index(p, row, col + 2 * j);
        const float c = PRE ? (j ? pre.rope.y : pre.rope.x) : (ij >= 0 ? p.rcos[ij] : 1.f);
        const float s = PRE ? (j ? pre.rope.w : pre.rope.z) : (ij >= 0 ? p.rsin[ij] : 0.f);
        const float x0 = o[2 * j], x1 = o[2 * j + 1];
        o[2 * j] = fmaf(x0, c, -x1 * s);
        o[2 * j + 1] = fmaf(x0, s, x1 * c);
      }
    }
  }
  const long long crow = (long long)row * p.ldc;
  const int ccol = out_col<E>(p, col);  // (a group of 4 never straddles a mapped block: cmap_w % 4 == 0)
  if (full) {
    if constexpr ((E & E_BETA) != 0) {
      const float4 c = *reinterpret_cast<const float4*>(C + crow + ccol);
      o[0] += p.beta * c.x; o[1] += p.beta * c.y; o[2] += p.beta * c.z; o[3] += p.beta * c.w;
    }
    if constexpr ((E & E_BIAS) != 0) {
      const float4 bv = PRE ? pre.bias : *reinterpret_cast<const float4*>(p.bias + col);
      o[0] += bv.x; o[1] += bv.y; o[2] += bv.z; o[3] += bv.w;
    }
    if constexpr ((E & E_RESID) != 0) {
      const float4 r = *reinterpret_cast<const float4*>(resid + (long long)row * p.ldr + col);
      o[0] += r.x; o[1] += r.y; o[2] += r.z; o[3] += r.w;
    }
    if constexpr ((E & (E_DGELU | E_DRELU)) != 0) {
      const float4 u = PRE ? pre.aux : *reinterpret_cast<const float4*>(p.aux + (long long)row * p.ldaux + col);
      const float uu[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr ((E & E_DGELU) != 0) o[j] *= uu[j];
        else o[j] = uu[j] > 0.f ? o[j] : 0.f;
      }
    }
    if constexpr ((E & E_GELU) != 0) {
      float dv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = gelu_fd(o[j], &dv[j]);
      if (p.aux) *reinterpret_cast<float4*>(p.aux + (long long)row * p.ldaux + col) = make_float4(dv[0], dv[1], dv[2], dv[3]);
    }
    if constexpr ((E & E_RELU) != 0) {
      if (p.aux) *reinterpret_cast<float4*>(p.aux + (long long)row * p.ldaux + col) = make_float4(o[0], o[1], o[2], o[3]);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = fmaxf(o[j], 0.f);
    }
    *reinterpret_cast<float4*>(C + crow + ccol) = make_float4(o[0], o[1], o[2], o[3]);
    return make_float4(o[0], o[1], o[2], o[3]);
  }
  if (row >= p.M) return make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int cj = col + j;
    if (cj >= p.N) break;
    float x = o[j];
    const int oc = out_col<E>(p, cj);
    if constexpr ((E & E_BETA) != 0) x += p.beta * C[crow + oc];
    if constexpr ((E & E_BIAS) != 0) x += p.bias[cj];
    if constexpr ((E & E_RESID) != 0) x += resid[(long long)row * p.ldr + cj];
    if constexpr ((E & E_DGELU) != 0) x *= p.aux[(long long)row * p.ldaux + cj];
    if constexpr ((E & E_DRELU) != 0) x = p.aux[(long long)row * p.ldaux + cj] > 0.f ? x : 0.f;
    if constexpr ((E & E_GELU) != 0) {
      float dx;
      x = gelu_fd(x, &dx);
      if (p.aux) p.aux[(long long)row * p.ldaux + cj] = dx;
    }
    if constexpr ((E & E_RELU) != 0) {
      if (p.aux) p.aux[(long long)row * p.ldaux + cj] = x;
      x = fmaxf(x, 0.f);
    }
    C[crow + oc] = x;
    o[j] = x;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (col + j >= p.N) o[j] = 0.f;  // columns past N take no part in a row norm
  return make_float4(o[0], o[1], o[2], o[3]);
}

// RMSNorm of the rows of a 128-wide tile from the epilogue's float4s: the 32 lanes of one
// half-wave hold one row (column groups 4 * (lane % 32)), so the row sum of squares is a
// shuffle reduction over that half-wave. Same arithmetic as rmsnorm_fwd_kernel.
// g: the gain piece of columns col..col+3 when they are all inside N, loaded by the caller once
// (a load here would follow the previous rows' stores and wait for them)
__device__ __forceinline__ void epi_norm4(const GemmArgs& p, float4 o, int row, int col, float4 g) {
  float ss = o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  const float r = 1.0f / sqrtf(ss / (float)p.N + p.norm_eps);
  if (row >= p.M) return;
  if ((threadIdx.x & 31) == 0 && p.norm_rstd) p.norm_rstd[row] = r;
  float* y = p.norm_out + (long long)row * p.ldn + col;
  if (col + 3 < p.N) {
    *reinterpret_cast<float4*>(y) = make_float4(o.x * r * g.x, o.y * r * g.y, o.z * r * g.z, o.w * r * g.w);
  } else {
    const float oo[4] = {o.x, o.y, o.z, o.w};
    for (int j = 0; j < 4 && col + j < p.N; ++j) y[j] = oo[j] * r * p.norm_gain[col + j];
  }
}

// RMSNorm backward of one row of a 128-wide tile from the epilogue's float4 gg = dL/dy (y the
// norm's output; the 32 lanes of a half-wave hold one row): dx = rstd * (gg * gain - x_hat * md)
// + the addends, md = mean(gg * gain * x_hat), x_hat = x * rstd; the lane's dgain terms gg * x_hat
// are added to dw (column group col). Same arithmetic as rmsnorm_bwd_kernel. Every lane of the
// half-wave takes part in the shuffle; rows past M contribute zeros. The row's x and rstd are
// loaded by normb_load one row ahead (normb_apply uses them), so the epilogue's loads overlap the
// previous row's work instead of each row waiting on memory.
struct NbIn {
  float4 x;
  float r;
};
__device__ __forceinline__ NbIn normb_load(const GemmArgs& p, int row, int col) {
  NbIn in;
  const bool on = row < p.M;
  in.r = on ? p.nb_rstd[row] : 0.f;
  in.x = on ? *reinterpret_cast<const float4*>(p.nb_x + (long long)row * p.N + col) : make_float4(0.f, 0.f, 0.f, 0.f);
  return in;
}
// Every operand of one row of the pipelined norm-backward epilogue (64-row tiles, E_NORMB without E_NBPRE),
// loaded kNbAhead rows ahead of its use with no branch around a load: the last-row addends are
// read for every row (a clamped, valid row) and kept only for the sample's last row, so the
// compiler can wait for exactly the loads a row needs instead of all of them.
struct NbRow {
  float4 x, add, dyl, addl;
  float r;
  bool last;
};
// q, rem: the row's sample and its index in the sample (row = q * seq + rem); LAST: the product
// may have last-row addends (E_NBLAST)
template <bool LAST>
__device__ __forceinline__ NbRow normb_row_load(const GemmArgs& p, int row, int q, int rem, int col) {
  NbRow in;
  const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
  const bool on = row < p.M;
  const int rr = on ? row : 0;
  in.r = on ? p.nb_rstd[rr] : 0.f;
  in.x = *reinterpret_cast<const float4*>(p.nb_x + (long long)rr * p.N + col);
  // the addend row is read from x's row when there is none and then zeroed: a load whose
  // pointer may be null would be compiled as a flat load from a zeroed stack slot instead
  const float4 add = *reinterpret_cast<const float4*>((p.nb_add ? p.nb_add : p.nb_x) + (long long)rr * p.N + col);
  in.add = p.nb_add ? add : z;
  if (!on) in.x = in.add = z;
  in.dyl = in.addl = z;
  in.last = false;
  if (LAST && (p.nb_add_last || p.nb_dy_last)) {  // uniform
    const int qq = on ? q : 0;
    int lr = p.nb_seq - 1;
    if (p.nb_lens) {
      const int L = p.nb_lens[qq];
      lr = (L < 1 ? 1 : (L > p.nb_seq ? p.nb_seq : L)) - 1;
    }
    in.last = on && rem == lr;
    // (absent rows read from x's first rows, [samples][N] fits inside x's [M][N], then zeroed)
    const float4 dy4 = *reinterpret_cast<const float4*>((p.nb_dy_last ? p.nb_dy_last : p.nb_x) + (long long)qq * p.N + col);
    const float4 ad4 = *reinterpret_cast<const float4*>((p.nb_add_last ? p.nb_add_last : p.nb_x) + (long long)qq * p.N + col);
    const float4 dyl = p.nb_dy_last ? dy4 : z;
    const float4 addl = p.nb_add_last ? ad4 : z;
    if (in.last) {
      in.dyl = dyl;
      in.addl = addl;
    }
  }
  return in;
}
// The row's norm backward from its preloaded operands (normb_apply's arithmetic).
__device__ __forceinline__ void normb_row_apply(const GemmArgs& p, float4 gg, int row, int col, const NbRow& in,
                                                const float4& g, float4& dw) {
  const bool on = row < p.M;
  gg.x += in.dyl.x;
  gg.y += in.dyl.y;
  gg.z += in.dyl.z;
  gg.w += in.dyl.w;
  if (!on) gg = make_float4(0.f, 0.f, 0.f, 0.f);
  const float r = in.r;
  const float4 xh = make_float4(in.x.x * r, in.x.y * r, in.x.z * r, in.x.w * r);
  float dot = gg.x * g.x * xh.x + gg.y * g.y * xh.y + gg.z * g.z * xh.z + gg.w * g.w * xh.w;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
  const float md = dot * (1.0f / (float)p.N);
  dw.x += gg.x * xh.x;
  dw.y += gg.y * xh.y;
  dw.z += gg.z * xh.z;
  dw.w += gg.w * xh.w;
  if (!on) return;
  float4 o = make_float4(r * (gg.x * g.x - xh.x * md), r * (gg.y * g.y - xh.y * md), r * (gg.z * g.z - xh.z * md),
                         r * (gg.w * g.w - xh.w * md));
  o.x += in.add.x + in.addl.x;
  o.y += in.add.y + in.addl.y;
  o.z += in.add.z + in.addl.z;
  o.w += in.add.w + in.addl.w;
  *reinterpret_cast<float4*>(p.nb_dx + (long long)row * p.N + col) = o;
}

template <bool PRE>
__device__ __forceinline__ void normb_apply(const GemmArgs& p, float4 gg, int row, int col, const NbIn& in,
                                            const float4& g, float4& dw) {
  const bool on = row < p.M;
  if constexpr (PRE) {  // the addend sum_h P[row][h] U[sample][h] (E_NBPRE), before anything else
    if (on) {
      const float4 w = *reinterpret_cast<const float4*>(p.nb_pre_p + (long long)row * 4);
      const float* u = p.nb_pre_u + (long long)(row / p.nb_seq) * 4 * p.N + col;
      const float wh[4] = {w.x, w.y, w.z, w.w};
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float4 uh = *reinterpret_cast<const float4*>(u + t * p.N);
        a = make_float4(fmaf(wh[t], uh.x, a.x), fmaf(wh[t], uh.y, a.y), fmaf(wh[t], uh.z, a.z), fmaf(wh[t], uh.w, a.w));
      }
      gg.x += a.x;
      gg.y += a.y;
      gg.z += a.z;
      gg.w += a.w;
    }
  }
  // the addend row, issued first: its latency runs under the row reduction below
  const float4 add = on && p.nb_add ? *reinterpret_cast<const float4*>(p.nb_add + (long long)row * p.N + col)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
  const bool last = (p.nb_add_last || p.nb_dy_last) && on &&
                    row % p.nb_seq == last_row(p.nb_lens, row / p.nb_seq, p.nb_seq);
  if (last && p.nb_dy_last) {
    const float4 a = *reinterpret_cast<const float4*>(p.nb_dy_last + (long long)(row / p.nb_seq) * p.N + col);
    gg.x += a.x;
    gg.y += a.y;
    gg.z += a.z;
    gg.w += a.w;
  }
  if (!on) gg = make_float4(0.f, 0.f, 0.f, 0.f);
  const float r = in.r;
  const float4 xh = make_float4(in.x.x * r, in.x.y * r, in.x.z * r, in.x.w * r);
  float dot = gg.x * g.x * xh.x + gg.y * g.y * xh.y + gg.z * g.z * xh.z + gg.w * g.w * xh.w;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) dot += __shfl_xor(dot, off, 64);
  const float md = dot * (1.0f / (float)p.N);
  dw.x += gg.x * xh.x;
  dw.y += gg.y * xh.y;
  dw.z += gg.z * xh.z;
  dw.w += gg.w * xh.w;
  if (!on) return;
  float4 o = make_float4(r * (gg.x * g.x - xh.x * md), r * (gg.y * g.y - xh.y * md), r * (gg.z * g.z - xh.z * md),
                         r * (gg.w * g.w - xh.w * md));
  o.x += add.x;
  o.y += add.y;
  o.z += add.z;
  o.w += add.w;
  if (last && p.nb_add_last) {
    const float4 a = *reinterpret_cast<const float4*>(p.nb_add_last + (long long)(row / p.nb_seq) * p.N + col);
    o.x += a.x;
    o.y += a.y;
    o.z += a.z;
    o.w += a.w;
  }
  *reinterpret_cast<float4*>(p.nb_dx + (long long)row * p.N + col) = o;
}

constexpr int T_S = 136;  // pitch of the staged output tile: rows h*4 apart land 32 banks apart
constexpr int T_ROWS = 64;  // the tile is staged 64 rows at a time
constexpr int SMEM_FLOATS = (2 * NBUF * PANEL > T_ROWS * T_S) ? 2 * NBUF * PANEL : T_ROWS * T_S;

// ---------------------------------------------------------------------------
// bf16-in / fp32-accumulate operand staging: panels of BKB = 64 k values are rounded to bf16 and
// stored k-contiguous (rows of PB bf16, 144 bytes: the 16-byte fragments of 8 consecutive rows
// fall on distinct banks), so one ds_read_b128 gives a lane the 8 k values of an MFMA step.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int BKB = 64;
constexpr int PB = BKB + 8;
// the bf16 main loop's LDS: two stages of the A and B panels (BM + BN rows of PB bf16), 73.7 KB
constexpr int SMEM_BF = 2 * (BM + BN) * PB / 2;

// round-to-nearest-even fp32 -> bf16 of two values, packed low | high: gfx950's
// v_cvt_pk_bf16_f32, one instruction a pair (an integer rounding sequence of about six
// instructions a pair made the staging, not the products, bound the bf16-in main loop)
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const floatx2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Loads the [rows r0.., k0..k0+64) panel of an operand X and packs it to bf16 pairs.
// KC = true: X[r][k] with k contiguous; thread t takes k = 4*(t%16) of rows t/16 + 16i.
// KC = false: X[k][r] with r contiguous; thread t takes r = 4*(t%32) .. + 3 and k = 8*(t/32) .. + 7
// (eight float4 rows), packed to four rows of eight k values.
template <bool KC>
__device__ __forceinline__ void load_bf(const float* __restrict__ X, long long ld, int r0, int rlim, int k0, int kend,
                                        bool fast, bool vec, uint32_t (&o)[16]) {
  const int t = threadIdx.x;
  if (KC) {
    const int k = k0 + 4 * (t & 15);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = r0 + (t >> 4) + 16 * i;
      const float* src = X + (long long)r * ld + k;
      float v[4];
      if (fast || (vec && r < rlim && k + 3 < kend)) {
        const float4 f = *reinterpret_cast<const float4*>(src);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (r < rlim && k + j < kend) ? src[j] : 0.f;
      }
      o[2 * i] = pack_bf16(v[0], v[1]);
      o[2 * i + 1] = pack_bf16(v[2], v[3]);
    }
  } else {
    const int r = r0 + 4 * (t & 31), kb = k0 + 8 * (t >> 5);
    float v[8][4];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int k = kb + u;
      const float* src = X + (long long)k * ld + r;
      if (fast || (vec && k < kend && r + 3 < rlim)) {
        const float4 f = *reinterpret_cast<const float4*>(src);
        v[u][0] = f.x; v[u][1] = f.y; v[u][2] = f.z; v[u][3] = f.w;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v[u][j] = (k < kend && r + j < rlim) ? src[j] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)  // row r + j: k pairs (kb + 2u, kb + 2u + 1)
#pragma unroll
      for (int u = 0; u < 4; ++u) o[4 * j + u] = pack_bf16(v[2 * u][j], v[2 * u + 1][j]);
  }
}

// A panel read from a bf16 copy of the operand (already rounded), in 16-byte loads of 8 bf16 (a
// panel is 4 loads a thread, half the load instructions of load_bf's float4 reads or of 8-byte
// reads, which is what bounds the bf16 main loop: the per-instruction cost of the texture
// address and data path, not bytes or latency). Layout of o[16] (store_bf16src):
//  KC = true  (rows r k-contiguous): o[4i .. 4i + 3] = row (t >> 3) + 32 i, k 8 (t & 7) .. + 7.
//  KC = false (k rows, r contiguous): thread (cg = t & 15, q = t >> 4) loads k rows 4q .. 4q + 3
//    of columns 8 cg .. 8 cg + 7; o[2c], o[2c + 1] = column 8 cg + c, k 4q .. 4q + 3 (pairs).
template <bool KC>
__device__ __forceinline__ void load_bf16src(const uint16_t* __restrict__ X, long long ld, int r0, int rlim, int k0,
                                             int kend, bool fast, bool vec, uint32_t (&o)[16]) {
  const int t = threadIdx.x;
  auto piece = [&](const uint16_t* src, bool full, int valid) {  // 8 values, zero past valid
    if (full) return *reinterpret_cast<const uint4*>(src);
    uint32_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = j < valid ? src[j] : 0u;
    return make_uint4(v[0] | (v[1] << 16), v[2] | (v[3] << 16), v[4] | (v[5] << 16), v[6] | (v[7] << 16));
  };
  if (KC) {
    const int k = k0 + 8 * (t & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + (t >> 3) + 32 * i;
      const int valid = r < rlim ? min(8, kend - k) : 0;
      const uint4 w = piece(X + (long long)r * ld + k, fast || (vec && valid == 8), valid);
      o[4 * i] = w.x;
      o[4 * i + 1] = w.y;
      o[4 * i + 2] = w.z;
      o[4 * i + 3] = w.w;
    }
  } else {
    const int r = r0 + 8 * (t & 15), kq = k0 + 4 * (t >> 4);
    uint4 w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = kq + j;
      const int valid = k < kend ? min(8, rlim - r) : 0;
      w[j] = piece(X + (long long)k * ld + r, fast || (vec && valid == 8), valid);
    }
    auto pack = [&](int u, uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3) {  // columns 2u, 2u + 1
      o[4 * u] = (x0 & 0xffffu) | (x1 << 16);
      o[4 * u + 1] = (x2 & 0xffffu) | (x3 << 16);
      o[4 * u + 2] = (x0 >> 16) | (x1 & 0xffff0000u);
      o[4 * u + 3] = (x2 >> 16) | (x3 & 0xffff0000u);
    };
    pack(0, w[0].x, w[1].x, w[2].x, w[3].x);
    pack(1, w[0].y, w[1].y, w[2].y, w[3].y);
    pack(2, w[0].z, w[1].z, w[2].z, w[3].z);
    pack(3, w[0].w, w[1].w, w[2].w, w[3].w);
  }
}

// Stores load_bf16src's o[16] into a k-contiguous panel (rows of PB bf16).
template <bool KC>
__device__ __forceinline__ void store_bf16src(uint16_t* S, const uint32_t (&o)[16]) {
  const int t = threadIdx.x;
  if (KC) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = (t >> 3) + 32 * i;
      *reinterpret_cast<uint4*>(S + r * PB + 8 * (t & 7)) = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
    }
  } else {
    // eight 8-byte pieces, rows 8 cg + c. Rows 8 apart are 8 * 36 = 32 mod 64 banks apart, so in
    // one store the 16 lanes of a row group would share two bank pairs; lane cg writes its columns
    // in the rotated order c = (i + cg) & 7 instead (rotation by three conditional shifts), which
    // leaves at most two lanes on a bank pair.
    const int cg = t & 15, kq = 4 * (t >> 4);
    uint2 g[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) g[c] = make_uint2(o[2 * c], o[2 * c + 1]);
#pragma unroll
    for (int sh = 1; sh < 8; sh *= 2) {
      if (cg & sh) {
        uint2 h[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) h[c] = g[(c + sh) & 7];
#pragma unroll
        for (int c = 0; c < 8; ++c) g[c] = h[c];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * cg + ((i + cg) & 7);
      *reinterpret_cast<uint2*>(S + r * PB + kq) = g[i];
    }
  }
}

template <bool KC>
__device__ __forceinline__ void store_bf(uint16_t* S, const uint32_t (&o)[16]) {
  const int t = threadIdx.x;
  if (KC) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = (t >> 4) + 16 * i;
      *reinterpret_cast<uint2*>(S + r * PB + 4 * (t & 15)) = make_uint2(o[2 * i], o[2 * i + 1]);
    }
  } else {
    // four 16-byte row pieces, rows 4 (t & 31) + j. Rows 4 apart are 4 * 36 = 16 mod 64 banks
    // apart, so in one store lanes 4 apart would meet on the same banks (4-way conflict); lane
    // group q = (t >> 2) & 3 writes its pieces in the rotated order j = (i + q) & 3 instead, which
    // moves those lanes 36 banks further per step and spreads 16 lanes over 16 distinct bank
    // groups. The rotation is two conditional swaps of whole pieces.
    const int q = (t >> 2) & 3;
    uint4 g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
    if (q & 1) {
      const uint4 g0 = g[0];
      g[0] = g[1];
      g[1] = g[2];
      g[2] = g[3];
      g[3] = g0;
    }
    if (q & 2) {
      const uint4 g0 = g[0], g1 = g[1];
      g[0] = g[2];
      g[1] = g[3];
      g[2] = g0;
      g[3] = g1;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * (t & 31) + ((i + q) & 3), k = 8 * (t >> 5);
      *reinterpret_cast<uint4*>(S + r * PB + k) = g[i];
    }
  }
}

// The XCD-aware order: the dispatcher sends workgroup i to XCD i % 8, so logical tiles are dealt
// out in contiguous runs per XCD; the N tiles of one M panel (and the tiles of one K split)
// then share that XCD's L2 instead of fetching the same operand panel once per XCD. The grid is
// padded to a multiple of 8; padding workgroups exit before any barrier.
__device__ __forceinline__ int xcd_logical() {
  const int per_xcd = (int)(gridDim.x >> 3);
  return (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
}

// One output tile of BMT (128 or 64) x 128 rows / columns for logical workgroup `logical` (in
// [0, p.nblocks)): four waves, wave (wm, wn) the [BMT / 2, 64] block at rows wm BMT / 2,
// columns 64 wn, as 2 x 2 (BMT = 128) or 1 x 2 (BMT = 64) 32 x 32 accumulators.
// The accumulators of the waves staging a 64-row half into the tile T (row pitch T_S): 128-row
// tiles (MT = 2) pass the half's waves' two 32-row blocks, 64-row tiles (MT = 1) every wave's one
// (accumulator layout of v_mfma_f32_32x32x2_f32: lane l, register r holds row
// 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32 of its 32 x 32 block).
template <int MT>
__device__ __forceinline__ void stage_acc(float* T, const floatx16 (&acc)[MT][2], int wm, int wn, int h, int l32,
                                          int) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = (MT == 1 ? wm * 32 : mt * 32) + 8 * (r >> 2) + 4 * h + (r & 3);
        const int c = wn * 64 + nt * 32 + l32;
        T[row * T_S + c] = acc[mt][nt][r];
      }
}

// The norm backward of the 64 staged rows of T (row pitch T_S; tile rows r0 - (t / 32) + 0..63):
// thread t takes column group cg of rows r0 + 8 i, i < 8, with the operands of AHEAD rows in
// flight ahead of the row it finishes; the row's sample q and its index rem in the sample are kept
// incrementally (no division per row).
// E_NBPRE on 64-row tiles: the four-term addend sum_h P[row][h] U[row / seq][h] added to the
// thread's own staged rows of T (the rows and columns normb_rows then reads), four rows' P and U
// loads in flight at once; normb_apply adds it to the product in the same order.
__device__ __forceinline__ void normb_pre_rows(const GemmArgs& p, float* T, int cg, int col, int r0) {
  constexpr int RT = T_ROWS / 8;
#pragma unroll
  for (int i0 = 0; i0 < RT; i0 += 4) {
    float4 w[4], u[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = r0 + 8 * (i0 + j);
      const int rr = row < p.M ? row : 0;
      w[j] = *reinterpret_cast<const float4*>(p.nb_pre_p + (long long)rr * 4);
      const float* ur = p.nb_pre_u + (long long)(rr / p.nb_seq) * 4 * p.N + col;
#pragma unroll
      for (int t = 0; t < 4; ++t) u[j][t] = *reinterpret_cast<const float4*>(ur + t * p.N);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (r0 + 8 * (i0 + j) >= p.M) continue;
      const float wh[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int t = 0; t < 4; ++t)
        a = make_float4(fmaf(wh[t], u[j][t].x, a.x), fmaf(wh[t], u[j][t].y, a.y), fmaf(wh[t], u[j][t].z, a.z),
                        fmaf(wh[t], u[j][t].w, a.w));
      float4* tp = reinterpret_cast<float4*>(T + ((threadIdx.x >> 5) + 8 * (i0 + j)) * T_S + cg);
      const float4 v = *tp;
      *tp = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
    }
  }
}

template <int AHEAD, bool LAST>
__device__ __forceinline__ void normb_rows(const GemmArgs& p, const float* T, int cg, int col, int r0,
                                           const float4& g, float4& nbw) {
  constexpr int RT = T_ROWS / 8;
  int lq = r0 / p.nb_seq, lrem = r0 - lq * p.nb_seq;  // of the next row to load
  auto load_next = [&](int i) {
    const NbRow in = normb_row_load<LAST>(p, r0 + 8 * i, lq, lrem, col);
    lrem += 8;
    while (lrem >= p.nb_seq) {
      lrem -= p.nb_seq;
      ++lq;
    }
    return in;
  };
  NbRow in[RT];
#pragma unroll
  for (int i = 0; i < AHEAD; ++i) in[i] = load_next(i);
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    if (i + AHEAD < RT) in[i + AHEAD] = load_next(i + AHEAD);
    const float4 v = *reinterpret_cast<const float4*>(T + ((threadIdx.x >> 5) + 8 * i) * T_S + cg);
    normb_row_apply(p, v, r0 + 8 * i, col, in[i], g, nbw);
  }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS panels (TALOS_GEMM_DLDS; NT products, whose two operands are both k-contiguous,
// on 128-row tiles: C4 2.361-2.370 -> 2.339 ms; the NN products, whose B panel is k-major, lost
// more than the NT ones gained, 235 -> 242 and 205 -> 219 us at C4): interior tiles stream their panels straight from global memory into LDS with
// global_load_lds_dwordx4 (no register staging, no LDS store instructions), DK = 16 k a chunk in
// two LDS stages. A wave's load writes 1 KB of consecutive LDS (16 bytes a lane), so the panels
// X[r][k] (16 floats a row, 16 rows a 1 KB block) are unpadded and their 16-byte pieces permuted
// instead, by choosing which global piece each lane fetches: piece p of row r sits in slot
// p ^ ((r >> 2) & 3), so the 16 rows one fragment read spans fall on 16 distinct bank groups.
// ---------------------------------------------------------------------------
#ifndef TALOS_GEMM_DLDS
#define TALOS_GEMM_DLDS 1
#endif
constexpr int DK = 16;
// The ROWS-row panel of X (k-contiguous rows of pitch ld) at rows r0.., k0.. into S: block b
// (rows 16 b .. 16 b + 15) by wave b % 4
template <int ROWS>
__device__ __forceinline__ void dl_panel(const float* __restrict__ X, long long ld, int r0, int k0, float* S) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int blk = w; blk < ROWS / 16; blk += 4) {
    const int row = 16 * blk + (lane >> 2), piece = (lane & 3) ^ ((row >> 2) & 3);
    __builtin_amdgcn_global_load_lds(X + (long long)(r0 + row) * ld + k0 + 4 * piece, S + 256 * blk, 16, 0, 0);
  }
}
// row r's (and, TWO, row r + 32's) values at k = k0 .. k0 + 3 of a direct-load panel
template <bool TWO>
__device__ __forceinline__ void dl_frag(const float* X, int r, int k0, float (&f0)[4], float (&f1)[4]) {
  const int o = 4 * ((k0 >> 2) ^ ((r >> 2) & 3));  // rows r and r + 32 share the permutation
  const float4 v0 = *reinterpret_cast<const float4*>(X + r * DK + o);
  f0[0] = v0.x; f0[1] = v0.y; f0[2] = v0.z; f0[3] = v0.w;
  if (TWO) {
    const float4 v1 = *reinterpret_cast<const float4*>(X + (r + 32) * DK + o);
    f1[0] = v1.x; f1[1] = v1.y; f1[2] = v1.z; f1[3] = v1.w;
  }
}

// The bf16 copies' k-contiguous 128-row panels (rows of BKB = 64 bf16, 128 bytes: eight rows a
// 1 KB block) straight into LDS; piece p (8 values) of row r sits in slot p ^ ((r >> 1) & 7), so
// a fragment read's 16 rows (8 even rows on one half of the banks, 8 odd on the other) fall on
// distinct 16-byte bank groups.
__device__ __forceinline__ void dl_panel_bf16(const uint16_t* __restrict__ X, long long ld, int r0, int k0,
                                              uint16_t* S) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int blk = w; blk < 16; blk += 4) {
    const int row = 8 * blk + (lane >> 3), piece = (lane & 7) ^ ((row >> 1) & 7);
    __builtin_amdgcn_global_load_lds(X + (long long)(r0 + row) * ld + k0 + 8 * piece, S + 512 * blk, 16, 0, 0);
  }
}
// row r's 8 values of piece pc (k = 8 pc .. 8 pc + 7) of a dl_panel_bf16 panel
__device__ __forceinline__ bf16x8 dl_frag_bf16(const uint16_t* S, int r, int pc) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(S + r * BKB + 8 * (pc ^ ((r >> 1) & 7))));
}

// The bf16 copies' k-major panels (X[k][c], c contiguous: BKB = 64 k rows of 128 columns, 256
// bytes a row, four rows a 1 KB block) straight into LDS; piece p (columns 8 p ..) of k row r sits
// in slot p ^ 4 (r mod 4), so the transposing fragment reads below (four consecutive k rows, four
// consecutive pieces, per half-wave) fall on 16 distinct 16-byte bank groups.
__device__ __forceinline__ void dl_panel_kmaj(const uint16_t* __restrict__ X, long long ld, int k0, int c0,
                                              uint16_t* S) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int blk = w; blk < 16; blk += 4) {
    const int row = 4 * blk + (lane >> 4), piece = (lane & 15) ^ (4 * (lane >> 4));
    __builtin_amdgcn_global_load_lds(X + (long long)(k0 + row) * ld + c0 + 8 * piece, S + 512 * blk, 16, 0, 0);
  }
}
// The four-stage form of the direct path takes 32-k chunks: k-contiguous panels with rows of
// DKB = 32 bf16 (64 bytes, sixteen rows a 1 KB block), piece p of row r in slot p ^ ((r / 4) mod
// 4), so a fragment read's 16 rows fall on distinct 16-byte bank groups; k-major panels as above
// with 32 k rows.
#ifndef TALOS_GEMM_BF_STAGES
#define TALOS_GEMM_BF_STAGES 4
#endif
constexpr int DKB = 32;
// One 16-byte piece a lane into LDS at lds + 16 lane (lds wave-uniform): global_load_lds_dwordx4
// issued from inline assembly. The compiler then does not track these LDS writes, so it puts no
// vmcnt(0) before later LDS reads (it does for the builtin, which drains every chunk in flight at
// each chunk); the caller waits for them itself (TALOS_WAIT_VM) before the barrier that publishes
// them. M0 holds the LDS address (the compiler sets M0 anew before each of its own uses).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16_untracked(const void* src, const void* lds) {
  const uint32_t off =
      __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(off), "v"(src) : "memory", "m0");
}
#pragma clang diagnostic pop
__device__ __forceinline__ void dl_panel_bf16_32(const uint16_t* __restrict__ X, long long ld, int r0, int k0,
                                                 uint16_t* S) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int blk = w; blk < 8; blk += 4) {
    const int row = 16 * blk + (lane >> 2), piece = (lane & 3) ^ ((row >> 2) & 3);
    dma16_untracked(X + (long long)(r0 + row) * ld + k0 + 8 * piece, S + 512 * blk);
  }
}
// dl_panel_kmaj for 32-k chunks, untracked as above
__device__ __forceinline__ void dl_panel_kmaj_32(const uint16_t* __restrict__ X, long long ld, int k0, int c0,
                                                 uint16_t* S) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int blk = w; blk < DKB / 4; blk += 4) {
    const int row = 4 * blk + (lane >> 4), piece = (lane & 15) ^ (4 * (lane >> 4));
    dma16_untracked(X + (long long)(k0 + row) * ld + c0 + 8 * piece, S + 512 * blk);
  }
}
__device__ __forceinline__ bf16x8 dl_frag_bf16_32(const uint16_t* S, int r, int pc) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(S + r * DKB + 8 * (pc ^ ((r >> 2) & 3))));
}
// s_waitcnt with vmcnt = n and the other counters left alone (gfx9 encoding: vmcnt bits 3:0,
// expcnt 6:4, lgkmcnt 11:8)
#define TALOS_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x0F70 | (n))
// A workgroup barrier that orders LDS accesses only: __syncthreads() also waits for every
// outstanding global load (vmcnt 0), which would drain the later chunks' direct loads at each
// barrier; their completion is waited for explicitly with TALOS_WAIT_VM instead.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The MFMA fragment of product s (k = 16 s + 8 h + 0..7, the slots of dl_frag_bf16's piece
// 2 s + h) for column cb + l32 (cb a multiple of 32) of a dl_panel_kmaj panel, by two
// ds_read_b64_tr_b16. That instruction works on groups of 16 lanes: lane 4a + j of a group gives
// the address of four consecutive values (row a of a 4 x 16 block, columns 4j .. 4j + 3) and lane
// l receives column l of the block's four rows. Group g = lane / 16 takes columns cb + 16 (g mod 2)
// .. + 15 of k rows 16 s + 8 (g / 2) + 0..3, then + 4..7.
__device__ __forceinline__ bf16x8 dl_frag_kmaj(const uint16_t* S, int s, int cb, int lane) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) shortx4* lds_x4;
  const int g = lane >> 4, a = (lane >> 2) & 3, j = lane & 3;
  const int k = 16 * s + 8 * (g >> 1) + a, pc = (cb >> 3) + 2 * (g & 1) + (j >> 1);
  const uint16_t* q = S + k * 128 + 8 * (pc ^ (4 * a)) + 4 * (j & 1);  // k mod 4 = a
  const shortx4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4)(q));
  const shortx4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_x4)(q + 4 * 128));
  const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
  const uint4 u = {l2.x, l2.y, h2.x, h2.y};
  return __builtin_bit_cast(bf16x8, u);
}

template <bool TA, bool TB, int E, bool BF, int BMT>
__device__ __forceinline__ void gemm_tile(GemmArgs p, int logical) {
  __shared__ __align__(16) float smem[BF ? SMEM_BF : SMEM_FLOATS];
  static_assert(BMT == 128 || (BMT == 64 && !BF), "64-row tiles are fp32 only");
  static_assert(SMEM_BF >= T_ROWS * T_S, "the staged output tile fits the bf16 panels");
  constexpr int MT = BMT / 64;  // 32-row accumulator blocks per wave
  // panels: As buffer i at smem + i*PANEL, Bs buffer i after the NBUF A buffers
  float* const Abase = smem;
  float* const Bbase = smem + NBUF * PANEL;

  const int tiles_n = (p.N + BN - 1) / BN;
  const int tiles = tiles_n * ((p.M + BMT - 1) / BMT);
  const int tile = logical % tiles;
  const int m0 = (tile / tiles_n) * BMT;
  const int n0 = (tile % tiles_n) * BN;
  const int bz = logical / tiles;
  const int b = bz / p.ksplit, split = bz % p.ksplit;
  const float* A = p.A + (long long)b * p.sA;
  const float* B = p.B + (long long)b * p.sB;
  const int kbeg = split * p.kper;
  const int kend = min(p.K, kbeg + p.kper);
  const bool interior = p.vecA && p.vecB && m0 + BMT <= p.M && n0 + BN <= p.N;

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int l32 = lane & 31, h = lane >> 5;

  floatx16 acc[MT][2];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  float csum = 0.f;  // E_DBIAS: this thread's column sum over its half of each panel
  if constexpr (BF && BMT == 128) {
    static_assert((E & E_DBIAS) == 0, "the bf16 path has no fused bias gradient");
    // Two LDS stages of [A panel | B panel] and two register sets: chunk i's products read stage
    // i & 1; then the registers holding chunk i + 1 (loaded two chunks earlier) go to the other
    // stage and take the loads of chunk i + 3. So a chunk's loads have two chunks of products and
    // barriers to land, and there is one barrier a chunk.
    constexpr int STAGE = (BM + BN) * PB;
    uint16_t* const S16 = reinterpret_cast<uint16_t*>(smem);
    uint32_t pa0[16], pb0[16], pa1[16], pb1[16];
    // from the operands' bf16 copies where given (uniform branches)
    const uint16_t* A16 = p.A16 ? p.A16 + (long long)b * p.sA : nullptr;
    const uint16_t* B16 = p.B16 ? p.B16 + (long long)b * p.sB : nullptr;
    const bool tile_in = m0 + BMT <= p.M && n0 + BN <= p.N;
    auto load = [&](int k0, uint32_t(&pa)[16], uint32_t(&pb)[16]) {
      if (A16)
        load_bf16src<!TA>(A16, p.lda, m0, p.M, k0, kend, tile_in && p.vecA16 && k0 + BKB <= kend, p.vecA16, pa);
      else
        load_bf<!TA>(A, p.lda, m0, p.M, k0, kend, interior && k0 + BKB <= kend, p.vecA, pa);
      if (B16)
        load_bf16src<TB>(B16, p.ldb, n0, p.N, k0, kend, tile_in && p.vecB16 && k0 + BKB <= kend, p.vecB16, pb);
      else
        load_bf<TB>(B, p.ldb, n0, p.N, k0, kend, interior && k0 + BKB <= kend, p.vecB, pb);
    };
    auto store = [&](uint16_t* S, const uint32_t(&pa)[16], const uint32_t(&pb)[16]) {
      if (A16)
        store_bf16src<!TA>(S, pa);
      else
        store_bf<!TA>(S, pa);
      if (B16)
        store_bf16src<TB>(S + BM * PB, pb);
      else
        store_bf<TB>(S + BM * PB, pb);
    };
    // chunk k0 from stage st; (ra, rb) hold chunk k0 + BKB
    auto step = [&](int k0, int st, uint32_t(&ra)[16], uint32_t(&rb)[16]) {
      const uint16_t* ap = S16 + st * STAGE + (wm * 64 + l32) * PB + 8 * h;
      const uint16_t* bp = S16 + st * STAGE + BM * PB + (wn * 64 + l32) * PB + 8 * h;
#pragma unroll
      for (int s = 0; s < BKB / 16; ++s) {
        const bf16x8 a0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(ap + 16 * s));
        const bf16x8 a1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(ap + 32 * PB + 16 * s));
        const bf16x8 b0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(bp + 16 * s));
        const bf16x8 b1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(bp + 32 * PB + 16 * s));
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
      }
      if (k0 + BKB < kend) {
        store(S16 + (st ^ 1) * STAGE, ra, rb);
        if (k0 + 3 * BKB < kend) load(k0 + 3 * BKB, ra, rb);
      }
      __syncthreads();
    };
    if (TALOS_GEMM_DLDS && TALOS_GEMM_BF_STAGES == 4 && A16 && B16 && tile_in && p.vecA16 && p.vecB16 &&
        kbeg < kend && (kend - kbeg) % DKB == 0) {
      // both bf16 copies, four stages of 32-k chunks: three chunks' loads in flight while one is
      // multiplied (four load instructions a wave a chunk), one barrier a chunk
      constexpr int NS = 4, STG = (BM + BN) * DKB;  // bf16 values a stage
      static_assert(NS * STG <= 2 * SMEM_BF, "four stages fit the bf16 LDS");
      auto issue = [&](int k0, int st) {
        if (TA)
          dl_panel_kmaj_32(A16, p.lda, k0, m0, S16 + st * STG);
        else
          dl_panel_bf16_32(A16, p.lda, m0, k0, S16 + st * STG);
        if (TB)
          dl_panel_bf16_32(B16, p.ldb, n0, k0, S16 + st * STG + BM * DKB);
        else
          dl_panel_kmaj_32(B16, p.ldb, k0, n0, S16 + st * STG + BM * DKB);
      };
      const int nch = (kend - kbeg) / DKB;
      for (int c = 0; c < NS - 1 && c < nch; ++c) issue(kbeg + c * DKB, c);
      for (int c = 0; c < nch; ++c) {
        // chunk c landed: only the chunks issued after it (at most two, four loads each) may be out
        const int after = min(NS - 2, nch - 1 - c);
        if (after >= 2)
          TALOS_WAIT_VM(8);
        else if (after == 1)
          TALOS_WAIT_VM(4);
        else
          TALOS_WAIT_VM(0);
        lds_barrier();  // every wave's pieces of chunk c are in; every wave is done with chunk c - 1
        if (c + NS - 1 < nch) issue(kbeg + (c + NS - 1) * DKB, (c + NS - 1) % NS);  // into chunk c - 1's stage
        const uint16_t* As = S16 + (c % NS) * STG;
        const uint16_t* Bs = As + BM * DKB;
#pragma unroll
        for (int s = 0; s < DKB / 16; ++s) {
          const bf16x8 a0 = TA ? dl_frag_kmaj(As, s, wm * 64, lane) : dl_frag_bf16_32(As, wm * 64 + l32, 2 * s + h);
          const bf16x8 a1 =
              TA ? dl_frag_kmaj(As, s, wm * 64 + 32, lane) : dl_frag_bf16_32(As, wm * 64 + 32 + l32, 2 * s + h);
          const bf16x8 b0 = TB ? dl_frag_bf16_32(Bs, wn * 64 + l32, 2 * s + h) : dl_frag_kmaj(Bs, s, wn * 64, lane);
          const bf16x8 b1 =
              TB ? dl_frag_bf16_32(Bs, wn * 64 + 32 + l32, 2 * s + h) : dl_frag_kmaj(Bs, s, wn * 64 + 32, lane);
          acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
          acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
          acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
        }
      }
      __syncthreads();  // the epilogue reuses the LDS
    } else if (TALOS_GEMM_DLDS && A16 && B16 && tile_in && p.vecA16 && p.vecB16 && kbeg < kend &&
        (kend - kbeg) % BKB == 0) {
      // both bf16 copies: the panels straight into LDS (k-contiguous operands by dl_panel_bf16,
      // k-major ones by dl_panel_kmaj, read back transposed), two stages, one barrier a chunk
      constexpr int STG = (BM + BN) * BKB;  // bf16 values a stage
      static_assert(2 * STG <= 2 * SMEM_BF, "two stages fit the bf16 LDS");
      auto issue = [&](int k0, int st) {
        if (TA)
          dl_panel_kmaj(A16, p.lda, k0, m0, S16 + st * STG);
        else
          dl_panel_bf16(A16, p.lda, m0, k0, S16 + st * STG);
        if (TB)
          dl_panel_bf16(B16, p.ldb, n0, k0, S16 + st * STG + BM * BKB);
        else
          dl_panel_kmaj(B16, p.ldb, k0, n0, S16 + st * STG + BM * BKB);
      };
      issue(kbeg, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      int st = 0;
      for (int k0 = kbeg; k0 < kend; k0 += BKB, st ^= 1) {
        if (k0 + BKB < kend) issue(k0 + BKB, st ^ 1);
        const uint16_t* As = S16 + st * STG;
        const uint16_t* Bs = As + BM * BKB;
#pragma unroll
        for (int s = 0; s < BKB / 16; ++s) {
          const bf16x8 a0 = TA ? dl_frag_kmaj(As, s, wm * 64, lane) : dl_frag_bf16(As, wm * 64 + l32, 2 * s + h);
          const bf16x8 a1 =
              TA ? dl_frag_kmaj(As, s, wm * 64 + 32, lane) : dl_frag_bf16(As, wm * 64 + 32 + l32, 2 * s + h);
          const bf16x8 b0 = TB ? dl_frag_bf16(Bs, wn * 64 + l32, 2 * s + h) : dl_frag_kmaj(Bs, s, wn * 64, lane);
          const bf16x8 b1 =
              TB ? dl_frag_bf16(Bs, wn * 64 + 32 + l32, 2 * s + h) : dl_frag_kmaj(Bs, s, wn * 64 + 32, lane);
          acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
          acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
          acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
      }
    } else if (A16 && B16) {
      if (kbeg < kend) {
        load(kbeg, pa0, pb0);
        store(S16, pa0, pb0);
        if (kbeg + BKB < kend) load(kbeg + BKB, pa1, pb1);
        if (kbeg + 2 * BKB < kend) load(kbeg + 2 * BKB, pa0, pb0);
      }
      __syncthreads();
      for (int k0 = kbeg; k0 < kend; k0 += 2 * BKB) {
        step(k0, 0, pa1, pb1);
        if (k0 + BKB < kend) step(k0 + BKB, 1, pa0, pb0);
      }
    } else {
      // an fp32 operand is rounded as it is loaded, which makes the wave wait for its loads
      // there: one register set and one stage, the next chunk's loads issued before the products
      if (kbeg < kend) {
        load(kbeg, pa0, pb0);
        store(S16, pa0, pb0);
      }
      __syncthreads();
      for (int k0 = kbeg; k0 < kend; k0 += BKB) {
        const bool more = k0 + BKB < kend;
        if (more) load(k0 + BKB, pa0, pb0);
        const uint16_t* ap = S16 + (wm * 64 + l32) * PB + 8 * h;
        const uint16_t* bp = S16 + BM * PB + (wn * 64 + l32) * PB + 8 * h;
#pragma unroll
        for (int s = 0; s < BKB / 16; ++s) {
          const bf16x8 a0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(ap + 16 * s));
          const bf16x8 a1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(ap + 32 * PB + 16 * s));
          const bf16x8 b0 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(bp + 16 * s));
          const bf16x8 b1 = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(bp + 32 * PB + 16 * s));
          acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
          acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
          acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
          acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
        if (more) {
          store(S16, pa0, pb0);
          __syncthreads();
        }
      }
    }
  } else {
  float ssq = 0.f;  // E_NORMIN: below
  bool direct = false;
  // (128-row tiles: on the 64-row tiles the direct loads measured 2-5% slower at C3; one column
  // tile: with four column tiles per row panel, N = 512 at C5, they measured 4% slower)
  if constexpr (TALOS_GEMM_DLDS && MT == 2 && !TA && TB && (E & (E_NORMIN | E_DBIAS)) == 0) {
    direct = interior && p.N <= BN && kbeg < kend && (kend - kbeg) % DK == 0;
    if (direct) {
      // stage s: the A panel (BMT rows) at smem + s (BMT + BN) DK, the B panel (BN rows) after it
      constexpr int STG = (BMT + BN) * DK;
      static_assert(2 * STG <= SMEM_FLOATS, "two stages fit the panels' LDS");
      auto issue = [&](int k0, int st) {
        dl_panel<BMT>(A, p.lda, m0, k0, smem + st * STG);
        dl_panel<BN>(B, p.ldb, n0, k0, smem + st * STG + BMT * DK);
      };
      issue(kbeg, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      int st = 0;
      for (int k0 = kbeg; k0 < kend; k0 += DK, st ^= 1) {
        if (k0 + DK < kend) issue(k0 + DK, st ^ 1);  // the other stage was read before the last barrier
        const float* Ap = smem + st * STG;
        const float* Bp = Ap + BMT * DK;
        __builtin_amdgcn_s_setprio(TALOS_GEMM_PRIO);
#pragma unroll
        for (int j = 0; j < DK / 8; ++j) {
          float fa0[4], fa1[4], fb0[4], fb1[4];
          dl_frag<MT == 2>(Ap, (MT == 2 ? wm * 64 : wm * 32) + l32, 8 * j + 4 * h, fa0, fa1);
          dl_frag<true>(Bp, wn * 64 + l32, 8 * j + 4 * h, fb0, fb1);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb0[q], acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb1[q], acc[0][1], 0, 0, 0);
            if constexpr (MT == 2) {
              acc[MT - 1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb0[q], acc[MT - 1][0], 0, 0, 0);
              acc[MT - 1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb1[q], acc[MT - 1][1], 0, 0, 0);
            }
          }
        }
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of the next chunk have landed
        __syncthreads();                // everyone's, and every wave is done with this stage
      }
    }
  }
  if (!direct) {
  float4 ra[BMT / 32], rb[4];
  // E_NORMIN: this thread's sum of squares over the A values it loads (thread t and t + 128 load
  // the halves of tile row t % 128), and the gain applied to the B rows as they are loaded
  auto normin = [&](int k0) {
    if constexpr ((E & E_NORMIN) != 0) {
      static_assert(!TA && !TB && BMT == 128, "input norm: A and B plain, 128-row tiles");
#pragma unroll
      for (int i = 0; i < BMT / 32; ++i) ssq += ra[i].x * ra[i].x + ra[i].y * ra[i].y + ra[i].z * ra[i].z + ra[i].w * ra[i].w;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = k0 + (threadIdx.x >> 5) + 8 * i;
        const float g = k < kend ? p.nin_gain[k] : 0.f;
        rb[i] = make_float4(rb[i].x * g, rb[i].y * g, rb[i].z * g, rb[i].w * g);
      }
    }
  };
  if (kbeg < kend) {
    load_chunk<TA, TB, BMT>(p, A, B, m0, n0, kbeg, kend, interior, ra, rb);
    normin(kbeg);
    store_a<TA, BMT>(Abase, ra);
    store_b<TB>(Bbase, rb);
  }
  __syncthreads();
  int buf = 0;
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) {
      load_chunk<TA, TB, BMT>(p, A, B, m0, n0, k0 + BK, kend, interior, ra, rb);
      normin(k0 + BK);
    }
    const float* Ap = Abase + buf * PANEL;
    const float* Bp = Bbase + buf * PANEL;
    // the chunk's products at a raised wave priority: a wave with products ready issues ahead of
    // the waves of the CU's other workgroups that are storing panels or waiting at the barrier
    __builtin_amdgcn_s_setprio(TALOS_GEMM_PRIO);
#pragma unroll
    for (int j = 0; j < BK / 8; ++j) {
      // fragments of steps 4j .. 4j+3: k = 8j + 4h + q for q = 0..3
      float fa0[4], fa1[4], fb0[4], fb1[4];
      if constexpr (MT == 2)
        frag4<!TA>(Ap, wm * 64 + l32, 8 * j + 4 * h, fa0, fa1);
      else
        frag1<!TA>(Ap, wm * 32 + l32, 8 * j + 4 * h, fa0);
      frag4<TB>(Bp, wn * 64 + l32, 8 * j + 4 * h, fb0, fb1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb0[q], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa0[q], fb1[q], acc[0][1], 0, 0, 0);
        if constexpr (MT == 2) {
          acc[MT - 1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb0[q], acc[MT - 1][0], 0, 0, 0);
          acc[MT - 1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa1[q], fb1[q], acc[MT - 1][1], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if constexpr ((E & E_DBIAS) != 0) {
      // column sums of the B panel Bs[k][n] (k-major): thread t sums column t%128 over half the rows
      if (m0 == 0) {
        const float* bc = Bbase + buf * PANEL + (threadIdx.x >> 7) * (BK / 2) * LDS_S + (threadIdx.x & 127);
#pragma unroll
        for (int kk = 0; kk < BK / 2; ++kk) csum += bc[kk * LDS_S];
      }
    }
    if (NBUF == 2) {
      // the other buffer was last read in the previous chunk, before the barrier that ended it
      if (more) {
        store_a<TA, BMT>(Abase + (buf ^ 1) * PANEL, ra);
        store_b<TB>(Bbase + (buf ^ 1) * PANEL, rb);
      }
      __syncthreads();
      buf ^= 1;
    } else {
      __syncthreads();
      if (more) {
        store_a<TA, BMT>(Abase, ra);
        store_b<TB>(Bbase, rb);
        __syncthreads();
      }
    }
  }
  if (NBUF == 2 || kbeg >= kend) __syncthreads();
  }  // !direct
  if constexpr ((E & E_NORMIN) != 0) {
    // rstd of each tile row, the accumulators scaled by their row's, and (first column tile) the
    // normalised rows and rstd written out
    __shared__ float nin_rs[BMT];
    smem[threadIdx.x] = ssq;
    __syncthreads();
    if (threadIdx.x < BMT)
      nin_rs[threadIdx.x] = 1.0f / sqrtf((smem[threadIdx.x] + smem[threadIdx.x + BMT]) / (float)p.K + p.nin_eps);
    __syncthreads();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][nt][r] *= nin_rs[wm * 64 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3)];
    {
      // the tile rows lr = tn, tn + tiles_n, ... are this column tile's to write (the work is shared
      // by the row's column tiles)
      const int tn = n0 / BN, k4 = p.K >> 2, mine = (BMT - tn + tiles_n - 1) / tiles_n;
      for (int i = threadIdx.x; i < mine * k4; i += NT) {
        const int lr = tn + tiles_n * (i / k4), c = 4 * (i % k4), row = m0 + lr;
        if (row >= p.M) continue;
        const float rs = nin_rs[lr];
        const float4 x = *reinterpret_cast<const float4*>(A + (long long)row * p.lda + c);
        const float4 g = *reinterpret_cast<const float4*>(p.nin_gain + c);
        *reinterpret_cast<float4*>(p.nin_out + (long long)row * p.K + c) =
            make_float4(x.x * rs * g.x, x.y * rs * g.y, x.z * rs * g.z, x.w * rs * g.w);
      }
      const int lr = tn + tiles_n * (int)threadIdx.x;
      if (lr < BMT && m0 + lr < p.M && p.nin_rstd) p.nin_rstd[m0 + lr] = nin_rs[lr];
    }
    __syncthreads();  // smem is the staging tile next
  }
  }  // fp32 main loop
  if constexpr ((E & E_DBIAS) != 0) {
    // combine the two row halves; the M-tile-0 workgroups write the bias-gradient row
    if (m0 == 0) {
      smem[threadIdx.x] = csum;
      __syncthreads();
      const int n = n0 + (int)threadIdx.x;
      if (threadIdx.x < 128 && n < p.N) {
        const float cs = smem[threadIdx.x] + smem[threadIdx.x + 128];
        if constexpr ((E & E_SPLIT) != 0) {
          p.part[(((long long)b * p.ksplit + split) * (p.M + 1) + p.M) * p.N + n] = cs;
        } else {
          float* db = p.dbias + (long long)b * p.N;
          db[n] = p.beta_dbias != 0.f ? db[n] + cs : cs;
        }
      }
      __syncthreads();
    }
  }

  // E_NBPRE on 128-row tiles whose samples are a multiple of 32 rows: each 32 x 32 accumulator
  // block lies in one sample, so its addend sum_h P[row][h] U[sample][h][col] is a 32 x 4 by 4 x 32
  // product, two more v_mfma_f32_32x32x2_f32 steps (lane half h supplies head 2 s + h at step s),
  // and the epilogue runs without the addend's per-row loads.
  bool pre_folded = false;
  if constexpr ((E & E_NBPRE) != 0 && MT == 2) {
    pre_folded = p.nb_seq % 32 == 0;
    if (pre_folded) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int r0 = m0 + wm * 64 + mt * 32, row = r0 + l32;
        // (a block that starts past M has zero P rows: any U row serves it)
        const long long smp = (long long)(r0 < p.M ? r0 : 0) / p.nb_seq;
        float pa[2], ub[2][2];  // P: [step]; U: [nt][step]
#pragma unroll
        for (int st = 0; st < 2; ++st) pa[st] = row < p.M ? p.nb_pre_p[(long long)row * 4 + 2 * st + h] : 0.f;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int col = n0 + wn * 64 + nt * 32 + l32;
#pragma unroll
          for (int st = 0; st < 2; ++st)
            ub[nt][st] = col < p.N ? p.nb_pre_u[(smp * 4 + 2 * st + h) * p.N + col] : 0.f;
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int st = 0; st < 2; ++st)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[st], ub[nt][st], acc[mt][nt], 0, 0, 0);
      }
    }
  }

  // Stage the tile through LDS 64 rows at a time (BMT = 128: one half, the two waves with
  // wm == half; BMT = 64: all four waves) (accumulator layout of v_mfma_f32_32x32x2_f32: lane l,
  // register r holds row 8*(r/4) + 4*(l/32) + r%4, column l%32 of its 32x32 block), then run the
  // epilogue on row-contiguous float4s: thread t handles column group t%32 of rows t/32 + 8i.
  float* T = smem;
  const int cg = 4 * (threadIdx.x & 31);
  const int col = n0 + cg;
  float4 nbw = make_float4(0.f, 0.f, 0.f, 0.f);  // E_NORMB: this thread's dgain terms
  float* C = p.C + (long long)b * p.sC;
  const float* resid = ((E & E_RESID) != 0) ? p.resid + (long long)b * p.sC : nullptr;
  // float4 path needs every row start 16-byte aligned in each operand the epilogue touches
  const bool full_cols = interior || (col + 3 < p.N);
  const bool aligned = ((p.ldc & 3) == 0) && (((E & E_RESID) == 0) || (p.ldr & 3) == 0) &&
                       (((E & (E_GELU | E_RELU | E_DGELU | E_DRELU)) == 0) || (p.ldaux & 3) == 0) &&
                       ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
  // E_NORMB on 64-row tiles: the whole tile is staged at once, so no accumulator is live in the
  // epilogue, and each thread keeps the x, rstd and addend rows of a few rows in flight ahead of
  // the row it finishes (normb_rows). (On 128-row tiles the second half's accumulators are live
  // through the first half's epilogue, which leaves registers for x one row ahead; there the
  // epilogue phase of the lockstep grid runs at the bandwidth of its mixed reads and writes, and
  // deeper prefetching of the second half measured the same.)
  constexpr bool NB_PIPE = (E & E_NORMB) != 0 && MT == 1;
  if constexpr (NB_PIPE) {
    constexpr bool LAST = (E & E_NBLAST) != 0;
    stage_acc<MT>(T, acc, wm, wn, h, l32, 0);
    __syncthreads();
    // (each thread reads and writes only its own rows' columns of T from here on)
    if constexpr ((E & E_NBPRE) != 0) normb_pre_rows(p, T, cg, col, m0 + (threadIdx.x >> 5));
    const float4 g = *reinterpret_cast<const float4*>(p.nb_gain + col);
    normb_rows<LAST ? TALOS_NB_AHEAD_LAST : TALOS_NB_AHEAD, LAST>(p, T, cg, col, m0 + (threadIdx.x >> 5), g, nbw);
  }
#pragma unroll
  for (int half = 0; half < (NB_PIPE ? 0 : BMT / T_ROWS); ++half) {
    if (half) __syncthreads();  // the first half has been read out
    if (MT == 1 || wm == half) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = (MT == 1 ? wm * 32 : mt * 32) + 8 * (r >> 2) + 4 * h + (r & 3);
            const int c = wn * 64 + nt * 32 + l32;
            T[row * T_S + c] = acc[mt][nt][r];
          }
    }
    __syncthreads();
    if constexpr ((E & E_SPLIT) != 0) {
      float* P = p.part + ((long long)b * p.ksplit + split) * (long long)(p.M + ((E & E_DBIAS) ? 1 : 0)) * p.N;
      const bool vec_out = (p.N & 3) == 0;
#pragma unroll 4
      for (int i = 0; i < T_ROWS / 8; ++i) {
        const int lr = (threadIdx.x >> 5) + 8 * i;
        const int row = m0 + half * T_ROWS + lr;
        const float4 v = *reinterpret_cast<const float4*>(T + lr * T_S + cg);
        if (row >= p.M) continue;
        if (vec_out && col + 3 < p.N) {
          *reinterpret_cast<float4*>(P + (long long)row * p.N + col) = v;
        } else {
          const float vv[4] = {v.x, v.y, v.z, v.w};
          for (int j = 0; j < 4 && col + j < p.N; ++j) P[(long long)row * p.N + col + j] = vv[j];
        }
      }
    } else if constexpr ((E & E_NORMB) != 0) {
      const float4 g = *reinterpret_cast<const float4*>(p.nb_gain + col);
      const int rbase = m0 + half * T_ROWS + (threadIdx.x >> 5);
      // the next row's x and rstd load under this row's work; with E_NBPRE, after the row (its
      // last-row terms leave no registers for them ahead: 16 bytes a lane spilled, 80.6 against
      // 79.3 us at C4), and the addend's P and U loaded in the row's own step unless the products
      // already added it (82.3 us when they did not)
      const bool pre = (E & E_NBPRE) != 0 && !pre_folded;
      NbIn cur = normb_load(p, rbase, col);
#pragma unroll 1
      for (int i = 0; i < T_ROWS / 8; ++i) {
        const int lr = (threadIdx.x >> 5) + 8 * i;
        NbIn nxt = cur;
        if ((E & E_NBPRE) == 0 && i + 1 < T_ROWS / 8) nxt = normb_load(p, rbase + 8 * (i + 1), col);
        const float4 v = *reinterpret_cast<const float4*>(T + lr * T_S + cg);
        if constexpr ((E & E_NBPRE) != 0) {
          if (pre)
            normb_apply<true>(p, v, rbase + 8 * i, col, cur, g, nbw);
          else
            normb_apply<false>(p, v, rbase + 8 * i, col, cur, g, nbw);
        } else {
          normb_apply<false>(p, v, rbase + 8 * i, col, cur, g, nbw);
        }
        if ((E & E_NBPRE) != 0 && i + 1 < T_ROWS / 8) nxt = normb_load(p, rbase + 8 * (i + 1), col);
        cur = nxt;
      }
    } else {
      // the row-dependent operands of four rows at a time (and the bias once) are loaded before
      // those rows' stores
      const bool fast = aligned && full_cols;
      float4 bias = make_float4(0.f, 0.f, 0.f, 0.f), ngain = make_float4(0.f, 0.f, 0.f, 0.f);
      if constexpr ((E & E_BIAS) != 0)
        if (fast) bias = *reinterpret_cast<const float4*>(p.bias + col);
      if constexpr ((E & E_NORM) != 0)
        if (col + 3 < p.N) ngain = *reinterpret_cast<const float4*>(p.norm_gain + col);
#pragma unroll 1
      for (int i0 = 0; i0 < T_ROWS / 8; i0 += 4) {
        EpiPre pre[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = m0 + half * T_ROWS + (threadIdx.x >> 5) + 8 * (i0 + j);
          pre[j] = epi_preload<E>(p, row, col, fast && row < p.M, bias);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int lr = (threadIdx.x >> 5) + 8 * (i0 + j);
          const int row = m0 + half * T_ROWS + lr;
          const float4 v = *reinterpret_cast<const float4*>(T + lr * T_S + cg);
          const float4 o = epi_store4<E, true>(p, v, row, col, C, resid, fast && row < p.M, pre[j]);
          if constexpr ((E & E_NORM) != 0) epi_norm4(p, o, row, col, ngain);
          if constexpr ((E & E_ROWDOT) != 0) {
            // the row's dot with rd_o over each head's columns: rd_w / 4 lanes a head (a 32-lane
            // group holds one row), the products and the lane sums in the attention row-dot
            // kernel's order (lane c holds columns 4c .. 4c + 3 of the head)
            const bool ok = fast && row < p.M;
            float dd = 0.f;
            if (ok) {
              const float4 x = *reinterpret_cast<const float4*>(p.rd_o + (long long)row * p.rd_ldo + col);
              dd = fmaf(o.x, x.x, fmaf(o.y, x.y, fmaf(o.z, x.z, fmaf(o.w, x.w, 0.f))));
            }
            dd += __shfl_xor(dd, 1, 64);
            dd += __shfl_xor(dd, 2, 64);
            dd += __shfl_xor(dd, 4, 64);
            if (p.rd_w == 64) dd += __shfl_xor(dd, 8, 64);
            if (ok && col % p.rd_w == 0)
              p.rd_D[((long long)(row / p.rd_seq) * p.rd_heads + col / p.rd_w) * p.rd_seq + row % p.rd_seq] = dd;
          }
          if constexpr (BF) {
            if (p.C16 && row < p.M) {  // the bf16 copy of the stored values
              uint16_t* c16 = p.C16 + (long long)b * p.sC + (long long)row * p.ldc + out_col<E>(p, col);
              if (fast && p.vecC16) {
                *reinterpret_cast<uint2*>(c16) = make_uint2(pack_bf16(o.x, o.y), pack_bf16(o.z, o.w));
              } else {
                const float oo[4] = {o.x, o.y, o.z, o.w};
                for (int q = 0; q < 4 && col + q < p.N; ++q) c16[q] = (uint16_t)(pack_bf16(oo[q], 0.f) & 0xffffu);
              }
            }
          }
        }
      }
    }
  }
  if constexpr ((E & E_NORMB) != 0) {
    // the tile's dgain partial: the 8 row groups' sums of each column added in f64, in order
    __syncthreads();  // T has been read out
    *reinterpret_cast<float4*>(T + (threadIdx.x >> 5) * BN + cg) = nbw;
    __syncthreads();
    if (threadIdx.x < BN) {
      double sum = 0.0;
#pragma unroll
      for (int g = 0; g < NT / 32; ++g) sum += (double)T[g * BN + threadIdx.x];
      p.nb_part[(long long)(m0 / BMT) * BN + threadIdx.x] = sum;
    }
  }
}

template <bool TA, bool TB, int E, bool BF>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(BF ? 2 : TALOS_GEMM_WAVES))) void gemm_f32_kernel(
    GemmArgs p) {
  const int logical = xcd_logical();
  if (logical >= p.nblocks) return;
  gemm_tile<TA, TB, E, BF, BM>(p, logical);
}

// 64 x 128 tiles for the products whose 128 x 128 tiles would leave each CU fewer than two
// workgroups (d = 128 outputs over 32K rows): twice the workgroups, half the serial chain each.
template <bool TA, bool TB, int E>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(TALOS_GEMM_WAVES))) void gemm_f32_m64_kernel(
    GemmArgs p) {
  const int logical = xcd_logical();
  if (logical >= p.nblocks) return;
  gemm_tile<TA, TB, E, false, 64>(p, logical);
}

// Two split-K products of one shape class in one grid (the weight gradients of a block's MLP):
// the logical workgroups alternate between the products (even: p0, odd: p1) while both have
// some left, then the larger one takes the rest, so every XCD runs both products in contiguous
// runs of each. Four workgroups per CU where each product alone would give two.
template <bool TA, bool TB, int E>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(TALOS_GEMM_WAVES))) void gemm_f32_pair_kernel(
    GemmArgs p0, GemmArgs p1) {
  const int logical = xcd_logical();
  const int m = min(p0.nblocks, p1.nblocks);
  if (logical < 2 * m) {
    if (logical & 1)
      gemm_tile<TA, TB, E, false, BM>(p1, logical >> 1);
    else
      gemm_tile<TA, TB, E, false, BM>(p0, logical >> 1);
  } else if (logical < p0.nblocks + p1.nblocks) {
    if (p0.nblocks > m)
      gemm_tile<TA, TB, E, false, BM>(p0, logical - m);
    else
      gemm_tile<TA, TB, E, false, BM>(p1, logical - m);
  }
}

// ---------------------------------------------------------------------------
// Small problems: 64x64 tiles. A product with fewer 128x128 tiles than half the CUs (the
// per-sample rows of the policy's last layer and heads, B = 4096 rows) would keep most of the
// chip idle while each workgroup walks K alone; a 64x64 tile gives four times the workgroups and
// a quarter of the serial MFMA chain each. Same 256 threads, one 32x32 accumulator per wave,
// the same panel layouts (k-contiguous pitch 36, k-major pitch 72) and the same epilogue code.
// ---------------------------------------------------------------------------
constexpr int SBM = 64, SBN = 64;
// k-major panel X[k][r] of 64 rows: rows k and k + 4 read by the two half-waves sit 4 * 72 = 32
// mod 64 banks apart
constexpr int S_LDS = 72;
constexpr int S_PANEL = (BK * S_LDS > SBM * KP) ? BK * S_LDS : SBM * KP;
constexpr int S_TS = 72;  // staged output tile pitch (the half-wave rows 4 apart: 32 banks apart)
constexpr int S_SMEM = (2 * S_PANEL > SBM * S_TS) ? 2 * S_PANEL : SBM * S_TS;

// op(X) panel [64 rows x 32 k] of chunk k0 into registers. KC: X[r][k] (k contiguous), thread t
// takes row t%64, k = 4*(t/64 + 4i); otherwise X[k][r] (r contiguous), thread t takes
// r = 4*(t%16), k = t/16 + 16i.
template <bool KC, bool CHECK>
__device__ __forceinline__ void s_load(const float* __restrict__ X, long long ld, int r0, int rlim, int k0, int kend,
                                       bool vec, float4 (&o)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int r, k;
    if (KC) {
      r = r0 + (t & 63);
      k = k0 + 4 * ((t >> 6) + 4 * i);
    } else {
      r = r0 + 4 * (t & 15);
      k = k0 + (t >> 4) + 16 * i;
    }
    const float* src = KC ? X + (long long)r * ld + k : X + (long long)k * ld + r;
    const bool ok = KC ? (r < rlim && k + 3 < kend) : (k < kend && r + 3 < rlim);
    if (!CHECK || (vec && ok)) {
      o[i] = *reinterpret_cast<const float4*>(src);
    } else {
      float v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = KC ? (r < rlim && k + j < kend) : (k < kend && r + j < rlim);
        v[j] = in ? src[j] : 0.f;
      }
      o[i] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}
template <bool KC>
__device__ __forceinline__ void s_store(float* X, const float4 (&o)[2]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (KC)
      *reinterpret_cast<float4*>(X + (t & 63) * KP + 4 * ((t >> 6) + 4 * i)) = o[i];
    else
      *reinterpret_cast<float4*>(X + ((t >> 4) + 16 * i) * S_LDS + 4 * (t & 15)) = o[i];
  }
}
// MFMA operand values of row r at k = k0 .. k0 + 3.
template <bool KC>
__device__ __forceinline__ void s_frag(const float* X, int r, int k0, float (&f)[4]) {
  if (KC) {
    const float4 v = *reinterpret_cast<const float4*>(X + r * KP + k0);
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) f[q] = X[(k0 + q) * S_LDS + r];
  }
}

template <bool TA, bool TB, int E>
__global__ __launch_bounds__(NT) void gemm_small_kernel(GemmArgs p) {
  __shared__ __align__(16) float smem[S_SMEM];
  float* const As = smem;
  float* const Bs = smem + S_PANEL;
  const int tiles_n = (p.N + SBN - 1) / SBN;
  const int tiles = tiles_n * ((p.M + SBM - 1) / SBM);
  // XCD-aware order, as in gemm_f32_kernel
  const int per_xcd = (int)(gridDim.x >> 3);
  const int logical = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (logical >= p.nblocks) return;
  const int tile = logical % tiles;
  const int m0 = (tile / tiles_n) * SBM;
  const int n0 = (tile % tiles_n) * SBN;
  const int bz = logical / tiles;
  const int b = bz / p.ksplit, split = bz % p.ksplit;
  const float* A = p.A + (long long)b * p.sA;
  const float* B = p.B + (long long)b * p.sB;
  const int kbeg = split * p.kper;
  const int kend = min(p.K, kbeg + p.kper);
  const bool interior = p.vecA && p.vecB && m0 + SBM <= p.M && n0 + SBN <= p.N;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w >> 1, wn = w & 1;
  const int l32 = lane & 31, h = lane >> 5;
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  float csum = 0.f;  // E_DBIAS: column t%64 of op(B) over rows 8*(t/64) .. +8 of each panel
  float4 ra[2], rb[2];
  auto load = [&](int k0) {
    if (interior && k0 + BK <= kend) {
      s_load<!TA, false>(A, p.lda, m0, p.M, k0, kend, p.vecA, ra);
      s_load<TB, false>(B, p.ldb, n0, p.N, k0, kend, p.vecB, rb);
    } else {
      s_load<!TA, true>(A, p.lda, m0, p.M, k0, kend, p.vecA, ra);
      s_load<TB, true>(B, p.ldb, n0, p.N, k0, kend, p.vecB, rb);
    }
  };
  if (kbeg < kend) {
    load(kbeg);
    s_store<!TA>(As, ra);
    s_store<TB>(Bs, rb);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load(k0 + BK);
#pragma unroll
    for (int j = 0; j < BK / 8; ++j) {
      float fa[4], fb[4];
      s_frag<!TA>(As, wm * 32 + l32, 8 * j + 4 * h, fa);
      s_frag<TB>(Bs, wn * 32 + l32, 8 * j + 4 * h, fb);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[q], fb[q], acc, 0, 0, 0);
    }
    if constexpr ((E & E_DBIAS) != 0) {
      if (m0 == 0) {
        const float* bc = Bs + (threadIdx.x >> 6) * 8 * S_LDS + (threadIdx.x & 63);
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) csum += bc[kk * S_LDS];
      }
    }
    __syncthreads();
    if (more) {
      s_store<!TA>(As, ra);
      s_store<TB>(Bs, rb);
      __syncthreads();
    }
  }
  if constexpr ((E & E_DBIAS) != 0) {
    if (m0 == 0) {
      smem[threadIdx.x] = csum;
      __syncthreads();
      const int n = n0 + (int)threadIdx.x;
      if (threadIdx.x < 64 && n < p.N) {
        const float cs = smem[threadIdx.x] + smem[threadIdx.x + 64] + smem[threadIdx.x + 128] + smem[threadIdx.x + 192];
        if constexpr ((E & E_SPLIT) != 0) {
          p.part[(((long long)b * p.ksplit + split) * (p.M + 1) + p.M) * p.N + n] = cs;
        } else {
          float* db = p.dbias + (long long)b * p.N;
          db[n] = p.beta_dbias != 0.f ? db[n] + cs : cs;
        }
      }
      __syncthreads();
    }
  }
  // stage the 64x64 tile through LDS, then the epilogue on row-contiguous float4s: thread t
  // handles column group t%16 of rows t/16 + 16i
  float* T = smem;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = wm * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
    T[row * S_TS + wn * 32 + l32] = acc[r];
  }
  __syncthreads();
  const int cg = 4 * (threadIdx.x & 15);
  const int col = n0 + cg;
  float* C = p.C + (long long)b * p.sC;
  const float* resid = ((E & E_RESID) != 0) ? p.resid + (long long)b * p.sC : nullptr;
  const bool full_cols = interior || (col + 3 < p.N);
  const bool aligned = ((p.ldc & 3) == 0) && (((E & E_RESID) == 0) || (p.ldr & 3) == 0) &&
                       (((E & (E_GELU | E_RELU | E_DGELU | E_DRELU)) == 0) || (p.ldaux & 3) == 0) &&
                       ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
#pragma unroll
  for (int i = 0; i < SBM / 16; ++i) {
    const int lr = (threadIdx.x >> 4) + 16 * i;
    const int row = m0 + lr;
    const float4 v = *reinterpret_cast<const float4*>(T + lr * S_TS + cg);
    if constexpr ((E & E_SPLIT) != 0) {
      if (row >= p.M) continue;
      float* P = p.part + ((long long)b * p.ksplit + split) * (long long)(p.M + ((E & E_DBIAS) ? 1 : 0)) * p.N;
      if ((p.N & 3) == 0 && col + 3 < p.N) {
        *reinterpret_cast<float4*>(P + (long long)row * p.N + col) = v;
      } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
        for (int j = 0; j < 4 && col + j < p.N; ++j) P[(long long)row * p.N + col + j] = vv[j];
      }
    } else {
      epi_store4<E>(p, v, row, col, C, resid, aligned && full_cols && row < p.M);
    }
  }
}

// Sums the split-K partials in f64 and applies the epilogue (beta and bias only). Workgroup of
// 256 threads = 4 waves: lane <-> one of 64 consecutive elements, wave w <-> splits w, w+4, ...
// (small workgroups, so the reduction finds room beside a product running on another stream).
// Row M of the partials (when present) holds the bias-gradient column sums.
template <int E>
__device__ __forceinline__ void splitk_reduce_tile(const GemmArgs& p, int blk, int b) {
  constexpr int W = 4;
  __shared__ double red[W][64];
  const int rows = p.M + (p.dbias ? 1 : 0);
  const long long RN = (long long)rows * p.N;
  const float* P = p.part + (long long)b * p.ksplit * RN;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const long long e = (long long)blk * 64 + lane;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  if (e < RN) {
    int k = w;
    for (; k + 3 * W < p.ksplit; k += 4 * W) {
      s0 += (double)P[k * RN + e];
      s1 += (double)P[(k + W) * RN + e];
      s2 += (double)P[(k + 2 * W) * RN + e];
      s3 += (double)P[(k + 3 * W) * RN + e];
    }
    for (; k < p.ksplit; k += W) s0 += (double)P[k * RN + e];
  }
  red[w][lane] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (w != 0 || e >= RN) return;
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < W; ++i) s += red[i][lane];
  const int row = (int)(e / p.N), col = (int)(e % p.N);
  if (row == p.M) {
    float* db = p.dbias + (long long)b * p.N;
    db[col] = (float)(p.beta_dbias != 0.f ? (double)db[col] + s : s);
    return;
  }
  float* C = p.C + (long long)b * p.sC;
  float v = p.alpha * (float)s;
  if constexpr ((E & E_BETA) != 0) v += p.beta * C[(long long)row * p.ldc + col];
  if constexpr ((E & E_BIAS) != 0) v += p.bias[col];
  C[(long long)row * p.ldc + col] = v;
}
template <int E>
__global__ __launch_bounds__(256) void gemm_splitk_reduce(GemmArgs p) {
  splitk_reduce_tile<E>(p, blockIdx.x, blockIdx.y);
}
// Held-back plain combinations in one launch: job k takes workgroups [start[k], start[k + 1]).
struct SplitBatch {
  SplitJob j[kSplitJobsMax];
  int start[kSplitJobsMax + 1];
  int n;
};
__global__ __launch_bounds__(256) void gemm_splitk_reduce_batch(SplitBatch sb) {
  int k = 0;
  while (k + 1 < sb.n && (int)blockIdx.x >= sb.start[k + 1]) ++k;  // uniform
  const SplitJob& J = sb.j[k];
  GemmArgs p{};
  p.part = const_cast<float*>(J.part);
  p.ksplit = J.ksplit;
  p.M = J.M;
  p.N = J.N;
  p.C = J.C;
  p.ldc = J.ldc;
  p.alpha = J.alpha;
  p.dbias = J.dbias;
  p.beta_dbias = J.beta_dbias;
  splitk_reduce_tile<0>(p, (int)blockIdx.x - sb.start[k], 0);
}

static GemmArgs to_args(const GemmDesc& d) {
  GemmArgs a;
  a.M = d.M;
  a.N = d.N;
  a.K = d.K;
  a.A = d.A;
  a.lda = d.lda;
  a.sA = d.sA;
  a.B = d.B;
  a.ldb = d.ldb;
  a.sB = d.sB;
  a.C = d.C;
  a.ldc = d.ldc;
  a.sC = d.sC;
  a.alpha = d.alpha;
  a.beta = d.beta;
  a.bias = d.bias;
  a.resid = d.resid;
  a.ldr = d.ldr;
  a.aux = d.aux;
  a.ldaux = d.ldaux;
  a.rcos = d.rope_cos;
  a.rsin = d.rope_sin;
  a.rope_cols = d.rope_cols;
  a.rope_dim = d.rope_dim > 0 ? d.rope_dim : 2;
  a.rope_seq = d.rope_seq > 0 ? d.rope_seq : 1;
  a.cmap_w = d.cmap_w;
  a.cmap_pitch = d.cmap_pitch;
  a.cmap_off = d.cmap_off;
  a.rd_o = d.rd_o;
  a.rd_ldo = d.rd_ldo;
  a.rd_D = d.rd_D;
  a.rd_w = d.rd_w;
  a.rd_seq = d.rd_seq > 0 ? d.rd_seq : 1;
  a.rd_heads = d.rd_heads > 0 ? d.rd_heads : 1;
  a.ksplit = d.ksplit < 1 ? 1 : d.ksplit;
  a.kper = d.K;
  a.part = d.workspace;
  a.dbias = d.dbias;
  a.beta_dbias = d.beta_dbias;
  a.norm_gain = d.norm_gain;
  a.norm_out = d.norm_out;
  a.ldn = d.ldn;
  a.norm_rstd = d.norm_rstd;
  a.norm_eps = d.norm_eps;
  a.nin_gain = d.nin_gain;
  a.nin_out = d.nin_out;
  a.nin_rstd = d.nin_rstd;
  a.nin_eps = d.nin_eps;
  a.nb_x = d.normb_x;
  a.nb_rstd = d.normb_rstd;
  a.nb_gain = d.normb_gain;
  a.nb_add = d.normb_add;
  a.nb_add_last = d.normb_add_last;
  a.nb_dy_last = d.normb_dy_last;
  a.nb_pre_p = d.normb_pre_p;
  a.nb_pre_u = d.normb_pre_u;
  a.nb_seq = d.normb_seq > 0 ? d.normb_seq : 1;
  a.nb_lens = d.normb_lens;
  a.nb_dx = d.normb_dx;
  a.nb_part = d.normb_ws;
  auto aligned = [](const void* ptr, long long ld) {
    return ((reinterpret_cast<uintptr_t>(ptr) & 15) == 0) && (ld % 4 == 0);
  };
  a.vecA = aligned(d.A, d.lda) && (d.batch == 1 || d.sA % 4 == 0);
  a.vecB = aligned(d.B, d.ldb) && (d.batch == 1 || d.sB % 4 == 0);
  auto aligned8 = [](const void* ptr, long long ld) {
    return ((reinterpret_cast<uintptr_t>(ptr) & 7) == 0) && (ld % 4 == 0);
  };
  auto aligned16 = [](const void* ptr, long long ld) {
    return ((reinterpret_cast<uintptr_t>(ptr) & 15) == 0) && (ld % 8 == 0);
  };
  a.A16 = d.bf16 ? d.A16 : nullptr;
  a.B16 = d.bf16 ? d.B16 : nullptr;
  a.C16 = d.bf16 ? d.C16 : nullptr;
  a.vecA16 = a.A16 && aligned16(d.A16, d.lda) && (d.batch == 1 || d.sA % 8 == 0);
  a.vecB16 = a.B16 && aligned16(d.B16, d.ldb) && (d.batch == 1 || d.sB % 8 == 0);
  a.vecC16 = a.C16 && aligned8(d.C16, d.ldc) && (d.batch == 1 || d.sC % 4 == 0);
  if (a.ksplit > 1) {
    const int chunk = d.bf16 ? BKB : BK;
    int kper = (d.K + a.ksplit - 1) / a.ksplit;
    kper = (kper + chunk - 1) / chunk * chunk;
    a.kper = kper;
    a.ksplit = (d.K + kper - 1) / kper;
  }
  return a;
}

static int epi_flags(const GemmDesc& d) {
  int e = 0;
  if (d.beta != 0.f) e |= E_BETA;
  if (d.bias) e |= E_BIAS;
  if (d.resid) e |= E_RESID;
  if (d.act == GEMM_ACT_GELU) e |= E_GELU;
  if (d.act == GEMM_ACT_RELU) e |= E_RELU;
  if (d.dact == GEMM_DACT_GELU) e |= E_DGELU;
  if (d.dact == GEMM_DACT_RELU) e |= E_DRELU;
  if (d.rope_cols > 0) e |= E_ROPE;
  if (d.dbias) e |= E_DBIAS;
  if (d.norm_out) e |= E_NORM;
  if (d.normb_dx) e |= E_NORMB;
  if (d.normb_dx && d.normb_pre_p) e |= E_NBPRE;
  if (d.normb_dx && (d.normb_add_last || d.normb_dy_last)) e |= E_NBLAST;
  if (d.nin_gain) e |= E_NORMIN;
  if (d.cmap_w) e |= E_CMAP;
  if (d.rd_D) e |= E_ROWDOT;
  return e;
}

// Whether a product runs on 64x64 tiles: fp32, fewer 128x128 tiles than CUs, and little work in
// all (at most 2^30 multiply-adds): long-K weight gradients over all tokens keep the 128x128 tiles
// and split K instead, which reads each operand half as often.
static void (*pick_m64(bool tA, bool tB, int e))(GemmArgs);
// The 64 x 64 tile kernel for products of fewer 128 x 128 tiles than CUs and at most 2^30 MACs;
// not for one 128-wide column of tiles over at least 64 rows a CU where the 64 x 128 tiles are
// instantiated (C5's M = 16384, N = 128 products: 1.669 -> 1.650 ms).
static bool use_small(const GemmDesc& d, int num_cu) {
  const long long tiles = (long long)((d.M + BM - 1) / BM) * ((d.N + BN - 1) / BN) * d.batch;
  const double macs = (double)d.M * d.N * d.K * d.batch;
  if (!d.bf16 && d.batch == 1 && d.N <= BN && d.M >= 64 * num_cu && !d.transA && d.ksplit <= 1 &&
      pick_m64(false, d.transB != 0, epi_flags(d)) != nullptr)
    return false;  // one 128-wide column of tiles over many rows: the 64-row tiles
  return !d.bf16 && d.cmap_w == 0 && !d.rd_D && tiles < num_cu && macs <= 1073741824.0;
}

size_t gemm_plan_split(GemmDesc& d, int num_cu) {
  const int e = epi_flags(d);
  if (d.ksplit == 0) {
    const bool small = use_small(d, num_cu);
    const int bm = small ? SBM : BM, bn = small ? SBN : BN;
    const long long tiles = (long long)((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn) * d.batch;
    // Split so that the grid holds TALOS_SPLITK_WG_PER_CU workgroups per CU (any split count,
    // not only powers of two: 3 tiles get 170 splits, not 128), keeping at least
    // TALOS_SPLITK_MIN_K of K per split: the partial traffic (ksplit * M * N floats) stays small
    // next to A and B.
    long long ks = (long long)TALOS_SPLITK_WG_PER_CU * num_cu / std::max(1LL, tiles);
    ks = std::min(ks, (long long)d.K / TALOS_SPLITK_MIN_K);
    d.ksplit = (int)std::max(1LL, ks);
  }
  if ((e & ~(E_BETA | E_BIAS | E_DBIAS)) != 0) d.ksplit = 1;  // only beta / bias survive a split
  if (d.C16) d.ksplit = 1;  // the bf16 copy of C is written by the epilogue
  if (d.cmap_w) d.ksplit = 1;  // the column map is the epilogue's
  if (d.ksplit <= 1) return 0;
  GemmArgs a = to_args(d);
  return (size_t)a.ksplit * (d.M + (d.dbias ? 1 : 0)) * d.N * d.batch * sizeof(float);
}

typedef void (*GemmKernel)(GemmArgs);

// Instantiated (transA, transB, epilogue) combinations; bf16 covers the same set minus the fused
// bias gradient.
#define GEMM_CASE(TA, TB, E)                                                                     \
  if (tA == TA && tB == TB && e == (E)) return bf ? &gemm_f32_kernel<TA, TB, (E), true>          \
                                                  : &gemm_f32_kernel<TA, TB, (E), false>;
#define GEMM_CASE_F32(TA, TB, E) \
  if (!bf && tA == TA && tB == TB && e == (E)) return &gemm_f32_kernel<TA, TB, (E), false>;
static GemmKernel pick_kernel(bool tA, bool tB, int e, bool bf) {
  GEMM_CASE(false, false, 0)
  GEMM_CASE(false, false, E_BETA)
  GEMM_CASE(false, false, E_BIAS)
  GEMM_CASE(false, false, E_ROPE)
  GEMM_CASE(false, false, E_CMAP)
  GEMM_CASE(false, false, E_ROPE | E_CMAP)
  GEMM_CASE(false, false, E_RESID)
  GEMM_CASE(false, false, E_BIAS | E_RESID)
  GEMM_CASE(false, false, E_BIAS | E_GELU)
  GEMM_CASE(false, false, E_BIAS | E_RELU)
  GEMM_CASE(false, false, E_SPLIT)
  GEMM_CASE_F32(false, false, E_BIAS | E_NORM)
  GEMM_CASE_F32(false, false, E_RESID | E_NORM)
  GEMM_CASE_F32(false, false, E_BIAS | E_RESID | E_NORM)
  GEMM_CASE_F32(false, false, E_NORMIN)
  GEMM_CASE_F32(false, false, E_ROPE | E_NORMIN)
  GEMM_CASE(false, true, 0)
  GEMM_CASE(false, true, E_BETA)
  GEMM_CASE(false, true, E_DGELU)
  GEMM_CASE(false, true, E_DRELU)
  GEMM_CASE(false, true, E_SPLIT)
  GEMM_CASE(false, true, E_ROWDOT)
  GEMM_CASE_F32(false, true, E_NORMB)
  GEMM_CASE_F32(false, true, E_NORMB | E_NBLAST)
  GEMM_CASE_F32(false, true, E_NORMB | E_NBPRE)
  GEMM_CASE_F32(false, true, E_NORMB | E_NBPRE | E_NBLAST)
  GEMM_CASE(true, false, 0)
  GEMM_CASE(true, false, E_BETA)
  GEMM_CASE(true, false, E_SPLIT)
  GEMM_CASE_F32(true, false, E_DBIAS)
  GEMM_CASE_F32(true, false, E_SPLIT | E_DBIAS)
  GEMM_CASE_F32(true, false, E_BETA | E_DBIAS)
  GEMM_CASE(true, true, 0)
  GEMM_CASE(true, true, E_BETA)
  GEMM_CASE(true, true, E_SPLIT)
  return nullptr;
}
#undef GEMM_CASE
#undef GEMM_CASE_F32

#define SMALL_CASE(TA, TB, E) \
  if (tA == TA && tB == TB && e == (E)) return &gemm_small_kernel<TA, TB, (E)>;
static GemmKernel pick_small(bool tA, bool tB, int e) {
  SMALL_CASE(false, false, 0)
  SMALL_CASE(false, false, E_BETA)
  SMALL_CASE(false, false, E_BIAS)
  SMALL_CASE(false, false, E_ROPE)
  SMALL_CASE(false, false, E_RESID)
  SMALL_CASE(false, false, E_BIAS | E_RESID)
  SMALL_CASE(false, false, E_BIAS | E_GELU)
  SMALL_CASE(false, false, E_BIAS | E_RELU)
  SMALL_CASE(false, false, E_SPLIT)
  SMALL_CASE(false, true, 0)
  SMALL_CASE(false, true, E_BETA)
  SMALL_CASE(false, true, E_DGELU)
  SMALL_CASE(false, true, E_DRELU)
  SMALL_CASE(false, true, E_SPLIT)
  SMALL_CASE(true, false, 0)
  SMALL_CASE(true, false, E_BETA)
  SMALL_CASE(true, false, E_SPLIT)
  SMALL_CASE(true, false, E_DBIAS)
  SMALL_CASE(true, false, E_SPLIT | E_DBIAS)
  SMALL_CASE(true, false, E_BETA | E_DBIAS)
  SMALL_CASE(true, true, 0)
  SMALL_CASE(true, true, E_BETA)
  SMALL_CASE(true, true, E_SPLIT)
  return nullptr;
}
#undef SMALL_CASE

// The 64 x 128 tile kernel: the d = 128-wide products of a block (norm backward, the MLP output
// with its residual, the attention output projection with the next norm).
static GemmKernel pick_m64(bool tA, bool tB, int e) {
  if (tA) return nullptr;
  if (tB) {
    if (e == E_NORMB) return &gemm_f32_m64_kernel<false, true, E_NORMB>;
    if (e == (E_NORMB | E_NBLAST)) return &gemm_f32_m64_kernel<false, true, E_NORMB | E_NBLAST>;
    if (e == (E_NORMB | E_NBPRE)) return &gemm_f32_m64_kernel<false, true, E_NORMB | E_NBPRE>;
    if (e == (E_NORMB | E_NBPRE | E_NBLAST)) return &gemm_f32_m64_kernel<false, true, E_NORMB | E_NBPRE | E_NBLAST>;
    if (e == 0) return &gemm_f32_m64_kernel<false, true, 0>;
    if (e == E_BETA) return &gemm_f32_m64_kernel<false, true, E_BETA>;
    return nullptr;
  }
  if (e == 0) return &gemm_f32_m64_kernel<false, false, 0>;
  if (e == (E_BIAS | E_RESID)) return &gemm_f32_m64_kernel<false, false, E_BIAS | E_RESID>;
  if (e == (E_RESID | E_NORM)) return &gemm_f32_m64_kernel<false, false, E_RESID | E_NORM>;
  if (e == (E_BIAS | E_RESID | E_NORM)) return &gemm_f32_m64_kernel<false, false, E_BIAS | E_RESID | E_NORM>;
  return nullptr;
}

static int num_cus();

// Rows per tile of an fp32 product on the 128-wide tiles with final epilogue e (after the
// split-K decision): 64 when the output is one tile wide, the 128-row tiles would give fewer
// than two workgroups per CU, K is not split and the 64-row kernel is instantiated for e
// (measured at 32768 rows: the norm-backward products 61 -> 56 us at K = 512 and 41 -> 36 us at
// K = 256; with 1024 or more tiles the 128-row tiles are 3-12% faster).
static int tile_rows(const GemmDesc& d, int e, int ksplit) {
  const long long tiles = (long long)((d.M + BM - 1) / BM) * ((d.N + BN - 1) / BN) * d.batch;
  if (d.bf16 || d.batch != 1 || d.N > BN || ksplit > 1) return BM;
  if (tiles >= 2LL * num_cus() && !(TALOS_NBPRE_M64 && (e & E_NBPRE) != 0)) return BM;
  return pick_m64(d.transA != 0, d.transB != 0, e) ? 64 : BM;
}

static int gemm_launch_one(const GemmDesc& d, hipStream_t stream);

// c[row][col] += sum_h p[row][h] u[row / seq][h][col] over four h, in the epilogue's order
__global__ void add_pre_kernel(int M, int N, int seq, const float* __restrict__ p, const float* __restrict__ u,
                               float* __restrict__ c) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)M * N) return;
  const long long row = i / N;
  const int col = (int)(i % N);
  float a = 0.f;
#pragma unroll
  for (int t = 0; t < 4; ++t) a = fmaf(p[row * 4 + t], u[((row / seq) * 4 + t) * N + col], a);
  c[i] += a;
}

// c[b * seq + last_row(b)][:] += add[b][:] for each sample b (rows of width n).
__global__ void add_last_rows_kernel(int nb, int seq, int n, const int32_t* __restrict__ lens,
                                     const float* __restrict__ add, float* __restrict__ c) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)nb * n) return;
  const int b = (int)(i / n), col = (int)(i % n);
  c[((long long)b * seq + last_row(lens, b, seq)) * n + col] += add[i];
}

bool gemm_normin_supported(const GemmDesc& d) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const int e = epi_flags(d) | E_NORMIN;
  return !d.bf16 && !d.transA && !d.transB && d.batch == 1 && d.ksplit <= 1 && d.K > 0 && d.K <= 512 && d.K % 4 == 0 &&
         (d.lda & 3) == 0 && a16(d.A) && a16(d.nin_gain) && a16(d.nin_out) && !use_small(d, num_cus()) &&
         tile_rows(d, e, 1) == BM && pick_kernel(false, false, e, false) != nullptr;
}

// Whether the RMSNorm backward of a product can run in its epilogue: 128x128 tiles holding the
// whole 128-wide row, fp32, one batch, float4 rows, and room for the per-tile partials.
static bool normb_fused(const GemmDesc& d) {
  auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  const int bm = tile_rows(d, epi_flags(d), 1);
  const int tiles_m = (d.M + bm - 1) / bm;
  return d.fuse_norm && d.N == BN && !d.bf16 && d.batch == 1 && !d.transA && d.transB && !use_small(d, num_cus()) &&
         d.beta == 0.f && !d.bias && !d.resid && d.act == GEMM_ACT_NONE && d.dact == GEMM_DACT_NONE &&
         d.rope_cols == 0 && !d.norm_out && !d.dbias && a16(d.normb_x) && a16(d.normb_dx) && a16(d.normb_gain) &&
         a16(d.normb_add) && a16(d.normb_add_last) && a16(d.normb_dy_last) && a16(d.normb_pre_p) && a16(d.normb_pre_u) && d.normb_ws &&
         d.normb_ws_bytes >= reduce_parts_workspace_bytes(tiles_m, d.N);
}

int gemm_splitk_batch_launch(int count, const SplitJob* jobs, hipStream_t stream) {
  TALOS_REQUIRE(count >= 0 && count <= kSplitJobsMax, TALOS_ERR_SHAPE, "split-K batch: %d jobs (at most %d)", count,
                kSplitJobsMax);
  SplitBatch sb{};
  sb.n = 0;
  sb.start[0] = 0;
  double moved = 0.0;
  for (int i = 0; i < count; ++i) {
    if (!jobs[i].part) continue;
    const long long RN = (long long)(jobs[i].M + (jobs[i].dbias ? 1 : 0)) * jobs[i].N;
    sb.j[sb.n] = jobs[i];
    sb.start[sb.n + 1] = sb.start[sb.n] + (int)((RN + 63) / 64);
    moved += 4.0 * (double)RN * (jobs[i].ksplit + 1);
    ++sb.n;
  }
  if (sb.n == 0) return TALOS_OK;
  ProfScope ps(stream, "gemm_splitk_reduce_batch", 0.0, moved);
  hipLaunchKernelGGL(gemm_splitk_reduce_batch, dim3(sb.start[sb.n]), dim3(256), 0, stream, sb);
  TALOS_LAUNCHED("gemm_splitk_reduce_batch");
  return TALOS_OK;
}

int gemm_launch(const GemmDesc& d, hipStream_t stream) {
  if (d.split_defer) d.split_defer->part = nullptr;  // (filled where the combination is held back)
  if (d.rd_D) {
    auto a16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    TALOS_REQUIRE(!d.transA && d.transB && epi_flags(d) == E_ROWDOT && d.batch == 1 && d.N % BN == 0 &&
                      (d.rd_w == 32 || d.rd_w == 64) && d.rd_seq > 0 && d.rd_heads > 0 &&
                      d.N == d.rd_w * d.rd_heads && d.M % d.rd_seq == 0 && d.ldc % 4 == 0 && d.rd_ldo % 4 == 0 &&
                      a16(d.C) && a16(d.rd_o),
                  TALOS_ERR_UNSUPPORTED,
                  "gemm: row dots need an NT product with a plain epilogue, N = rd_w * rd_heads a multiple of "
                  "128 (rd_w 32 or 64), 16-byte rows");
  }
  if (d.cmap_w) {
    const int e = epi_flags(d);
    TALOS_REQUIRE(d.cmap_w > 0 && d.cmap_w % 4 == 0 && d.cmap_pitch % 4 == 0 && d.cmap_off % 4 == 0 &&
                      d.cmap_off + d.cmap_w <= d.cmap_pitch && d.batch == 1 && !d.normb_dx &&
                      (e & ~(E_BETA | E_BIAS | E_ROPE | E_CMAP)) == 0,
                  TALOS_ERR_UNSUPPORTED,
                  "gemm: an output column map needs widths, pitch and offset in multiples of 4 and a plain, bias or "
                  "RoPE epilogue");
  }
  if (d.normb_dx) {
    if (d.normb_defer) d.normb_defer->cols = 0;  // (filled below where held back)
    if (!normb_fused(d)) {
      // the product into C, then the row-norm backward kernel
      TALOS_REQUIRE(d.C != nullptr && d.ldc == d.N, TALOS_ERR_UNSUPPORTED,
                    "gemm: a row-norm backward after the product needs C with ldc == N");
      GemmDesc g = d;
      g.normb_dx = nullptr;
      g.normb_pre_p = g.normb_pre_u = nullptr;
      if (int rc = gemm_launch(g, stream)) return rc;
      if (d.normb_pre_p) {
        const size_t n = (size_t)d.M * d.N;
        ProfScope ps(stream, "add_pre_kernel", 8.0 * n, 8.0 * n);
        hipLaunchKernelGGL(add_pre_kernel, dim3(ceil_div(n, 256)), dim3(256), 0, stream, d.M, d.N,
                           d.normb_seq > 0 ? d.normb_seq : 1, d.normb_pre_p, d.normb_pre_u, d.C);
        TALOS_LAUNCHED("add_pre_kernel");
      }
      if (d.normb_dy_last) {
        const int nb = d.M / (d.normb_seq > 0 ? d.normb_seq : 1);
        ProfScope ps(stream, "add_last_rows_kernel", (double)nb * d.N, 12.0 * nb * d.N);
        hipLaunchKernelGGL(add_last_rows_kernel, dim3(ceil_div((size_t)nb * d.N, 256)), dim3(256), 0, stream, nb,
                           d.normb_seq > 0 ? d.normb_seq : 1, d.N, d.normb_lens, d.normb_dy_last, d.C);
        TALOS_LAUNCHED("add_last_rows_kernel");
      }
      return rmsnorm_bwd_launch(d.M, d.N, d.normb_x, d.normb_gain, d.normb_rstd, d.C, 0.f, d.normb_dx,
                                d.normb_beta_dw, d.normb_dw, d.normb_ws, stream, d.normb_add, d.normb_add_last,
                                d.normb_seq, d.normb_lens);
    }
    GemmDesc g = d;
    g.ksplit = 1;
    if (int rc = gemm_launch_one(g, stream)) return rc;
    if (!d.normb_dw) return TALOS_OK;
    const int bm = tile_rows(d, epi_flags(d), 1);
    const int nparts = (d.M + bm - 1) / bm;
    if (d.normb_defer && nparts <= kPartsOnePass) {
      PartsJob& J = *d.normb_defer;
      J.cols = d.N;
      J.nparts = nparts;
      J.part = d.normb_ws;
      J.beta = d.normb_beta_dw;
      J.out = d.normb_dw;
      J.split = -1;
      J.out2 = nullptr;
      return TALOS_OK;
    }
    return reduce_parts_launch(d.N, nparts, d.normb_ws, d.normb_beta_dw, d.normb_dw, stream);
  }
  return gemm_launch_one(d, stream);
}

// The fixed-order f64 combination of a split-K product's partials (and the bias epilogue).
static int split_reduce(const GemmDesc& d, const GemmArgs& a, int e, hipStream_t stream) {
  const long long RN = (long long)(d.M + (d.dbias ? 1 : 0)) * d.N;
  if (d.split_defer && (e & (E_BETA | E_BIAS)) == 0 && d.batch == 1) {
    SplitJob& J = *d.split_defer;
    J.part = a.part;
    J.ksplit = a.ksplit;
    J.M = d.M;
    J.N = d.N;
    J.C = d.C;
    J.ldc = d.ldc;
    J.alpha = a.alpha;
    J.dbias = d.dbias;
    J.beta_dbias = d.beta_dbias;
    return TALOS_OK;
  }
  dim3 rg((unsigned)((RN + 63) / 64), d.batch);
  const int re = e & (E_BETA | E_BIAS);
  char rname[48];
  snprintf(rname, sizeof(rname), "gemm_splitk_reduce<%d>", re);
  ProfScope ps(stream, rname, 0.0, 4.0 * (double)RN * d.batch * (a.ksplit + 1 + (d.beta != 0.f)));
  if (re == 0) hipLaunchKernelGGL(gemm_splitk_reduce<0>, rg, dim3(256), 0, stream, a);
  else if (re == E_BETA) hipLaunchKernelGGL(gemm_splitk_reduce<E_BETA>, rg, dim3(256), 0, stream, a);
  else if (re == E_BIAS) hipLaunchKernelGGL(gemm_splitk_reduce<E_BIAS>, rg, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL(gemm_splitk_reduce<E_BETA | E_BIAS>, rg, dim3(256), 0, stream, a);
  TALOS_LAUNCHED("gemm_splitk_reduce");
  return TALOS_OK;
}

static int gemm_launch_one(const GemmDesc& d, hipStream_t stream) {
  if (d.norm_out && (!d.fuse_norm || d.N != BN || d.bf16 || d.batch != 1 || use_small(d, num_cus()))) {
    // the fused row norm needs the whole 128-wide row in one 128x128 tile: otherwise the product,
    // then the separate row-norm kernel
    TALOS_REQUIRE(d.ldc == d.N && d.ldn == d.N, TALOS_ERR_UNSUPPORTED,
                  "gemm: a row norm after the product needs ldc == ldn == N");
    GemmDesc g = d;
    g.norm_out = nullptr;
    if (int rc = gemm_launch(g, stream)) return rc;
    return rmsnorm_fwd_launch(d.M, d.N, d.norm_eps, d.C, d.norm_gain, d.norm_out, d.norm_rstd, stream);
  }
  GemmArgs a = to_args(d);
  if (d.M == 0 || d.N == 0 || d.batch == 0) return TALOS_OK;
  const bool small = use_small(d, num_cus());
  if (d.K == 0) {
    // C = beta*C (+ epilogue): run the kernel with an empty K loop.
    a.ksplit = 1;
    a.kper = 0;
  }
  const int e = epi_flags(d);
  const bool split = a.ksplit > 1;
  const int ke = split ? (E_SPLIT | (e & E_DBIAS)) : e;
  const int bm = small ? SBM : tile_rows(d, ke, a.ksplit);
  const unsigned tiles = small ? ceil_div(d.M, SBM) * ceil_div(d.N, SBN) : ceil_div(d.M, bm) * ceil_div(d.N, BN);
  a.nblocks = (int)(tiles * (unsigned)d.batch * (unsigned)a.ksplit);
  dim3 grid((unsigned)((a.nblocks + 7) / 8 * 8));
  GemmKernel kern = small      ? pick_small(d.transA != 0, d.transB != 0, ke)
                    : bm == 64 ? pick_m64(d.transA != 0, d.transB != 0, ke)
                               : pick_kernel(d.transA != 0, d.transB != 0, ke, d.bf16);
  if (kern == nullptr) {
    set_error("gemm: epilogue combination 0x%x is not instantiated for transA=%d transB=%d%s", e, d.transA, d.transB,
              d.bf16 ? " (bf16)" : "");
    return TALOS_ERR_UNSUPPORTED;
  }
  // profiler name = the kernel symbol's template arguments as rocprofv3 prints them
  char name[64];
  if (small)
    snprintf(name, sizeof(name), "gemm_small_kernel<%s, %s, %d>", d.transA ? "true" : "false",
             d.transB ? "true" : "false", ke);
  else if (bm == 64)
    snprintf(name, sizeof(name), "gemm_f32_m64_kernel<%s, %s, %d>", d.transA ? "true" : "false",
             d.transB ? "true" : "false", ke);
  else
    snprintf(name, sizeof(name), "gemm_f32_kernel<%s, %s, %d, %s>", d.transA ? "true" : "false",
             d.transB ? "true" : "false", ke, d.bf16 ? "true" : "false");
  {
    // algorithmic work: 2MNK flops; A, B read once, C written once (+ C / residual / aux reads)
    const double MN = (double)d.M * d.N;
    double bytes = 4.0 * ((double)d.M * d.K + (double)d.K * d.N + MN);
    if (!split) {
      if (d.beta != 0.f) bytes += 4.0 * MN;
      if (d.resid) bytes += 4.0 * MN;
      if (d.aux) bytes += 4.0 * MN;
      if (d.norm_out) bytes += 4.0 * (MN + d.M + d.N);
      // E_NORMB: x (and the addend) read, dx written instead of C, rstd and gain read
      if (d.normb_dx) bytes += 4.0 * (MN * (1 + (d.normb_add != nullptr)) + d.M + d.N) + 8.0 * (d.M / bm + 1) * d.N;
      if (d.bias) bytes += 4.0 * d.N;
    }
    ProfScope ps(stream, name, 2.0 * MN * d.K * d.batch, bytes * d.batch);
    hipLaunchKernelGGL(kern, grid, dim3(NT), 0, stream, a);
    TALOS_LAUNCHED(small ? "gemm_small_kernel" : bm == 64 ? "gemm_f32_m64_kernel" : "gemm_f32_kernel");
  }
  if (split) return split_reduce(d, a, e, stream);
  return TALOS_OK;
}

// Two products launched as one grid (gemm_f32_pair_kernel) when both are fp32 split-K weight
// gradients (transA, op(B) plain, one batch) on 128-row tiles with the same epilogue (with or
// without the fused bias gradient), each with its own workspace; otherwise one after the other.
// Each product's partials are then combined by its own reduction, as gemm_launch does.
bool gemm_pairable(const GemmDesc& d0, const GemmDesc& d1) {
  const GemmArgs a0 = to_args(d0), a1 = to_args(d1);
  const int e0 = epi_flags(d0), e1 = epi_flags(d1);
  // (a product planned for 64x64 tiles runs on the 128x128 body here: the split-K partial layout
  // does not depend on the tile; the two products' splits must be of similar length, or the
  // longer one's workgroups run on alone)
  auto pairable = [&](const GemmDesc& d, const GemmArgs& a, int e) {
    return d.transA && !d.transB && !d.bf16 && d.batch == 1 && d.M > 0 && d.N > 0 && d.K > 0 && a.ksplit > 1 &&
           (e & ~E_DBIAS) == 0 && d.workspace != nullptr;
  };
  const int klo = std::min(a0.kper, a1.kper), khi = std::max(a0.kper, a1.kper);
  return pairable(d0, a0, e0) && pairable(d1, a1, e1) && e0 == e1 && d0.workspace != d1.workspace && 2 * khi <= 3 * klo;
}

int gemm_launch_pair(const GemmDesc& d0, const GemmDesc& d1, hipStream_t stream) {
  if (!gemm_pairable(d0, d1)) {
    if (int rc = gemm_launch(d0, stream)) return rc;
    return gemm_launch(d1, stream);
  }
  GemmArgs a0 = to_args(d0), a1 = to_args(d1);
  const int e0 = epi_flags(d0), e1 = epi_flags(d1);
  const int ke = E_SPLIT | (e0 & E_DBIAS);
  a0.nblocks = (int)(ceil_div(d0.M, BM) * ceil_div(d0.N, BN) * (unsigned)a0.ksplit);
  a1.nblocks = (int)(ceil_div(d1.M, BM) * ceil_div(d1.N, BN) * (unsigned)a1.ksplit);
  dim3 grid((unsigned)((a0.nblocks + a1.nblocks + 7) / 8 * 8));
  {
    const double f = 2.0 * ((double)d0.M * d0.N * d0.K + (double)d1.M * d1.N * d1.K);
    const double bytes = 4.0 * ((double)d0.M * d0.K + (double)d0.K * d0.N + (double)d0.M * d0.N +
                                (double)d1.M * d1.K + (double)d1.K * d1.N + (double)d1.M * d1.N);
    char name[64];
    snprintf(name, sizeof(name), "gemm_f32_pair_kernel<true, false, %d>", ke);
    ProfScope ps(stream, name, f, bytes);
    void (*kern)(GemmArgs, GemmArgs) = ke == E_SPLIT ? &gemm_f32_pair_kernel<true, false, E_SPLIT>
                                                     : &gemm_f32_pair_kernel<true, false, E_SPLIT | E_DBIAS>;
    hipLaunchKernelGGL(kern, grid, dim3(NT), 0, stream, a0, a1);
    TALOS_LAUNCHED("gemm_f32_pair_kernel");
  }
  if (int rc = split_reduce(d0, a0, e0, stream)) return rc;
  return split_reduce(d1, a1, e1, stream);
}

static int num_cus() {
  static int n = -1;
  if (n < 0) {
    hipDeviceProp_t prop;
    n = (hipGetDeviceProperties(&prop, 0) == hipSuccess) ? prop.multiProcessorCount : 256;
  }
  return n;
}

// Host validation shared by the kernel-level GEMM entry points.
static int check_gemm(const char* fn, int transA, int transB, int M, int N, int K, const void* A, long long lda,
                      const void* B, long long ldb, float beta, const void* C, long long ldc, int batch) {
  TALOS_REQUIRE(A && B && C, TALOS_ERR_NULL, "%s: null matrix pointer", fn);
  TALOS_REQUIRE(M >= 0 && N >= 0 && K >= 0 && batch >= 0, TALOS_ERR_SHAPE, "%s: negative size (M=%d N=%d K=%d batch=%d)",
                fn, M, N, K, batch);
  TALOS_REQUIRE((transA == 0 || transA == 1) && (transB == 0 || transB == 1), TALOS_ERR_DTYPE,
                "%s: trans flags must be 0 or 1", fn);
  TALOS_REQUIRE(lda >= (transA ? M : K) && lda >= 1, TALOS_ERR_SHAPE, "%s: lda=%lld too small for %s A", fn, lda,
                transA ? "transposed" : "plain");
  TALOS_REQUIRE(ldb >= (transB ? K : N) && ldb >= 1, TALOS_ERR_SHAPE, "%s: ldb=%lld too small for %s B", fn, ldb,
                transB ? "transposed" : "plain");
  TALOS_REQUIRE(ldc >= N && ldc >= 1, TALOS_ERR_SHAPE, "%s: ldc=%lld < N=%d", fn, ldc, N);
  TALOS_REQUIRE(beta == 0.f || beta == 1.f, TALOS_ERR_UNSUPPORTED, "%s: beta must be 0 or 1 (got %g)", fn, beta);
  return TALOS_OK;
}

// Split-K partials of a kernel-level product: with a workspace bound on this thread the split
// count shrinks until the partials fit it (down to no split), so the call allocates nothing;
// without one the partials are allocated on the stream for the call.
static int run_gemm(GemmDesc& d, hipStream_t stream) {
  size_t ws = gemm_plan_split(d, num_cus());
  const size_t bound = bound_workspace_bytes();
  if (ws && bound && ws > bound) {
    note_workspace_need(ws);
    const size_t per_split = (size_t)(d.M + (d.dbias ? 1 : 0)) * d.N * d.batch * sizeof(float);
    d.ksplit = (int)std::max<size_t>(1, bound / per_split);
    ws = d.ksplit > 1 ? gemm_plan_split(d, num_cus()) : 0;
    if (ws > bound) {  // the rounding of K to whole chunks can add a split
      d.ksplit = 1;
      ws = 0;
    }
  }
  EntryScratch scratch;
  if (int rc = scratch.acquire(ws, stream)) return rc;
  d.workspace = static_cast<float*>(scratch.ptr);
  const int rc = gemm_launch(d, stream);
  const int rel = scratch.release();
  return rc ? rc : rel;
}

}  // namespace talos

using namespace talos;

extern "C" {

int talos_gemm_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda, const float* B,
                   int ldb, float beta, float* C, int ldc, talos_stream_t stream) {
  int rc = check_gemm(__func__, transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc, 1);
  if (rc) return rc;
  TALOS_DEVICE();
  GemmDesc d;
  d.transA = transA;
  d.transB = transB;
  d.M = M;
  d.N = N;
  d.K = K;
  d.A = A;
  d.lda = lda;
  d.B = B;
  d.ldb = ldb;
  d.C = C;
  d.ldc = ldc;
  d.alpha = alpha;
  d.beta = beta;
  d.ksplit = 0;
  return entry_done(run_gemm(d, as_stream(stream)), as_stream(stream));
}

int talos_gemm_bf16acc_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                           const float* B, int ldb, float beta, float* C, int ldc, talos_stream_t stream) {
  int rc = check_gemm(__func__, transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc, 1);
  if (rc) return rc;
  TALOS_DEVICE();
  GemmDesc d;
  d.transA = transA;
  d.transB = transB;
  d.M = M;
  d.N = N;
  d.K = K;
  d.A = A;
  d.lda = lda;
  d.B = B;
  d.ldb = ldb;
  d.C = C;
  d.ldc = ldc;
  d.alpha = alpha;
  d.beta = beta;
  d.bf16 = true;
  d.ksplit = 0;
  return entry_done(run_gemm(d, as_stream(stream)), as_stream(stream));
}

int talos_gemm_batched_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                           long long sA, const float* B, int ldb, long long sB, float beta, float* C, int ldc,
                           long long sC, int batch, talos_stream_t stream) {
  int rc = check_gemm(__func__, transA, transB, M, N, K, A, lda, B, ldb, beta, C, ldc, batch);
  if (rc) return rc;
  TALOS_REQUIRE(sA >= 0 && sB >= 0 && sC >= 0, TALOS_ERR_SHAPE, "%s: negative batch stride", __func__);
  TALOS_DEVICE();
  GemmDesc d;
  d.transA = transA;
  d.transB = transB;
  d.M = M;
  d.N = N;
  d.K = K;
  d.batch = batch;
  d.A = A;
  d.lda = lda;
  d.sA = sA;
  d.B = B;
  d.ldb = ldb;
  d.sB = sB;
  d.C = C;
  d.ldc = ldc;
  d.sC = sC;
  d.alpha = alpha;
  d.beta = beta;
  d.ksplit = 0;
  return entry_done(run_gemm(d, as_stream(stream)), as_stream(stream));
}

}  // extern "C"
