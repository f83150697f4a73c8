// gemm.hpp -- internal interface of the fp32 MFMA GEMM (gemm.hip) used by the kernel-level
// entry points and by the fused block / policy plans.
#pragma once

#include "common.hpp"
#include "rowops.hpp"

namespace talos {

enum GemmAct { GEMM_ACT_NONE = 0, GEMM_ACT_GELU = 1, GEMM_ACT_RELU = 2 };
// Epilogue of the backward of an activation: C = acc * aux for GELU (aux holds gelu' saved by
// the forward), C = acc where aux > 0 for ReLU (aux holds the pre-activation).
enum GemmDAct { GEMM_DACT_NONE = 0, GEMM_DACT_GELU = 1, GEMM_DACT_RELU = 2 };

// C[b][M,N] = alpha * op(A[b]) . op(B[b]) + beta * C[b]  (+ bias[N]) (+ resid[M,N]),
// then optionally act(.) storing to aux what its backward needs (gelu'(v) for GELU, the
// pre-activation v for ReLU), or that saved value applied (GEMM_DACT_*); RoPE on columns
// [0, rope_cols) with position row % rope_seq.
// Row-major storage; op(A) is [M,K]: A[m*lda + k] (transA = 0) or A[k*lda + m] (transA = 1);
// op(B) is [K,N]: B[k*ldb + n] (transB = 0) or B[n*ldb + k] (transB = 1).
// A split-K product's partials' combination held back (GemmDesc::split_defer). part null: none.
struct SplitJob {
  const float* part = nullptr;
  int ksplit = 0, M = 0, N = 0;
  float* C = nullptr;
  long long ldc = 0;
  float alpha = 1.f;
  float* dbias = nullptr;
  float beta_dbias = 0.f;
};
constexpr int kSplitJobsMax = 8;

struct GemmDesc {
  int transA = 0, transB = 0;
  int M = 0, N = 0, K = 0;
  int batch = 1;
  const float* A = nullptr;
  long long lda = 0, sA = 0;
  const float* B = nullptr;
  long long ldb = 0, sB = 0;
  float* C = nullptr;
  long long ldc = 0, sC = 0;
  // bf16-in products (bf16 = true): optional bf16 copies of A / B (same layout, leading dimensions
  // and batch strides, each value rounded to nearest even), which the staging reads instead of
  // loading and rounding the fp32 operand; and C16, a bf16 copy of C (leading dimension ldc) that
  // the epilogue also writes (not with a split K, the row norm or its backward, or an activation's
  // saved input).
  const uint16_t* A16 = nullptr;
  const uint16_t* B16 = nullptr;
  uint16_t* C16 = nullptr;
  float alpha = 1.f, beta = 0.f;
  const float* bias = nullptr;
  const float* resid = nullptr;
  long long ldr = 0;
  int act = GEMM_ACT_NONE;
  int dact = GEMM_DACT_NONE;
  float* aux = nullptr;  // act: output of what the backward needs; dact: that input
  long long ldaux = 0;
  // RoPE epilogue (interleaved pairs (2i, 2i+1) inside each rot_dim-wide head)
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int rope_cols = 0, rope_dim = 0, rope_seq = 1;
  // Output column map (cmap_w > 0): product column c is stored at column
  // (c / cmap_w) * cmap_pitch + cmap_off + c % cmap_w of C (ldc wide), e.g. a head's content or
  // rope part into a head-interleaved row; the epilogue's own arithmetic (RoPE) sees c. cmap_w a
  // multiple of 4; not with a split K (the library keeps it unsplit), the row norms or activations.
  int cmap_w = 0, cmap_pitch = 0, cmap_off = 0;
  // Row dots by head (rd_D given; transA = 0, transB = 1, a plain epilogue, N % 128 == 0, rd_w
  // 32 or 64): rd_D[((row / rd_seq) * rd_heads + c / rd_w) * rd_seq + row % rd_seq] = sum over
  // the rd_w columns c of that head of C[row][c] * rd_o[row][c] (ldc and rd_ldo multiples of 4,
  // 16-byte aligned), summed as the attention backward's D = rowsum(dO . O) would be when this
  // product forms dO: that kernel's lanes and order, so the values are the same.
  const float* rd_o = nullptr;
  long long rd_ldo = 0;
  float* rd_D = nullptr;
  int rd_w = 0, rd_seq = 1, rd_heads = 1;
  // Split-K: the K range is cut into ksplit parts of kper (multiple of 32) whose fp32 partial
  // tiles are summed in f64 by a second kernel. ksplit = 0 lets the library choose.
  int ksplit = 1;
  float* workspace = nullptr;  // >= gemm_plan_split(desc) bytes when ksplit > 1
  // Fused bias gradient (transA = 1, transB = 0 only): dbias[n] = beta_dbias * dbias[n] +
  // sum_k B[k][n], the column sums of op(B) accumulated from the panels already in LDS.
  float* dbias = nullptr;
  float beta_dbias = 0.f;
  // Row norm after the epilogue (RMSNorm, rmsnorm_fwd_launch's arithmetic): norm_out[row] =
  // C[row] * rstd * norm_gain with rstd = 1 / sqrt(mean(C[row]^2) + norm_eps), stored to
  // norm_rstd[row]. Fused into the epilogue when N = 128 (one tile holds the row); other shapes
  // run the row-norm kernel after the product (ldc = ldn = N).
  const float* norm_gain = nullptr;
  float* norm_out = nullptr;
  long long ldn = 0;
  float* norm_rstd = nullptr;
  float norm_eps = 0.f;
  // RMSNorm of A's rows before the product (A plain, K = the norm's width): the product is
  // rmsnorm(A) * nin_gain times op(B), formed as rstd[row] * (A . (nin_gain (x) B)) with rstd =
  // 1 / sqrt(mean(A[row]^2) + nin_eps) from the A rows the tile loads anyway; the normalised rows
  // go to nin_out (row stride K) and rstd to nin_rstd. Only where gemm_normin_supported holds.
  const float* nin_gain = nullptr;
  float* nin_out = nullptr;
  float* nin_rstd = nullptr;
  float nin_eps = 0.f;
  // RMSNorm backward after the product, C = dL/d(the norm's output) (rmsnorm_bwd_launch's
  // arithmetic): normb_dx = rstd * (C * gain - x_hat * mean(C * gain * x_hat)) + normb_add (+
  // normb_add_last[b] on the last row of each sample b, rows of normb_seq; normb_dy_last[b] is
  // added to C on those rows before anything else), x_hat = x * rstd, and
  // normb_dw = normb_beta_dw * normb_dw + the column sums of C * x_hat, through f64 partials in
  // normb_ws. Fused into the epilogue when N = 128 (one tile holds the row; C is not written);
  // other shapes write C (ldc = N) and run the row-norm backward kernel after the product.
  const float* normb_x = nullptr;
  const float* normb_rstd = nullptr;
  const float* normb_gain = nullptr;
  const float* normb_add = nullptr;
  const float* normb_add_last = nullptr;
  const float* normb_dy_last = nullptr;  // added to C on the last row of each sample first
  // [M][4] and [M / normb_seq][4][N]: C[row] += sum_h normb_pre_p[row][h] normb_pre_u[sample][h]
  // on every row first (h = 0..3, fmaf from zero in h order)
  const float* normb_pre_p = nullptr;
  const float* normb_pre_u = nullptr;
  int normb_seq = 1;
  const int32_t* normb_lens = nullptr;
  float* normb_dx = nullptr;
  float* normb_dw = nullptr;
  float normb_beta_dw = 0.f;
  double* normb_ws = nullptr;
  size_t normb_ws_bytes = 0;
  // Where the gain gradient's combination would be one reduce_parts pass after the fused
  // product: held back into *normb_defer instead of launched (for reduce_parts_batch_launch;
  // normb_ws must then stay untouched until that runs). Otherwise normb_defer->cols is set to 0
  // and it runs here.
  PartsJob* normb_defer = nullptr;
  // A split-K product whose partials' combination is plain (beta 0, no bias; the fused bias
  // gradient allowed), one batch: that combination held back into *split_defer instead of
  // launched, for gemm_splitk_batch_launch (the workspace must stay untouched until then).
  // Otherwise split_defer->part is set to null and it runs here.
  SplitJob* split_defer = nullptr;
  // bf16-in / fp32-accumulate: operands are rounded to bf16 (nearest even) as they are staged
  // into LDS and multiplied with v_mfma_f32_32x32x16_bf16; HBM layout and outputs stay fp32.
  bool bf16 = false;
  // false: the row norm (norm_out) and the row-norm backward (normb_dx) always run as the separate
  // row kernels after the product, never in its epilogue (the cross-check of the fused epilogues)
  bool fuse_norm = true;
};

// Whether a product can normalise its A rows itself (nin_*): fp32, A plain with K <= 512 and a
// multiple of 4 and 16-byte rows, 128-row tiles, one batch, no split, an instantiated epilogue.
bool gemm_normin_supported(const GemmDesc& d);

// Fills in ksplit (when 0) and returns the workspace bytes the descriptor needs.
size_t gemm_plan_split(GemmDesc& d, int num_cu);
// Enqueues the GEMM. Validation of shapes and pointers is the caller's job.
int gemm_launch(const GemmDesc& d, hipStream_t stream);
// Up to kSplitJobsMax held-back split-K combinations in one launch, each summed as the
// product's own combination would be (the same workgroups' arithmetic and order: the same
// results); their outputs must be distinct.
int gemm_splitk_batch_launch(int count, const SplitJob* jobs, hipStream_t stream);
// Two products in one launch where both are split-K weight gradients of one shape class (each
// with its own workspace); otherwise gemm_launch on each.
int gemm_launch_pair(const GemmDesc& d0, const GemmDesc& d1, hipStream_t stream);
// Whether gemm_launch_pair runs the two as one grid (split-K weight gradients of one epilogue
// with splits within 1.5x of each other in length).
bool gemm_pairable(const GemmDesc& d0, const GemmDesc& d1);

}  // namespace talos
