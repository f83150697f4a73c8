// rowops.hpp -- internal launchers of the row / element-wise kernels (rowops.hip) shared with
// the fused plans.
#pragma once

#include <vector>

#include "common.hpp"

namespace talos {

int fill_zero(void* dst, size_t bytes, hipStream_t s);

size_t colsum_workspace_bytes(int rows, int cols);
int colsum_launch(int rows, int cols, const float* dy, long long ld, float beta, float* out, double* ws,
                  hipStream_t s);

size_t rmsnorm_bwd_workspace_bytes(int rows, int dim);
// Bytes of the workspace reduce_parts_launch needs for nparts partial rows of cols doubles, and
// the launch: out = beta * out + the fixed-order f64 sum of the partial rows (columns from split
// on into out2 instead, when out2 is given).
size_t reduce_parts_workspace_bytes(int nparts, int cols);
// A reduce_parts_launch held back to run in a batch (one pass: nparts <= 4096): the same
// arguments. cols == 0: none.
struct PartsJob {
  int cols = 0, nparts = 0;
  const double* part = nullptr;
  float beta = 0.f;
  float* out = nullptr;
  int split = -1;
  float* out2 = nullptr;
};
constexpr int kPartsJobsMax = 8;
constexpr int kPartsOnePass = 4096;  // partial rows one reduce_parts pass takes
// Up to kPartsJobsMax held-back reductions in one launch, each summed as reduce_parts_launch
// would (the same workgroups' arithmetic and order: the same results); their outputs must be
// distinct.
int reduce_parts_batch_launch(int count, const PartsJob* jobs, hipStream_t s);
int reduce_parts_launch(int cols, int nparts, double* part, float beta, float* out, hipStream_t s, int split = -1,
                        float* out2 = nullptr);
// y16 (optional): also y's bf16 copy (nearest even, as cvt_bf16_launch rounds), same layout
int rmsnorm_fwd_launch(int rows, int dim, float eps, const float* x, const float* w, float* y, float* rstd,
                       hipStream_t s, uint16_t* y16 = nullptr);
// bf16 copies (rounded to nearest even, the GEMM staging's conversion) of count <= 8 fp32 tensors
// of n[i] elements in one launch
int cvt_bf16_launch(int count, const float* const* src, uint16_t* const* dst, const long long* n, hipStream_t s);
// dx = (dres ? dres : beta_dx * dx) + d rmsnorm / dx . dy; dres (the residual branch's gradient)
// may equal dx. dres_last ([rows / seq, dim]) adds a gradient that is non-zero on the last token
// of each sample only: row b * seq + last_row(lens, b, seq) receives dres_last[b].
int rmsnorm_bwd_launch(int rows, int dim, const float* x, const float* w, const float* rstd, const float* dy,
                       float beta_dx, float* dx, float beta_dw, float* dw, double* ws, hipStream_t s,
                       const float* dres = nullptr, const float* dres_last = nullptr, int seq = 1,
                       const int32_t* lens = nullptr);

// out[r] = [a[r] | b[r]]; split: da[r] (+)= g[r][:ca], db[r] (+)= g[r][ca:]
int concat_launch(size_t rows, int ca, int cb, const float* a, const float* b, float* out, hipStream_t s);
int split_launch(size_t rows, int ca, int cb, const float* g, float* da, float* db, bool accumulate, hipStream_t s);

void rope_table_host(int max_len, int dim, double base, std::vector<float>& c, std::vector<float>& s);
int rope_table_device(int need_len, int dim, float base, const float** cosv, const float** sinv);
int rope_launch(int n_seq, int seq, int heads, int dim, int start_pos, const float* cosv, const float* sinv,
                const float* x, float beta, float* y, bool backward, hipStream_t s);

}  // namespace talos
