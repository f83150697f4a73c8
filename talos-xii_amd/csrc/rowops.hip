// rowops.hip -- HBM-bound row and element-wise kernels of the autograd tape:
// RMSNorm (src/nn.rs:182-296), softmax (src/transformer.rs:1074-1121), RoPE
// (src/transformer.rs:219-337), the Linear bias gradient (src/autograd.rs:530-544) and the
// element-wise / layout ops (src/autograd.rs:356-792, 1606-1862; src/transformer.rs:1123-1183).
//
// Row kernels give each row to one wave64: a lane holds dim/64 consecutive elements read with
// 16-byte loads, row statistics are wave shuffles (no LDS, no block barriers), and per-feature
// reductions over rows (RMSNorm dgain, bias grads) write one f64 partial per workgroup that a
// second pass sums in f64.
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "rowops.hpp"

namespace talos {

// ---------------------------------------------------------------------------
// Fill / copy
// ---------------------------------------------------------------------------
__global__ void fill_zero_kernel(uint32_t* __restrict__ p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}
__global__ void fill_zero_bytes_kernel(uint8_t* __restrict__ p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

static unsigned grid_for(size_t n, unsigned block = 256, unsigned cap = 65536) {
  size_t g = (n + block - 1) / block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (unsigned)g;
}

int fill_zero(void* dst, size_t bytes, hipStream_t s) {
  if (bytes == 0) return TALOS_OK;
  if ((reinterpret_cast<uintptr_t>(dst) & 3) == 0 && bytes % 4 == 0) {
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(bytes / 4)), dim3(256), 0, s, (uint32_t*)dst, bytes / 4);
  } else {
    hipLaunchKernelGGL(fill_zero_bytes_kernel, dim3(grid_for(bytes)), dim3(256), 0, s, (uint8_t*)dst, bytes);
  }
  TALOS_LAUNCHED("fill_zero");
  return TALOS_OK;
}

// ---------------------------------------------------------------------------
// Column sums (bias gradient): db[c] = beta*db[c] + sum_r dy[r, c]
// ---------------------------------------------------------------------------
// Row chunks: at most kMaxParts partials per column, each over >= 64 rows.
constexpr int kMaxParts = 256;

static int colsum_parts(int rows) {
  int p = (rows + 63) / 64;
  return p < 1 ? 1 : (p > kMaxParts ? kMaxParts : p);
}

// Workgroup (x = 64-column group, y = row chunk): lane = column, the 4 waves stride over the
// chunk's rows (each row read is one 256-byte segment), f64 accumulation, LDS combine.
__global__ __launch_bounds__(256) void colsum_partial_kernel(int rows, int cols, const float* __restrict__ dy,
                                                             long long ld, int nparts, double* __restrict__ part) {
  __shared__ double red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int per = (rows + nparts - 1) / nparts;
  const int r0 = blockIdx.y * per, r1 = min(rows, r0 + per);
  double s0 = 0.0, s1 = 0.0;
  if (c < cols) {
    int r = r0 + w;
    for (; r + 4 < r1; r += 8) {
      s0 += (double)dy[(long long)r * ld + c];
      s1 += (double)dy[(long long)(r + 4) * ld + c];
    }
    if (r < r1) s0 += (double)dy[(long long)r * ld + c];
  }
  red[w][lane] = s0 + s1;
  __syncthreads();
  if (w == 0 && c < cols) part[(long long)blockIdx.y * cols + c] = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
}

// out[c] = beta*out[c] + sum_p part[p][c] in one pass: a workgroup takes 16 columns with 16
// waves; lane (column lane % 16, q = lane / 16) of wave w adds partials p = 4w + q + 64i in i
// order with eight loads in flight, so a wave reads four 128-byte row pieces per load; the 64
// sums of a column are then added in a fixed order.
constexpr int kOnePassParts = kPartsOnePass;
// Columns from split on go to out2[c - split] (two gradients reduced in one launch). blk: the
// workgroup's 16-column group.
__device__ __forceinline__ void reduce_parts_cols(int cols, int nparts, const double* __restrict__ part, float beta,
                                                  float* __restrict__ out, int split, float* __restrict__ out2,
                                                  int blk) {
  __shared__ double red[64][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int cl = lane & 15, q = lane >> 4;
  const int c = blk * 16 + cl;
  double acc = 0.0;
  if (c < cols) {
    const long long step = 64LL * cols;
    int p = 4 * w + q;
    for (; p + 7 * 64 < nparts; p += 8 * 64) {
      const double* r = part + (long long)p * cols + c;
      double a[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = r[u * step];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += a[u];
    }
    for (; p < nparts; p += 64) acc += part[(long long)p * cols + c];
  }
  red[4 * w + q][cl] = acc;
  __syncthreads();
  // 64 threads add 16 of a column's 64 sums each, then 16 threads the four, in a fixed order
  __shared__ double red4[4][16];
  if (threadIdx.x < 64) {
    const int col = threadIdx.x & 15, quarter = threadIdx.x >> 4;
    double t = 0.0;
#pragma unroll
    for (int j = 0; j < 16; ++j) t += red[16 * quarter + j][col];
    red4[quarter][col] = t;
  }
  __syncthreads();
  if (threadIdx.x < 16 && c < cols) {
    const double t = (red4[0][cl] + red4[1][cl]) + (red4[2][cl] + red4[3][cl]);
    float* o = c < split ? out + c : out2 + (c - split);
    *o = (float)(t + (beta != 0.f ? (double)*o : 0.0));
  }
}
__global__ __launch_bounds__(1024) void reduce_parts_kernel(int cols, int nparts, const double* __restrict__ part,
                                                            float beta, float* __restrict__ out, int split,
                                                            float* __restrict__ out2) {
  reduce_parts_cols(cols, nparts, part, beta, out, split, out2, blockIdx.x);
}
// Held-back reductions in one launch: job k takes workgroups [start[k], start[k + 1]).
struct PartsBatch {
  PartsJob j[kPartsJobsMax];
  int start[kPartsJobsMax + 1];
  int n;
};
__global__ __launch_bounds__(1024) void reduce_parts_batch_kernel(PartsBatch b) {
  int k = 0;
  while (k + 1 < b.n && (int)blockIdx.x >= b.start[k + 1]) ++k;  // uniform
  const PartsJob& J = b.j[k];
  reduce_parts_cols(J.cols, J.nparts, J.part, J.beta, J.out, J.split, J.out2, (int)blockIdx.x - b.start[k]);
}

// First level for many partials: workgroup (x = 64-column group, y = group of kGroupParts
// partials) sums its group in a fixed order into part2[y][c], so the final pass reads at most
// nparts / kGroupParts rows instead of one workgroup per 64 columns reading all of them.
constexpr int kGroupParts = 32;
__global__ __launch_bounds__(256) void group_parts_kernel(int cols, int nparts, const double* __restrict__ part,
                                                          double* __restrict__ part2) {
  __shared__ double red[4][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  const int p0 = blockIdx.y * kGroupParts, p1 = min(nparts, p0 + kGroupParts);
  double acc = 0.0;
  if (c < cols)
    for (int p = p0 + w; p < p1; p += 4) acc += part[(long long)p * cols + c];
  red[w][lane] = acc;
  __syncthreads();
  if (w == 0 && c < cols)
    part2[(long long)blockIdx.y * cols + c] = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
}

static int grouped_parts(int nparts) { return nparts > kOnePassParts ? (nparts + kGroupParts - 1) / kGroupParts : 0; }

// Workspace rows (of cols doubles) a reduction over nparts partials needs: the partials and the
// first level's group sums after them.
static size_t parts_rows(int nparts) { return (size_t)nparts + grouped_parts(nparts); }

int reduce_parts_launch(int cols, int nparts, double* part, float beta, float* out, hipStream_t s, int split,
                        float* out2) {
  if (split < 0 || split > cols || out2 == nullptr) split = cols;
  const int groups = grouped_parts(nparts);
  if (groups > 0) {
    // part is the start of a workspace of parts_rows(nparts) rows (every caller sizes it so)
    double* part2 = part + (size_t)nparts * cols;
    ProfScope ps(s, "group_parts_kernel", (double)nparts * cols, 8.0 * (nparts + groups) * cols);
    hipLaunchKernelGGL(group_parts_kernel, dim3(ceil_div(cols, 64), groups), dim3(256), 0, s, cols, nparts, part,
                       part2);
    TALOS_LAUNCHED("group_parts_kernel");
    part = part2;
    nparts = groups;
  }
  ProfScope ps(s, "reduce_parts_kernel", (double)nparts * cols, 8.0 * nparts * cols + 4.0 * cols);
  hipLaunchKernelGGL(reduce_parts_kernel, dim3(ceil_div(cols, 16)), dim3(1024), 0, s, cols, nparts, part, beta, out,
                     split, out2);
  TALOS_LAUNCHED("reduce_parts_kernel");
  return TALOS_OK;
}

size_t reduce_parts_workspace_bytes(int nparts, int cols) { return parts_rows(nparts) * cols * sizeof(double); }

int reduce_parts_batch_launch(int count, const PartsJob* jobs, hipStream_t s) {
  TALOS_REQUIRE(count >= 0 && count <= kPartsJobsMax, TALOS_ERR_SHAPE, "reduction batch: %d jobs (at most %d)", count,
                kPartsJobsMax);
  PartsBatch b{};
  b.n = 0;
  b.start[0] = 0;
  double cells = 0.0;
  for (int i = 0; i < count; ++i) {
    PartsJob J = jobs[i];
    if (J.cols <= 0) continue;
    TALOS_REQUIRE(J.nparts >= 0 && J.nparts <= kOnePassParts && J.part && J.out, TALOS_ERR_SHAPE,
                  "reduction batch: a job needs one pass (at most %d partials), partials and an output", kOnePassParts);
    if (J.split < 0 || J.split > J.cols || J.out2 == nullptr) J.split = J.cols;
    b.j[b.n] = J;
    b.start[b.n + 1] = b.start[b.n] + (int)ceil_div(J.cols, 16);
    cells += (double)J.nparts * J.cols;
    ++b.n;
  }
  if (b.n == 0) return TALOS_OK;
  ProfScope ps(s, "reduce_parts_batch_kernel", cells, 8.0 * cells);
  hipLaunchKernelGGL(reduce_parts_batch_kernel, dim3(b.start[b.n]), dim3(1024), 0, s, b);
  TALOS_LAUNCHED("reduce_parts_batch_kernel");
  return TALOS_OK;
}

size_t colsum_workspace_bytes(int rows, int cols) { return parts_rows(colsum_parts(rows)) * cols * sizeof(double); }

int colsum_launch(int rows, int cols, const float* dy, long long ld, float beta, float* out, double* ws,
                  hipStream_t s) {
  if (cols == 0) return TALOS_OK;
  const int nparts = rows > 0 ? colsum_parts(rows) : 0;
  if (nparts > 0) {
    dim3 g(ceil_div(cols, 64), nparts);
    ProfScope ps(s, "colsum_partial_kernel", (double)rows * cols, 4.0 * rows * cols + 8.0 * nparts * cols);
    hipLaunchKernelGGL(colsum_partial_kernel, g, dim3(256), 0, s, rows, cols, dy, ld, nparts, ws);
    TALOS_LAUNCHED("colsum_partial_kernel");
  }
  return reduce_parts_launch(cols, nparts, ws, beta, out, s);
}

// ---------------------------------------------------------------------------
// fp32 -> bf16 copies (the bf16 operands of bf16-in products)
// ---------------------------------------------------------------------------
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));
// two values rounded to nearest even (v_cvt_pk_bf16_f32, the conversion the GEMM staging makes),
// lo in the low half
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  const floatx2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// Up to kCvtMax tensors in one launch: blockIdx.y picks the tensor, the x grid strides its
// elements four at a time (float4 in, 8 bytes out; a scalar tail).
constexpr int kCvtMax = 8;
struct CvtList {
  const float* src[kCvtMax];
  uint16_t* dst[kCvtMax];
  long long n[kCvtMax];
};
__global__ __launch_bounds__(256) void cvt_bf16_kernel(CvtList l) {
  const int t = blockIdx.y;
  const float* x = l.src[t];
  uint16_t* y = l.dst[t];
  const long long n = l.n[t];
  // float4 reads and 8-byte writes where both ends allow, else element by element
  const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) | (reinterpret_cast<uintptr_t>(y) & 7)) == 0;
  const long long n4 = vec ? n / 4 : 0;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    reinterpret_cast<uint2*>(y)[i] = make_uint2(bf16_pair(v.x, v.y), bf16_pair(v.z, v.w));
  }
  for (long long i = 4 * n4 + (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (uint16_t)(bf16_pair(x[i], 0.f) & 0xffffu);
}

int cvt_bf16_launch(int count, const float* const* src, uint16_t* const* dst, const long long* n, hipStream_t s) {
  CvtList l{};
  long long most = 0, bytes = 0;
  TALOS_REQUIRE(count >= 0 && count <= kCvtMax, TALOS_ERR_SHAPE, "bf16 conversion: %d tensors (at most %d)", count,
                kCvtMax);
  for (int i = 0; i < count; ++i) {
    TALOS_REQUIRE((reinterpret_cast<uintptr_t>(src[i]) & 3) == 0 && (reinterpret_cast<uintptr_t>(dst[i]) & 1) == 0,
                  TALOS_ERR_SHAPE, "bf16 conversion: misaligned fp32 source or bf16 destination");
    l.src[i] = src[i];
    l.dst[i] = dst[i];
    l.n[i] = n[i];
    most = std::max(most, n[i]);
    bytes += 6 * n[i];
  }
  if (count == 0 || most == 0) return TALOS_OK;
  const unsigned gx = (unsigned)std::min<long long>(2048, (most / 4 + 255) / 256 + 1);
  ProfScope ps(s, "cvt_bf16_kernel", 0.0, (double)bytes);
  hipLaunchKernelGGL(cvt_bf16_kernel, dim3(gx, count), dim3(256), 0, s, l);
  TALOS_LAUNCHED("cvt_bf16_kernel");
  return TALOS_OK;
}

// ---------------------------------------------------------------------------
// RMSNorm
// ---------------------------------------------------------------------------
// Each wave handles rows; lane l holds elements [4*l + 256*j, +4) for j < dim/256 (dim % 4 == 0,
// dim <= 1024 on the vector path). Generic dims fall back to a strided scalar loop.
// Y16: each lane also writes its four values' bf16 copy (8 bytes) to y16.
template <int V, bool Y16 = false>  // float4 vectors per lane
__global__ __launch_bounds__(256) void rmsnorm_fwd_kernel(int rows, int dim, float eps, const float* __restrict__ x,
                                                          const float* __restrict__ w, float* __restrict__ y,
                                                          float* __restrict__ rstd, uint16_t* __restrict__ y16) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + (long long)row * dim;
  float4 v[V];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = 4 * lane + 256 * j;
    v[j] = c < dim ? *reinterpret_cast<const float4*>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  if (lane == 0 && rstd) rstd[row] = r;
  float* yr = y + (long long)row * dim;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = 4 * lane + 256 * j;
    if (c < dim) {
      const float4 g = *reinterpret_cast<const float4*>(w + c);
      const float4 o = make_float4(v[j].x * r * g.x, v[j].y * r * g.y, v[j].z * r * g.z, v[j].w * r * g.w);
      *reinterpret_cast<float4*>(yr + c) = o;
      if (Y16)
        *reinterpret_cast<uint2*>(y16 + (long long)row * dim + c) = make_uint2(bf16_pair(o.x, o.y), bf16_pair(o.z, o.w));
    }
  }
}

__global__ __launch_bounds__(256) void rmsnorm_fwd_generic(int rows, int dim, float eps, const float* __restrict__ x,
                                                           const float* __restrict__ w, float* __restrict__ y,
                                                           float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + (long long)row * dim;
  float ss = 0.f;
  for (int c = lane; c < dim; c += 64) ss += xr[c] * xr[c];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)dim + eps);
  if (lane == 0 && rstd) rstd[row] = r;
  for (int c = lane; c < dim; c += 64) y[(long long)row * dim + c] = xr[c] * r * w[c];
}

// Backward: a bounded grid of 16-wave workgroups strides over the rows, one row per wave up to
// 16 * kRmsMaxBlocks rows, and beyond that kRmsRowsPerWave rows of a wave's stride class per pass
// (their loads in flight together). Each lane keeps its columns' dgain sums in registers; a
// workgroup adds its 16 waves' sums in LDS in a fixed order and writes one f64 partial row, which
// reduce_parts_kernel combines. (The generic kernel runs 4-wave workgroups on the same grid.)
constexpr int kRmsWaves = 16, kRmsThreads = 64 * kRmsWaves;
constexpr int kRmsRowsPerWave = 2;
// one 16-wave workgroup per CU; 256 x dim f64 partials at most (at 16384 rows of 512 the
// workgroups' waves take four rows each, two passes of two: 24.3 us against 28.3 with 1024
// workgroups of one row a wave, which run in two rounds of two workgroups per CU)
constexpr int kRmsMaxBlocks = 256;
static int rms_bwd_blocks(int rows) {
  int b = (rows + kRmsWaves - 1) / kRmsWaves;
  return b < 1 ? 1 : (b > kRmsMaxBlocks ? kRmsMaxBlocks : b);
}

template <int V>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_bwd_kernel(int rows, int dim, const float* __restrict__ x,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ rstd,
                                                          const float* __restrict__ dy, const float* add,
                                                          float* dx, double* __restrict__ dw_part,
                                                          const float* __restrict__ add_last, int seq,
                                                          const int32_t* __restrict__ lens) {
  __shared__ float red[kRmsWaves][V * 256];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float4 gw[V], dwacc[V];
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = 4 * lane + 256 * j;
    gw[j] = c < dim ? *reinterpret_cast<const float4*>(w + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    dwacc[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float inv_dim = 1.0f / (float)dim;
  const int stride = gridDim.x * kRmsWaves;
  // kRmsRowsPerWave rows per pass, all of their loads issued before the first row is reduced
  for (int row0 = blockIdx.x * kRmsWaves + wv; row0 < rows; row0 += kRmsRowsPerWave * stride) {
    float4 xh[kRmsRowsPerWave][V], gg[kRmsRowsPerWave][V], ad[kRmsRowsPerWave][V];
    float r[kRmsRowsPerWave];
#pragma unroll
    for (int k = 0; k < kRmsRowsPerWave; ++k) {
      const int row = row0 + k * stride;
      const bool live = row < rows;
      r[k] = live ? rstd[row] : 0.f;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int c = 4 * lane + 256 * j;
        ad[k][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live && c < dim) {
          xh[k][j] = *reinterpret_cast<const float4*>(x + (long long)row * dim + c);
          gg[k][j] = *reinterpret_cast<const float4*>(dy + (long long)row * dim + c);
          // the addend row too, so a row waits on memory once (before its reduction)
          if (add) ad[k][j] = *reinterpret_cast<const float4*>(add + (long long)row * dim + c);
        } else {
          xh[k][j] = gg[k][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kRmsRowsPerWave; ++k) {
      const int row = row0 + k * stride;
      if (row >= rows) break;
      const float rk = r[k];
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        float4& h = xh[k][j];
        const float4 g = gg[k][j];
        h = make_float4(h.x * rk, h.y * rk, h.z * rk, h.w * rk);
        dot += g.x * gw[j].x * h.x + g.y * gw[j].y * h.y + g.z * gw[j].z * h.z + g.w * gw[j].w * h.w;
        dwacc[j].x += g.x * h.x;
        dwacc[j].y += g.y * h.y;
        dwacc[j].z += g.z * h.z;
        dwacc[j].w += g.w * h.w;
      }
      const float md = wave_sum(dot) * inv_dim;
      float* dxr = dx + (long long)row * dim;
      const bool last = add_last && row % seq == last_row(lens, row / seq, seq);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int c = 4 * lane + 256 * j;
        if (c < dim) {
          const float4 h = xh[k][j], g = gg[k][j];
          float4 o = make_float4(rk * (g.x * gw[j].x - h.x * md), rk * (g.y * gw[j].y - h.y * md),
                                 rk * (g.z * gw[j].z - h.z * md), rk * (g.w * gw[j].w - h.w * md));
          if (add) {
            const float4 old = ad[k][j];
            o.x += old.x;
            o.y += old.y;
            o.z += old.z;
            o.w += old.w;
          }
          if (last) {
            const float4 ex = *reinterpret_cast<const float4*>(add_last + (long long)(row / seq) * dim + c);
            o.x += ex.x;
            o.y += ex.y;
            o.z += ex.z;
            o.w += ex.w;
          }
          *reinterpret_cast<float4*>(dxr + c) = o;
        }
      }
    }
  }
  if (dw_part == nullptr) return;
#pragma unroll
  for (int j = 0; j < V; ++j) *reinterpret_cast<float4*>(&red[wv][4 * lane + 256 * j]) = dwacc[j];
  __syncthreads();
  for (int c = threadIdx.x; c < dim; c += kRmsThreads) {
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < kRmsWaves; ++i) s += (double)red[i][c];
    dw_part[(long long)blockIdx.x * dim + c] = s;
  }
}

__global__ __launch_bounds__(256) void rmsnorm_bwd_generic(int rows, int dim, const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ rstd,
                                                           const float* __restrict__ dy, const float* add,
                                                           float* dx, double* __restrict__ dw_part,
                                                           const float* __restrict__ add_last, int seq,
                                                           const int32_t* __restrict__ lens) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int row = blockIdx.x * 4 + wv; row < rows; row += gridDim.x * 4) {
    const float r = rstd[row];
    const float* xr = x + (long long)row * dim;
    const float* gr = dy + (long long)row * dim;
    float dot = 0.f;
    for (int c = lane; c < dim; c += 64) dot += gr[c] * w[c] * xr[c] * r;
    const float md = wave_sum(dot) / (float)dim;
    for (int c = lane; c < dim; c += 64) {
      float o = r * (gr[c] * w[c] - xr[c] * r * md);
      if (add) o += add[(long long)row * dim + c];
      if (add_last && row % seq == last_row(lens, row / seq, seq)) o += add_last[(long long)(row / seq) * dim + c];
      dx[(long long)row * dim + c] = o;
    }
  }
  if (dw_part == nullptr) return;
  // per-feature partial over the rows this workgroup visited
  for (int c = threadIdx.x; c < dim; c += 256) {
    double s = 0.0;
    for (int r0 = blockIdx.x * 4; r0 < rows; r0 += gridDim.x * 4)
      for (int row = r0; row < r0 + 4 && row < rows; ++row)
        s += (double)dy[(long long)row * dim + c] * (double)(x[(long long)row * dim + c] * rstd[row]);
    dw_part[(long long)blockIdx.x * dim + c] = s;
  }
}

size_t rmsnorm_bwd_workspace_bytes(int rows, int dim) {
  return parts_rows(rms_bwd_blocks(rows)) * dim * sizeof(double);
}

int rmsnorm_fwd_launch(int rows, int dim, float eps, const float* x, const float* w, float* y, float* rstd,
                       hipStream_t s, uint16_t* y16) {
  if (rows == 0) return TALOS_OK;
  dim3 g(ceil_div(rows, 4)), b(256);
  const bool vec = dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y) |
                                     reinterpret_cast<uintptr_t>(w)) & 15) == 0;
  if (y16) {
    if (vec && dim <= 1024 && (reinterpret_cast<uintptr_t>(y16) & 7) == 0) {
      // x read, y and its bf16 copy written, gain read, rstd written
      ProfScope ps(s, dim <= 256 ? "rmsnorm_fwd_kernel<1, true>" : dim <= 512 ? "rmsnorm_fwd_kernel<2, true>"
                                                                              : "rmsnorm_fwd_kernel<4, true>",
                   4.0 * rows * dim, 4.0 * (2.0 * rows * dim + dim + (rstd ? rows : 0)) + 2.0 * rows * dim);
      if (dim <= 256)
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<1, true>), g, b, 0, s, rows, dim, eps, x, w, y, rstd, y16);
      else if (dim <= 512)
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<2, true>), g, b, 0, s, rows, dim, eps, x, w, y, rstd, y16);
      else
        hipLaunchKernelGGL((rmsnorm_fwd_kernel<4, true>), g, b, 0, s, rows, dim, eps, x, w, y, rstd, y16);
      TALOS_LAUNCHED("rmsnorm_fwd");
      return TALOS_OK;
    }
    if (int rc = rmsnorm_fwd_launch(rows, dim, eps, x, w, y, rstd, s)) return rc;
    const float* src[1] = {y};
    uint16_t* dst[1] = {y16};
    const long long n[1] = {(long long)rows * dim};
    return cvt_bf16_launch(1, src, dst, n, s);
  }
  // x read, y written, gain read, rstd written
  ProfScope ps(s, vec && dim <= 256 ? "rmsnorm_fwd_kernel<1>" : vec && dim <= 512 ? "rmsnorm_fwd_kernel<2>"
                  : vec && dim <= 1024 ? "rmsnorm_fwd_kernel<4>" : "rmsnorm_fwd_generic",
               4.0 * rows * dim, 4.0 * (2.0 * rows * dim + dim + (rstd ? rows : 0)));
  if (vec && dim <= 256) hipLaunchKernelGGL(rmsnorm_fwd_kernel<1>, g, b, 0, s, rows, dim, eps, x, w, y, rstd, nullptr);
  else if (vec && dim <= 512) hipLaunchKernelGGL(rmsnorm_fwd_kernel<2>, g, b, 0, s, rows, dim, eps, x, w, y, rstd, nullptr);
  else if (vec && dim <= 1024) hipLaunchKernelGGL(rmsnorm_fwd_kernel<4>, g, b, 0, s, rows, dim, eps, x, w, y, rstd, nullptr);
  else hipLaunchKernelGGL(rmsnorm_fwd_generic, g, b, 0, s, rows, dim, eps, x, w, y, rstd);
  TALOS_LAUNCHED("rmsnorm_fwd");
  return TALOS_OK;
}

int rmsnorm_bwd_launch(int rows, int dim, const float* x, const float* w, const float* rstd, const float* dy,
                       float beta_dx, float* dx, float beta_dw, float* dw, double* ws, hipStream_t s,
                       const float* dres, const float* dres_last, int seq, const int32_t* lens) {
  const int nblk = rows > 0 ? rms_bwd_blocks(rows) : 0;
  if (nblk > 0) {
    dim3 g(nblk), b(256);
    double* part = dw ? ws : nullptr;
    // the addend: the residual branch's gradient, or dx itself when accumulating
    const float* add = dres ? dres : (beta_dx != 0.f ? dx : nullptr);
    const bool vec = dim % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) |
                                       reinterpret_cast<uintptr_t>(dx) | reinterpret_cast<uintptr_t>(w) |
                                       reinterpret_cast<uintptr_t>(add) | reinterpret_cast<uintptr_t>(dres_last)) & 15) == 0;
    // x, dy read, dx written (the addend read too), gain + rstd read, dgain partials written
    ProfScope ps(s, vec && dim <= 256 ? "rmsnorm_bwd_kernel<1>" : vec && dim <= 512 ? "rmsnorm_bwd_kernel<2>"
                    : "rmsnorm_bwd_generic",
                 8.0 * rows * dim, 4.0 * ((3.0 + (add != nullptr)) * rows * dim + dim + rows) +
                                       (part ? 8.0 * nblk * dim : 0.0));
    const int sq = seq > 0 ? seq : 1;
    const dim3 bv(kRmsThreads);
    if (vec && dim <= 256)
      hipLaunchKernelGGL(rmsnorm_bwd_kernel<1>, g, bv, 0, s, rows, dim, x, w, rstd, dy, add, dx, part, dres_last, sq,
                         lens);
    else if (vec && dim <= 512)
      hipLaunchKernelGGL(rmsnorm_bwd_kernel<2>, g, bv, 0, s, rows, dim, x, w, rstd, dy, add, dx, part, dres_last, sq,
                         lens);
    else
      hipLaunchKernelGGL(rmsnorm_bwd_generic, g, b, 0, s, rows, dim, x, w, rstd, dy, add, dx, part, dres_last, sq,
                         lens);
    TALOS_LAUNCHED("rmsnorm_bwd");
  }
  if (dw) return reduce_parts_launch(dim, nblk, ws, beta_dw, dw, s);
  return TALOS_OK;
}

// ---------------------------------------------------------------------------
// Softmax over rows of length cols (optionally causal: row r is query q = r mod cols and keys
// j > q are masked to probability 0).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void softmax_fwd_kernel(int rows, int cols, int causal, const float* __restrict__ x,
                                                          float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lim = causal ? (row % cols) + 1 : cols;
  const float* xr = x + (long long)row * cols;
  float* yr = y + (long long)row * cols;
  float mx = -INFINITY;
  for (int c = lane; c < lim; c += 64) mx = fmaxf(mx, xr[c]);
  mx = wave_max(mx);
  float s = 0.f;
  for (int c = lane; c < lim; c += 64) s += expf(xr[c] - mx);
  s = wave_sum(s);
  const float inv = 1.0f / s;
  for (int c = lane; c < cols; c += 64) yr[c] = c < lim ? expf(xr[c] - mx) * inv : 0.f;
}

// dx = beta*dx + y * (g - sum(g*y)); masked entries (y = 0) get exactly 0 and are not read.
// Vector path: each lane owns float4 groups; a group entirely past the causal limit is skipped.
// Single-pass backward for rows of at most 256 * V columns on the float4 path: a lane keeps its
// columns' y and dy in registers, so each is read from memory once; keys past the causal limit
// are neither read nor summed (dx there is 0 plus the accumulated old value).
template <int V>
__global__ __launch_bounds__(256) void softmax_bwd_rows_kernel(int rows, int cols, int causal,
                                                               const float* __restrict__ y,
                                                               const float* __restrict__ dy, float beta,
                                                               float* __restrict__ dx) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lim = causal ? (row % cols) + 1 : cols;
  const long long base = (long long)row * cols;
  float4 yv[V], gv[V], old[V];
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = 4 * lane + 256 * j;
    yv[j] = gv[j] = old[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < lim) {
      yv[j] = *reinterpret_cast<const float4*>(y + base + c);
      gv[j] = *reinterpret_cast<const float4*>(dy + base + c);
      // entries at or past lim are masked: drop them from the dot product and the output
      if (c + 1 >= lim) yv[j].y = gv[j].y = 0.f;
      if (c + 2 >= lim) yv[j].z = gv[j].z = 0.f;
      if (c + 3 >= lim) yv[j].w = gv[j].w = 0.f;
    }
    if (beta != 0.f && c < cols) old[j] = *reinterpret_cast<const float4*>(dx + base + c);
    dot += yv[j].x * gv[j].x + yv[j].y * gv[j].y + yv[j].z * gv[j].z + yv[j].w * gv[j].w;
  }
  dot = wave_sum(dot);
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int c = 4 * lane + 256 * j;
    if (c < cols) {
      const float4 o = make_float4(yv[j].x * (gv[j].x - dot) + old[j].x, yv[j].y * (gv[j].y - dot) + old[j].y,
                                   yv[j].z * (gv[j].z - dot) + old[j].z, yv[j].w * (gv[j].w - dot) + old[j].w);
      *reinterpret_cast<float4*>(dx + base + c) = o;
    }
  }
}

__global__ __launch_bounds__(256) void softmax_bwd_kernel(int rows, int cols, int causal, const float* __restrict__ y,
                                                          const float* __restrict__ dy, float beta,
                                                          float* __restrict__ dx, int vec) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lim = causal ? (row % cols) + 1 : cols;
  const long long base = (long long)row * cols;
  if (vec) {
    // pass 1: sum(g*y) over the unmasked prefix
    float dot = 0.f;
    for (int c = 4 * lane; c < lim; c += 256) {
      const float4 yv = *reinterpret_cast<const float4*>(y + base + c);
      const float4 gv = *reinterpret_cast<const float4*>(dy + base + c);
      dot += yv.x * gv.x;
      if (c + 1 < lim) dot += yv.y * gv.y;
      if (c + 2 < lim) dot += yv.z * gv.z;
      if (c + 3 < lim) dot += yv.w * gv.w;
    }
    dot = wave_sum(dot);
    for (int c = 4 * lane; c < cols; c += 256) {
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c < lim) {
        const float4 yv = *reinterpret_cast<const float4*>(y + base + c);
        const float4 gv = *reinterpret_cast<const float4*>(dy + base + c);
        o.x = yv.x * (gv.x - dot);
        o.y = c + 1 < lim ? yv.y * (gv.y - dot) : 0.f;
        o.z = c + 2 < lim ? yv.z * (gv.z - dot) : 0.f;
        o.w = c + 3 < lim ? yv.w * (gv.w - dot) : 0.f;
      }
      if (beta != 0.f) {
        const float4 old = *reinterpret_cast<const float4*>(dx + base + c);
        o.x += old.x;
        o.y += old.y;
        o.z += old.z;
        o.w += old.w;
      }
      *reinterpret_cast<float4*>(dx + base + c) = o;
    }
    return;
  }
  float dot = 0.f;
  for (int c = lane; c < lim; c += 64) dot += y[base + c] * dy[base + c];
  dot = wave_sum(dot);
  for (int c = lane; c < cols; c += 64) {
    float o = c < lim ? y[base + c] * (dy[base + c] - dot) : 0.f;
    if (beta != 0.f) o += dx[base + c];
    dx[base + c] = o;
  }
}

// ---------------------------------------------------------------------------
// RoPE on [n_seq, seq, heads, dim], interleaved pairs, position start_pos + t.
// ---------------------------------------------------------------------------
__global__ void rope_kernel(long long npairs, int seq, int heads, int dim, int start_pos, float sign,
                            const float* __restrict__ cosv, const float* __restrict__ sinv,
                            const float* __restrict__ x, float beta, float* __restrict__ y) {
  const int half = dim >> 1;
  for (long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x; p < npairs;
       p += (long long)gridDim.x * blockDim.x) {
    const int i = (int)(p % half);
    const long long tok = p / half / heads;
    const int t = (int)(tok % seq);
    const int ci = (start_pos + t) * half + i;
    const float c = cosv[ci], s = sign * sinv[ci];
    const float2 v = reinterpret_cast<const float2*>(x)[p];
    float2 o = make_float2(v.x * c - v.y * s, v.x * s + v.y * c);
    if (beta != 0.f) {
      const float2 old = reinterpret_cast<const float2*>(y)[p];
      o.x += old.x;
      o.y += old.y;
    }
    reinterpret_cast<float2*>(y)[p] = o;
  }
}

// Host-side table cache: cos/sin(pos * theta_i), theta_i = 1 / base^(2i/dim), evaluated in f64
// as the reference does (src/transformer.rs:239-251) and rounded to fp32.
void rope_table_host(int max_len, int dim, double base, std::vector<float>& c, std::vector<float>& s) {
  const int half = dim / 2;
  c.resize((size_t)max_len * half);
  s.resize((size_t)max_len * half);
  for (int pos = 0; pos < max_len; ++pos)
    for (int i = 0; i < half; ++i) {
      const double theta = 1.0 / std::pow(base, (double)(2 * i) / (double)dim);
      const double ang = (double)pos * theta;
      c[(size_t)pos * half + i] = (float)std::cos(ang);
      s[(size_t)pos * half + i] = (float)std::sin(ang);
    }
}

struct RopeTable {
  float* cos = nullptr;
  float* sin = nullptr;
  int max_len = 0;
};
static std::mutex g_rope_mu;
static std::map<std::tuple<int, uint32_t>, RopeTable> g_rope_tables;  // (dim, base bits) -> table

// Returns device cos/sin tables covering positions [0, need_len). Tables are kept for the life
// of the process and only grow.
int rope_table_device(int need_len, int dim, float base, const float** cosv, const float** sinv) {
  uint32_t bb;
  std::memcpy(&bb, &base, 4);
  std::lock_guard<std::mutex> lk(g_rope_mu);
  RopeTable& t = g_rope_tables[std::make_tuple(dim, bb)];
  if (t.max_len < need_len) {
    int len = std::max(need_len, 256);
    std::vector<float> c, s;
    rope_table_host(len, dim, (double)base, c, s);
    float *dc = nullptr, *ds = nullptr;
    TALOS_HIP(hipMalloc(&dc, c.size() * 4));
    TALOS_HIP(hipMalloc(&ds, s.size() * 4));
    TALOS_HIP(hipMemcpy(dc, c.data(), c.size() * 4, hipMemcpyHostToDevice));
    TALOS_HIP(hipMemcpy(ds, s.data(), s.size() * 4, hipMemcpyHostToDevice));
    // Older tables stay allocated: work already enqueued on other streams may still read them.
    t.cos = dc;
    t.sin = ds;
    t.max_len = len;
  }
  *cosv = t.cos;
  *sinv = t.sin;
  return TALOS_OK;
}

// Two interleaved pairs (four consecutive elements) per thread for dim % 4 == 0 with 16-byte
// aligned rows: one float4 of x, one float2 each of the cos / sin table (pairs i, i + 1 of the
// same position), 32-bit index arithmetic (the launcher checks the element count fits).
__global__ __launch_bounds__(256) void rope4_kernel(unsigned n4, int seq, int heads, int dim, int start_pos,
                                                    float sign, const float* __restrict__ cosv,
                                                    const float* __restrict__ sinv, const float* __restrict__ x,
                                                    float beta, float* __restrict__ y) {
  const unsigned q = blockIdx.x * 256u + threadIdx.x;
  if (q >= n4) return;
  const unsigned per_row = (unsigned)dim >> 2;  // float4s per (token, head) row
  const unsigned row = q / per_row;
  const int i = 2 * (int)(q - row * per_row);  // first pair of the four elements
  const int t = (int)((row / (unsigned)heads) % (unsigned)seq);
  const int ci = (start_pos + t) * (dim >> 1) + i;
  const float2 c = *reinterpret_cast<const float2*>(cosv + ci);
  const float2 sn = *reinterpret_cast<const float2*>(sinv + ci);
  const float s0 = sign * sn.x, s1 = sign * sn.y;
  const float4 v = reinterpret_cast<const float4*>(x)[q];
  float4 o = make_float4(v.x * c.x - v.y * s0, v.x * s0 + v.y * c.x, v.z * c.y - v.w * s1, v.z * s1 + v.w * c.y);
  if (beta != 0.f) {
    const float4 old = reinterpret_cast<const float4*>(y)[q];
    o.x += old.x;
    o.y += old.y;
    o.z += old.z;
    o.w += old.w;
  }
  reinterpret_cast<float4*>(y)[q] = o;
}

int rope_launch(int n_seq, int seq, int heads, int dim, int start_pos, const float* cosv, const float* sinv,
                const float* x, float beta, float* y, bool backward, hipStream_t s) {
  const long long npairs = (long long)n_seq * seq * heads * (dim / 2);
  if (npairs == 0) return TALOS_OK;
  const long long n4 = npairs / 2;
  if (dim % 4 == 0 && n4 < (1LL << 31) &&
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15) == 0) {
    hipLaunchKernelGGL(rope4_kernel, dim3((unsigned)ceil_div((size_t)n4, 256)), dim3(256), 0, s, (unsigned)n4, seq,
                       heads, dim, start_pos, backward ? -1.f : 1.f, cosv, sinv, x, beta, y);
    TALOS_LAUNCHED("rope4_kernel");
    return TALOS_OK;
  }
  hipLaunchKernelGGL(rope_kernel, dim3(grid_for((size_t)npairs)), dim3(256), 0, s, npairs, seq, heads, dim,
                     start_pos, backward ? -1.f : 1.f, cosv, sinv, x, beta, y);
  TALOS_LAUNCHED("rope_kernel");
  return TALOS_OK;
}

// ---------------------------------------------------------------------------
// Element-wise ops
// ---------------------------------------------------------------------------
__device__ __forceinline__ float unary_f(int op, float v, float p0, float p1) {
  switch (op) {
    case TALOS_RELU: return v > 0.f ? v : 0.f;
    case TALOS_LOG: return logf(v);
    case TALOS_EXP: return expf(v);
    case TALOS_SIN: return sinf(v);
    case TALOS_COS: return cosf(v);
    case TALOS_SQRT: return sqrtf(v);
    case TALOS_NEG: return -v;
    case TALOS_SCALE: return v * p0;
    case TALOS_CLIP: return fminf(fmaxf(v, p0), p1);
    case TALOS_GELU: return gelu_f(v);
    default: return v;
  }
}
// d op / dx at x (the reference closures, src/autograd.rs:356-792).
__device__ __forceinline__ float unary_d(int op, float v, float p0, float p1) {
  switch (op) {
    case TALOS_RELU: return v > 0.f ? 1.f : 0.f;
    case TALOS_LOG: return 1.f / v;
    case TALOS_EXP: return expf(v);
    case TALOS_SIN: return cosf(v);
    case TALOS_COS: return -sinf(v);
    case TALOS_SQRT: return v > 0.f ? 0.5f / sqrtf(v) : 0.f;
    case TALOS_NEG: return -1.f;
    case TALOS_SCALE: return p0;
    case TALOS_CLIP: return (v >= p0 && v <= p1) ? 1.f : 0.f;
    case TALOS_GELU: return gelu_d(v);
    default: return 1.f;
  }
}

__global__ void unary_fwd_kernel(int op, size_t n, float p0, float p1, const float* __restrict__ x,
                                 float* __restrict__ y) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    y[i] = unary_f(op, x[i], p0, p1);
}
__global__ void unary_bwd_kernel(int op, size_t n, float p0, float p1, const float* __restrict__ x,
                                 const float* __restrict__ dy, float* __restrict__ dx) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dx[i] += unary_d(op, x[i], p0, p1) * dy[i];
}
// GELU (y = x Phi(x)) and its backward (dx = beta dx + dy (Phi(x) + x phi(x))), HBM-bound: 8 bytes
// per element forward, 12 (beta 0) or 16 (beta 1) backward. vec: n % 4 == 0 and every pointer
// 16-byte aligned, so each thread moves float4s; otherwise one element per thread.
template <bool BWD>
__global__ __launch_bounds__(256) void gelu_kernel(size_t n, float beta, const float* __restrict__ x,
                                                   const float* __restrict__ dy, float* __restrict__ out, int vec) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (vec) {
    for (; i < n / 4; i += stride) {
      const float4 v = reinterpret_cast<const float4*>(x)[i];
      float4 r;
      if (BWD) {
        const float4 g = reinterpret_cast<const float4*>(dy)[i];
        r = make_float4(gelu_d(v.x) * g.x, gelu_d(v.y) * g.y, gelu_d(v.z) * g.z, gelu_d(v.w) * g.w);
        if (beta != 0.f) {
          const float4 o = reinterpret_cast<const float4*>(out)[i];
          r = make_float4(o.x + r.x, o.y + r.y, o.z + r.z, o.w + r.w);
        }
      } else {
        r = make_float4(gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w));
      }
      reinterpret_cast<float4*>(out)[i] = r;
    }
    return;
  }
  for (; i < n; i += stride) {
    if (BWD) {
      const float r = gelu_d(x[i]) * dy[i];
      out[i] = beta != 0.f ? out[i] + r : r;
    } else {
      out[i] = gelu_f(x[i]);
    }
  }
}

__global__ void binary_fwd_kernel(int op, size_t n, const float* __restrict__ a, const float* __restrict__ b,
                                  float* __restrict__ y) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float u = a[i], v = b[i];
    y[i] = op == TALOS_ADD ? u + v : op == TALOS_SUB ? u - v : op == TALOS_MUL ? u * v : u / v;
  }
}
// da / db may alias (x op x): then the two partial derivatives are summed into one write.
__global__ void binary_bwd_kernel(int op, size_t n, const float* a, const float* b, const float* __restrict__ dy,
                                  float* da, float* db) {
  const bool alias = da == db;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float g = dy[i], u = a[i], v = b[i];
    float ga, gb;
    switch (op) {
      case TALOS_ADD: ga = g; gb = g; break;
      case TALOS_SUB: ga = g; gb = -g; break;
      case TALOS_MUL: ga = g * v; gb = g * u; break;
      default: ga = g / v; gb = -g * u / (v * v); break;
    }
    if (alias) {
      if (da) da[i] += ga + gb;
    } else {
      if (da) da[i] += ga;
      if (db) db[i] += gb;
    }
  }
}

__global__ void reduce_partial_kernel(size_t n, const float* __restrict__ x, double* __restrict__ part) {
  __shared__ double red[4];
  double s = 0.0;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    s += (double)x[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}
__global__ void reduce_final_kernel(int nparts, float scale, const double* __restrict__ part, float* __restrict__ out) {
  __shared__ double red[4];
  double s = 0.0;
  for (int i = threadIdx.x; i < nparts; i += blockDim.x) s += part[i];
  s = block_sum(s, red);
  if (threadIdx.x == 0) out[0] = (float)(s * (double)scale);
}
__global__ void fill_add_kernel(size_t n, float scale, const float* __restrict__ g, float* __restrict__ dx) {
  const float v = scale * g[0];
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) dx[i] += v;
}

struct TShape {
  long long d[6];
  long long stride_in[6];
  int rank;
};
__global__ void transpose_kernel(size_t n, TShape s, const float* __restrict__ x, float* __restrict__ y, int acc) {
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < n; o += (size_t)gridDim.x * blockDim.x) {
    size_t rem = o;
    long long src = 0;
    for (int k = s.rank - 1; k >= 0; --k) {
      const long long idx = (long long)(rem % (size_t)s.d[k]);
      rem /= (size_t)s.d[k];
      src += idx * s.stride_in[k];
    }
    if (acc) y[o] += x[src];
    else y[o] = x[src];
  }
}
__global__ void concat_kernel(size_t rows, int ca, int cb, const float* __restrict__ a, const float* __restrict__ b,
                              float* __restrict__ out) {
  const int w = ca + cb;
  const size_t n = rows * w;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / w;
    const int c = (int)(i % w);
    out[i] = c < ca ? a[r * ca + c] : b[r * cb + (c - ca)];
  }
}
__global__ void concat_bwd_kernel(size_t rows, int ca, int cb, const float* __restrict__ g, float* __restrict__ da,
                                  float* __restrict__ db, int accumulate) {
  const int w = ca + cb;
  const size_t n = rows * w;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const size_t r = i / w;
    const int c = (int)(i % w);
    float* dst = c < ca ? &da[r * ca + c] : &db[r * cb + (c - ca)];
    *dst = accumulate ? *dst + g[i] : g[i];
  }
}

// The same copies four floats per thread when both widths are multiples of 4 and every buffer is
// 16-byte aligned (each float4 then lies inside one of a / b), with 32-bit index arithmetic.
__global__ __launch_bounds__(256) void concat4_kernel(unsigned n4, int ca4, int cb4, const float4* __restrict__ a,
                                                      const float4* __restrict__ b, float4* __restrict__ out) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n4) return;
  const unsigned w4 = (unsigned)(ca4 + cb4), r = i / w4;
  const int c = (int)(i - r * w4);
  out[i] = c < ca4 ? a[r * (unsigned)ca4 + c] : b[r * (unsigned)cb4 + (c - ca4)];
}
__global__ __launch_bounds__(256) void split4_kernel(unsigned n4, int ca4, int cb4, const float4* __restrict__ g,
                                                     float4* __restrict__ da, float4* __restrict__ db,
                                                     int accumulate) {
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= n4) return;
  const unsigned w4 = (unsigned)(ca4 + cb4), r = i / w4;
  const int c = (int)(i - r * w4);
  float4* dst = c < ca4 ? &da[r * (unsigned)ca4 + c] : &db[r * (unsigned)cb4 + (c - ca4)];
  float4 v = g[i];
  if (accumulate) {
    const float4 o = *dst;
    v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
  }
  *dst = v;
}
static bool concat_vec(size_t rows, int ca, int cb, const void* p0, const void* p1, const void* p2) {
  return ca % 4 == 0 && cb % 4 == 0 && rows * (size_t)(ca + cb) / 4 < (1ull << 31) &&
         ((reinterpret_cast<uintptr_t>(p0) | reinterpret_cast<uintptr_t>(p1) | reinterpret_cast<uintptr_t>(p2)) & 15) == 0;
}

int concat_launch(size_t rows, int ca, int cb, const float* a, const float* b, float* out, hipStream_t s) {
  if (rows == 0 || ca + cb == 0) return TALOS_OK;
  const size_t n = rows * (size_t)(ca + cb);
  if (concat_vec(rows, ca, cb, a, b, out)) {
    ProfScope ps(s, "concat4_kernel", 0.0, 8.0 * n);
    hipLaunchKernelGGL(concat4_kernel, dim3(ceil_div(n / 4, 256)), dim3(256), 0, s, (unsigned)(n / 4), ca / 4, cb / 4,
                       reinterpret_cast<const float4*>(a), reinterpret_cast<const float4*>(b),
                       reinterpret_cast<float4*>(out));
    TALOS_LAUNCHED("concat4_kernel");
    return TALOS_OK;
  }
  ProfScope ps(s, "concat_kernel", 0.0, 8.0 * n);
  hipLaunchKernelGGL(concat_kernel, dim3(grid_for(n)), dim3(256), 0, s, rows, ca, cb, a, b, out);
  TALOS_LAUNCHED("concat_kernel");
  return TALOS_OK;
}

int split_launch(size_t rows, int ca, int cb, const float* g, float* da, float* db, bool accumulate, hipStream_t s) {
  if (rows == 0 || ca + cb == 0) return TALOS_OK;
  const size_t n = rows * (size_t)(ca + cb);
  if (concat_vec(rows, ca, cb, g, da, db)) {
    ProfScope ps(s, "split4_kernel", 0.0, (accumulate ? 12.0 : 8.0) * n);
    hipLaunchKernelGGL(split4_kernel, dim3(ceil_div(n / 4, 256)), dim3(256), 0, s, (unsigned)(n / 4), ca / 4, cb / 4,
                       reinterpret_cast<const float4*>(g), reinterpret_cast<float4*>(da), reinterpret_cast<float4*>(db),
                       accumulate ? 1 : 0);
    TALOS_LAUNCHED("split4_kernel");
    return TALOS_OK;
  }
  ProfScope ps(s, "concat_bwd_kernel", 0.0, (accumulate ? 12.0 : 8.0) * n);
  hipLaunchKernelGGL(concat_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, s, rows, ca, cb, g, da, db,
                     accumulate ? 1 : 0);
  TALOS_LAUNCHED("concat_bwd_kernel");
  return TALOS_OK;
}
__global__ void broadcast_rows_kernel(size_t rows, int cols, const float* __restrict__ v, float* __restrict__ out) {
  const size_t n = rows * cols;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = v[i % cols];
}

}  // namespace talos

using namespace talos;

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

int talos_fill_zero(void* dst, size_t bytes, talos_stream_t stream) {
  TALOS_NONNULL(dst);
  TALOS_DEVICE();
  return entry_done(fill_zero(dst, bytes, as_stream(stream)), as_stream(stream));
}

int talos_bias_grad_f32(int rows, int cols, const float* dy, float beta, float* db, talos_stream_t stream) {
  TALOS_NONNULL(dy);
  TALOS_NONNULL(db);
  TALOS_REQUIRE(rows >= 0 && cols >= 0, TALOS_ERR_SHAPE, "%s: negative size", __func__);
  TALOS_REQUIRE(beta == 0.f || beta == 1.f, TALOS_ERR_UNSUPPORTED, "%s: beta must be 0 or 1", __func__);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  EntryScratch ws;
  int rc = ws.acquire(colsum_workspace_bytes(rows, cols), s);
  if (rc) return rc;
  rc = colsum_launch(rows, cols, dy, cols, beta, db, static_cast<double*>(ws.ptr), s);
  const int rel = ws.release();
  return entry_done(rc ? rc : rel, as_stream(stream));
}

int talos_rmsnorm_fwd_f32(int rows, int dim, float eps, const float* x, const float* w, float* y, float* rstd,
                          talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(w);
  TALOS_NONNULL(y);
  TALOS_REQUIRE(rows >= 0 && dim > 0, TALOS_ERR_SHAPE, "%s: bad shape rows=%d dim=%d", __func__, rows, dim);
  TALOS_REQUIRE(eps >= 0.f, TALOS_ERR_SHAPE, "%s: eps must be >= 0", __func__);
  TALOS_DEVICE();
  return entry_done(rmsnorm_fwd_launch(rows, dim, eps, x, w, y, rstd, as_stream(stream)), as_stream(stream));
}

int talos_rmsnorm_bwd_f32(int rows, int dim, const float* x, const float* w, const float* rstd, const float* dy,
                          float beta_dx, float* dx, float beta_dw, float* dw, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(w);
  TALOS_NONNULL(rstd);
  TALOS_NONNULL(dy);
  TALOS_NONNULL(dx);
  TALOS_REQUIRE(rows >= 0 && dim > 0, TALOS_ERR_SHAPE, "%s: bad shape rows=%d dim=%d", __func__, rows, dim);
  TALOS_REQUIRE((beta_dx == 0.f || beta_dx == 1.f) && (beta_dw == 0.f || beta_dw == 1.f), TALOS_ERR_UNSUPPORTED,
                "%s: beta_dx / beta_dw must be 0 or 1", __func__);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  EntryScratch ws;
  int rc = ws.acquire(dw ? rmsnorm_bwd_workspace_bytes(rows, dim) : 0, s);
  if (rc) return rc;
  rc = rmsnorm_bwd_launch(rows, dim, x, w, rstd, dy, beta_dx, dx, beta_dw, dw, static_cast<double*>(ws.ptr), s);
  const int rel = ws.release();
  return entry_done(rc ? rc : rel, as_stream(stream));
}

int talos_softmax_fwd_f32(int rows, int cols, int causal, const float* x, float* y, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(y);
  TALOS_REQUIRE(rows >= 0 && cols > 0, TALOS_ERR_SHAPE, "%s: bad shape rows=%d cols=%d", __func__, rows, cols);
  TALOS_REQUIRE(causal == 0 || causal == 1, TALOS_ERR_DTYPE, "%s: causal must be 0 or 1", __func__);
  TALOS_DEVICE();
  if (rows == 0) return TALOS_OK;
  hipLaunchKernelGGL(softmax_fwd_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, as_stream(stream), rows, cols, causal,
                     x, y);
  TALOS_LAUNCHED("softmax_fwd_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_softmax_bwd_f32(int rows, int cols, int causal, const float* y, const float* dy, float beta, float* dx,
                          talos_stream_t stream) {
  TALOS_NONNULL(y);
  TALOS_NONNULL(dy);
  TALOS_NONNULL(dx);
  TALOS_REQUIRE(rows >= 0 && cols > 0, TALOS_ERR_SHAPE, "%s: bad shape rows=%d cols=%d", __func__, rows, cols);
  TALOS_REQUIRE(causal == 0 || causal == 1, TALOS_ERR_DTYPE, "%s: causal must be 0 or 1", __func__);
  TALOS_REQUIRE(beta == 0.f || beta == 1.f, TALOS_ERR_UNSUPPORTED, "%s: beta must be 0 or 1", __func__);
  TALOS_DEVICE();
  if (rows == 0) return TALOS_OK;
  const int vec = cols % 4 == 0 && ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(dy) |
                                     reinterpret_cast<uintptr_t>(dx)) & 15) == 0;
  const hipStream_t s = as_stream(stream);
  const dim3 g(ceil_div(rows, 4)), b(256);
  if (vec && cols <= 256)
    hipLaunchKernelGGL(softmax_bwd_rows_kernel<1>, g, b, 0, s, rows, cols, causal, y, dy, beta, dx);
  else if (vec && cols <= 512)
    hipLaunchKernelGGL(softmax_bwd_rows_kernel<2>, g, b, 0, s, rows, cols, causal, y, dy, beta, dx);
  else if (vec && cols <= 1024)
    hipLaunchKernelGGL(softmax_bwd_rows_kernel<4>, g, b, 0, s, rows, cols, causal, y, dy, beta, dx);
  else
    hipLaunchKernelGGL(softmax_bwd_kernel, g, b, 0, s, rows, cols, causal, y, dy, beta, dx, vec);
  TALOS_LAUNCHED("softmax_bwd");
  return entry_done(TALOS_OK, s);
}

static int check_rope(const char* fn, int n_seq, int seq_len, int heads, int dim, int start_pos, float base) {
  TALOS_REQUIRE(n_seq >= 0 && seq_len >= 0 && heads >= 0 && dim > 0, TALOS_ERR_SHAPE, "%s: bad shape", fn);
  TALOS_REQUIRE(dim % 2 == 0, TALOS_ERR_SHAPE, "%s: dim=%d must be even (interleaved pairs)", fn, dim);
  TALOS_REQUIRE(start_pos >= 0, TALOS_ERR_SHAPE, "%s: start_pos must be >= 0", fn);
  TALOS_REQUIRE(base > 0.f, TALOS_ERR_SHAPE, "%s: base must be > 0", fn);
  return TALOS_OK;
}

int talos_rope_fwd_f32(int n_seq, int seq_len, int heads, int dim, int start_pos, float base, const float* x, float* y,
                       talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(y);
  int rc = check_rope(__func__, n_seq, seq_len, heads, dim, start_pos, base);
  if (rc) return rc;
  TALOS_DEVICE();
  const float *c, *s;
  rc = rope_table_device(start_pos + seq_len, dim, base, &c, &s);
  if (rc) return rc;
  return entry_done(rope_launch(n_seq, seq_len, heads, dim, start_pos, c, s, x, 0.f, y, false, as_stream(stream)), as_stream(stream));
}

int talos_rope_bwd_f32(int n_seq, int seq_len, int heads, int dim, int start_pos, float base, const float* dy,
                       float beta, float* dx, talos_stream_t stream) {
  TALOS_NONNULL(dy);
  TALOS_NONNULL(dx);
  int rc = check_rope(__func__, n_seq, seq_len, heads, dim, start_pos, base);
  if (rc) return rc;
  TALOS_REQUIRE(beta == 0.f || beta == 1.f, TALOS_ERR_UNSUPPORTED, "%s: beta must be 0 or 1", __func__);
  TALOS_DEVICE();
  const float *c, *s;
  rc = rope_table_device(start_pos + seq_len, dim, base, &c, &s);
  if (rc) return rc;
  return entry_done(rope_launch(n_seq, seq_len, heads, dim, start_pos, c, s, dy, beta, dx, true, as_stream(stream)), as_stream(stream));
}

int talos_rope_table_f32(int max_len, int dim, float base, float* cos_out, float* sin_out, talos_stream_t stream) {
  TALOS_NONNULL(cos_out);
  TALOS_NONNULL(sin_out);
  TALOS_REQUIRE(max_len >= 0 && dim > 0 && dim % 2 == 0, TALOS_ERR_SHAPE, "%s: bad shape", __func__);
  TALOS_DEVICE();
  std::vector<float> c, s;
  rope_table_host(max_len, dim, (double)base, c, s);
  if (c.empty()) return TALOS_OK;
  TALOS_HIP(hipMemcpyAsync(cos_out, c.data(), c.size() * 4, hipMemcpyHostToDevice, as_stream(stream)));
  TALOS_HIP(hipMemcpyAsync(sin_out, s.data(), s.size() * 4, hipMemcpyHostToDevice, as_stream(stream)));
  TALOS_HIP(hipStreamSynchronize(as_stream(stream)));
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_unary_fwd_f32(int op, size_t n, float p0, float p1, const float* x, float* y, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(y);
  TALOS_REQUIRE(op >= TALOS_RELU && op <= TALOS_COPY, TALOS_ERR_DTYPE, "%s: unknown op %d", __func__, op);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  hipLaunchKernelGGL(unary_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), op, n, p0, p1, x, y);
  TALOS_LAUNCHED("unary_fwd_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_unary_bwd_f32(int op, size_t n, float p0, float p1, const float* x, const float* dy, float* dx,
                        talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(dy);
  TALOS_NONNULL(dx);
  TALOS_REQUIRE(op >= TALOS_RELU && op <= TALOS_COPY, TALOS_ERR_DTYPE, "%s: unknown op %d", __func__, op);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  hipLaunchKernelGGL(unary_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), op, n, p0, p1, x, dy, dx);
  TALOS_LAUNCHED("unary_bwd_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

static int gelu_launch(bool bwd, size_t n, float beta, const float* x, const float* dy, float* out,
                       hipStream_t s) {
  const int vec = n % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) |
                                  reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  const unsigned grid = grid_for(vec ? n / 4 : n);
  if (bwd)
    hipLaunchKernelGGL(gelu_kernel<true>, dim3(grid), dim3(256), 0, s, n, beta, x, dy, out, vec);
  else
    hipLaunchKernelGGL(gelu_kernel<false>, dim3(grid), dim3(256), 0, s, n, beta, x, dy, out, vec);
  return launch_status(bwd ? "gelu_kernel<true>" : "gelu_kernel<false>");
}

int talos_gelu_fwd_f32(size_t n, const float* x, float* y, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(y);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  return entry_done(gelu_launch(false, n, 0.f, x, nullptr, y, as_stream(stream)), as_stream(stream));
}

int talos_gelu_bwd_f32(size_t n, const float* x, const float* dy, float beta, float* dx, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(dy);
  TALOS_NONNULL(dx);
  TALOS_REQUIRE(beta == 0.f || beta == 1.f, TALOS_ERR_UNSUPPORTED, "%s: beta must be 0 or 1", __func__);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  return entry_done(gelu_launch(true, n, beta, x, dy, dx, as_stream(stream)), as_stream(stream));
}

int talos_binary_fwd_f32(int op, size_t n, const float* a, const float* b, float* y, talos_stream_t stream) {
  TALOS_NONNULL(a);
  TALOS_NONNULL(b);
  TALOS_NONNULL(y);
  TALOS_REQUIRE(op >= TALOS_ADD && op <= TALOS_DIV, TALOS_ERR_DTYPE, "%s: unknown op %d", __func__, op);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  hipLaunchKernelGGL(binary_fwd_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), op, n, a, b, y);
  TALOS_LAUNCHED("binary_fwd_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_binary_bwd_f32(int op, size_t n, const float* a, const float* b, const float* dy, float* da, float* db,
                         talos_stream_t stream) {
  TALOS_NONNULL(a);
  TALOS_NONNULL(b);
  TALOS_NONNULL(dy);
  TALOS_REQUIRE(da || db, TALOS_ERR_NULL, "%s: da and db are both null", __func__);
  TALOS_REQUIRE(op >= TALOS_ADD && op <= TALOS_DIV, TALOS_ERR_DTYPE, "%s: unknown op %d", __func__, op);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  hipLaunchKernelGGL(binary_bwd_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), op, n, a, b, dy, da, db);
  TALOS_LAUNCHED("binary_bwd_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_reduce_sum_f32(size_t n, float scale, const float* x, float* out, talos_stream_t stream) {
  TALOS_NONNULL(x);
  TALOS_NONNULL(out);
  TALOS_DEVICE();
  hipStream_t s = as_stream(stream);
  const int nparts = (int)std::min<size_t>(1024, std::max<size_t>(1, (n + 1023) / 1024));
  EntryScratch scratch;
  int rc = scratch.acquire(nparts * sizeof(double), s);
  if (rc) return rc;
  double* ws = static_cast<double*>(scratch.ptr);
  hipLaunchKernelGGL(reduce_partial_kernel, dim3(nparts), dim3(256), 0, s, n, x, ws);
  rc = launch_status("reduce_partial_kernel");
  if (rc == TALOS_OK) {
    hipLaunchKernelGGL(reduce_final_kernel, dim3(1), dim3(256), 0, s, nparts, scale, ws, out);
    rc = launch_status("reduce_final_kernel");
  }
  const int rel = scratch.release();
  return entry_done(rc ? rc : rel, as_stream(stream));
}

int talos_fill_add_f32(size_t n, float scale, const float* g, float* dx, talos_stream_t stream) {
  TALOS_NONNULL(g);
  TALOS_NONNULL(dx);
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  hipLaunchKernelGGL(fill_add_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), n, scale, g, dx);
  TALOS_LAUNCHED("fill_add_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_transpose_f32(int rank, const long long* shape, int dim0, int dim1, const float* x, float* y, int accumulate,
                        talos_stream_t stream) {
  TALOS_NONNULL(shape);
  TALOS_NONNULL(x);
  TALOS_NONNULL(y);
  TALOS_REQUIRE(rank >= 1 && rank <= 6, TALOS_ERR_SHAPE, "%s: rank %d outside [1, 6]", __func__, rank);
  TALOS_REQUIRE(dim0 >= 0 && dim0 < rank && dim1 >= 0 && dim1 < rank, TALOS_ERR_SHAPE,
                "%s: dims (%d, %d) out of range for rank %d", __func__, dim0, dim1, rank);
  size_t n = 1;
  long long in_stride[6];
  for (int k = rank - 1; k >= 0; --k) {
    TALOS_REQUIRE(shape[k] >= 0, TALOS_ERR_SHAPE, "%s: negative extent", __func__);
    in_stride[k] = (long long)n;
    n *= (size_t)shape[k];
  }
  TALOS_DEVICE();
  if (n == 0) return TALOS_OK;
  TShape ts;
  ts.rank = rank;
  for (int k = 0; k < rank; ++k) {
    ts.d[k] = shape[k];
    ts.stride_in[k] = in_stride[k];
  }
  // output shape = input shape with dim0, dim1 swapped; output index k reads input stride of the swapped dim
  std::swap(ts.d[dim0], ts.d[dim1]);
  std::swap(ts.stride_in[dim0], ts.stride_in[dim1]);
  hipLaunchKernelGGL(transpose_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream), n, ts, x, y, accumulate);
  TALOS_LAUNCHED("transpose_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

int talos_concat_last_f32(size_t rows, int ca, int cb, const float* a, const float* b, float* out,
                          talos_stream_t stream) {
  TALOS_NONNULL(a);
  TALOS_NONNULL(b);
  TALOS_NONNULL(out);
  TALOS_REQUIRE(ca >= 0 && cb >= 0, TALOS_ERR_SHAPE, "%s: negative width", __func__);
  TALOS_DEVICE();
  if (rows == 0 || ca + cb == 0) return TALOS_OK;
  return entry_done(concat_launch(rows, ca, cb, a, b, out, as_stream(stream)), as_stream(stream));
}

int talos_concat_last_bwd_f32(size_t rows, int ca, int cb, const float* dout, float* da, float* db,
                              talos_stream_t stream) {
  TALOS_NONNULL(dout);
  TALOS_NONNULL(da);
  TALOS_NONNULL(db);
  TALOS_REQUIRE(ca >= 0 && cb >= 0, TALOS_ERR_SHAPE, "%s: negative width", __func__);
  TALOS_DEVICE();
  // the reference's closure accumulates into both parents (src/transformer.rs:1162-1179)
  return entry_done(split_launch(rows, ca, cb, dout, da, db, true, as_stream(stream)), as_stream(stream));
}

int talos_broadcast_rows_f32(size_t rows, int cols, const float* v, float* out, talos_stream_t stream) {
  TALOS_NONNULL(v);
  TALOS_NONNULL(out);
  TALOS_REQUIRE(cols >= 0, TALOS_ERR_SHAPE, "%s: negative width", __func__);
  TALOS_DEVICE();
  if (rows == 0 || cols == 0) return TALOS_OK;
  hipLaunchKernelGGL(broadcast_rows_kernel, dim3(grid_for(rows * cols)), dim3(256), 0, as_stream(stream), rows, cols, v,
                     out);
  TALOS_LAUNCHED("broadcast_rows_kernel");
  return entry_done(TALOS_OK, as_stream(stream));
}

}  // extern "C"
