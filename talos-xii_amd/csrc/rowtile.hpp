// rowtile.hpp -- device building blocks for kernels that keep 16 rows (environments, samples) of
// activations in LDS and run their per-row products on the fp32 matrix cores, one
// v_mfma_f32_16x16x4f32 tile row per row: products with register-prefetched weights, a row RMSNorm
// with 16 lanes per row, DPP group sums and an LDS-only workgroup barrier. Used by the one-launch
// rollout step (decode.hip) and the last-row tails of the PPO plan (plans.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace talos {

typedef float rt_floatx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) void* rt_gptr;  // global, for direct-to-LDS loads
typedef __attribute__((address_space(3))) void* rt_lptr;  // LDS
constexpr int kRowTileRows = 16;  // the rows of a v_mfma_f32_16x16x4f32 tile
constexpr int kVmcnt0 = 0x0F70;   // s_waitcnt vmcnt(0), expcnt / lgkmcnt not waited

// out(e, n, sum_k X[e][k] W(k, n) (+ bias[n])) for 16 rows on the matrix cores, W(k, n) =
// W[k * LDW + n] (or W[n * LDW + k] when TRANS). The 16-column tiles of Y go round the WAVES
// waves of the workgroup (tile t to wave (t + woff) % WAVES); for the 16 k of group g a lane
// (row i = lane % 16, quad kq = lane / 16) reads X[i][16g + 4kq .. +3] as one float4 from LDS and
// feeds the four v_mfma_f32_16x16x4f32 of the group (product u takes k = 16g + 4kq + u) with
// B = W(16g + 4kq + u, n). The result tile holds D[4kq + r][lane % 16] in register r. K % 4 == 0;
// k past K (K % 16 != 0) and columns past N contribute zeros.
//
// The lane's weights (K / 4 a tile) and bias are loaded by RowTileW::load, a phase or more before
// rowtile_mm uses them, so the loads of the next product are in flight while the current phase
// runs. No __restrict__ on the weights: loads the compiler cannot prove invariant are not
// re-issued at their use.
template <int K, int N, int LDW, bool TRANS, int WAVES>
struct RowTileW {
  static constexpr int TILES = (N + 15) / 16, TPW = (TILES + WAVES - 1) / WAVES;
  static constexpr int KG = (K + 15) / 16;
  float w[TPW][4 * KG];
  float b[TPW];
  int woff;
  bool has_bias;
  __device__ __forceinline__ int tile_of(int tp) const {
    return ((int)(threadIdx.x >> 6) + WAVES - woff % WAVES) % WAVES + tp * WAVES;
  }
  __device__ __forceinline__ void load(const float* W, const float* bias, int wo = 0) {
    const int row = threadIdx.x & 15, kq = (threadIdx.x >> 4) & 3;
    woff = wo;
    has_bias = bias != nullptr;
#pragma unroll
    for (int tp = 0; tp < TPW; ++tp) {
      const int t = tile_of(tp), n = t * 16 + row;
      const bool nv = t < TILES && n < N;
#pragma unroll
      for (int g = 0; g < KG; ++g)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = 16 * g + 4 * kq + u;
          w[tp][4 * g + u] = nv && k < K ? W[TRANS ? n * LDW + k : k * LDW + n] : 0.f;
        }
      b[tp] = nv && bias ? bias[n] : 0.f;
    }
  }
};
template <int K, int N, int LDX, int LDW, bool TRANS, int WAVES, class Out>
__device__ __forceinline__ void rowtile_mm(const float* X, const RowTileW<K, N, LDW, TRANS, WAVES>& wt, Out out) {
  static_assert(K % 4 == 0 && LDX % 4 == 0, "float4 rows");
  using FW = RowTileW<K, N, LDW, TRANS, WAVES>;
  const int row = threadIdx.x & 15, kq = (threadIdx.x >> 4) & 3;
#pragma unroll
  for (int tp = 0; tp < FW::TPW; ++tp) {
    const int t = wt.tile_of(tp), n = t * 16 + row;
    if (t >= FW::TILES) continue;  // wave-uniform
    rt_floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < FW::KG; ++g) {
      const int k = 16 * g + 4 * kq;
      const float4 xa = k < K ? *reinterpret_cast<const float4*>(X + row * LDX + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      rt_floatx4& acc = (g & 1) ? acc1 : acc0;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, wt.w[tp][4 * g], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, wt.w[tp][4 * g + 1], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, wt.w[tp][4 * g + 2], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, wt.w[tp][4 * g + 3], acc, 0, 0, 0);
    }
    if (n < N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sum = acc0[r] + acc1[r];
        out(4 * kq + r, n, wt.has_bias ? sum + wt.b[tp] : sum);
      }
    }
  }
}

// The same product (W(k, n) = W[k * LDW + n], or W[n * LDW + k] when TRANS) with the weights
// streamed: the N / 16 tiles in passes over the WAVES waves
// (tile wave + WAVES * pass), K in chunks of KC, each chunk's weights (KC / 4 per lane) loaded one
// chunk ahead into a second register buffer while the current chunk multiplies. For products too
// wide (F-wide N) or too deep (F-wide K) to hold all of a lane's weights in registers.
template <int K, int N, int LDX, int LDW, int WAVES, int KC, bool TRANS, class Out>
__device__ __forceinline__ void rowtile_mm_stream(const float* X, const float* W, const float* bias, Out out) {
  static_assert(K % KC == 0 && KC % 16 == 0 && LDX % 4 == 0, "whole chunks of float4 groups");
  constexpr int TILES = (N + 15) / 16, PASSES = (TILES + WAVES - 1) / WAVES, NKC = K / KC, J = KC / 4;
  const int row = threadIdx.x & 15, kq = (threadIdx.x >> 4) & 3, wave = (int)(threadIdx.x >> 6);
  float wb[2][J];
  auto load = [&](float (&w)[J], int step) {
    const int t = wave + WAVES * (step / NKC), n = t * 16 + row, k0 = (step % NKC) * KC;
    const bool nv = t < TILES && n < N;
#pragma unroll
    for (int g = 0; g < KC / 16; ++g)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const long long k = k0 + 16 * g + 4 * kq + u;
        w[4 * g + u] = nv ? W[TRANS ? n * (long long)LDW + k : k * LDW + n] : 0.f;
      }
  };
  load(wb[0], 0);
#pragma unroll
  for (int pass = 0; pass < PASSES; ++pass) {
    const int t = wave + WAVES * pass, n = t * 16 + row;
    const float b = bias && t < TILES && n < N ? bias[n] : 0.f;
    rt_floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < NKC; ++kc) {
      const int step = pass * NKC + kc;
      if (step + 1 < PASSES * NKC) load(wb[(step + 1) & 1], step + 1);
      const float(&w)[J] = wb[step & 1];
      if (t < TILES) {  // wave-uniform
#pragma unroll
        for (int g = 0; g < KC / 16; ++g) {
          const float4 xa = *reinterpret_cast<const float4*>(X + row * LDX + kc * KC + 16 * g + 4 * kq);
          rt_floatx4& acc = (g & 1) ? acc1 : acc0;
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.x, w[4 * g], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.y, w[4 * g + 1], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.z, w[4 * g + 2], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa.w, w[4 * g + 3], acc, 0, 0, 0);
        }
      }
    }
    if (t < TILES && n < N) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sum = acc0[r] + acc1[r];
        out(4 * kq + r, n, bias ? sum + b : sum);
      }
    }
  }
}

// A workgroup barrier that orders LDS only: for kernels whose threads share data through LDS alone
// (global results are read by later launches, direct-to-LDS copies are waited for explicitly), so
// outstanding global loads and stores need not drain at every barrier, as behind __syncthreads().
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over aligned groups of W adjacent lanes (W a power of two <= 16) with DPP lane moves, every
// lane of a group getting its sum; all lanes of the wave must be active.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(W >= 1 && W <= 16 && (W & (W - 1)) == 0, "group width");
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  if constexpr (W >= 2) v += dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v += dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if constexpr (W >= 16) v += dpp(v, std::integral_constant<int, 0x140>{});  // row_mirror
  return v;
}

// y = x / sqrt(mean(x^2) + eps) * g over the 16 rows, 16 lanes per row (threads 0..255; the
// rstd of each row optionally stored); the lane's gains are loaded by RowGain::load ahead of the
// phase.
template <int D>
struct RowGain {
  static constexpr int LPR = 16, PER = (D + LPR - 1) / LPR;
  float g[PER];
  __device__ __forceinline__ void load(const float* gain) {
    const int l = threadIdx.x % LPR;
#pragma unroll
    for (int j = 0; j < PER; ++j) g[j] = l + j * LPR < D ? gain[l + j * LPR] : 0.f;
  }
};
template <int D, int LD>
__device__ __forceinline__ void row_norm(const float* x, float* y, float eps, const RowGain<D>& gn,
                                         float* rstd = nullptr) {
  constexpr int LPR = RowGain<D>::LPR, PER = RowGain<D>::PER;
  if (threadIdx.x >= kRowTileRows * LPR) return;  // whole waves
  const int row = threadIdx.x / LPR, l = threadIdx.x % LPR;
  float xv[PER];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = l + j * LPR;
    xv[j] = c < D ? x[row * LD + c] : 0.f;
    ss = fmaf(xv[j], xv[j], ss);
  }
  ss = group_sum<LPR>(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (rstd && l == 0) rstd[row] = r;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int c = l + j * LPR;
    if (c < D) y[row * LD + c] = xv[j] * r * gn.g[j];
  }
}

}  // namespace talos
