// attention.hpp -- internal interface of the fused attention kernels (attention.hip).
#pragma once

#include "common.hpp"

namespace talos {

// q/k: [batch, seq, heads, dk] and v/o/dout: [batch, seq, heads, dv], token rows of stride ld*;
// lse (and the backward workspace D) are [batch, heads, seq].
struct AttnDesc {
  int batch = 0, seq = 0, heads = 0, dk = 0, dv = 0;
  float scale = 1.f;
  int causal = 0;
  const float* q = nullptr;
  long long ldq = 0;
  const float* k = nullptr;
  long long ldk = 0;
  const float* v = nullptr;
  long long ldv = 0;
  float* o = nullptr;
  long long ldo = 0;
  float* lse = nullptr;
  const float* dout = nullptr;
  long long lddo = 0;
  float* dq = nullptr;
  long long lddq = 0;
  float* dk_out = nullptr;
  long long lddk = 0;
  float* dv_out = nullptr;
  long long lddv = 0;
  // optional R^T applied to dims [rope_off, rope_off + rope_dim) of dq and dk before they are
  // stored (the q/k inputs are the rotated projections); position = sequence index
  const float* rope_cos = nullptr;
  const float* rope_sin = nullptr;
  int rope_off = 0, rope_dim = 0;
  // optional per-batch key counts: keys >= lens[b] (clamped to [0, seq]) are masked for every
  // query of batch entry b, so right-padded sequences attend only to their own tokens
  const int32_t* lens = nullptr;
};

int attn_fwd_launch(const AttnDesc& d, hipStream_t s);
size_t attn_bwd_workspace_bytes(const AttnDesc& d);
int attn_bwd_launch(const AttnDesc& d, float* ws, hipStream_t s);

}  // namespace talos
