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
  // last-query kernels only: the query of batch entry b is row b of q_last ([batch, heads * dk],
  // not yet rotated: the kernels apply RoPE at the last row's position), and the backward writes
  // the query gradient to row b of dq_last instead of every row of dq
  const float* q_last = nullptr;
  long long ldq_last = 0;
  float* dq_last = nullptr;
  long long lddq_last = 0;
  // optional scratch of attn_bwd_ds_bytes(d) bytes (16-byte aligned): where attn_bwd_ds_supported
  // holds (attn_ds_path), the backward forms D = rowsum(dO * O) first, stores dS
  // ([batch * heads][seq][seq]) from its dK / dV kernel and forms dQ = dS . K from it instead of
  // forming S, P and dP a second time
  float* ds = nullptr;
  // on that path only (attn_ds_path): columns [dsplit, dk) of each head's dq / dk go to dq2 /
  // dk2 (head width dk - dsplit, row pitch lddq2 / lddk2) and columns [0, dsplit) to dq / dk_out
  // at head width dsplit, instead of one [.., heads * dk] row each
  float* dq2 = nullptr;
  long long lddq2 = 0;
  float* dk2 = nullptr;
  long long lddk2 = 0;
  int dsplit = 0;
  // 1: where the backward takes the dS path (ds given, attn_bwd_ds_supported), the tiled forward
  // and that backward take bf16 operands in their QK^T, PV and gradient contractions (rounded to
  // nearest even as staged, fp32 accumulation; softmax, lse and D in fp32, dS formed in fp32 and
  // kept in ds as bf16 rows), for plans whose products are bf16-in. Other shapes run in fp32,
  // forward and backward alike.
  int bf16 = 0;
  // 1 (with bf16, on the dS path only): the backward writes dq, dq2, dk_out, dk2 and dv_out as bf16
  // (nearest even) into uint16_t buffers at those pointers, with the same leading dimensions in
  // elements, instead of fp32, for plans whose later products read only bf16 copies of them.
  int out_bf16 = 0;
  // 1 (on the dS path): D = rowsum(dO . O) is already in the backward's workspace (ws[(b * heads +
  // h) * seq + query], e.g. from the product that formed dO, GemmDesc::rd_*), so it is not formed.
  int d_ready = 0;
};

int attn_fwd_launch(const AttnDesc& d, hipStream_t s);

// The attention forward fused with the output projection, its residual and the following
// RMSNorm (S <= 64, four 32-wide heads, d = 128, o rows of 128): besides o and lse it writes
// h2 = resid + o.Wo, xn = rmsnorm(h2) * gain and rstd (optional), all rows of 128 floats.
struct AttnWoDesc {
  const float* wo = nullptr;  // [128, 128], row = input feature
  const float* resid = nullptr;
  float* h2 = nullptr;
  const float* gain = nullptr;
  float* xn = nullptr;
  float* rstd = nullptr;
  float eps = 1e-5f;
};
int attn_fwd_wo_supported(const AttnDesc& d, const AttnWoDesc& w);
int attn_fwd_wo_launch(const AttnDesc& d, const AttnWoDesc& w, hipStream_t s);

// Attention of the last query row of each batch entry only (row lens[b] - 1, or seq - 1), over all
// of that entry's keys: o_last / do_last are [batch, heads * dv] with row strides ldol / lddol,
// lse_last is [batch * heads]. The backward takes dO on that row only and writes every row of
// dq (zero except the last), dk and dv. Head dims 32 or 64 with dk == dv and 16-byte aligned
// q / k / v rows (attn_lastq_supported).
int attn_lastq_supported(const AttnDesc& d);
int attn_fwd_lastq_launch(const AttnDesc& d, float* o_last, long long ldol, float* lse_last, hipStream_t s);
int attn_bwd_lastq_launch(const AttnDesc& d, const float* o_last, long long ldol, const float* lse_last,
                          const float* do_last, long long lddol, hipStream_t s);
// The last query with the value projection absorbed (v_j = xn_j . Wv carries no rotation): the
// forward writes z[b][h] = sum_j p_j xn_j ([B][H][128], the caller forms o_h = z_h . Wv_h) and
// lse; the backward takes u[b][h] = Wv_h . dO_h ([B][H][128]) and writes dk (d.dk_out), the last
// query's dq (d.dq_last) and every row's weights prow[b*S + j][h] = p_j^h ([B*S][4],
// zero past each sample's keys). Head dims 32, four heads, xn rows of 128 (attn_lastq_vabs_supported).
int attn_lastq_vabs_supported(const AttnDesc& d, const float* xn, long long ldx);
int attn_fwd_lastq_z_launch(const AttnDesc& d, const float* xn, long long ldx, float* z, float* lse_last,
                            hipStream_t s);
int attn_bwd_lastq_z_launch(const AttnDesc& d, const float* xn, long long ldx, const float* u, const float* o_last,
                            long long ldol, const float* lse_last, const float* do_last, long long lddol, float* prow,
                            hipStream_t s);
size_t attn_bwd_workspace_bytes(const AttnDesc& d);
bool attn_bwd_ds_supported(const AttnDesc& d);
// The one predicate of the dS path: ds given, 16-byte aligned, on attn_bwd_ds_supported's shapes.
// The forward's bf16 kernel and the backward both follow it, so a forward
// and its backward always form P from the same products (the backward then needs the workspace).
bool attn_ds_path(const AttnDesc& d);
// bytes of the dS scratch: batch * heads * seq^2 entries of 4 bytes, 2 for bf16 (d.bf16)
size_t attn_bwd_ds_bytes(const AttnDesc& d);
// Whether attn_bwd_launch reads its workspace: the split dQ / dK-dV kernels of seq > 32 keep
// D = rowsum(dO * O) there; the single-block kernel of seq <= 32 forms D in registers.
bool attn_bwd_uses_workspace(const AttnDesc& d);
int attn_bwd_launch(const AttnDesc& d, float* ws, hipStream_t s);
// The S <= 32 backward with the output projection's input gradient folded in (four 32-wide
// heads, d = 128): dO = gh2 . Wo^T is formed in the kernel from gh2 = dL/dh2 (rows of 128) and
// Wo ([128, 128]); d.dout is not read. Writes dq, dk, dv as attn_bwd_launch does.
int attn_bwd_wo_supported(const AttnDesc& d, const float* wo, const float* gh2);
int attn_bwd_wo_launch(const AttnDesc& d, const float* wo, const float* gh2, hipStream_t s);

}  // namespace talos
