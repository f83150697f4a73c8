// plans.hpp -- internal access to the model plans (plans.hip) for the other translation units:
// the flat parameter layouts of talos_block_cfg / talos_ppo_cfg and the configuration checks.
#pragma once

#include <cstddef>

#include "common.hpp"

namespace talos {

// The configuration of a PPO plan, or nullptr when plan is not one.
const talos_ppo_cfg* ppo_plan_cfg(talos_plan plan);

// Shape of one latent attention (a TALOS_ATTN_MLA block, or an MLA plan).
struct MlaDims {
  int batch, seq, d, H, L, r, hd, vd, causal;
};
MlaDims mla_dims(const talos_block_cfg& c);
MlaDims mla_dims(const talos_mla_cfg& c);

// Offsets of the latent-attention weights W_dkv | W_uk | W_uv | W_q | W_kr | W_qr | W_o (the
// order of MultiHeadLatentAttention::parameters, src/transformer.rs:466-476) from base.
struct MlaW {
  size_t wdkv, wuk, wuv, wq, wkr, wqr, wo, end;
};
MlaW mla_weights(const MlaDims& D, size_t base);

// Width of a block's attention output (the rows of Wo) and of its RoPE table.
int attn_width(const talos_block_cfg& c);
int rope_width(const talos_block_cfg& c);

// Offsets of one block's parameters inside a flat buffer.
struct BlockOff {
  size_t g1, wqkv, wo, g2, w1, b1, w2, b2, end;
  MlaW mla;  // TALOS_ATTN_MLA: the attention weights (mla.wo == wo)
};
BlockOff block_offsets(const talos_block_cfg& c, size_t base);
size_t block_params(const talos_block_cfg& c);

// The policy's layout: embed | blocks | final gain | out_proj | actor | critic.
struct PpoOff {
  size_t we, be, blocks, gf, wout, bout, wa, ba, wc, bc, end;
};
PpoOff ppo_offsets(const talos_ppo_cfg& c);
talos_block_cfg block_cfg_of(const talos_ppo_cfg& p);

// Host-side configuration checks (TALOS_OK or a status with the message set).
int check_block_cfg(const talos_block_cfg& c);
int check_ppo_cfg(const talos_ppo_cfg& c);

}  // namespace talos
