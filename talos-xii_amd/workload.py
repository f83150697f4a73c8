"""Synthetic inputs and parameter layouts of the benchmark configurations.

Seeded numpy generators for the flat parameter layouts of talos_block_cfg / talos_ppo_cfg
(include/talos_hip.h) and for the 8-feature gacha states of the PPO configuration, whose layout
follows build_features (src/sim.rs:328-357).
"""
import math

import numpy as np


ATTN_MHA, ATTN_MLA = 0, 1  # talos_attention

# The reference's ActorCritic (ActorCritic::new, src/ppo.rs:254-258; LuckTransformer::new,
# src/transformer.rs:48-69) as talos_ppo_cfg fields after batch and seq: in_dim, d_model,
# n_layers, n_heads, head_dim, ffn_dim, n_actions, causal, activation (ReLU), eps, rope_base,
# clip_eps, value_coef, entropy_coef, attention, kv_latent, rope_dim, v_dim.
REFERENCE_ACTOR_CRITIC = (8, 64, 1, 4, 16, 128, 5, 0, 1, 1e-5, 10000.0, 0.2, 0.5, 0.01, ATTN_MLA, 32, 16, 16)


def xavier(rng, fan_in, fan_out, shape=None):
    """Xavier-uniform U(-l, l), l = sqrt(6 / (fan_in + fan_out)) (the limit of Linear::new,
    src/nn.rs:20-23, drawn over the full range)."""
    lim = math.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-lim, lim, size=shape or (fan_in, fan_out))


def block_params(rng, d, F, gain_jitter=False):
    """Flat talos_block_cfg parameters: g1 | Wqkv | Wo | g2 | W1 | b1 | W2 | b2."""
    g1 = rng.uniform(0.9, 1.1, d) if gain_jitter else np.ones(d)
    g2 = rng.uniform(0.9, 1.1, d) if gain_jitter else np.ones(d)
    parts = [g1, xavier(rng, d, d, (d, 3 * d)), xavier(rng, d, d), g2, xavier(rng, d, F),
             rng.normal(0, 0.02, F) if gain_jitter else np.zeros(F), xavier(rng, F, d),
             rng.normal(0, 0.02, d) if gain_jitter else np.zeros(d)]
    return np.concatenate([p.ravel() for p in parts])


def mla_block_params(rng, cfg, gain_jitter=False):
    """Flat talos_block_cfg parameters of a TALOS_ATTN_MLA block (the order of
    LuckTransformer::parameters, src/transformer.rs:205-215): g1 | W_dkv | W_uk | W_uv | W_q |
    W_kr | W_qr | W_o | g2 | W1 | b1 | W2 | b2."""
    d, F, H = cfg.d_model, cfg.ffn_dim, cfg.n_heads
    L, r, hd, vd = cfg.kv_latent, cfg.rope_dim, cfg.head_dim, cfg.v_dim
    gain = (lambda: rng.uniform(0.9, 1.1, d)) if gain_jitter else (lambda: np.ones(d))
    parts = [gain()] + [xavier(rng, a, b) for a, b in ((d, L), (L, H * hd), (L, H * vd), (d, H * hd), (d, H * r),
                                                          (d, H * r), (H * vd, d))]
    parts += [gain(), xavier(rng, d, F), rng.normal(0, 0.02, F) if gain_jitter else np.zeros(F), xavier(rng, F, d),
              rng.normal(0, 0.02, d) if gain_jitter else np.zeros(d)]
    return np.concatenate([p.ravel() for p in parts])


def ppo_params(rng, cfg, jitter=True):
    """Flat talos_ppo_cfg parameters (Xavier weights; gains / biases jittered when jitter)."""
    d, F, I, A = cfg.d_model, cfg.ffn_dim, cfg.in_dim, cfg.n_actions
    parts = [xavier(rng, I, d), rng.normal(0, 0.02, d) if jitter else np.zeros(d)]
    for _ in range(cfg.n_layers):
        if getattr(cfg, "attention", 0) == ATTN_MLA:
            parts.append(mla_block_params(rng, cfg, gain_jitter=jitter))
        else:
            parts.append(block_params(rng, d, F, gain_jitter=jitter))
    parts += [rng.uniform(0.9, 1.1, d) if jitter else np.ones(d), xavier(rng, d, d),
              rng.normal(0, 0.02, d) if jitter else np.zeros(d), xavier(rng, d, A),
              rng.normal(0, 0.02, A) if jitter else np.zeros(A), xavier(rng, d, 1),
              rng.normal(0, 0.02, 1) if jitter else np.zeros(1)]
    return np.concatenate([p.ravel() for p in parts])


def gacha_states(rng, B, S):
    """[B,S,8] synthetic gacha states (layout of build_features, src/sim.rs:328-357):
    pity int 0..79 normalised by 80, guarantee flag, currency U(0,1e4) log-scaled,
    pulls U(0,300) normalised, pity*flag, (pulls mod 120)/120 and its square, noise U(-1,1)."""
    pity = rng.integers(0, 80, size=(B, S)).astype(np.float64)
    flag = rng.integers(0, 2, size=(B, S)).astype(np.float64)
    cur = rng.uniform(0, 1e4, size=(B, S))
    pulls = rng.uniform(0, 300, size=(B, S))
    tn = np.mod(pulls, 120.0) / 120.0
    feats = [pity / 80.0, flag, np.log1p(cur) / np.log1p(1e4), pulls / 300.0, (pity / 80.0) * flag, tn, tn * tn,
             rng.uniform(-1, 1, size=(B, S))]
    return np.stack(feats, axis=-1)


def mla_params(rng, ci):
    """Flat MLA block parameters: g | W_dkv | W_uk | W_uv | W_q | W_kr | W_qr | W_o."""
    B, S, d, H, L, r, hd, vd = ci[:8]
    shapes = [(d, L), (L, H * hd), (L, H * vd), (d, H * hd), (d, H * r), (d, H * r), (H * vd, d)]
    parts = [rng.uniform(0.9, 1.1, d)] + [xavier(rng, s[0], s[1]) for s in shapes]
    return np.concatenate([p.ravel() for p in parts])


def log_softmax(z):
    mx = z.max(-1, keepdims=True)
    return z - mx - np.log(np.exp(z - mx).sum(-1, keepdims=True))


def ppo_step_flops(B, S, in_dim, d, L, H, F, A, causal=True, live=True):
    """Algorithmic flops of one minibatch forward + backward (multiply-add = 2 flops): per layer
    the QKV / O projections (4 * 2 M d^2), the MLP (2 * 2 M d F) and attention (QK^T and PV over
    the kept (query, key) pairs, 2 * 2 * B * H * hd * pairs); the embedding (2 M in d), and on the
    B last-token rows out_proj (2 B d^2) and the heads (2 B d (A+1)). The backward is twice the
    forward (dX and dW of every product) minus the embedding's input gradient, which is not formed.

    live=False counts the whole graph the reference builds. live=True counts the work the loss
    depends on: the heads read only the last token of each sample and everything after attention
    acts per row, so in the last layer the query projection, attention, output projection and MLP
    matter on those B rows only, while keys and values (and their gradients) still cover all M
    rows. The live attention backward of one (sample, head) is 5 products of 2 * S * hd (the last
    query's scores and dP recomputed, dq, dk, dv)."""
    M = B * S
    hd = d // H
    pairs = S * (S + 1) / 2 if causal else S * S
    layer = 4 * 2 * M * d * d + 2 * 2 * M * d * F + 2 * 2 * B * H * hd * pairs
    embed = 2 * M * in_dim * d
    heads = 2 * B * d * d + 2 * B * d * (A + 1)
    if not live or L == 0:
        return 3 * (L * layer + embed + heads) - embed
    proj_kv, proj_q, proj_o = 2 * 2 * M * d * d, 2 * B * d * d, 2 * B * d * d
    mlp = 2 * 2 * B * d * F
    last_fwd = proj_kv + proj_q + 2 * 2 * B * H * hd * S + proj_o + mlp
    last_bwd = 2 * (proj_kv + proj_q + proj_o + mlp) + 5 * 2 * B * H * hd * S
    rest = (L - 1) * layer + embed + heads
    return 3 * rest - embed + last_fwd + last_bwd

def ppo_step_executed_flops(B, S, in_dim, d, L, H, F, A, causal=True):
    """The flops the PPO plan's kernels execute for the live work (ppo_step_flops(live=True)),
    where the last layer's value projection is absorbed into its last-query attention (four heads
    of 32 at d 128): the value rows v_j = xn1_j Wv over all M rows (forward, their input gradient
    and Wv's gradient, 3 * 2 M d^2) are never formed. In their place the forward forms
    z_h = sum_j p_j xn1_j per (sample, head) and o_h = z_h Wv_h; the backward u_h = Wv_h dO_h,
    dP_j = xn1_j . u_h, the value path's share sum_h p_j^h u_h of each row's input gradient, and
    dWv = sum_b z_bh^T dO_bh."""
    live = ppo_step_flops(B, S, in_dim, d, L, H, F, A, causal)
    if L == 0 or not (H == 4 and d == 128):
        return live
    M = B * S
    absorbed = 3 * 2 * B * H * S * d + 3 * 2 * B * d * d
    return live - 3 * 2 * M * d * d + absorbed
