"""Independent float64 forward definitions in PyTorch, differentiated by torch.autograd.

Used only by the tests to pin the oracle's hand-written backward closures: the gradients
here come from torch's automatic differentiation of a forward written from the textbook
definitions (RMSNorm, interleaved-pair RoPE, causal scaled-dot-product attention, exact GELU,
the PPO clipped objective), not from the oracle's formulas.
"""
import math

import numpy as np
import torch

torch.set_default_dtype(torch.float64)


def t64(a, grad=False):
    return torch.tensor(np.asarray(a, dtype=np.float64), dtype=torch.float64, requires_grad=grad)


def rmsnorm(x, w, eps):
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w


def rope_angles(seq, dim, base, start_pos=0):
    i = torch.arange(dim // 2, dtype=torch.float64)
    theta = 1.0 / (base ** (2.0 * i / dim))
    pos = torch.arange(start_pos, start_pos + seq, dtype=torch.float64)
    ang = pos[:, None] * theta[None, :]
    return torch.cos(ang), torch.sin(ang)


def rope(x, base, start_pos=0):
    """x [..., S, H, D] rotated by position along S, pairs (2i, 2i+1) as complex numbers."""
    S, H, D = x.shape[-3], x.shape[-2], x.shape[-1]
    c, s = rope_angles(S, D, base, start_pos)
    xc = torch.view_as_complex(x.reshape(*x.shape[:-1], D // 2, 2).contiguous())
    rot = torch.complex(c, s)[:, None, :]  # [S,1,D/2]
    return torch.view_as_real(xc * rot).reshape(x.shape)


def attention(q, k, v, scale, causal):
    """q,k [B,S,H,dk], v [B,S,H,dv] -> [B,S,H,dv]."""
    qh, kh, vh = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) * scale
    if causal:
        S = s.shape[-1]
        mask = torch.ones(S, S, dtype=torch.bool).triu(1)
        s = s.masked_fill(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vh).transpose(1, 2)


def gelu(x):
    return 0.5 * x * (1.0 + torch.erf(x / math.sqrt(2.0)))


def split_block_params(p, d, F):
    sizes = [("g1", (d,)), ("wqkv", (d, 3 * d)), ("wo", (d, d)), ("g2", (d,)), ("w1", (d, F)), ("b1", (F,)),
             ("w2", (F, d)), ("b2", (d,))]
    out, o = {}, 0
    for name, shp in sizes:
        n = int(np.prod(shp))
        out[name] = p[o:o + n].reshape(shp)
        o += n
    return out, o


def block(x, P, H, hd, eps, base, causal, act="gelu"):
    B, S, d = x.shape
    xn = rmsnorm(x, P["g1"], eps)
    qkv = xn @ P["wqkv"]
    q, k, v = qkv[..., :d], qkv[..., d:2 * d], qkv[..., 2 * d:]
    q = rope(q.reshape(B, S, H, hd), base)
    k = rope(k.reshape(B, S, H, hd), base)
    v = v.reshape(B, S, H, hd)
    o = attention(q, k, v, 1.0 / math.sqrt(hd), causal).reshape(B, S, d)
    h2 = x + o @ P["wo"]
    xn2 = rmsnorm(h2, P["g2"], eps)
    u = xn2 @ P["w1"] + P["b1"]
    a = gelu(u) if act == "gelu" else torch.relu(u)
    return h2 + a @ P["w2"] + P["b2"]


def policy(states, p, cfg):
    """Returns logits [B,A], values [B] of the talos_ppo_cfg parameter layout."""
    d, F, I, A = cfg.d_model, cfg.ffn_dim, cfg.in_dim, cfg.n_actions
    o = 0

    def take(shape):
        nonlocal o
        n = int(np.prod(shape))
        t = p[o:o + n].reshape(shape)
        o += n
        return t

    We, be = take((I, d)), take((d,))
    h = states @ We + be
    for _ in range(cfg.n_layers):
        if getattr(cfg, "attention", 0) == 1:
            h, n = mla_ffn_block(h, p[o:], cfg)
            o += n
            continue
        P, n = split_block_params(p[o:], d, F)
        o += n
        h = block(h, P, cfg.n_heads, cfg.head_dim, cfg.eps, cfg.rope_base, bool(cfg.causal),
                  "gelu" if cfg.activation == 0 else "relu")
    gf = take((d,))
    Wout, bout = take((d, d)), take((d,))
    Wa, ba = take((d, A)), take((A,))
    Wc, bc = take((d, 1)), take((1,))
    hf = rmsnorm(h, gf, cfg.eps) @ Wout + bout
    last = hf[:, -1, :]
    return last @ Wa + ba, (last @ Wc + bc)[:, 0]


def ppo_loss(logits, values, actions, old_logp, adv, ret, clip_eps, vc, ec):
    """Clipped PPO objective of src/ppo.rs:702-755 written with torch ops (mean over batch)."""
    lp = torch.log_softmax(logits, dim=-1)
    a = torch.as_tensor(np.asarray(actions, dtype=np.int64))
    logp = lp.gather(1, a[:, None])[:, 0]
    ratio = torch.exp(logp - old_logp)
    s1 = ratio * adv
    rc = torch.clamp(ratio, 1.0 - clip_eps, 1.0 + clip_eps)
    s2 = rc * adv
    pol = torch.where(s1 < s2, s1, s2)
    vl = (values - ret) ** 2
    ent = -(torch.exp(lp) * lp).sum(-1)
    return (-pol + vc * vl - ec * ent).mean()


def mla_block(x, p, ci, eps, base):
    """x + MLA(rmsnorm(x)) of src/transformer.rs:478-557 with sequence-position RoPE."""
    B, S, d, H, L, r, hd, vd, causal, literal = [int(v) for v in ci]
    o = 0

    def take(shape):
        nonlocal o
        n = int(np.prod(shape))
        t = p[o:o + n].reshape(shape)
        o += n
        return t

    g = take((d,))
    Wdkv, Wuk, Wuv = take((d, L)), take((L, H * hd)), take((L, H * vd))
    Wq, Wkr, Wqr, Wo = take((d, H * hd)), take((d, H * r)), take((d, H * r)), take((H * vd, d))
    xn = rmsnorm(x, g, eps)
    ckv = xn @ Wdkv
    kc, vc = (ckv @ Wuk).reshape(B, S, H, hd), (ckv @ Wuv).reshape(B, S, H, vd)
    qc = (xn @ Wq).reshape(B, S, H, hd)
    kr, qr = (xn @ Wkr).reshape(B, S, H, r), (xn @ Wqr).reshape(B, S, H, r)
    if literal:
        # rotate along the head axis (index along shape[-2] of [B,S,H,R])
        kr, qr = _rope_heads(kr, base), _rope_heads(qr, base)
    else:
        kr, qr = rope(kr, base), rope(qr, base)
    q = torch.cat([qc, qr], -1)
    k = torch.cat([kc, kr], -1)
    att = attention(q, k, vc, 1.0 / math.sqrt(hd + r), bool(causal)).reshape(B, S, H * vd)
    return x + att @ Wo


def _rope_heads(x, base):
    """Rotation by the head index (the reference's training-path quirk): x [B,S,H,R]."""
    B, S, H, R = x.shape
    c, s = rope_angles(H, R, base)
    xc = torch.view_as_complex(x.reshape(B, S, H, R // 2, 2).contiguous())
    return torch.view_as_real(xc * torch.complex(c, s)[None, None]).reshape(x.shape)


def mla_param_count(d, H, L, r, hd, vd):
    return d + d * L + L * H * hd + L * H * vd + d * H * hd + 2 * d * H * r + H * vd * d


def mla_ffn_block(x, p, cfg):
    """A talos_block_cfg block with MLA attention: x + MLA(rmsnorm(x)) followed by the pre-norm
    MLP, the wiring of LuckTransformer::forward (src/transformer.rs:71-90). Returns (out, number of
    parameters consumed)."""
    B, S, _ = x.shape
    d, F, H = cfg.d_model, cfg.ffn_dim, cfg.n_heads
    ci = [B, S, d, H, cfg.kv_latent, cfg.rope_dim, cfg.head_dim, cfg.v_dim, cfg.causal, 0]
    o = mla_param_count(d, H, cfg.kv_latent, cfg.rope_dim, cfg.head_dim, cfg.v_dim)
    h2 = mla_block(x, p[:o], ci, cfg.eps, cfg.rope_base)
    sizes = [(d,), (d, F), (F,), (F, d), (d,)]
    ws = []
    for shp in sizes:
        n = int(np.prod(shp))
        ws.append(p[o:o + n].reshape(shp))
        o += n
    g2, w1, b1, w2, b2 = ws
    u = rmsnorm(h2, g2, cfg.eps) @ w1 + b1
    a = gelu(u) if cfg.activation == 0 else torch.relu(u)
    return h2 + a @ w2 + b2, o
