"""Shared input generators and the comparison rule of the parity tests."""
import math

import numpy as np

# Tolerances of the north star: fp32 within 1e-4 relative with a 1e-5 absolute floor,
# bf16-input MFMA variants within 2e-2 relative (floor scaled the same way).
FP32_RTOL, FP32_ATOL = 1e-4, 1e-5
BF16_RTOL, BF16_ATOL = 2e-2, 2e-3


def f32(a):
    """Rounds to fp32 and back to f64: the exact values the GPU path sees."""
    return np.asarray(a, dtype=np.float32).astype(np.float64)


# Parameter gradients that are sums over many token rows (dW = X^T dY, dgain, db) with an
# unscaled loss hold elements that cancel to a tiny fraction of the tensor's scale; there the
# fp32 rounding of the inputs alone exceeds 1e-5 absolute (torch's own fp32 CPU autograd fails
# the plain rule on the C3 block: 118 of 197504 parameter-gradient elements at batch 64). For
# those tensors the absolute floor is raised to 1e-6 of the tensor's largest |ref| (16 fp32 ulps
# of its largest element); everything else uses the plain floor.
GRAD_SCALE_FLOOR = 1e-6


def check_close(got, ref, rtol=FP32_RTOL, atol=FP32_ATOL, name="", scale_floor=0.0):
    """Element-wise |got - ref| <= rtol * |ref| + max(atol, scale_floor * max|ref|); reports the
    worst element."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    err = np.abs(got - ref)
    if scale_floor and ref.size:
        atol = max(atol, scale_floor * float(np.abs(ref).max()))
    bound = rtol * np.abs(ref) + atol
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{name}: {int(bad.sum())}/{err.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} err {err[i]:.3e} bound {bound[i]:.3e}")
    return float((err / (np.abs(ref) + atol)).max()) if err.size else 0.0


def xavier(rng, fan_in, fan_out, shape=None):
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


def ppo_params(rng, cfg, jitter=True):
    """Flat talos_ppo_cfg parameters (Xavier weights; biases small random when jitter)."""
    d, F, I, A = cfg.d_model, cfg.ffn_dim, cfg.in_dim, cfg.n_actions
    parts = [xavier(rng, I, d), rng.normal(0, 0.02, d) if jitter else np.zeros(d)]
    for _ in range(cfg.n_layers):
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
    B, S, d, H, L, r, hd, vd = ci[:8]
    shapes = [(d, L), (L, H * hd), (L, H * vd), (d, H * hd), (d, H * r), (d, H * r), (H * vd, d)]
    parts = [rng.uniform(0.9, 1.1, d)] + [xavier(rng, s[0], s[1]) for s in shapes]
    return np.concatenate([p.ravel() for p in parts])
