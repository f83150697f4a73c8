"""The fused plans at BASELINE.json's full sizes against the f64 oracle over the whole batch:
C3 block B512 S64, C4 PPO minibatch 4096 x 32 (and a ragged minibatch of 1536 samples of lengths
1..32 on the same plan), C5 MLA block B64 S256 d512.

At these sizes the plans take their fused paths: the RMSNorm backward in the epilogue of the
d = 128 dX products (with the residual, the last-row addends and the per-sample lengths), the
RMSNorm forward in the epilogue of the 128-wide products, the embedding + norm kernel, the heads /
loss kernel and the last-row tail kernels. Each test also builds the plan with
TALOS_PLAN_UNFUSED=1, which sends every one of those through its separate-kernel path, and checks
both against the oracle (and against each other).

The oracle runs the whole batch. The PPO loss is a mean over samples, so the C4 oracle is
evaluated in chunks of samples (each a batched f64 graph; a ragged minibatch grouped by length, a
sample of length L run at seq L) and the chunks' losses and gradients are combined with weights
n_chunk / n: the same f64 mean, in a memory footprint of a few GB.

Tolerance: the fp32 rule of the other parity tests (parameter gradients with the magnitude-derived
allowance of common.check_grad, whose use conftest.py reports); bf16 at its normwise 2e-2.
"""
import contextlib
import os

import numpy as np
import pytest

import talos_hip as th
from common import (BF16_RTOL, FP32_ATOL, FP32_RTOL, GRAD_KAPPA, block_params, check_close, check_grad, check_grad_bf16, f32,
                    gacha_states, mla_params, ppo_params)
from test_gpu_models import block_slices, mla_slices, ppo_slices

pytestmark = pytest.mark.gpu
DA = th.DeviceArray

C4_ARGS = (4096, 32, 8, 128, 2, 4, 32, 512, 3, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)


@contextlib.contextmanager
def plan_mode(unfused):
    """Plans created inside take the separate-kernel paths when unfused (TALOS_PLAN_UNFUSED=1)."""
    old = os.environ.get("TALOS_PLAN_UNFUSED")
    if unfused:
        os.environ["TALOS_PLAN_UNFUSED"] = "1"
    else:
        os.environ.pop("TALOS_PLAN_UNFUSED", None)
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("TALOS_PLAN_UNFUSED", None)
        else:
            os.environ["TALOS_PLAN_UNFUSED"] = old


# ---------------------------------------------------------------------------------------------
# C4: PPO minibatch
# ---------------------------------------------------------------------------------------------
def _ppo_inputs(seed, n, lens=None, seq=None):
    rng = np.random.default_rng(seed)
    ocfg_args = list(C4_ARGS)
    p = f32(ppo_params(rng, th.PpoCfg(*ocfg_args)))
    S = seq or C4_ARGS[1]
    states = f32(gacha_states(rng, n, S))
    if lens is not None:
        for b, L in enumerate(lens):  # padding rows hold finite garbage: they must not leak
            states[b, L:] = f32(rng.normal(size=(S - L, 8)) * 5.0)
    actions = rng.integers(0, 3, n).astype(np.int32)
    adv, ret = f32(rng.normal(size=n)), f32(rng.normal(size=n))
    old = f32(rng.normal(size=n) * 0.2 - 1.1)
    return p, states, actions, adv, ret, old


def _ppo_oracle(oracle, p, states, lens, actions, adv, ret, old, chunk=512):
    """Loss, dparams (means over the n samples), logits, values and the parameter gradients'
    magnitude sums of the whole minibatch."""
    n, S = states.shape[0], states.shape[1]
    lens = np.full(n, S) if lens is None else np.asarray(lens)
    loss, dp, mag = 0.0, np.zeros(p.size), np.zeros(p.size)
    logits, values = np.zeros((n, 3)), np.zeros(n)
    for L in np.unique(lens):
        idx = np.nonzero(lens == L)[0]
        for c0 in range(0, idx.size, chunk):
            sel = idx[c0:c0 + chunk]
            a = list(C4_ARGS)
            a[0], a[1] = int(sel.size), int(L)
            lc, lg, vl, dc, mc = oracle.ppo_fwd_bwd(oracle.PpoCfg(*a), p, states[sel, :L], actions[sel], adv[sel],
                                                    ret[sel], old[sel], mag=True)
            w = sel.size / n
            loss += w * lc
            dp += w * dc
            mag += w * mc
            logits[sel], values[sel] = lg, vl
    return loss, dp, logits, values, mag


def _ppo_gpu(unfused, p, states, lens, actions, adv, ret, old):
    n = states.shape[0]
    args = list(C4_ARGS)
    args[1] = states.shape[1]  # the plan's sequence length is the inputs'
    with plan_mode(unfused):
        plan = th.Plan("ppo", th.PpoCfg(*args))
    P, St, Ac = DA.from_numpy(p), DA.from_numpy(states), DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    Ln = DA.from_numpy(np.asarray(lens), np.int32) if lens is not None else None
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    lg, vl = DA.zeros((n, 3)), DA.zeros(n)
    if lens is None and n == C4_ARGS[0]:
        th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
        th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, vl.ptr, None)
    else:
        lp = Ln.ptr if Ln is not None else None
        th.call("talos_ppo_minibatch_f32", plan.h, n, P.ptr, St.ptr, lp, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr,
                dp.ptr, None, 0, None)
        th.call("talos_ppo_forward_n_f32", plan.h, n, P.ptr, St.ptr, lp, lg.ptr, vl.ptr, None)
    res = float(loss.numpy()[0]), dp.numpy().astype(np.float64), lg.numpy(), vl.numpy()
    plan.destroy()
    return res


def _check_ppo(tag, got, ref):
    loss, dp, logits, values = got
    loss_r, dp_r, logits_r, values_r, mag = ref
    check_close(logits, logits_r, name=f"{tag} logits")
    check_close(values, values_r, name=f"{tag} values")
    check_close(loss, loss_r, name=f"{tag} loss")
    for name, sl in ppo_slices(th.PpoCfg(*C4_ARGS)).items():
        check_grad(dp[sl], dp_r[sl], mag[sl], name=f"{tag} d{name}")


def test_c4_ppo_full_size(oracle):
    B = C4_ARGS[0]
    p, states, actions, adv, ret, old = _ppo_inputs(44, B)
    ref = _ppo_oracle(oracle, p, states, None, actions, adv, ret, old)
    fused = _ppo_gpu(False, p, states, None, actions, adv, ret, old)
    _check_ppo("fused", fused, ref)
    unfused = _ppo_gpu(True, p, states, None, actions, adv, ret, old)
    _check_ppo("unfused", unfused, ref)
    # the two paths against each other: each is within the bound of the oracle, so they are within
    # twice it of each other
    check_grad(fused[1], unfused[1], ref[4], name="fused vs unfused dparams", kappa=2 * GRAD_KAPPA,
               rtol=2 * FP32_RTOL, atol=2 * FP32_ATOL)


def test_c4_ppo_ragged_full_size(oracle):
    # 1536 samples of lengths 1..32 on the 4096-sample plan: large enough for every fused path
    # (the per-sample last rows and key masks inside the fused norm-backward epilogue)
    n = 1536
    lens = np.random.default_rng(7).integers(1, 33, n)
    lens[:4] = [32, 1, 2, 31]
    p, states, actions, adv, ret, old = _ppo_inputs(45, n, lens)
    ref = _ppo_oracle(oracle, p, states, lens, actions, adv, ret, old)
    for unfused in (False, True):
        got = _ppo_gpu(unfused, p, states, lens, actions, adv, ret, old)
        _check_ppo("unfused" if unfused else "fused", got, ref)


def test_c4_ppo_seq24_full_size(oracle):
    # 4096 samples of 24 tokens: the last layer's key-gradient product still runs on 128-row
    # tiles, whose 32-row accumulator blocks now straddle samples, so it adds the value-path addend
    # row by row in its epilogue (at 32 tokens it adds it with two more matrix steps a block)
    B = C4_ARGS[0]
    p, states, actions, adv, ret, old = _ppo_inputs(47, B, seq=24)
    ref = _ppo_oracle(oracle, p, states, None, actions, adv, ret, old)
    _check_ppo("seq 24", _ppo_gpu(False, p, states, None, actions, adv, ret, old), ref)


# ---------------------------------------------------------------------------------------------
# C3: one pre-norm block
# ---------------------------------------------------------------------------------------------
def _block_run(unfused, cfg, p, x, G):
    with plan_mode(unfused):
        plan = th.Plan("block", cfg)
    P, X, Gd = DA.from_numpy(p), DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(p.size), DA.zeros(x.shape)
    th.call("talos_block_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    res = out.numpy(), dp.numpy().astype(np.float64), dx.numpy()
    plan.destroy()
    return res


@pytest.mark.parametrize("B,S,causal", [(512, 64, 1), (289, 61, 0)])
def test_c3_block_full_size(oracle, B, S, causal):
    # (289, 61): 17629 rows, not a multiple of 64, so the 64-row tiles of the d = 128 products
    # (norm backward at K = 512, the MLP output with its residual) end in a partial tile
    d, H, F = 128, 4, 512
    rng = np.random.default_rng(33 + S)
    p = f32(block_params(rng, d, F, gain_jitter=True))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    args = (B, S, d, H, d // H, F, causal, 0, 1e-6, 1e4)
    out_r, dp_r, dx_r, mag = oracle.block_fwd_bwd(oracle.BlockCfg(*args), p, x, G, mag=True)
    for unfused in (False, True):
        tag = "unfused" if unfused else "fused"
        out, dp, dx = _block_run(unfused, th.BlockCfg(*args), p, x, G)
        check_close(out, out_r, name=f"{tag} out")
        check_close(dx, dx_r, name=f"{tag} dx")
        for n, sl in block_slices(d, F).items():
            check_grad(dp[sl], dp_r[sl], mag[sl], name=f"{tag} d{n}")


# ---------------------------------------------------------------------------------------------
# C5: MLA block, fp32 and bf16-in / fp32-accumulate
# ---------------------------------------------------------------------------------------------
C5 = [64, 256, 512, 8, 128, 32, 64, 64, 0, 0]  # batch, seq, d, heads, latent, rope, head, v, causal, literal


@pytest.fixture(scope="module")
def c5_case(oracle):
    rng = np.random.default_rng(55)
    p = f32(mla_params(rng, C5))
    B, S, d = C5[0], C5[1], C5[2]
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    return p, x, G, oracle.mla_fwd_bwd(C5, 1e-5, 1e4, p, x, G, mag=True)


@pytest.mark.parametrize("prec", [th.PREC_FP32, th.PREC_BF16])
def test_c5_mla_full_size(c5_case, prec):
    p, x, G, (out_r, dp_r, dx_r, mag) = c5_case
    B, S, d, H, L, r, hd, vd, causal = C5[:9]
    plan = th.Plan("mla", th.MlaCfg(B, S, d, H, L, r, hd, vd, causal, prec, 1e-5, 1e4))
    P, X, Gd = DA.from_numpy(p), DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(p.size), DA.zeros(x.shape)
    th.call("talos_mla_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    out, dp, dx = out.numpy(), dp.numpy().astype(np.float64), dx.numpy()
    plan.destroy()
    if prec == th.PREC_FP32:
        check_close(out, out_r, name="out")
        check_close(dx, dx_r, name="dx")
        for n, sl in mla_slices(C5).items():
            check_grad(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")
    else:
        pairs = [("out", out, out_r), ("dx", dx, dx_r)] + [(f"d{n}", dp[sl], dp_r[sl])
                                                           for n, sl in mla_slices(C5).items()]
        for name, got, ref in pairs:
            rel = float(np.abs(got - ref).max() / np.abs(ref).max())
            assert rel <= BF16_RTOL, f"{name}: normwise relative error {rel:.3e}"
        for n, sl in mla_slices(C5).items():  # and element-wise, with the magnitude-derived allowance
            check_grad_bf16(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")
