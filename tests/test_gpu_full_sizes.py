"""The fused plans at BASELINE.json's full sizes (C3 block B512 S64, C4 PPO minibatch 4096 x 32,
C5 MLA block B64 S256 d512), where the f64 oracle of the whole batch would take minutes.

Two size-independent checks stand in for it:
* batch entries are independent in the forward pass and in dx, so rows of the full run equal the
  oracle run on just those entries (the first and the last);
* the loss is a sum (C3, C5) or a mean (C4) over batch entries, so the full run's parameter
  gradient equals the sum (mean) of the gradients of disjoint sub-batches run separately. The
  sub-batches take other grid shapes and split-K counts, so this also checks that the full-size
  launch geometry changes nothing.
Tolerance: the fp32 rule of the other parity tests (parameter gradients with the scale floor);
bf16 at its normwise 2e-2.
"""
import numpy as np
import pytest

import talos_hip as th
from common import BF16_RTOL, GRAD_SCALE_FLOOR, block_params, check_close, f32, gacha_states, mla_params, ppo_params

pytestmark = pytest.mark.gpu
DA = th.DeviceArray


def _block_run(cfg, P, x, G):
    plan = th.Plan("block", cfg)
    X, Gd = DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(P.size), DA.zeros(x.shape)
    th.call("talos_block_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    res = out.numpy(), dp.numpy(), dx.numpy()
    plan.destroy()
    for a in (X, Gd, out, dp, dx):
        a.free()
    return res


def test_c3_block_full_size(oracle):
    B, S, d, H, F = 512, 64, 128, 4, 512
    rng = np.random.default_rng(33)
    p = f32(block_params(rng, d, F, gain_jitter=True))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    P = DA.from_numpy(p)
    out, dp, dx = _block_run(th.BlockCfg(B, S, d, H, d // H, F, 1, 0, 1e-6, 1e4), P, x, G)
    # entries 0 and B-1 against the oracle
    sel = [0, B - 1]
    ocfg = oracle.BlockCfg(2, S, d, H, d // H, F, 1, 0, 1e-6, 1e4)
    out_r, _, dx_r = oracle.block_fwd_bwd(ocfg, p, x[sel], G[sel])
    check_close(out[sel], out_r, name="out rows")
    check_close(dx[sel], dx_r, name="dx rows")
    # loss = sum(out * G) is additive over the batch
    half = th.BlockCfg(B // 2, S, d, H, d // H, F, 1, 0, 1e-6, 1e4)
    _, dp0, _ = _block_run(half, P, x[:B // 2], G[:B // 2])
    _, dp1, _ = _block_run(half, P, x[B // 2:], G[B // 2:])
    check_close(dp, dp0.astype(np.float64) + dp1, name="dparams = sum over halves", scale_floor=GRAD_SCALE_FLOOR)


def test_c4_ppo_full_size(oracle):
    B, S = 4096, 32
    args = (B, S, 8, 128, 2, 4, 32, 512, 3, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    rng = np.random.default_rng(44)
    p = f32(ppo_params(rng, ocfg))
    states = f32(gacha_states(rng, B, S))
    actions = rng.integers(0, 3, B).astype(np.int32)
    adv, ret = f32(rng.normal(size=B)), f32(rng.normal(size=B))
    old = f32(rng.normal(size=B) * 0.2 - 1.1)
    plan = th.Plan("ppo", cfg)
    P, St, Ac = DA.from_numpy(p), DA.from_numpy(states), DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
    full_loss, full_dp = float(loss.numpy()[0]), dp.numpy()
    lg = DA.zeros((B, 3))
    th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, None, None)
    # samples 0 and B-1 against the oracle
    sel = [0, B - 1]
    a2 = list(args)
    a2[0] = 2
    _, logits_r, _, _ = oracle.ppo_fwd_bwd(oracle.PpoCfg(*a2), p, states[sel], actions[sel], adv[sel], ret[sel],
                                           old[sel])
    check_close(lg.numpy()[sel], logits_r, name="logits rows")
    # the loss is a mean over samples: four minibatches of 1024 on the same plan
    q = B // 4
    losses, dps = [], []
    for c in range(4):
        th.call("talos_ppo_minibatch_f32", plan.h, q, P.ptr, St.offset(c * q * S * 8), None, Ac.offset(c * q),
                Ad.offset(c * q), Re.offset(c * q), Ol.offset(c * q), loss.ptr, dp.ptr, None, 0, None)
        losses.append(float(loss.numpy()[0]))
        dps.append(dp.numpy().astype(np.float64))
    check_close(full_loss, np.mean(losses), name="loss = mean over quarters")
    check_close(full_dp, np.mean(dps, axis=0), name="dparams = mean over quarters", scale_floor=GRAD_SCALE_FLOOR)
    plan.destroy()


def _mla_run(ci, prec, P, x, G):
    B, S, d, H, L, r, hd, vd, causal = ci[:9]
    plan = th.Plan("mla", th.MlaCfg(B, S, d, H, L, r, hd, vd, causal, prec, 1e-5, 1e4))
    X, Gd = DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(P.size), DA.zeros(x.shape)
    th.call("talos_mla_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    res = out.numpy(), dp.numpy(), dx.numpy()
    plan.destroy()
    for a in (X, Gd, out, dp, dx):
        a.free()
    return res


@pytest.mark.parametrize("prec", [th.PREC_FP32, th.PREC_BF16])
def test_c5_mla_full_size(oracle, prec):
    ci = [64, 256, 512, 8, 128, 32, 64, 64, 0, 0]
    B = ci[0]
    rng = np.random.default_rng(55)
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(B, ci[1], ci[2]))), f32(rng.normal(size=(B, ci[1], ci[2])))
    P = DA.from_numpy(p)
    out, dp, dx = _mla_run(ci, prec, P, x, G)
    sel = [0, B - 1]
    c2 = list(ci)
    c2[0] = 2
    out_r, _, dx_r = oracle.mla_fwd_bwd(c2, 1e-5, 1e4, p, x[sel], G[sel])
    half = list(ci)
    half[0] = B // 2
    _, dp0, _ = _mla_run(half, prec, P, x[:B // 2], G[:B // 2])
    _, dp1, _ = _mla_run(half, prec, P, x[B // 2:], G[B // 2:])
    if prec == th.PREC_FP32:
        check_close(out[sel], out_r, name="out rows")
        check_close(dx[sel], dx_r, name="dx rows")
        check_close(dp, dp0.astype(np.float64) + dp1, name="dparams = sum over halves", scale_floor=GRAD_SCALE_FLOOR)
    else:
        for name, got, ref in (("out rows", out[sel], out_r), ("dx rows", dx[sel], dx_r),
                               ("dparams = sum over halves", dp, dp0.astype(np.float64) + dp1)):
            rel = float(np.abs(got - ref).max() / np.abs(ref).max())
            assert rel <= BF16_RTOL, f"{name}: normwise relative error {rel:.3e}"
