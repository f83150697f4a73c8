"""GPU parity of the PPO update harness (src/ppo.rs:625-770): GAE + advantage normalisation
against the f64 oracle, the minibatch entry with per-sample lengths and n < batch against
per-sample oracle graphs of the unpadded lengths, and talos_ppo_update_f32 against the same
sequence of component calls made from the host.

Comparison rules: GAE advantages (f64) within 1e-12 relative to the largest; fp32 outputs
(returns, normalised advantages) within 1e-6 relative to the largest; minibatch loss, logits and
gradients at the fp32 rule of the other model tests (parameter gradients with the scale floor);
the harness and the host-driven sequence run the same deterministic kernels in the same order, so
they must agree bit for bit.
"""
import ctypes

import numpy as np
import pytest

import talos_hip as th
from common import check_close, check_grad, f32, gacha_states, ppo_params
from test_gpu_models import ppo_slices

pytestmark = pytest.mark.gpu
DA = th.DeviceArray


def cfg_args(B, S, causal, d=64, L=2, H=2, F=128, A=3):
    return (B, S, 8, d, L, H, d // H, F, A, causal, 0, 1e-5, 10000.0, 0.2, 0.5, 0.01)


@pytest.mark.parametrize("n,p_done", [(1, 0.0), (7, 0.3), (1000, 0.05), (4096, 0.01), (100003, 0.02)])
def test_gae_vs_oracle(oracle, n, p_done):
    rng = np.random.default_rng(n)
    rew, val = rng.normal(size=n) * 2.0 + 0.3, rng.normal(size=n)
    done = (rng.random(n) < p_done).astype(np.uint8)
    mu, var = 0.2, 3.0
    a_r, ret_r, an_r = oracle.ppo_gae(rew, val, done, mu, var, 10.0, 0.99, 0.95)
    R, V = DA.from_numpy(rew, np.float64), DA.from_numpy(val, np.float64)
    D = DA.zeros(n, np.uint8)
    th.call("talos_memcpy_h2d", D.ptr, done.ctypes.data, n, None)
    adv, ret, raw = DA.zeros(n), DA.zeros(n), DA.zeros(n, np.float64)
    th.call("talos_ppo_gae_f64", n, R.ptr, V.ptr, D.ptr, mu, var, 10.0, 0.99, 0.95, adv.ptr, ret.ptr, raw.ptr, None)
    got = raw.numpy()
    assert np.abs(got - a_r).max() <= 1e-12 * max(1.0, np.abs(a_r).max()), np.abs(got - a_r).max()
    assert np.abs(ret.numpy() - ret_r).max() <= 1e-6 * np.abs(ret_r).max()
    if n > 1:
        assert np.abs(adv.numpy() - an_r).max() <= 1e-6 * np.abs(an_r).max()


def test_gae_empty_is_a_no_op():
    th.call("talos_ppo_gae_f64", 0, None, None, None, 0.0, 1.0, 10.0, 0.99, 0.95, None, None, None, None)


def _varlen_inputs(rng, ocfg, n, lens):
    S = ocfg.seq
    states = f32(gacha_states(rng, n, S))
    for b, L in enumerate(lens):  # padding rows hold finite garbage: they must not leak
        states[b, L:] = f32(rng.normal(size=(S - L, ocfg.in_dim)) * 5.0)
    actions = rng.integers(0, ocfg.n_actions, n).astype(np.int32)
    adv, ret = f32(rng.normal(size=n)), f32(rng.normal(size=n))
    old = f32(rng.normal(size=n) * 0.2 - 1.1)
    return states, actions, adv, ret, old


def _oracle_varlen(oracle, args, p, states, lens, actions, adv, ret, old):
    """Per-sample oracle graphs at each sample's own length; the minibatch mean (loss, parameter
    gradients, logits, and the gradients' magnitude sums)."""
    n = len(lens)
    loss, dp, mag, logits = 0.0, np.zeros(p.size), np.zeros(p.size), []
    for b, L in enumerate(lens):
        a = list(args)
        a[0], a[1] = 1, int(L)
        oc = oracle.PpoCfg(*a)
        lb, lg, _, db, mb = oracle.ppo_fwd_bwd(oc, p, states[b:b + 1, :L], actions[b:b + 1], adv[b:b + 1],
                                               ret[b:b + 1], old[b:b + 1], mag=True)
        loss += lb / n
        dp += db / n
        mag += mb / n
        logits.append(lg[0])
    return loss, dp, np.array(logits), mag


@pytest.mark.parametrize("causal,H,S,lens,d", [(1, 2, 12, [12, 1, 7, 12, 3], 64), (0, 2, 12, [12, 1, 7, 12, 3], 64),
                                               (1, 1, 12, [12, 1, 7, 12, 3], 64), (1, 2, 40, [40, 1, 33, 17, 40], 64),
                                               (0, 2, 40, [40, 1, 33, 17, 40], 64),
                                               (1, 4, 47, [47, 1, 33, 20, 32], 128),
                                               (0, 4, 64, [64, 2, 40, 31, 64], 128),
                                               (1, 4, 32, [32, 1, 17, 20, 31], 128),
                                               (0, 4, 20, [20, 3, 20, 9, 1], 128)])
def test_minibatch_varlen_vs_oracle(oracle, causal, H, S, lens, d):
    # head dim 32 (H = 2) and 64 (H = 1): both last-query attention kernels of the last layer;
    # seq 40 at head dim 32: the first layer's backward on the four-block kernel, keys masked past
    # each sample's length; d = 128 with four heads of 32 at seq 47 / 64: the first layer's
    # forward on the eight-wave attention kernel with o.Wo, the residual and RMSNorm2 fused
    rng = np.random.default_rng(11 + causal + H + S)
    args = cfg_args(8, S, causal, d=d, H=H)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    p = f32(ppo_params(rng, ocfg))
    n = len(lens)
    states, actions, adv, ret, old = _varlen_inputs(rng, ocfg, n, lens)
    loss_r, dp_r, logits_r, mag = _oracle_varlen(oracle, args, p, states, lens, actions, adv, ret, old)

    plan = th.Plan("ppo", cfg)
    P, St, Ln = DA.from_numpy(p), DA.from_numpy(states), DA.from_numpy(np.array(lens), np.int32)
    Ac = DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    stats = DA.zeros(th.PPO_NSTATS, np.float64)
    th.call("talos_ppo_minibatch_f32", plan.h, n, P.ptr, St.ptr, Ln.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr,
            dp.ptr, stats.ptr, 0, None)
    lg = DA.zeros((n, cfg.n_actions))
    th.call("talos_ppo_forward_n_f32", plan.h, n, P.ptr, St.ptr, Ln.ptr, lg.ptr, None, None)
    check_close(lg.numpy(), logits_r, name="logits")
    check_close(loss.numpy()[0], loss_r, name="loss")
    got = dp.numpy()
    for name, sl in ppo_slices(ocfg).items():
        check_grad(got[sl], dp_r[sl], mag[sl], name=f"d{name}")
    # statistics: approx_kl and the sample count from the oracle's logits
    z = logits_r - logits_r.max(1, keepdims=True)
    lp = z - np.log(np.exp(z).sum(1, keepdims=True))
    log_ratio = lp[np.arange(n), actions] - old
    st = stats.numpy()
    check_close(st[th.STAT_KL], np.sum(np.exp(log_ratio) - 1.0 - log_ratio), name="kl sum")
    check_close(st[th.STAT_ENTROPY], -np.sum(np.exp(lp) * lp), name="entropy sum")
    assert st[th.STAT_COUNT] == n
    # a second call accumulates
    th.call("talos_ppo_minibatch_f32", plan.h, n, P.ptr, St.ptr, Ln.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, None,
            dp.ptr, stats.ptr, 1, None)
    assert stats.numpy()[th.STAT_COUNT] == 2 * n
    plan.destroy()


def test_minibatch_rejects_n_outside_the_plan():
    cfg = th.PpoCfg(*cfg_args(4, 6, 1))
    plan = th.Plan("ppo", cfg)
    p = ctypes.c_void_p(16)
    for n in (0, 5):
        rc = th.lib().talos_ppo_minibatch_f32(plan.h, n, p, p, None, p, p, p, p, None, p, None, 0, None)
        assert rc == th.ERR_SHAPE
    plan.destroy()


class _Rollout:
    def __init__(self, oracle, seed, n, B=8, S=10):
        rng = np.random.default_rng(seed)
        self.args = cfg_args(B, S, 1, L=1)
        self.cfg, ocfg = th.PpoCfg(*self.args), oracle.PpoCfg(*self.args)
        self.p0 = f32(ppo_params(rng, ocfg))
        self.lens = rng.integers(1, S + 1, n).astype(np.int32)
        st, self.actions, _, _, self.old = _varlen_inputs(rng, ocfg, n, self.lens)
        self.states = st
        self.rew = rng.normal(size=n) * 2.0
        self.val = rng.normal(size=n)
        self.done = (rng.random(n) < 0.1).astype(np.uint8)
        self.n = n

    def device(self):
        d = {k: DA.from_numpy(getattr(self, k)) for k in ("states", "old")}
        d["lens"] = DA.from_numpy(self.lens, np.int32)
        d["actions"] = DA.from_numpy(self.actions, np.int32)
        d["rew"] = DA.from_numpy(self.rew, np.float64)
        d["val"] = DA.from_numpy(self.val, np.float64)
        d["done"] = DA.zeros(self.n, np.uint8)
        th.call("talos_memcpy_h2d", d["done"].ptr, self.done.ctypes.data, self.n, None)
        d["P"] = DA.from_numpy(self.p0)
        d["m"], d["v"] = DA.zeros(self.p0.size), DA.zeros(self.p0.size)
        return d


RM, RV, CLIP, GAMMA, LAM, LR = 0.1, 2.0, 10.0, 0.99, 0.95, 1e-3


def _run_harness(plan, ro, d, k_epochs, target_kl, t0=0):
    work = DA.zeros(th.lib().talos_ppo_update_work_bytes(plan.h, ro.n) // 4 + 1)
    a = th.PpoUpdateArgs(ro.n, d["states"].ptr, d["lens"].ptr, d["actions"].ptr, d["old"].ptr, d["rew"].ptr,
                         d["val"].ptr, d["done"].ptr, RM, RV, CLIP, GAMMA, LAM, target_kl, k_epochs, LR, d["P"].ptr,
                         d["m"].ptr, d["v"].ptr, t0, work.ptr)
    res = th.PpoUpdateResult()
    th.call("talos_ppo_update_f32", plan.h, ctypes.byref(a), ctypes.byref(res), None)
    return a, res


def _run_components(plan, ro, d, k_epochs):
    """PPO::update's loop written out on the host with the component entry points."""
    n, B = ro.n, ro.cfg.batch
    S, I = ro.cfg.seq, ro.cfg.in_dim
    adv, ret = DA.zeros(n), DA.zeros(n)
    th.call("talos_ppo_gae_f64", n, d["rew"].ptr, d["val"].ptr, d["done"].ptr, RM, RV, CLIP, GAMMA, LAM, adv.ptr,
            ret.ptr, None, None)
    grads, stats = DA.zeros(ro.p0.size), DA.zeros(th.PPO_NSTATS, np.float64)
    t, kls = 0, []
    for _ in range(k_epochs):
        for start in range(0, n, B):
            nb = min(B, n - start)
            th.call("talos_ppo_minibatch_f32", plan.h, nb, d["P"].ptr, d["states"].offset(start * S * I),
                    d["lens"].offset(start), d["actions"].offset(start), adv.offset(start), ret.offset(start),
                    d["old"].offset(start), None, grads.ptr, stats.ptr, int(start > 0), None)
            t += 1
            th.call("talos_adam_step_f32", ro.p0.size, d["P"].ptr, grads.ptr, d["m"].ptr, d["v"].ptr, t, LR, 0.9,
                    0.999, 1e-8, None, 0.0, None)
        st = stats.numpy()
        kls.append(st[th.STAT_KL] / st[th.STAT_COUNT])
    return t, kls


def test_update_equals_component_sequence(oracle):
    ro = _Rollout(oracle, 21, n=20)
    plan = th.Plan("ppo", ro.cfg)
    d1, d2 = ro.device(), ro.device()
    a, res = _run_harness(plan, ro, d1, 3, target_kl=1e9)
    t, kls = _run_components(plan, ro, d2, 3)
    assert res.epochs_run == 3 and res.stopped_early == 0
    assert a.adam_t == t == 9  # 3 epochs x ceil(20 / 8) minibatches
    assert res.approx_kl == kls[-1]
    for k in ("P", "m", "v"):
        assert np.array_equal(d1[k].numpy(), d2[k].numpy()), k
    assert not np.array_equal(d1["P"].numpy(), ro.p0)  # the update moved the parameters
    plan.destroy()


def test_update_kl_early_stop(oracle):
    ro = _Rollout(oracle, 22, n=13)
    plan = th.Plan("ppo", ro.cfg)
    d = ro.device()
    # approx_kl >= 0 with equality only at ratio 1; old log-probs differ from the policy's, so a
    # target of 0 stops after the first epoch (src/ppo.rs:761-768)
    a, res = _run_harness(plan, ro, d, 4, target_kl=0.0, t0=5)
    assert res.epochs_run == 1 and res.stopped_early == 1
    assert a.adam_t == 5 + 2
    assert res.approx_kl > 0
    # an empty rollout returns at once
    empty = th.PpoUpdateArgs()
    out = th.PpoUpdateResult()
    th.call("talos_ppo_update_f32", plan.h, ctypes.byref(empty), ctypes.byref(out), None)
    assert out.epochs_run == 0
    plan.destroy()


def test_update_one_step_vs_oracle(oracle):
    """One epoch over one minibatch: GAE, the minibatch gradient and the first Adam step, against
    the oracle's GAE, per-sample graphs and f64 Adam. At t = 1 Adam moves each parameter by
    lr * g / (|g| + eps), i.e. by about lr * sign(g), so the comparison keeps the parameters whose
    oracle gradient is not tiny (|g| > 1e-3 max|g|): for the others fp32 rounding may flip the
    sign."""
    ro = _Rollout(oracle, 23, n=8)  # n = the plan's batch: a single minibatch
    plan = th.Plan("ppo", ro.cfg)
    d = ro.device()
    a, res = _run_harness(plan, ro, d, 1, target_kl=1e9)
    assert res.epochs_run == 1 and a.adam_t == 1
    _, _, adv_n = oracle.ppo_gae(ro.rew, ro.val, ro.done, RM, RV, CLIP, GAMMA, LAM)
    _, ret_r, _ = oracle.ppo_gae(ro.rew, ro.val, ro.done, RM, RV, CLIP, GAMMA, LAM)
    _, g_r, _, _ = _oracle_varlen(oracle, ro.args, ro.p0, ro.states, list(ro.lens), ro.actions, f32(adv_n),
                                  f32(ret_r), ro.old)
    p_r, m_r, v_r = ro.p0.astype(np.float64), np.zeros(ro.p0.size), np.zeros(ro.p0.size)
    oracle.adam_step(p_r, g_r, m_r, v_r, 1, LR)
    keep = np.abs(g_r) > 1e-3 * np.abs(g_r).max()
    assert keep.sum() > 0.5 * keep.size
    got = d["P"].numpy().astype(np.float64) - ro.p0
    check_close(got[keep], (p_r - ro.p0)[keep], rtol=1e-3, atol=1e-7, name="first Adam step")
    plan.destroy()
