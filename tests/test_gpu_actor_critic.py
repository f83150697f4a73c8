"""GPU parity of blocks with latent attention (TALOS_ATTN_MLA) and of the PPO plan on the
reference's own ActorCritic (ActorCritic::new, src/ppo.rs:254-258: in 8, d 64, one MLA layer with
4 heads, latent 32, rope 16, head 16, ReLU FFN 128, 5 actions, no mask) against the f64 oracle.

The sequence length 16 is the reference trainer's ppo_context_len (data/config.json:53-54).
Tolerance: the fp32 rule of the other parity tests (parameter gradients with the magnitude-derived
allowance of common.check_grad).
"""
import ctypes

import numpy as np
import pytest

import talos_hip as th
import workload
from common import check_close, check_grad, f32, gacha_states, ppo_params

pytestmark = pytest.mark.gpu
DA = th.DeviceArray

MLA_BLOCK_NAMES = ["g1", "W_dkv", "W_uk", "W_uv", "W_q", "W_kr", "W_qr", "W_o", "g2", "W1", "b1", "W2", "b2"]


def mla_block_sizes(c):
    d, F, H, L, r, hd, vd = c.d_model, c.ffn_dim, c.n_heads, c.kv_latent, c.rope_dim, c.head_dim, c.v_dim
    return [d, d * L, L * H * hd, L * H * vd, d * H * hd, d * H * r, d * H * r, H * vd * d, d, d * F, F, F * d, d]


def ac_slices(c):
    """Named slices of the talos_ppo_cfg layout with MLA blocks."""
    d, I, A = c.d_model, c.in_dim, c.n_actions
    names = [("We", I * d), ("be", d)]
    for layer in range(c.n_layers):
        names += [(f"L{layer}.{n}", s) for n, s in zip(MLA_BLOCK_NAMES, mla_block_sizes(c))]
    names += [("gf", d), ("Wout", d * d), ("bout", d), ("Wa", d * A), ("ba", A), ("Wc", d), ("bc", 1)]
    out, o = {}, 0
    for n, s in names:
        out[n] = slice(o, o + s)
        o += s
    return out


@pytest.mark.parametrize("B,S,causal", [(3, 16, 0), (2, 37, 1)])
def test_mla_block_plan_vs_oracle(oracle, B, S, causal):
    rng = np.random.default_rng(300 + S)
    args = (B, S, 64, 4, 16, 128, causal, th.ACT_RELU, 1e-5, 10000.0, th.ATTN_MLA, 32, 16, 16)
    cfg, ocfg = th.BlockCfg(*args), oracle.BlockCfg(*args)
    p = f32(workload.mla_block_params(rng, ocfg, gain_jitter=True))
    x, G = f32(rng.normal(size=(B, S, 64))), f32(rng.normal(size=(B, S, 64)))
    out_r, dp_r, dx_r, mag = oracle.block_fwd_bwd(ocfg, p, x, G, mag=True)
    plan = th.Plan("block", cfg)
    P, X, Gd = DA.from_numpy(p), DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(p.size), DA.zeros(x.shape)
    th.call("talos_block_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    check_close(out.numpy(), out_r, name="out")
    check_close(dx.numpy(), dx_r, name="dx")
    got, o = dp.numpy(), 0
    for n, sz in zip(MLA_BLOCK_NAMES, mla_block_sizes(ocfg)):
        check_grad(got[o:o + sz], dp_r[o:o + sz], mag[o:o + sz], name=f"d{n}")
        o += sz
    plan.destroy()


def ac_args(B, S, L=1, causal=0):
    a = list(workload.REFERENCE_ACTOR_CRITIC)
    a[2], a[7] = L, causal
    return (B, S, *a)


def ac_inputs(rng, ocfg, p, oracle, spread=0.3):
    B, A = ocfg.batch, ocfg.n_actions
    states = f32(gacha_states(rng, B, ocfg.seq))
    actions = rng.integers(0, A, B).astype(np.int32)
    adv, ret = f32(rng.normal(size=B)), f32(rng.normal(size=B))
    _, logits, _, _ = oracle.ppo_fwd_bwd(ocfg, p, states, actions, adv, ret, np.zeros(B))
    mx = logits.max(1, keepdims=True)
    lp = logits - mx - np.log(np.exp(logits - mx).sum(1, keepdims=True))
    old = f32(lp[np.arange(B), actions] + rng.uniform(-spread, spread, B))
    return states, actions, adv, ret, old


@pytest.mark.parametrize("B,S,L,causal", [(16, 16, 1, 0), (5, 16, 2, 1), (64, 16, 1, 0)])
def test_actor_critic_minibatch_vs_oracle(oracle, B, S, L, causal):
    rng = np.random.default_rng(400 + B + L)
    args = ac_args(B, S, L, causal)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    p = f32(ppo_params(rng, ocfg))
    states, actions, adv, ret, old = ac_inputs(rng, ocfg, p, oracle)
    loss_r, logits_r, values_r, dp_r, mag = oracle.ppo_fwd_bwd(ocfg, p, states, actions, adv, ret, old, mag=True)
    plan = th.Plan("ppo", cfg)
    P, St = DA.from_numpy(p), DA.from_numpy(states)
    Ac = DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
    first = dp.numpy()
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
    assert np.array_equal(first, dp.numpy()), "a repeated call on the same plan changed the gradients"
    lg, vl = DA.zeros((B, cfg.n_actions)), DA.zeros(B)
    th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, vl.ptr, None)
    check_close(lg.numpy(), logits_r, name="logits")
    check_close(vl.numpy(), values_r, name="values")
    check_close(float(loss.numpy()[0]), loss_r, name="loss")
    for n, sl in ac_slices(ocfg).items():
        check_grad(first[sl], dp_r[sl], mag[sl], name=f"d{n}")
    plan.destroy()


def test_actor_critic_varlen_vs_per_sample_oracle(oracle):
    """Variable-length samples (the trainer's sequences are 1..context_len long, src/ppo.rs:856-866)
    against one oracle graph per sample at its own length."""
    rng = np.random.default_rng(500)
    S = 16
    args = ac_args(8, S)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    p = f32(ppo_params(rng, ocfg))
    lens = [16, 1, 9, 4, 16, 2]
    n = len(lens)
    states = f32(gacha_states(rng, n, S))
    for b, L in enumerate(lens):  # padding rows hold finite garbage: they must not leak
        states[b, L:] = f32(rng.normal(size=(S - L, ocfg.in_dim)) * 5.0)
    actions = rng.integers(0, ocfg.n_actions, n).astype(np.int32)
    adv, ret = f32(rng.normal(size=n)), f32(rng.normal(size=n))
    old = f32(rng.normal(size=n) * 0.2 - 1.6)
    loss_r, dp_r, mag, logits_r = 0.0, np.zeros(p.size), np.zeros(p.size), []
    for b, L in enumerate(lens):
        a = list(args)
        a[0], a[1] = 1, L
        lb, lg, _, db, mb = oracle.ppo_fwd_bwd(oracle.PpoCfg(*a), p, states[b:b + 1, :L], actions[b:b + 1],
                                               adv[b:b + 1], ret[b:b + 1], old[b:b + 1], mag=True)
        loss_r += lb / n
        dp_r += db / n
        mag += mb / n
        logits_r.append(lg[0])
    plan = th.Plan("ppo", cfg)
    P, St, Ln = DA.from_numpy(p), DA.from_numpy(states), DA.from_numpy(np.array(lens), np.int32)
    Ac = DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    th.call("talos_ppo_minibatch_f32", plan.h, n, P.ptr, St.ptr, Ln.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr,
            dp.ptr, None, 0, None)
    lg = DA.zeros((n, cfg.n_actions))
    th.call("talos_ppo_forward_n_f32", plan.h, n, P.ptr, St.ptr, Ln.ptr, lg.ptr, None, None)
    check_close(lg.numpy(), np.array(logits_r), name="logits")
    check_close(float(loss.numpy()[0]), loss_r, name="loss")
    got = dp.numpy()
    for name, sl in ac_slices(ocfg).items():
        check_grad(got[sl], dp_r[sl], mag[sl], name=f"d{name}")
    plan.destroy()


def test_actor_critic_update_runs_and_moves_params(oracle):
    """PPO::update on the reference model: two epochs over three minibatches."""
    rng = np.random.default_rng(600)
    B, S, n = 8, 16, 20
    cfg, ocfg = th.PpoCfg(*ac_args(B, S)), oracle.PpoCfg(*ac_args(B, S))
    p0 = f32(ppo_params(rng, ocfg))
    lens = rng.integers(1, S + 1, n).astype(np.int32)
    states = f32(gacha_states(rng, n, S))
    actions = rng.integers(0, ocfg.n_actions, n).astype(np.int32)
    old = f32(rng.normal(size=n) * 0.2 - 1.6)
    rew, val = rng.normal(size=n), rng.normal(size=n)
    done = (rng.random(n) < 0.1).astype(np.uint8)
    plan = th.Plan("ppo", cfg)
    P, St, Ln = DA.from_numpy(p0), DA.from_numpy(states), DA.from_numpy(lens, np.int32)
    Ac, Ol = DA.from_numpy(actions, np.int32), DA.from_numpy(old)
    Rw, Vl = DA.from_numpy(rew, np.float64), DA.from_numpy(val, np.float64)
    Dn = DA.zeros(n, np.uint8)
    th.call("talos_memcpy_h2d", Dn.ptr, done.ctypes.data, n, None)
    m, v = DA.zeros(p0.size), DA.zeros(p0.size)
    work = DA.zeros(th.lib().talos_ppo_update_work_bytes(plan.h, n) // 4 + 1)
    a = th.PpoUpdateArgs(n, St.ptr, Ln.ptr, Ac.ptr, Ol.ptr, Rw.ptr, Vl.ptr, Dn.ptr, 0.0, 1.0, 10.0, 0.99, 0.95, 1e9,
                         2, 3e-4, P.ptr, m.ptr, v.ptr, 0, work.ptr)
    res = th.PpoUpdateResult()
    th.call("talos_ppo_update_f32", plan.h, ctypes.byref(a), ctypes.byref(res), None)
    assert res.epochs_run == 2 and a.adam_t == 6
    p1 = P.numpy()
    assert np.all(np.isfinite(p1)) and not np.array_equal(p1, p0)
    # every parameter group of the backbone moved: gradients reach it through the last token
    for name, sl in ac_slices(ocfg).items():
        assert np.any(p1[sl] != p0[sl]), name
    plan.destroy()


def test_checkpoint_interop_with_the_device_path(oracle, tmp_path):
    """A reference-format checkpoint of f64 weights (the JSON document a serde_json writer would
    produce) loads into the plan, whose forward then matches the oracle run on the f64 weights;
    parameters updated on the device save back exactly (the f64 in the file is the fp32 value)."""
    import json
    from test_checkpoint import _jsonable, _tree

    rng = np.random.default_rng(700)
    B, S = 6, 16
    args = ac_args(B, S)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    p64 = ppo_params(rng, ocfg)
    path = str(tmp_path / "ppo.cache")
    with open(path, "w") as f:
        json.dump(_jsonable(_tree(cfg, p64)), f)
    p = th.load_ppo_model(cfg, path)
    assert np.array_equal(p, p64.astype(np.float32))
    states, actions, adv, ret, old = ac_inputs(rng, ocfg, p64, oracle)
    _, logits_r, values_r, _ = oracle.ppo_fwd_bwd(ocfg, p64, states, actions, adv, ret, old)
    plan = th.Plan("ppo", cfg)
    P, St = DA.from_numpy(p), DA.from_numpy(states)
    lg, vl = DA.zeros((B, cfg.n_actions)), DA.zeros(B)
    th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, vl.ptr, None)
    check_close(lg.numpy(), logits_r, name="logits from a loaded checkpoint")
    check_close(vl.numpy(), values_r, name="values from a loaded checkpoint")
    # one Adam step on the device, then save: the file holds the device's fp32 values exactly
    Ac = DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    g, m, v = DA.zeros(p.size), DA.zeros(p.size), DA.zeros(p.size)
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, None, g.ptr, None)
    th.call("talos_adam_step_f32", p.size, P.ptr, g.ptr, m.ptr, v.ptr, 1, 3e-4, 0.9, 0.999, 1e-8, None, 0.0, None)
    p1 = P.numpy()
    assert not np.array_equal(p1, p)
    th.save_ppo_model(cfg, p1, path)
    doc = json.load(open(path))
    assert doc["backbone"]["embed"]["weight"]["data"] == p1[:8 * 64].astype(np.float64).tolist()
    assert th.load_ppo_model(cfg, path).tobytes() == p1.tobytes()
    plan.destroy()
