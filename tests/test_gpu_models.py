"""GPU parity of the fused block (C3) and PPO policy minibatch (C4) plans against the f64 oracle.

Reduced batch sizes keep the oracle within seconds; the kernels and launch geometry are the
ones of the full configurations (d_model 128, 4 heads x 32, seq 64 / 32, 4x GELU MLP).
"""
import ctypes

import numpy as np
import pytest

import talos_hip as th
from common import block_params, check_close, check_grad, f32, gacha_states, ppo_params

pytestmark = pytest.mark.gpu
DA = th.DeviceArray

BLOCK_NAMES = ["g1", "wqkv", "wo", "g2", "w1", "b1", "w2", "b2"]


def block_slices(d, F):
    sizes = [d, 3 * d * d, d * d, d, d * F, F, F * d, d]
    out, o = {}, 0
    for n, s in zip(BLOCK_NAMES, sizes):
        out[n] = slice(o, o + s)
        o += s
    return out


def run_block(cfg, p, x, G):
    plan = th.Plan("block", cfg)
    P, X, Gd = DA.from_numpy(p), DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(p.size), DA.zeros(x.shape)
    th.call("talos_block_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    res = out.numpy(), dp.numpy(), dx.numpy()
    plan.destroy()
    return res


# head dims 6 and 10 (not multiples of 4): the RoPE epilogue's interleaved pairs straddle the
# float4 column groups and the heads, so each pair must take its own head's table entry.
# S <= 32 with four 32-wide heads at d 128 (causal and not) runs the attention kernel that also
# forms o.Wo, the residual and RMSNorm2.
@pytest.mark.parametrize("B,S,d,H,F,causal,act", [(2, 6, 16, 4, 64, 1, 0), (3, 64, 128, 4, 512, 1, 0),
                                                  (2, 33, 64, 2, 128, 0, 1), (2, 5, 24, 4, 48, 1, 0),
                                                  (3, 9, 40, 4, 80, 0, 1), (3, 23, 128, 4, 256, 0, 0),
                                                  (2, 32, 128, 4, 512, 1, 1), (2, 47, 128, 4, 256, 0, 1)])
def test_block_fwd_bwd_vs_oracle(oracle, B, S, d, H, F, causal, act):
    rng = np.random.default_rng(1000 + S + d)
    cfg = th.BlockCfg(B, S, d, H, d // H, F, causal, act, 1e-6, 10000.0)
    ocfg = oracle.BlockCfg(B, S, d, H, d // H, F, causal, act, 1e-6, 10000.0)
    p = f32(block_params(rng, d, F, gain_jitter=True))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    out_r, dp_r, dx_r, mag = oracle.block_fwd_bwd(ocfg, p, x, G, mag=True)
    out, dp, dx = run_block(cfg, p, x, G)
    check_close(out, out_r, name="out")
    check_close(dx, dx_r, name="dx")
    for n, sl in block_slices(d, F).items():
        check_grad(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")


def ppo_cfgs(oracle, B, S=32, d=128, L=2, H=4, F=512, A=3, act=0):
    args = (B, S, 8, d, L, H, d // H, F, A, 1, act, 1e-5, 10000.0, 0.2, 0.5, 0.01)
    return th.PpoCfg(*args), oracle.PpoCfg(*args)


def ppo_inputs(rng, ocfg, p, oracle, spread=0.3):
    B, A = ocfg.batch, ocfg.n_actions
    states = f32(gacha_states(rng, B, ocfg.seq))
    actions = rng.integers(0, A, B).astype(np.int32)
    adv, ret = f32(rng.normal(size=B)), f32(rng.normal(size=B))
    _, logits, _, _ = oracle.ppo_fwd_bwd(ocfg, p, states, actions, adv, ret, np.zeros(B))
    mx = logits.max(1, keepdims=True)
    lp = logits - mx - np.log(np.exp(logits - mx).sum(1, keepdims=True))
    old = f32(lp[np.arange(B), actions] + rng.uniform(-spread, spread, B))
    return states, actions, adv, ret, old


def run_ppo(cfg, p, states, actions, adv, ret, old):
    plan = th.Plan("ppo", cfg)
    P, St = DA.from_numpy(p), DA.from_numpy(states)
    Ac = DA.from_numpy(actions, np.int32)
    Ad, Re, Ol = DA.from_numpy(adv), DA.from_numpy(ret), DA.from_numpy(old)
    loss, dp = DA.zeros(1), DA.zeros(p.size)
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
    first = dp.numpy()
    # a second call on the same plan must give the same result: no state leaks between calls
    th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dp.ptr, None)
    assert np.array_equal(first, dp.numpy()), "a repeated call on the same plan changed the gradients"
    lg, vl = DA.zeros((cfg.batch, cfg.n_actions)), DA.zeros(cfg.batch)
    th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, vl.ptr, None)
    res = float(loss.numpy()[0]), dp.numpy(), lg.numpy(), vl.numpy()
    plan.destroy()
    return res


def ppo_slices(cfg):
    d, F, I, A = cfg.d_model, cfg.ffn_dim, cfg.in_dim, cfg.n_actions
    names = [("We", I * d), ("be", d)]
    for l in range(cfg.n_layers):
        names += [(f"L{l}.{n}", s) for n, s in zip(BLOCK_NAMES, [d, 3 * d * d, d * d, d, d * F, F, F * d, d])]
    names += [("gf", d), ("Wout", d * d), ("bout", d), ("Wa", d * A), ("ba", A), ("Wc", d), ("bc", 1)]
    out, o = {}, 0
    for n, s in names:
        out[n] = slice(o, o + s)
        o += s
    return out


# (B, S, layers, activation, actions): B = 6 and 40 leave a partial 16-row tile in the last-row
# kernels; act 1 (ReLU) takes their ReLU branch at the C4 width (d 128, F 512); 8 actions make the
# heads' per-wave gradient rows (d (A + 1) + A + 1 = 1161 floats) too wide for the fused heads
# kernel, so the loss kernel and the head products run instead.
@pytest.mark.parametrize("B,S,L,act,A", [(6, 5, 2, 0, 3), (64, 32, 2, 0, 3), (16, 32, 1, 0, 3), (40, 16, 2, 1, 3),
                                         (40, 16, 2, 0, 8)])
def test_ppo_minibatch_vs_oracle(oracle, B, S, L, act, A):
    rng = np.random.default_rng(2000 + B + S + A)
    cfg, ocfg = ppo_cfgs(oracle, B, S=S, L=L, act=act, A=A)
    p = f32(ppo_params(rng, ocfg))
    states, actions, adv, ret, old = ppo_inputs(rng, ocfg, p, oracle)
    loss_r, logits_r, values_r, dp_r, mag = oracle.ppo_fwd_bwd(ocfg, p, states, actions, adv, ret, old, mag=True)
    loss, dp, logits, values = run_ppo(cfg, p, states, actions, adv, ret, old)
    check_close(logits, logits_r, name="logits")
    check_close(values, values_r, name="values")
    check_close(loss, loss_r, name="loss")
    for n, sl in ppo_slices(ocfg).items():
        check_grad(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")


@pytest.mark.parametrize("B,L", [(256, 3), (1024, 2)])
def test_ppo_side_stream_backward_matches(oracle, monkeypatch, B, L):
    """The weight-gradient products on the backward's side stream (TALOS_BWD_SIDE_STREAM=1) give
    the same bits as the one-stream backward: the same products with the same splits, only
    overlapped. Three layers exercise the guards on buffers a lower layer overwrites; B = 1024
    runs the fused norm-backward epilogues and the full-width products."""
    rng = np.random.default_rng(2100 + B)
    cfg, ocfg = ppo_cfgs(oracle, B, S=32, L=L)
    p = f32(ppo_params(rng, ocfg))
    states, actions, adv, ret, old = ppo_inputs(rng, ocfg, p, oracle)
    monkeypatch.delenv("TALOS_BWD_SIDE_STREAM", raising=False)
    one = run_ppo(cfg, p, states, actions, adv, ret, old)
    monkeypatch.setenv("TALOS_BWD_SIDE_STREAM", "1")
    two = run_ppo(cfg, p, states, actions, adv, ret, old)
    assert one[0] == two[0]
    assert np.array_equal(one[1], two[1])


def test_ppo_bad_action_is_nan_not_a_fault(oracle):
    rng = np.random.default_rng(7)
    cfg, ocfg = ppo_cfgs(oracle, 4, S=4, L=1)
    p = f32(ppo_params(rng, ocfg))
    states = f32(gacha_states(rng, 4, 4))
    actions = np.array([0, 1, 5, 2], np.int32)  # 5 is out of range for 3 actions
    z = np.zeros(4, np.float32)
    loss, dp, _, _ = run_ppo(cfg, p, states, actions, z, z, z)
    assert np.isnan(loss)


MLA_NAMES = ["g", "W_dkv", "W_uk", "W_uv", "W_q", "W_kr", "W_qr", "W_o"]


def mla_slices(ci):
    B, S, d, H, L, r, hd, vd = ci[:8]
    sizes = [d, d * L, L * H * hd, L * H * vd, d * H * hd, d * H * r, d * H * r, H * vd * d]
    out, o = {}, 0
    for n, s in zip(MLA_NAMES, sizes):
        out[n] = slice(o, o + s)
        o += s
    return out


def run_mla(ci, prec, p, x, G, eps=1e-5, base=10000.0):
    B, S, d, H, L, r, hd, vd, causal = ci[:9]
    cfg = th.MlaCfg(B, S, d, H, L, r, hd, vd, causal, prec, eps, base)
    plan = th.Plan("mla", cfg)
    assert plan.n_params == p.size
    P, X, Gd = DA.from_numpy(p), DA.from_numpy(x), DA.from_numpy(G)
    out, dp, dx = DA.zeros(x.shape), DA.zeros(p.size), DA.zeros(x.shape)
    th.call("talos_mla_fwd_bwd_f32", plan.h, P.ptr, X.ptr, Gd.ptr, out.ptr, dp.ptr, dx.ptr, None)
    res = out.numpy(), dp.numpy(), dx.numpy()
    plan.destroy()
    return res


@pytest.mark.parametrize("ci", [[2, 5, 16, 2, 8, 4, 8, 8, 0, 0], [2, 37, 64, 2, 32, 8, 16, 16, 1, 0],
                                [2, 64, 512, 8, 128, 32, 64, 64, 0, 0], [2, 100, 64, 2, 32, 8, 16, 16, 1, 0],
                                [1, 132, 512, 8, 128, 32, 64, 64, 1, 0]])
def test_mla_fwd_bwd_vs_oracle(oracle, ci):
    # the third case is C5's block (d512, 8 heads, latent 128, rope 32, head 64, v 64) at batch 2;
    # the last two (seq 100, 132: a partial last key block, causal) take the backward that stores
    # dS from its dK / dV kernel and forms dQ from it
    from common import mla_params
    rng = np.random.default_rng(3000 + ci[1] + ci[2])
    B, S, d = ci[:3]
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    out_r, dp_r, dx_r, mag = oracle.mla_fwd_bwd(ci, 1e-5, 10000.0, p, x, G, mag=True)
    out, dp, dx = run_mla(ci, th.PREC_FP32, p, x, G)
    check_close(out, out_r, name="out")
    check_close(dx, dx_r, name="dx")
    for n, sl in mla_slices(ci).items():
        check_grad(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_mla_without_ds_buffer_vs_oracle(oracle, monkeypatch, prec):
    """With the dS budget at 0 (TALOS_DS_BUDGET_MB=0 at plan creation) the MLA plan keeps no dS
    rows: its forward and backward both take the tiled path (fp32 attention, also in a bf16 plan)
    and still match the oracle, at seq 132 (causal, C5's head dims) where the dS path would run."""
    from common import BF16_RTOL, mla_params
    monkeypatch.setenv("TALOS_DS_BUDGET_MB", "0")
    ci = [1, 132, 512, 8, 128, 32, 64, 64, 1, 0]
    rng = np.random.default_rng(4100)
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(1, 132, 512))), f32(rng.normal(size=(1, 132, 512)))
    out_r, dp_r, dx_r, mag = oracle.mla_fwd_bwd(ci, 1e-5, 10000.0, p, x, G, mag=True)
    out, dp, dx = run_mla(ci, th.PREC_FP32 if prec == "fp32" else th.PREC_BF16, p, x, G)
    if prec == "fp32":
        check_close(out, out_r, name="out")
        check_close(dx, dx_r, name="dx")
        for n, sl in mla_slices(ci).items():
            check_grad(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")
    else:
        for name, got, ref in [("out", out, out_r), ("dx", dx, dx_r)] + [(f"d{n}", dp[sl], dp_r[sl])
                                                                          for n, sl in mla_slices(ci).items()]:
            assert float(np.abs(got - ref).max() / np.abs(ref).max()) <= BF16_RTOL, name


@pytest.mark.parametrize("ci", [[2, 64, 512, 8, 128, 32, 64, 64, 0, 0], [2, 100, 64, 2, 32, 8, 16, 16, 1, 0],
                                [2, 37, 20, 3, 12, 4, 12, 4, 1, 0], [64, 256, 512, 8, 128, 32, 64, 64, 0, 0]])
def test_mla_bf16_copies_bit_identical(monkeypatch, ci):
    """The bf16 plan's copies (weights, output gradient, activations and attention results
    converted to bf16 once, products reading them) give bit-identical results to the same plan
    rounding the fp32 operands at staging (TALOS_BF16_COPIES=0): the roundings, the products'
    accumulation order and the splits are the same, so any difference is a copy that is stale,
    misplaced or read at the wrong offset."""
    from common import mla_params
    rng = np.random.default_rng(4200 + ci[1] + ci[2])
    B, S, d = ci[:3]
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    with_copies = run_mla(ci, th.PREC_BF16, p, x, G)
    monkeypatch.setenv("TALOS_BF16_COPIES", "0")
    without = run_mla(ci, th.PREC_BF16, p, x, G)
    for name, a, b in zip(("out", "dparams", "dx"), with_copies, without):
        assert np.array_equal(a, b), f"{name}: {int((a != b).sum())} elements differ, max {np.abs(a - b).max():.3e}"


@pytest.mark.parametrize("prec", [th.PREC_FP32, th.PREC_BF16])
@pytest.mark.parametrize("ci", [[2, 100, 128, 4, 32, 8, 24, 32, 1, 0], [1, 132, 512, 8, 128, 32, 64, 64, 1, 0],
                                [2, 256, 512, 8, 128, 32, 64, 64, 0, 0]])
def test_mla_fused_rowdot_bit_identical(monkeypatch, ci, prec):
    """The attention backward's D = rowsum(dO . O) formed in the epilogue of the product that
    forms dO gives bit-identical results to the row-dot kernel (TALOS_MLA_ROWDOT=0): the epilogue
    sums each head's products in that kernel's lanes and order, so a difference is a wrong row,
    head or D index. Head widths 32 and 64, causal and not."""
    from common import mla_params
    rng = np.random.default_rng(4300 + ci[1] + ci[2])
    B, S, d = ci[:3]
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    fused = run_mla(ci, prec, p, x, G)
    monkeypatch.setenv("TALOS_MLA_ROWDOT", "0")
    apart = run_mla(ci, prec, p, x, G)
    for name, a, b in zip(("out", "dparams", "dx"), fused, apart):
        assert np.array_equal(a, b), f"{name}: {int((a != b).sum())} elements differ, max {np.abs(a - b).max():.3e}"


@pytest.mark.parametrize("kind", ["block", "mla_fp32", "mla_bf16"])
def test_held_split_combinations_bit_identical(monkeypatch, kind):
    """The block and MLA backward hold their split-K weight gradients' combinations back and run
    them as one batched launch at the end (each product's partials in a workspace slot of its
    own); the batch sums each as the product's own combination would, so the results equal the
    backward that combines each product at once (TALOS_BWD_SIDE_STREAM=1, under which nothing is
    held: a side stream's products would not be ordered before the batch)."""
    from common import mla_params
    rng = np.random.default_rng(4400 + len(kind))
    if kind == "block":
        B, S, d, F = 64, 64, 128, 512
        cfg = th.BlockCfg(B, S, d, 4, d // 4, F, 1, 0, 1e-6, 10000.0)
        p = f32(block_params(rng, d, F, gain_jitter=True))
        x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
        run = lambda: run_block(cfg, p, x, G)  # noqa: E731
    else:
        ci = [8, 256, 512, 8, 128, 32, 64, 64, 0, 0]
        prec = th.PREC_BF16 if kind == "mla_bf16" else th.PREC_FP32
        p = f32(mla_params(rng, ci))
        x, G = f32(rng.normal(size=(ci[0], ci[1], ci[2]))), f32(rng.normal(size=(ci[0], ci[1], ci[2])))
        run = lambda: run_mla(ci, prec, p, x, G)  # noqa: E731
    monkeypatch.delenv("TALOS_BWD_SIDE_STREAM", raising=False)
    held = run()
    monkeypatch.setenv("TALOS_BWD_SIDE_STREAM", "1")
    at_once = run()
    for name, a, b in zip(("out", "dparams", "dx"), held, at_once):
        assert np.array_equal(a, b), f"{name}: {int((a != b).sum())} elements differ, max {np.abs(a - b).max():.3e}"


def test_mla_plan_over_ds_budget_is_created():
    """A plan whose dS rows would exceed the budget (seq 2048 at batch 64, 8 heads: 8.6 GB in
    fp32, 4.3 GB in bf16, against 4 GiB) is still created, on the tiled path."""
    for prec in (th.PREC_FP32, th.PREC_BF16):
        plan = th.Plan("mla", th.MlaCfg(64, 2048, 512, 8, 128, 32, 64, 64, 0, prec, 1e-5, 10000.0))
        plan.destroy()


# seq 100 / 132 / 256 reach the bf16 tiled forward and dS backward (causal with ragged tiles,
# C5's head dims non-causal); at 37 and 64 attention runs in fp32. The d = 20 case has row lengths
# (20, 36, 12, 12) that are multiples of 4, as the plan requires, but not of 8, so the products
# read their operands' bf16 copies element by element instead of in 16-byte pieces.
@pytest.mark.parametrize("ci", [[2, 37, 20, 3, 12, 4, 12, 4, 1, 0],
                                [2, 37, 64, 2, 32, 8, 16, 16, 1, 0], [2, 64, 512, 8, 128, 32, 64, 64, 0, 0],
                                [2, 100, 64, 2, 32, 8, 16, 16, 1, 0], [1, 132, 512, 8, 128, 32, 64, 64, 1, 0],
                                [1, 256, 512, 8, 128, 32, 64, 64, 0, 0]])
def test_mla_bf16_vs_oracle(oracle, ci):
    # bf16-in / fp32-accumulate GEMMs against the f64 oracle: out and dx within 2e-2 relative in the
    # max norm, max|got - ref| <= 2e-2 * max|ref|; every parameter-gradient element within 2e-2 of
    # its own value plus the magnitude-derived allowance (common.check_grad_bf16), the form of the
    # fp32 rule with bf16's unit roundoff (bf16 keeps 8 significand bits, so an element that cancels
    # toward zero has no element-wise relative bound of its own)
    from common import BF16_RTOL, check_grad_bf16, mla_params
    rng = np.random.default_rng(4000 + ci[1] + ci[2])
    B, S, d = ci[:3]
    p = f32(mla_params(rng, ci))
    x, G = f32(rng.normal(size=(B, S, d))), f32(rng.normal(size=(B, S, d)))
    out_r, dp_r, dx_r, mag = oracle.mla_fwd_bwd(ci, 1e-5, 10000.0, p, x, G, mag=True)
    out, dp, dx = run_mla(ci, th.PREC_BF16, p, x, G)

    def chk(got, ref, name):
        assert np.all(np.isfinite(got)), name
        rel = float(np.abs(got - ref).max() / np.abs(ref).max())
        print(f"{name}: max|err| / max|ref| = {rel:.3e}")
        assert rel <= BF16_RTOL, f"{name}: normwise relative error {rel:.3e} > {BF16_RTOL}"

    chk(out, out_r, "out")
    chk(dx, dx_r, "dx")
    for n, sl in mla_slices(ci).items():
        chk(dp[sl], dp_r[sl], f"d{n}")
        check_grad_bf16(dp[sl], dp_r[sl], mag[sl], name=f"d{n}")
