"""Pins the f64 oracle before it is trusted as the checker of the HIP path.

Three kinds of evidence, chosen so that a dropped term, a wrong sign or index or a
transposed operand fails at least one of them:
  1. the reference's own known-answer tests (src/grad_check.rs, src/autograd.rs and
     src/transformer.rs #[cfg(test)] blocks), restated on the oracle's tape;
  2. central finite differences of every op's forward against its hand-written backward;
  3. closed forms and invariants, and torch float64 autograd (an independent library)
     on the composite models.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import torch_ref as tr
from common import block_params, gacha_states, mla_params, ppo_params, reference_init_actor_critic, xavier
from workload import REFERENCE_ACTOR_CRITIC, mla_block_params

# ---------------------------------------------------------------------------
# 1. Reference known-answer tests
# ---------------------------------------------------------------------------


def test_kat_matmul_grad(oracle):
    # src/grad_check.rs:30-63: A=[[2,3],[4,5]], x=[1,2]^T, L=sum(Ax): dx=[6,8], dA=[[1,2],[1,2]]
    T = oracle.T
    a = T.new([2.0, 3.0, 4.0, 5.0], [2, 2])
    x = T.new([1.0, 2.0], [2, 1])
    loss = a.matmul(x).sum()
    loss.backward()
    assert np.allclose(x.grad.ravel(), [6.0, 8.0], atol=1e-6)
    assert np.allclose(a.grad.ravel(), [1.0, 2.0, 1.0, 2.0], atol=1e-6)
    assert loss.data.ravel()[0] == 22.0


def test_kat_broadcast_grad(oracle):
    # src/grad_check.rs:66-90: z = x + broadcast(y): dx=[1,1], dy=2
    T = oracle.T
    x = T.new([1.0, 2.0], [2])
    y = T.new([10.0], [1])
    z = x + y.broadcast([2])
    z.sum().backward()
    assert np.allclose(x.grad, [1.0, 1.0])
    assert np.allclose(y.grad, [2.0])


def test_kat_numerical_gradient(oracle):
    # src/grad_check.rs:93-114: f = x^2 * sin x at 2.0 (x*x takes Mul's aliasing path)
    T = oracle.T
    x = T.new([2.0], [1])
    y = (x * x) * x.sin()
    y.backward()
    f = lambda v: v * v * math.sin(v)
    num = (f(2.0 + 1e-6) - f(2.0 - 1e-6)) / 2e-6
    assert abs(x.grad[0] - num) < 1e-4
    assert abs(x.grad[0] - (4.0 * math.sin(2.0) + 4.0 * math.cos(2.0))) < 1e-12


def test_kat_detach_and_broadcast_fwd(oracle):
    # src/grad_check.rs:6-27 (detach drops the graph) and src/autograd.rs:1868-1875 (broadcast fwd)
    T = oracle.T
    a = T.new([2.0], [1])
    b = a
    for _ in range(100):
        b = b * T.new([1.1], [1])
    assert b.has_ctx and not b.detach().has_ctx
    t = T.new([5.0], [1]).broadcast([2, 2])
    assert t.shape == (2, 2) and np.all(t.data == 5.0)


def test_kat_transpose_and_reshape(oracle):
    # src/transformer.rs:1211-1225 (transpose) and :1191-1209 (reshape is a copy)
    T = oracle.T
    t = T.new([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [2, 3])
    tt = t.transpose(0, 1)
    assert tt.shape == (3, 2)
    assert list(tt.data.ravel()) == [1.0, 4.0, 2.0, 5.0, 3.0, 6.0]
    r = T.new([1.0, 2.0, 3.0, 4.0], [2, 2]).reshape([4])
    assert r.shape == (4,) and r.data[0] == 1.0


def test_tensor_rand_lcg_half_range(oracle):
    # Tensor::rand (src/autograd.rs:114-124): r = (x>>33)/u32::MAX lies in [0, 0.5), so values of
    # rand(min, max) cover [min, (min+max)/2). For rand(-1, 1, seed 42) over 100000 draws the
    # extremes are -0.99999 and -1.08e-5 (established for the reference independently).
    v = oracle.lcg_rand(100000, -1.0, 1.0, 42)
    assert v.max() < 0.0 and v.min() >= -1.0
    assert abs(v.min() - (-0.99999)) < 1e-5 and abs(v.max() - (-1.08e-5)) < 5e-8
    # first draw from the recurrence x1 = 42 * 6364136223846793005 + 1 (mod 2^64), integer-exact
    x1 = (42 * 6364136223846793005 + 1) % (1 << 64)
    assert v[0] == -1.0 + ((x1 >> 33) / 4294967295.0) * 2.0


# ---------------------------------------------------------------------------
# 2. Finite differences of every op's forward against its backward
# ---------------------------------------------------------------------------


def _fd_check(oracle, build, inputs, seed=0, h=1e-6, tol=1e-6):
    """build(list_of_T) -> output T. Checks d sum(out*G) / d input against central differences."""
    T = oracle.T
    rng = np.random.default_rng(seed)
    ts = [T.new(a, a.shape) for a in inputs]
    out = build(ts)
    G = rng.normal(size=out.shape)
    loss = out * T.new(G, out.shape)
    loss.sum().backward()
    for idx, a in enumerate(inputs):
        g = ts[idx].grad
        num = np.zeros_like(a)
        flat = a.ravel()
        for j in range(flat.size):
            vals = []
            for sgn in (1.0, -1.0):
                b = flat.copy()
                b[j] += sgn * h
                args = [T.new(b.reshape(a.shape), a.shape) if k == idx else T.new(inputs[k], inputs[k].shape)
                        for k in range(len(inputs))]
                vals.append(float((build(args).data * G).sum()))
            num.ravel()[j] = (vals[0] - vals[1]) / (2 * h)
        scale = max(1.0, np.abs(num).max())
        assert np.abs(g - num).max() <= tol * scale, f"input {idx}: max |fd - grad| = {np.abs(g - num).max()}"
    oracle.free_all()


R = np.random.default_rng(1234)


@pytest.mark.parametrize("name,fn,make", [
    ("relu", lambda t: t[0].relu(), lambda: [R.normal(size=(3, 4)) + 0.05]),
    ("log", lambda t: t[0].log(), lambda: [R.uniform(0.5, 2.0, (3, 4))]),
    ("exp", lambda t: t[0].exp(), lambda: [R.normal(size=(3, 4))]),
    ("sin", lambda t: t[0].sin(), lambda: [R.normal(size=(5,))]),
    ("cos", lambda t: t[0].cos(), lambda: [R.normal(size=(5,))]),
    ("sqrt", lambda t: t[0].sqrt(), lambda: [R.uniform(0.5, 2.0, (5,))]),
    ("neg", lambda t: -t[0], lambda: [R.normal(size=(5,))]),
    ("gelu", lambda t: t[0].gelu(), lambda: [R.normal(size=(4, 3)) * 2]),
    ("clip", lambda t: t[0].clip(-0.5, 0.7), lambda: [R.uniform(-1.5, 1.5, (4, 5))]),
    ("scale", lambda t: t[0].scale(0.37), lambda: [R.normal(size=(4,))]),
    ("sum", lambda t: t[0].sum(), lambda: [R.normal(size=(3, 2))]),
    ("mean", lambda t: t[0].mean(), lambda: [R.normal(size=(3, 2))]),
    ("broadcast", lambda t: t[0].broadcast([2, 3]), lambda: [R.normal(size=(1,))]),
    ("broadcast_to_batch", lambda t: t[0].broadcast_to_batch(4), lambda: [R.normal(size=(3,))]),
    ("transpose", lambda t: t[0].transpose(1, 3), lambda: [R.normal(size=(2, 3, 2, 4))]),
    ("reshape", lambda t: t[0].reshape([6, 2]), lambda: [R.normal(size=(3, 4))]),
    ("add", lambda t: t[0] + t[1], lambda: [R.normal(size=(3, 2)), R.normal(size=(3, 2))]),
    ("sub", lambda t: t[0] - t[1], lambda: [R.normal(size=(3, 2)), R.normal(size=(3, 2))]),
    ("mul", lambda t: t[0] * t[1], lambda: [R.normal(size=(3, 2)), R.normal(size=(3, 2))]),
    ("mul_alias", lambda t: t[0] * t[0], lambda: [R.normal(size=(3, 2))]),
    ("div", lambda t: t[0] / t[1], lambda: [R.normal(size=(3, 2)), R.uniform(0.5, 2, (3, 2))]),
    ("div_alias_plus", lambda t: (t[0] / t[0]) + t[0], lambda: [R.uniform(0.5, 2, (4,))]),
    ("matmul", lambda t: t[0].matmul(t[1]), lambda: [R.normal(size=(3, 4)), R.normal(size=(4, 5))]),
    ("matmul_vec", lambda t: t[0].matmul(t[1]), lambda: [R.normal(size=(4,)), R.normal(size=(4, 2))]),
    ("mse", lambda t: t[0].mse_loss(t[1]), lambda: [R.normal(size=(3, 2)), R.normal(size=(3, 2))]),
    ("softmax", lambda t: t[0].softmax(5), lambda: [R.normal(size=(3, 5))]),
    ("softmax_causal", lambda t: t[0].softmax(4, True), lambda: [R.normal(size=(8, 4))]),
    ("rmsnorm", lambda t: t[0].rmsnorm(t[1], 1e-5), lambda: [R.normal(size=(3, 6)), R.uniform(0.9, 1.1, 6)]),
    ("rope", lambda t: t[0].rope(8, 10000.0, 2), lambda: [R.normal(size=(2, 3, 6))]),
    ("bmm_qt_k", lambda t: oracle_mod().bmm_qt_k(t[0], t[1]), lambda: [R.normal(size=(2, 3, 4)),
                                                                    R.normal(size=(2, 3, 4))]),
    ("bmm_p_v", lambda t: oracle_mod().bmm_p_v(t[0], t[1]), lambda: [R.uniform(0.1, 1, (2, 3, 3)),
                                                                  R.normal(size=(2, 3, 2))]),
    ("concat", lambda t: oracle_mod().concat_last(t[0], t[1]), lambda: [R.normal(size=(2, 3, 2)),
                                                                     R.normal(size=(2, 3, 3))]),
    ("last_token", lambda t: t[0].last_token(True), lambda: [R.normal(size=(2, 3, 4))]),
])
def test_finite_differences(oracle, name, fn, make):
    _fd_check(oracle, fn, make())


def oracle_mod():
    import pyoracle
    return pyoracle


def test_last_token_reference_literal_cuts_graph(oracle):
    # Reference last_token (src/transformer.rs:92-109) builds a fresh Tensor: no gradient flows back.
    T = oracle.T
    x = T.new(np.arange(24.0), [2, 3, 4])
    y = (x * T.new(np.ones(24), [2, 3, 4])).last_token(False)
    assert not y.has_ctx
    assert np.array_equal(y.data, np.arange(24.0).reshape(2, 3, 4)[:, -1, :])


# ---------------------------------------------------------------------------
# 3. Closed forms, invariants, torch float64
# ---------------------------------------------------------------------------


def test_rmsnorm_closed_form_and_invariant(oracle):
    rng = np.random.default_rng(3)
    rows, dim, eps = 16, 32, 1e-2
    x, w, g = rng.normal(size=(rows, dim)), rng.uniform(0.9, 1.1, dim), rng.normal(size=(rows, dim))
    y, dx, dw = oracle.rmsnorm_fwd_bwd(x, w, g, eps)
    ms = (x * x).mean(1, keepdims=True)
    xh = x / np.sqrt(ms + eps)
    assert np.allclose(y, xh * w, rtol=1e-13, atol=1e-14)
    # sum_i dx_i x_i = (sum_i g_i w_i xhat_i) * eps / (mean(x^2) + eps), per row
    lhs = (dx * x).sum(1)
    rhs = (g * w * xh).sum(1) * eps / (ms[:, 0] + eps)
    assert np.allclose(lhs, rhs, rtol=1e-10, atol=1e-12)
    assert np.allclose(dw, (g * xh).sum(0), rtol=1e-12)
    xt, wt = tr.t64(x, True), tr.t64(w, True)
    (tr.rmsnorm(xt, wt, eps) * tr.t64(g)).sum().backward()
    assert np.allclose(dx, xt.grad.numpy(), rtol=1e-11, atol=1e-13)
    assert np.allclose(dw, wt.grad.numpy(), rtol=1e-11, atol=1e-13)


@pytest.mark.parametrize("causal", [False, True])
def test_softmax_invariants(oracle, causal):
    rng = np.random.default_rng(4)
    L = 16
    x, g = rng.normal(size=(3 * L, L)) * 3, rng.normal(size=(3 * L, L))
    y, dx = oracle.softmax_fwd_bwd(x, g, causal)
    assert np.allclose(y.sum(1), 1.0, atol=1e-14)
    assert np.allclose(dx.sum(1), 0.0, atol=1e-12)
    if causal:
        q = np.arange(3 * L) % L
        mask = np.arange(L)[None, :] > q[:, None]
        assert np.all(y[mask] == 0.0) and np.all(dx[mask] == 0.0)
        assert np.all(dx[q == 0] == 0.0)  # query 0 sees only itself: probability 1, zero gradient
        assert np.all(y[q == 0, 0] == 1.0)
    xt = tr.t64(x, True)
    xs = xt
    if causal:
        xs = xt.masked_fill(torch.as_tensor(mask), float("-inf"))
    (torch.softmax(xs, -1) * tr.t64(g)).sum().backward()
    assert np.allclose(dx, xt.grad.numpy(), atol=1e-13)


def test_rope_properties(oracle):
    rng = np.random.default_rng(5)
    x, g = rng.normal(size=(3, 16, 4, 8)), rng.normal(size=(3, 16, 4, 8))
    y, dx = oracle.rope_fwd_bwd(x, g, 10000.0)
    pair = lambda a: (a.reshape(*a.shape[:-1], -1, 2) ** 2).sum(-1)
    assert np.allclose(pair(y), pair(x), rtol=1e-13)  # rotation keeps each pair's norm
    assert np.array_equal(y[:, 0], x[:, 0])            # position 0 is the identity, bit-exact
    # backward is the rotation by -theta: rotating dx forward again gives g back
    back, _ = oracle.rope_fwd_bwd(dx, np.zeros_like(dx), 10000.0)
    assert np.allclose(back, g, atol=1e-13)
    xt = tr.t64(x, True)
    (tr.rope(xt, 10000.0) * tr.t64(g)).sum().backward()
    assert np.allclose(y, tr.rope(tr.t64(x), 10000.0).numpy(), atol=1e-13)
    assert np.allclose(dx, xt.grad.numpy(), atol=1e-13)
    # the table is the reference's cos/sin(pos * base^(-2i/dim))
    c, s = oracle.rope_table(64, 8, 10000.0)
    ang = np.arange(64)[:, None] * (1.0 / 10000.0 ** (np.arange(4) * 2 / 8.0))[None]
    assert np.allclose(c, np.cos(ang), atol=1e-15) and np.allclose(s, np.sin(ang), atol=1e-15)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_vs_torch(oracle, causal):
    rng = np.random.default_rng(6)
    B, S, H, dk, dv = 2, 7, 3, 5, 4
    q, k = rng.normal(size=(B, S, H, dk)), rng.normal(size=(B, S, H, dk))
    v, g = rng.normal(size=(B, S, H, dv)), rng.normal(size=(B, S, H, dv))
    sc = 1 / math.sqrt(dk)
    o, dq, dk_, dv_ = oracle.attention_fwd_bwd(q, k, v, g, sc, causal)
    qt, kt, vt = tr.t64(q, True), tr.t64(k, True), tr.t64(v, True)
    ot = tr.attention(qt, kt, vt, sc, causal)
    (ot * tr.t64(g)).sum().backward()
    assert np.allclose(o, ot.detach().numpy(), atol=1e-12)
    for a, b in ((dq, qt), (dk_, kt), (dv_, vt)):
        assert np.allclose(a, b.grad.numpy(), atol=1e-12)


def _block_cfg(oracle, B, S, d, H, F, causal=1, act=0, eps=1e-6):
    return oracle.BlockCfg(B, S, d, H, d // H, F, causal, act, eps, 10000.0)


@pytest.mark.parametrize("act", [0, 1])
def test_block_vs_torch(oracle, act):
    rng = np.random.default_rng(7)
    B, S, d, H, F = 2, 6, 16, 4, 64
    cfg = _block_cfg(oracle, B, S, d, H, F, act=act)
    p = block_params(rng, d, F, gain_jitter=True)
    x, G = rng.normal(size=(B, S, d)), rng.normal(size=(B, S, d))
    out, dp, dx = oracle.block_fwd_bwd(cfg, p, x, G)
    pt, xt = tr.t64(p, True), tr.t64(x, True)
    P, _ = tr.split_block_params(pt, d, F)
    ot = tr.block(xt, P, H, d // H, 1e-6, 10000.0, True, "gelu" if act == 0 else "relu")
    (ot * tr.t64(G)).sum().backward()
    assert np.allclose(out, ot.detach().numpy(), atol=1e-11)
    assert np.allclose(dp, pt.grad.numpy(), atol=1e-10)
    assert np.allclose(dx, xt.grad.numpy(), atol=1e-10)


def _ppo_cfg(oracle, B, S=5, d=16, L=2, H=4, F=64, A=3):
    return oracle.PpoCfg(B, S, 8, d, L, H, d // H, F, A, 1, 0, 1e-5, 10000.0, 0.2, 0.5, 0.01)


def _ppo_inputs(rng, cfg, params, oracle, spread=0.3):
    states = gacha_states(rng, cfg.batch, cfg.seq)
    actions = rng.integers(0, cfg.n_actions, cfg.batch)
    adv, ret = rng.normal(size=cfg.batch), rng.normal(size=cfg.batch)
    # old log-probs: the initial policy's, perturbed so that both surrogate branches and both
    # sides of the clip range occur
    _, logits, _, _ = oracle.ppo_fwd_bwd(cfg, params, states, actions, adv, ret, np.zeros(cfg.batch))
    lp = logits - np.log(np.exp(logits - logits.max(1, keepdims=True)).sum(1, keepdims=True)) - \
        logits.max(1, keepdims=True)
    old = lp[np.arange(cfg.batch), actions] + rng.uniform(-spread, spread, cfg.batch)
    return states, actions, adv, ret, old


def test_ppo_loss_closed_form_vs_reference_graph_and_torch(oracle):
    rng = np.random.default_rng(8)
    cfg = _ppo_cfg(oracle, 64)
    B, A = 64, 3
    logits, values = rng.normal(size=(B, A)), rng.normal(size=(B, 1))
    actions = rng.integers(0, A, B)
    old = rng.normal(size=B) - 1.0
    adv, ret = rng.normal(size=B), rng.normal(size=B)
    loss, dl, dv = oracle.ppo_batched_loss(cfg, logits, values, actions, old, adv, ret)
    # the per-sample reference graph (src/ppo.rs:702-755), summed and divided by B
    tot, dl_ref, dv_ref = 0.0, np.zeros_like(dl), np.zeros_like(dv)
    for b in range(B):
        l, g, gv = oracle.ppo_sample_loss(cfg, logits[b], values[b, 0], int(actions[b]), old[b], adv[b], ret[b])
        tot += l
        dl_ref[b], dv_ref[b, 0] = g / B, gv / B
    assert abs(loss - tot / B) < 1e-13
    assert np.allclose(dl, dl_ref, atol=1e-14) and np.allclose(dv, dv_ref, atol=1e-14)
    zt, vt = tr.t64(logits, True), tr.t64(values[:, 0], True)
    lt = tr.ppo_loss(zt, vt, actions, tr.t64(old), tr.t64(adv), tr.t64(ret), cfg.clip_eps, cfg.value_coef,
                     cfg.entropy_coef)
    lt.backward()
    assert abs(loss - lt.item()) < 1e-13
    assert np.allclose(dl, zt.grad.numpy(), atol=1e-14)
    assert np.allclose(dv[:, 0], vt.grad.numpy(), atol=1e-14)
    # both branches and clipped ratios occur in this sample
    ratio = np.exp(np.log(np.exp(logits - logits.max(1, keepdims=True)) /
                          np.exp(logits - logits.max(1, keepdims=True)).sum(1, keepdims=True))[np.arange(B), actions]
                   - old)
    assert (ratio > 1.2).any() and (ratio < 0.8).any()


def test_ppo_policy_batched_vs_per_sample_and_torch(oracle):
    rng = np.random.default_rng(9)
    cfg = _ppo_cfg(oracle, 6)
    p = ppo_params(rng, cfg)
    assert p.size == oracle.ppo_param_count(cfg)
    states, actions, adv, ret, old = _ppo_inputs(rng, cfg, p, oracle)
    loss, logits, values, dp = oracle.ppo_fwd_bwd(cfg, p, states, actions, adv, ret, old)
    # the reference-faithful per-sample graphs (backbone evaluated twice per sample)
    loss2, dp2 = oracle.ppo_fwd_bwd_per_sample(cfg, p, states, actions, adv, ret, old, diff_last=True)
    assert abs(loss - loss2) < 1e-12
    assert np.allclose(dp, dp2, atol=1e-12)
    pt = tr.t64(p, True)
    lt_, vt_ = tr.policy(tr.t64(states), pt, cfg)
    assert np.allclose(logits, lt_.detach().numpy(), atol=1e-12)
    lt = tr.ppo_loss(lt_, vt_, actions, tr.t64(old), tr.t64(adv), tr.t64(ret), cfg.clip_eps, cfg.value_coef,
                     cfg.entropy_coef)
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12
    assert np.allclose(dp, pt.grad.numpy(), atol=1e-11)


def test_ppo_reference_literal_graph_cut(oracle):
    # With the reference's last_token (no graph) only the actor/critic heads get gradients
    # (src/ppo.rs:274-276, 292-294): every backbone gradient is exactly 0.
    rng = np.random.default_rng(10)
    cfg = _ppo_cfg(oracle, 3)
    p = ppo_params(rng, cfg)
    states, actions, adv, ret, old = _ppo_inputs(rng, cfg, p, oracle)
    _, dp = oracle.ppo_fwd_bwd_per_sample(cfg, p, states, actions, adv, ret, old, diff_last=False)
    d, A = cfg.d_model, cfg.n_actions
    nheads = d * A + A + d + 1
    assert np.all(dp[:-nheads] == 0.0) and np.any(dp[-nheads:] != 0.0)


@pytest.mark.parametrize("literal,causal", [(0, 0), (0, 1), (1, 0)])
def test_mla_vs_torch(oracle, literal, causal):
    rng = np.random.default_rng(11)
    ci = [2, 5, 16, 2, 8, 4, 8, 6, causal, literal]
    p = mla_params(rng, ci)
    assert p.size == oracle.mla_param_count(ci)
    x, G = rng.normal(size=(2, 5, 16)), rng.normal(size=(2, 5, 16))
    out, dp, dx = oracle.mla_fwd_bwd(ci, 1e-5, 10000.0, p, x, G)
    pt, xt = tr.t64(p, True), tr.t64(x, True)
    ot = tr.mla_block(xt, pt, ci, 1e-5, 10000.0)
    (ot * tr.t64(G)).sum().backward()
    assert np.allclose(out, ot.detach().numpy(), atol=1e-12)
    assert np.allclose(dp, pt.grad.numpy(), atol=1e-11)
    assert np.allclose(dx, xt.grad.numpy(), atol=1e-11)


def test_mla_reference_config_shapes(oracle):
    # MLAConfig used by the reference test (src/transformer.rs:1227-1266): dim 16, 2 heads,
    # kv 8, rope 4, v 8, input rand([1,3,16], -0.1, 0.1, 123); the reference asserts non-zero grads.
    rng = np.random.default_rng(12)
    ci = [1, 3, 16, 2, 8, 4, 8, 8, 0, 1]
    p = mla_params(rng, ci)
    x = oracle.lcg_rand(48, -0.1, 0.1, 123).reshape(1, 3, 16)
    out, dp, dx = oracle.mla_fwd_bwd(ci, 1e-5, 10000.0, p, x, np.full((1, 3, 16), 1.0 / 48))
    d, L = 16, 8
    assert abs(dp[d:d + d * L].sum()) > 0.0
    assert out.shape == (1, 3, 16)


def _mla_block_cfg(oracle, B, S, causal=0):
    # the reference block's shape family (LuckTransformer::new, src/transformer.rs:48-69) at d 16
    return oracle.BlockCfg(B, S, 16, 2, 4, 32, causal, 1, 1e-5, 10000.0, 1, 8, 4, 4)


@pytest.mark.parametrize("causal", [0, 1])
def test_mla_block_vs_torch(oracle, causal):
    rng = np.random.default_rng(13)
    cfg = _mla_block_cfg(oracle, 2, 5, causal)
    p = mla_block_params(rng, cfg, gain_jitter=True)
    assert p.size == oracle.block_param_count(cfg)
    x, G = rng.normal(size=(2, 5, 16)), rng.normal(size=(2, 5, 16))
    out, dp, dx = oracle.block_fwd_bwd(cfg, p, x, G)
    pt, xt = tr.t64(p, True), tr.t64(x, True)
    ot, n = tr.mla_ffn_block(xt, pt, cfg)
    assert n == p.size
    (ot * tr.t64(G)).sum().backward()
    assert np.allclose(out, ot.detach().numpy(), atol=1e-12)
    assert np.allclose(dp, pt.grad.numpy(), atol=1e-11)
    assert np.allclose(dx, xt.grad.numpy(), atol=1e-11)


def test_reference_actor_critic_vs_per_sample_and_torch(oracle):
    # the reference's own ActorCritic shape (in 8, d 64, one MLA layer, 5 actions, no mask)
    rng = np.random.default_rng(14)
    B, S = 4, 6
    cfg = oracle.PpoCfg(B, S, *REFERENCE_ACTOR_CRITIC)
    p = ppo_params(rng, cfg)
    assert p.size == oracle.ppo_param_count(cfg)
    states, actions, adv, ret, old = _ppo_inputs(rng, cfg, p, oracle)
    loss, logits, values, dp = oracle.ppo_fwd_bwd(cfg, p, states, actions, adv, ret, old)
    loss2, dp2 = oracle.ppo_fwd_bwd_per_sample(cfg, p, states, actions, adv, ret, old, diff_last=True)
    assert abs(loss - loss2) < 1e-12
    assert np.allclose(dp, dp2, atol=1e-12)
    pt = tr.t64(p, True)
    lt_, vt_ = tr.policy(tr.t64(states), pt, cfg)
    assert np.allclose(logits, lt_.detach().numpy(), atol=1e-12)
    assert np.allclose(values, vt_.detach().numpy(), atol=1e-12)
    lt = tr.ppo_loss(lt_, vt_, actions, tr.t64(old), tr.t64(adv), tr.t64(ret), cfg.clip_eps, cfg.value_coef,
                     cfg.entropy_coef)
    lt.backward()
    assert abs(loss - lt.item()) < 1e-12
    assert np.allclose(dp, pt.grad.numpy(), atol=1e-11)


# ---------------------------------------------------------------------------
# Rollout inference with the KV cache
# ---------------------------------------------------------------------------
def _ac_cfg(oracle, B, S, **over):
    c = oracle.PpoCfg(B, S, *REFERENCE_ACTOR_CRITIC)
    for k, v in over.items():
        setattr(c, k, v)
    return c


def _full_last_logits(oracle, cfg, p, tokens):
    """The full-graph forward of one sequence (positions 0..S-1): logits and value of its last token."""
    S = tokens.shape[0]
    c = type(cfg)()
    ctypes.pointer(c)[0] = cfg
    c.batch, c.seq = 1, S
    _, lg, val, _ = oracle.ppo_fwd_bwd(c, p, tokens[None], np.zeros(1, np.int32), np.zeros(1), np.zeros(1),
                                       np.zeros(1))
    return lg[0], val[0]


def test_decoder_reference_fast_slow_alignment(oracle):
    """The reference's own check (src/sim.rs:1180-1216): ActorCritic::new(12345), six tokens
    flat[t, i] = 0.01 t + 0.001 i; the full forward's probabilities and those of six cached steps
    differ by less than 1e-6 in sum. With RoPE by sequence position (not the head index of the
    training path) they agree to rounding."""
    cfg = _ac_cfg(oracle, 1, 6)
    p = reference_init_actor_critic(oracle, 12345)
    assert p.size == oracle.ppo_param_count(cfg)
    flat = np.array([[t * 0.01 + i * 0.001 for i in range(8)] for t in range(6)])
    slow, _ = _full_last_logits(oracle, cfg, p, flat)
    dec = oracle.Decoder(cfg, p, 256, 1)
    for t in range(6):
        fast, _, _ = dec.step(0, flat[t], t)

    def sm(z):
        e = np.exp(z - z.max())
        return e / e.sum()

    assert np.abs(sm(slow) - sm(fast)).sum() < 1e-6
    assert np.allclose(fast, slow, rtol=1e-12, atol=1e-13)


@pytest.mark.parametrize("attention,layers,causal", [(1, 1, 0), (0, 2, 1), (1, 2, 1)])
def test_decoder_equals_full_forward_last_token(oracle, attention, layers, causal):
    """Feeding a sequence one token at a time gives the full graph's last-token logits and value:
    with one layer for any mask (the last query sees every key either way), with several layers
    when the mask is causal (earlier tokens never see later ones)."""
    rng = np.random.default_rng(15 + layers)
    if attention == 1:
        cfg = _ac_cfg(oracle, 1, 7, n_layers=layers, causal=causal)
    else:
        cfg = oracle.PpoCfg(1, 7, 8, 32, layers, 2, 16, 64, 3, causal, 0, 1e-5, 10000.0, 0.2, 0.5, 0.01)
    p = ppo_params(rng, cfg)
    toks = gacha_states(rng, 1, 7)[0]
    lg_r, v_r = _full_last_logits(oracle, cfg, p, toks)
    dec = oracle.Decoder(cfg, p, 64, 1)
    for t in range(7):
        lg, v, _ = dec.step(0, toks[t], t)
    assert np.allclose(lg, lg_r, rtol=1e-11, atol=1e-12)
    assert abs(v - v_r) < 1e-11 * (1 + abs(v_r))
    k, vv = dec.cache(0, layers - 1)
    assert k.shape == (7, cfg.n_heads, cfg.head_dim + (cfg.rope_dim if attention == 1 else 0))


def test_decoder_prune_keeps_a_sliding_window(oracle):
    """After prune_kv_cache to W rows, a step attends to the newest W + 1 tokens; RoPE scores
    depend only on position differences, so the step equals the full forward of that window
    re-based to positions 0..W."""
    rng = np.random.default_rng(16)
    cfg = _ac_cfg(oracle, 1, 16)
    p = ppo_params(rng, cfg)
    toks = gacha_states(rng, 1, 12)[0]
    W, p0 = 4, 9
    dec = oracle.Decoder(cfg, p, 256, 1)
    for t in range(12):
        lg, _, _ = dec.step(0, toks[t], p0 + t)
        lo = max(0, t - W)
        lg_r, _ = _full_last_logits(oracle, cfg, p, toks[lo:t + 1])
        assert np.allclose(lg, lg_r, rtol=1e-9, atol=1e-11), t
        dec.prune(0, W)
        assert dec.cache(0)[0].shape[0] == min(t + 1, W)
    dec.clear(0)
    assert dec.cache(0)[0].shape[0] == 0


def test_decoder_positions_past_the_rope_cache_are_not_rotated(oracle):
    """forward_inference_cached skips the rotation when pos * rope_dim / 2 is past the cos cache
    (src/transformer.rs:718-721): positions >= max_seq_len act as position 0 (the identity)."""
    rng = np.random.default_rng(17)
    cfg = _ac_cfg(oracle, 1, 8)
    p = ppo_params(rng, cfg)
    toks = gacha_states(rng, 1, 5)[0]
    a, b, c = oracle.Decoder(cfg, p, 32, 1), oracle.Decoder(cfg, p, 32, 1), oracle.Decoder(cfg, p, 32, 1)
    for t in range(5):
        la, _, _ = a.step(0, toks[t], 32 + 7 * t)  # all past the 32-position cache
        lb, _, _ = b.step(0, toks[t], 0)
        lc, _, _ = c.step(0, toks[t], t)
    assert np.array_equal(la, lb)
    assert not np.allclose(la, lc)  # while in range the rotation matters


def test_sample_action_rule(oracle):
    z = np.array([0.3, -1.0, 2.0, 0.0, 0.5])
    e = np.exp(z - z.max())
    pr = e / e.sum()
    edges = np.cumsum(pr)
    for a in range(5):
        lo = 0.0 if a == 0 else edges[a - 1]
        for r in (lo + 1e-6, (lo + edges[a]) / 2, edges[a] - 1e-6):
            got, lp = oracle.sample_action(z, r)
            assert got == a, (a, r)
            assert abs(lp - math.log(pr[a])) < 1e-14
    # no bucket (a draw at or past the rounded total): the index keeps its initial 0, since the
    # reference's `action_idx == ACTION_SPACE` fallback never fires (src/ppo.rs:336-346)
    assert oracle.sample_action(z, 1.5)[0] == 0


def test_linear_mse_closed_form(oracle):
    # C1 at its full size: closed forms dX = dY W^T, dW = X^T dY, db = sum dY with dY = 2(XW+b-Y)/N
    rng = np.random.default_rng(13)
    X, W, b, Y = rng.normal(size=(256, 64)), xavier(rng, 64, 64), np.zeros(64), rng.normal(size=(256, 64))
    loss, dx, dw, db = oracle.linear_mse(X, W, b, Y)
    r = X @ W + b - Y
    dY = 2 * r / r.size
    assert abs(loss - (r * r).mean()) < 1e-12
    assert np.allclose(dx, dY @ W.T, atol=1e-15) and np.allclose(dw, X.T @ dY, atol=1e-14)
    assert np.allclose(db, dY.sum(0), atol=1e-15)


# ---------------------------------------------------------------------------
# Optimizer step: Adam (src/ppo.rs:519-533) and the DQN global-norm clip (src/dqn.rs:207-226)
# ---------------------------------------------------------------------------
def test_adam_vs_torch_adam_f64(oracle):
    """Five steps of the oracle's Adam equal torch.optim.Adam in float64 (same update written as
    p -= (lr / (1 - b1^t)) * m / (sqrt(v) / sqrt(1 - b2^t) + eps))."""
    rng = np.random.default_rng(7)
    n = 1000
    p0 = rng.normal(size=n)
    p, m, v = p0.copy(), np.zeros(n), np.zeros(n)
    tp = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.Adam([tp], lr=3e-3, betas=(0.9, 0.999), eps=1e-8)
    for t in range(1, 6):
        g = rng.normal(size=n) * (0.1 * t)
        oracle.adam_step(p, g, m, v, t, 3e-3)
        tp.grad = torch.tensor(g, dtype=torch.float64)
        opt.step()
        np.testing.assert_allclose(p - p0, tp.detach().numpy() - p0, rtol=1e-10, atol=1e-15)
        st = opt.state[tp]
        # torch forms m with lerp (m + (1 - b1)(g - m)): the same value up to f64 rounding
        np.testing.assert_allclose(m, st["exp_avg"].numpy(), rtol=1e-10, atol=1e-16)
        np.testing.assert_allclose(v, st["exp_avg_sq"].numpy(), rtol=1e-10, atol=1e-18)


def test_adam_first_step_closed_form(oracle):
    """At t = 1 from zero state the bias corrections cancel: m_hat = g, v_hat = g^2, so the update
    is lr * g / (|g| + eps) (exactly 0 where g = 0)."""
    rng = np.random.default_rng(8)
    g = rng.normal(size=257)
    g[::17] = 0.0
    p0 = rng.normal(size=257)
    p, m, v = p0.copy(), np.zeros(257), np.zeros(257)
    oracle.adam_step(p, g, m, v, 1, 1e-2)
    np.testing.assert_allclose(p0 - p, 1e-2 * g / (np.abs(g) + 1e-8), rtol=1e-12, atol=1e-18)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-15)
    np.testing.assert_allclose(v, 0.001 * g * g, rtol=1e-12)


@pytest.mark.parametrize("scale", [5.0, 0.01])
def test_adam_global_norm_clip(oracle, scale):
    """The DQN step equals the plain step on g / ||g|| when ||g|| > 1 and on g itself otherwise."""
    rng = np.random.default_rng(9)
    n = 300
    g = rng.normal(size=n) * scale / math.sqrt(n)
    norm = float(np.linalg.norm(g))
    g_eff = g / norm if norm > 1.0 else g
    p0 = rng.normal(size=n)
    pa, ma, va = p0.copy(), np.zeros(n), np.zeros(n)
    pb, mb, vb = p0.copy(), np.zeros(n), np.zeros(n)
    for t in (1, 2):
        oracle.adam_step(pa, g, ma, va, t, 1e-2, max_norm=1.0)
        oracle.adam_step(pb, g_eff, mb, vb, t, 1e-2)
    np.testing.assert_allclose(ma, mb, rtol=1e-13, atol=0)
    np.testing.assert_allclose(va, vb, rtol=1e-12, atol=0)
    np.testing.assert_allclose(pa - p0, pb - p0, rtol=1e-11, atol=1e-16)
    if norm > 1.0:  # the clipped first moment has norm (1 - b1) * 1 after one step
        m1 = np.zeros(n)
        oracle.adam_step(p0.copy(), g, m1, np.zeros(n), 1, 1e-2, max_norm=1.0)
        assert abs(np.linalg.norm(m1) - 0.1) < 1e-12


# ---------------------------------------------------------------------------
# PPO::update prologue: reward normalisation, GAE, advantage normalisation (src/ppo.rs:650-676)
# ---------------------------------------------------------------------------
def _gae_by_sum(r, v, done, gamma, lam):
    """A_t = sum_l (gamma lambda)^l (prod_{j<l} (1 - done_{t+j})) delta_{t+l}: the definition as a
    sum, independent of the backward recursion."""
    n = r.size
    nonterm = 1.0 - done.astype(np.float64)
    v_next = np.append(v[1:], 0.0)
    delta = r + gamma * v_next * nonterm - v
    a = np.zeros(n)
    for t in range(n):
        w = 1.0
        for k in range(t, n):
            a[t] += w * delta[k]
            w *= gamma * lam * nonterm[k]
            if w == 0.0:
                break
    return a


@pytest.mark.parametrize("n,p_done", [(1, 0.0), (17, 0.2), (300, 0.05), (300, 1.0)])
def test_gae_vs_sum_definition(oracle, n, p_done):
    rng = np.random.default_rng(n)
    rew, val = rng.normal(size=n) * 3.0, rng.normal(size=n)
    done = rng.random(n) < p_done
    mu, var = 0.4, 2.5
    a, ret, an = oracle.ppo_gae(rew, val, done, mu, var, 10.0, 0.99, 0.95)
    r = np.clip((rew - mu) / (np.sqrt(var) + 1e-8), -10.0, 10.0)
    ref = _gae_by_sum(r, val, done, 0.99, 0.95)
    np.testing.assert_allclose(a, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(ret, ref + val, rtol=1e-12, atol=1e-12)
    if n > 1:
        np.testing.assert_allclose(an.mean(), 0.0, atol=1e-12)
        np.testing.assert_allclose(an, (a - a.mean()) / (a.std() + 1e-8), rtol=1e-12, atol=1e-12)


def test_gae_special_cases(oracle):
    rng = np.random.default_rng(5)
    rew, val = rng.normal(size=50), rng.normal(size=50)
    done = rng.random(50) < 0.3
    v_next = np.append(val[1:], 0.0)
    r = rew / (1.0 + 1e-8)  # normalised with mean 0, var 1: (r - 0) / (sqrt(1) + 1e-8)
    # lambda = 0: A is the one-step TD error
    a, _, _ = oracle.ppo_gae(rew, val, done, 0.0, 1.0, 10.0, 0.9, 0.0)
    np.testing.assert_allclose(a, r + 0.9 * v_next * (1 - done) - val, rtol=1e-12, atol=1e-13)
    # gamma = 0: A = r - V
    a, _, _ = oracle.ppo_gae(rew, val, done, 0.0, 1.0, 10.0, 0.0, 0.95)
    np.testing.assert_allclose(a, r - val, rtol=1e-12, atol=1e-13)
    # the reward clip: |r_norm| <= clip
    a, _, _ = oracle.ppo_gae(rew * 1e6, val * 0, np.ones(50, bool), 0.0, 1.0, 10.0, 0.99, 0.95)
    np.testing.assert_allclose(a, np.clip(rew * 1e6 / (1.0 + 1e-8), -10, 10), rtol=1e-15, atol=0)


# ---------------------------------------------------------------------------
# 4. Gradient magnitude sums (the allowance of the parameter-gradient bound, common.check_grad)
# ---------------------------------------------------------------------------


def test_magnitude_sums_closed_forms(oracle):
    """Under track_mag the oracle's leaves carry, per gradient element, the sum of |term| over its
    terms: (|X|^T |G|) for a weight, sum_r |g x_hat| for an RMSNorm gain, sum_r |g| for a bias,
    |G| |W|^T for the input of a product."""
    T = oracle.T
    rng = np.random.default_rng(8)
    rows, k, n = 37, 6, 5
    X, W, b, G = rng.normal(size=(rows, k)), rng.normal(size=(k, n)), rng.normal(size=n), rng.normal(size=(rows, n))
    oracle.track_mag(True)
    try:
        x, w, bb, g = T.new(X, X.shape), T.new(W, W.shape), T.new(b, b.shape), T.new(G, G.shape)
        y = x.matmul(w) + bb.broadcast_to_batch(rows)
        (y * g).sum().backward()
        assert np.allclose(w.mag, np.abs(X).T @ np.abs(G), rtol=1e-13)
        assert np.allclose(bb.mag, np.abs(G).sum(0), rtol=1e-13)
        assert np.allclose(x.mag, np.abs(G) @ np.abs(W).T, rtol=1e-13)
        assert np.allclose(w.grad, X.T @ G, rtol=1e-12)  # the gradients themselves are unchanged
        # RMSNorm gain: sum_r |g x_hat|
        gain = rng.uniform(0.9, 1.1, k)
        x2, w2 = T.new(X, X.shape), T.new(gain, gain.shape)
        G2 = rng.normal(size=(rows, k))
        (x2.rmsnorm(w2, 1e-6) * T.new(G2, G2.shape)).sum().backward()
        xh = X / np.sqrt((X * X).mean(1, keepdims=True) + 1e-6)
        assert np.allclose(w2.mag, np.abs(G2 * xh).sum(0), rtol=1e-13)
    finally:
        oracle.track_mag(False)
    # untracked leaves report zeros
    z = T.new(W, W.shape)
    assert not z.mag.any()


def test_magnitude_sums_bound_the_model_gradients(oracle):
    """On the composite models every parameter's magnitude sum is at least |grad| (the triangle
    inequality; equality when no term cancels), and the returned gradients do not depend on
    tracking."""
    rng = np.random.default_rng(9)
    B, S, d, H, F = 2, 7, 16, 2, 32
    args = (B, S, d, H, d // H, F, 1, 0, 1e-6, 1e4)
    p = block_params(rng, d, F, gain_jitter=True)
    x, G = rng.normal(size=(B, S, d)), rng.normal(size=(B, S, d))
    out0, dp0, dx0 = oracle.block_fwd_bwd(oracle.BlockCfg(*args), p, x, G)
    out1, dp1, dx1, mag = oracle.block_fwd_bwd(oracle.BlockCfg(*args), p, x, G, mag=True)
    assert np.array_equal(dp0, dp1) and np.array_equal(dx0, dx1) and np.array_equal(out0, out1)
    assert np.all(mag >= np.abs(dp1) * (1 - 1e-12)) and mag.min() > 0
    ci = [2, 9, 16, 2, 8, 4, 8, 8, 1, 0]
    pm = mla_params(rng, ci)
    xm, Gm = rng.normal(size=(2, 9, 16)), rng.normal(size=(2, 9, 16))
    _, dpm, _, magm = oracle.mla_fwd_bwd(ci, 1e-5, 1e4, pm, xm, Gm, mag=True)
    assert np.all(magm >= np.abs(dpm) * (1 - 1e-12)) and magm.min() > 0
    cfg = oracle.PpoCfg(5, 6, 8, 16, 2, 2, 8, 32, 3, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)
    pp = ppo_params(rng, cfg)
    st = gacha_states(rng, 5, 6)
    acts = rng.integers(0, 3, 5).astype(np.int32)
    adv, ret, old = rng.normal(size=5), rng.normal(size=5), rng.normal(size=5) * 0.2 - 1.1
    _, _, _, dpp, magp = oracle.ppo_fwd_bwd(cfg, pp, st, acts, adv, ret, old, mag=True)
    assert np.all(magp >= np.abs(dpp) * (1 - 1e-12)) and magp.min() > 0
    # per-sample graphs (biases reach the loss through reshape and element-wise adds)
    _, dps, mags = oracle.ppo_fwd_bwd_per_sample(cfg, pp, st, acts, adv, ret, old, mag=True)
    assert np.all(mags >= np.abs(dps) * (1 - 1e-12))
    # a product of non-negative factors has no cancellation: magnitude == |grad|
    T = oracle.T
    oracle.track_mag(True)
    try:
        A, Gp = rng.uniform(0, 1, (50, 4)), rng.uniform(0, 1, (50, 3))
        a, w = T.new(A, A.shape), T.new(np.ones((4, 3)), (4, 3))
        (a.matmul(w) * T.new(Gp, Gp.shape)).sum().backward()
        assert np.allclose(w.mag, w.grad, rtol=1e-13)
    finally:
        oracle.track_mag(False)


def test_gradient_bound_accepts_fp32_rounding_and_rejects_planted_mistakes(oracle):
    """The parameter-gradient bound of common.check_grad, 1e-4 |r| + max(1e-5, 32 u M), on a
    weight gradient over 32768 rows with N(0,1) factors (sums of +-terms that cancel to ~0.6 % of
    their magnitude): an fp32 evaluation (numpy float32 products, blocked accumulation) passes it,
    and so does one in 512-row fp32 splits combined in f64 (the device's weight-gradient shape);
    a dropped row, a doubled row, a transposed index and a sign error each fail it."""
    from common import check_grad
    rng = np.random.default_rng(10)
    rows, k, n = 32768, 16, 16
    X = rng.normal(size=(rows, k)).astype(np.float32).astype(np.float64)
    G = rng.normal(size=(rows, n)).astype(np.float32).astype(np.float64)
    ref = X.T @ G
    mag = np.abs(X).T @ np.abs(G)
    got32 = (X.astype(np.float32).T @ G.astype(np.float32)).astype(np.float64)
    check_grad(got32, ref, mag, name="fp32 evaluation")
    split = sum((X[s:s + 512].astype(np.float32).T @ G[s:s + 512].astype(np.float32)).astype(np.float64)
                for s in range(0, rows, 512))
    check_grad(split, ref, mag, name="fp32 splits")
    r = int(np.argmax(np.abs(X).sum(1) * np.abs(G).sum(1) < 1e9))  # any row
    mistakes = {
        "dropped row": ref - np.outer(X[r], G[r]),
        "doubled row": ref + np.outer(X[r], G[r]),
        "transposed index": ref.T.copy(),
        "sign error": -ref,
    }
    for what, bad in mistakes.items():
        with pytest.raises(AssertionError):
            check_grad(bad, ref, mag, name=what, audit=False)
