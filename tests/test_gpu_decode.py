"""GPU parity of rollout inference with the KV cache (talos_ppo_decoder_*) against the oracle's
restatement of LuckTransformer::forward_inference_step / forward_inference_cached /
prune_kv_cache (src/transformer.rs:157-196, 688-840) and the action draw of
ActorCritic::step_inference_cached (src/ppo.rs:391-433).

Each test drives several environments with their own positions, resets and uniform draws, step
after step, and compares every step's logits and values, the final caches and the actions.
Tolerance: the fp32 rule of the other parity tests. An action is compared where the draw is not
within 1e-4 of a bucket edge of the oracle's probabilities (an fp32 rounding may move it across).

Every test runs on both device paths: the one-launch step (chosen for small policies with a
window of at most 64) and the layered step (TALOS_DECODER_LAYERED=1 at decoder creation, and any
configuration past the one-launch limits).
"""
import numpy as np
import pytest

import talos_hip as th
import workload
from common import check_close, f32, gacha_states, ppo_params

pytestmark = pytest.mark.gpu
DA = th.DeviceArray


@pytest.fixture(autouse=True, params=["fused", "layered"])
def decoder_path(request, monkeypatch):
    if request.param == "layered":
        monkeypatch.setenv("TALOS_DECODER_LAYERED", "1")
    else:
        monkeypatch.delenv("TALOS_DECODER_LAYERED", raising=False)
    return request.param


def _probs(z):
    e = np.exp(z - z.max())
    return e / e.sum()


def _run(oracle, args, p, T, n, W, max_seq_len, pos0, reset_at=(), seed=0, n_active=None):
    """T steps of n environments on the device and in the oracle; returns the device decoder,
    the oracle decoder and per-step records."""
    rng = np.random.default_rng(seed)
    cfg, ocfg = th.PpoCfg(*args), oracle.PpoCfg(*args)
    na = n if n_active is None else n_active
    dec = th.Decoder(cfg, n, W, max_seq_len)
    odec = oracle.Decoder(ocfg, p, max_seq_len or 256, n)
    P = DA.from_numpy(p)
    A = cfg.n_actions
    lg, vl = DA.zeros((na, A)), DA.zeros(na)
    act, lp = DA.zeros(na, np.int32), DA.zeros(na)
    for t in range(T):
        toks = f32(gacha_states(rng, na, 1)[:, 0])
        pos = (np.asarray(pos0[:na]) + t).astype(np.int32)
        reset = np.array([1 if (t, e) in reset_at else 0 for e in range(na)], np.uint8)
        u = f32(rng.random(na))
        Tk, Ps, Un = DA.from_numpy(toks), DA.from_numpy(pos, np.int32), DA.from_numpy(u)
        Rs = DA.zeros(na, np.uint8)
        th.call("talos_memcpy_h2d", Rs.ptr, reset.ctypes.data, na, None)
        dec.step(na, P, Tk, Ps, Rs, Un, lg, vl, act, lp)
        g_lg, g_v, g_a, g_lp = lg.numpy(), vl.numpy(), act.numpy(), lp.numpy()
        for e in range(na):
            if reset[e]:
                odec.clear(e)
            r_lg, r_v, _ = odec.step(e, toks[e], int(pos[e]))
            odec.prune(e, W)
            check_close(g_lg[e], r_lg, name=f"logits step {t} env {e}")
            check_close(g_v[e], r_v, name=f"value step {t} env {e}")
            edges = np.cumsum(_probs(r_lg))
            if np.min(np.abs(edges - u[e])) > 1e-4:
                a_r, lp_r = oracle.sample_action(r_lg, float(u[e]))
                assert g_a[e] == a_r, (t, e)
                check_close(g_lp[e], lp_r, name=f"logp step {t} env {e}")
        for a in (Tk, Ps, Un, Rs):
            a.free()
    return dec, odec, cfg


def _check_caches(dec, odec, cfg, envs):
    for layer in range(cfg.n_layers):
        for e in envs:
            k, v = dec.cache(layer, e)
            k_r, v_r = odec.cache(e, layer)
            assert k.shape == k_r.shape, (layer, e)
            check_close(k, k_r, name=f"k cache layer {layer} env {e}")
            check_close(v, v_r, name=f"v cache layer {layer} env {e}")


def test_reference_actor_critic_rollout(oracle):
    """The reference's model, 5 environments, a window of 4, positions crossing the 256-entry
    RoPE cache (past it no rotation), resets mid-rollout."""
    args = (1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    p = f32(ppo_params(np.random.default_rng(800), oracle.PpoCfg(*args)))
    dec, odec, cfg = _run(oracle, args, p, T=10, n=5, W=4, max_seq_len=256, pos0=[0, 3, 250, 7, 300],
                          reset_at={(6, 1), (3, 4)}, seed=801)
    _check_caches(dec, odec, cfg, range(5))
    dec.destroy()


@pytest.mark.parametrize("attention,layers", [(0, 2), (1, 2)])
def test_multi_layer_rollout(oracle, attention, layers):
    """Several layers (one cache each), standard and latent attention, a window longer than the
    rollout (no pruning) and one shorter."""
    if attention == 1:
        a = list(workload.REFERENCE_ACTOR_CRITIC)
        a[2], a[7] = layers, 1
        args = (1, 16, *a)
    else:
        args = (1, 16, 8, 64, layers, 2, 32, 256, 3, 1, 0, 1e-5, 10000.0, 0.2, 0.5, 0.01)
    p = f32(ppo_params(np.random.default_rng(810 + attention), oracle.PpoCfg(*args)))
    for W in (16, 3):
        dec, odec, cfg = _run(oracle, args, p, T=7, n=3, W=W, max_seq_len=64, pos0=[0, 5, 60], seed=811 + W)
        _check_caches(dec, odec, cfg, range(3))
        dec.destroy()


def test_window_past_the_one_launch_limit(oracle):
    """A window of 70 (> 64: the layered step on both parametrisations) with pruning reached."""
    args = (1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    p = f32(ppo_params(np.random.default_rng(830), oracle.PpoCfg(*args)))
    dec, odec, cfg = _run(oracle, args, p, T=73, n=2, W=70, max_seq_len=256, pos0=[0, 180], seed=831)
    _check_caches(dec, odec, cfg, range(2))
    dec.destroy()


def test_many_environments_and_a_partial_step(oracle):
    """1000 environments (thousands of waves per launch), then steps over the first 600 only: the
    others keep their caches."""
    args = (1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    p = f32(ppo_params(np.random.default_rng(820), oracle.PpoCfg(*args)))
    rng = np.random.default_rng(821)
    pos0 = rng.integers(0, 200, 1000)
    dec, odec, cfg = _run(oracle, args, p, T=3, n=1000, W=16, max_seq_len=256, pos0=pos0, seed=822)
    k_before, _ = dec.cache(0, 900)
    assert k_before.shape[0] == 3
    # a fourth step on the first 600 environments
    P = DA.from_numpy(p)
    toks = f32(gacha_states(rng, 600, 1)[:, 0])
    pos = (pos0[:600] + 3).astype(np.int32)
    lg = DA.zeros((600, cfg.n_actions))
    dec.step(600, P, DA.from_numpy(toks), DA.from_numpy(pos, np.int32), None, None, lg)
    g = lg.numpy()
    for e in (0, 299, 599):
        r_lg, _, _ = odec.step(e, toks[e], int(pos[e]))
        check_close(g[e], r_lg, name=f"logits env {e}")
    assert dec.cache(0, 599)[0].shape[0] == 4 and dec.cache(0, 600)[0].shape[0] == 3
    k_after, _ = dec.cache(0, 900)
    assert np.array_equal(k_before, k_after)
    dec.destroy()


def test_decoder_argument_errors():
    cfg = th.PpoCfg(1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    dec = th.Decoder(cfg, 4, 8)
    p = DA.zeros(th.lib().talos_ppo_param_count(cfg))
    x, pos, u = DA.zeros((4, 8)), DA.zeros(4, np.int32), DA.zeros(4)
    L = th.lib()
    assert L.talos_ppo_decoder_step_f32(dec.h, 5, p.ptr, x.ptr, pos.ptr, None, None, None, None, None, None,
                                        None) == th.ERR_SHAPE
    assert L.talos_ppo_decoder_step_f32(dec.h, 4, p.ptr, x.ptr, pos.ptr, None, None, None, None, u.ptr, None,
                                        None) == th.ERR_NULL  # actions need the draws
    assert L.talos_ppo_decoder_read_cache(dec.h, 1, 0, None, None, None) != th.OK
    dec.destroy()
