"""GPU parity of the optimizer step (talos_adam_step_f32, talos_grad_sumsq_f32) against the f64
oracle's Adam (src/ppo.rs:519-533) and the DQN global-norm clip (src/dqn.rs:207-226).

Comparison rule: parameter deltas (p_t - p_0) and m within 1e-4 * |ref| + 1e-5 element-wise over
five consecutive steps (the device keeps fp32 state, the oracle f64); v, whose entries are
1e-3 * g^2 and smaller, within 1e-4 * |ref| + 1e-6 * max|ref|; the f64 squared norm within 1e-12
relative (only the summation order differs).
"""
import numpy as np
import pytest

import talos_hip as th
from common import check_close, f32

pytestmark = pytest.mark.gpu
DA = th.DeviceArray
B1, B2, EPS = 0.9, 0.999, 1e-8


def _grads(rng, n, t, scale=1.0):
    g = rng.normal(size=n) * scale * (1.0 + 0.3 * t)
    if n > 8:
        g[::9] = 0.0  # exact zeros: the first update there is exactly 0
    return f32(g)


def _dev(a, offset):
    """Device copy of a at an element offset (offset 1 makes the pointer 4-byte, not 16-byte,
    aligned and selects the scalar path)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    d = DA.zeros(a.size + offset)
    th.call("talos_memcpy_h2d", d.offset(offset), a.ctypes.data, a.nbytes, None)
    return d


def _host(d, n, offset):
    th.call("talos_stream_sync", None)
    out = np.empty(n, np.float32)
    if n:
        th.call("talos_memcpy_d2h", out.ctypes.data, d.offset(offset), 4 * n, None)
    return out


def _check_state(n, off, dp, dm, dv, p0, rp, rm, rv, tag):
    check_close(_host(dp, n, off).astype(np.float64) - p0, rp - p0, name=f"{tag} delta p")
    check_close(_host(dm, n, off), rm, name=f"{tag} m")
    # v is a positive combination of g^2 terms (no cancellation), each step's update formed in f64
    # and rounded once to fp32: a relative error of a few 2^-24, so purely relative, no floor
    check_close(_host(dv, n, off), rv, atol=0.0, name=f"{tag} v")


@pytest.mark.parametrize("n", [1, 3, 4, 4099, 1000003])
@pytest.mark.parametrize("offset", [0, 1])
def test_adam_steps_match_oracle(oracle, n, offset):
    rng = np.random.default_rng(n + 10 * offset)
    p0 = f32(rng.normal(size=n) * 0.5)
    dp, dm, dv = _dev(p0, offset), DA.zeros(n + offset), DA.zeros(n + offset)
    rp, rm, rv = p0.astype(np.float64), np.zeros(n), np.zeros(n)
    lr = 1e-2
    for t in range(1, 6):
        g = _grads(rng, n, t)
        dg = _dev(g, offset)
        th.call("talos_adam_step_f32", n, dp.offset(offset), dg.offset(offset), dm.offset(offset), dv.offset(offset),
                t, lr, B1, B2, EPS, None, 0.0, None)
        oracle.adam_step(rp, g, rm, rv, t, lr)
        _check_state(n, offset, dp, dm, dv, p0.astype(np.float64), rp, rm, rv, f"n={n} off={offset} t={t}")
        dg.free()
    for d in (dp, dm, dv):
        d.free()


@pytest.mark.parametrize("scale", [4.0, 0.02])
def test_adam_global_norm_clip_multi_tensor(oracle, scale):
    """Three parameter tensors of ragged sizes share one norm (sumsq accumulated over them), as
    the DQN optimizer's norm loop runs over every parameter; scale 4 clips, 0.02 does not."""
    rng = np.random.default_rng(int(scale * 100))
    sizes = [517, 64, 130001]
    n = sum(sizes)
    p0 = f32(rng.normal(size=n) * 0.3)
    rp, rm, rv = p0.astype(np.float64), np.zeros(n), np.zeros(n)
    dps = [DA.from_numpy(x) for x in np.split(p0, np.cumsum(sizes)[:-1])]
    dms = [DA.zeros(s) for s in sizes]
    dvs = [DA.zeros(s) for s in sizes]
    sumsq = DA.zeros(1, np.float64)
    ws = DA.zeros(th.lib().talos_grad_sumsq_workspace_bytes() // 8, np.float64)  # caller workspace from t = 2
    lr = 1e-2
    for t in range(1, 4):
        g = f32(rng.normal(size=n) * scale / np.sqrt(n))
        dgs = [DA.from_numpy(x) for x in np.split(g, np.cumsum(sizes)[:-1])]
        for i, dg in enumerate(dgs):
            th.call("talos_grad_sumsq_f32", sizes[i], dg.ptr, int(i > 0), sumsq.ptr, ws.ptr if t > 1 else None, None)
        ref_ss = float(np.sum(g.astype(np.float64) ** 2))
        got_ss = float(sumsq.numpy()[0])
        assert abs(got_ss - ref_ss) <= 1e-12 * ref_ss, (got_ss, ref_ss)
        assert (np.sqrt(ref_ss) > 1.0) == (scale > 1.0)
        for i, dg in enumerate(dgs):
            th.call("talos_adam_step_f32", sizes[i], dps[i].ptr, dg.ptr, dms[i].ptr, dvs[i].ptr, t, lr, B1, B2, EPS,
                    sumsq.ptr, 1.0, None)
        oracle.adam_step(rp, g, rm, rv, t, lr, max_norm=1.0)
        got_p = np.concatenate([d.numpy() for d in dps]).astype(np.float64)
        check_close(got_p - p0, rp - p0, name=f"clip scale={scale} t={t} delta p")
        check_close(np.concatenate([d.numpy() for d in dms]), rm, name=f"clip t={t} m")
        check_close(np.concatenate([d.numpy() for d in dvs]), rv, atol=0.0, name=f"clip t={t} v")
        for dg in dgs:
            dg.free()


def test_grad_sumsq_edges_and_determinism():
    rng = np.random.default_rng(3)
    sumsq = DA.from_numpy(np.array([2.5]), np.float64)
    th.call("talos_grad_sumsq_f32", 0, None, 1, sumsq.ptr, None, None)  # empty, accumulate: unchanged
    assert sumsq.numpy()[0] == 2.5
    th.call("talos_grad_sumsq_f32", 0, None, 0, sumsq.ptr, None, None)  # empty, overwrite: zero
    assert sumsq.numpy()[0] == 0.0
    g = f32(rng.normal(size=3_000_001))
    dg = DA.from_numpy(g)
    results = []
    for off in (0, 0, 1):
        th.call("talos_grad_sumsq_f32", g.size - off, dg.offset(off), 0, sumsq.ptr, None, None)
        results.append(float(sumsq.numpy()[0]))
    assert results[0] == results[1]  # fixed partition: bit-identical repeats
    ref = float(np.sum(g.astype(np.float64) ** 2))
    assert abs(results[0] - ref) <= 1e-12 * ref
    ref1 = float(np.sum(g[1:].astype(np.float64) ** 2))
    assert abs(results[2] - ref1) <= 1e-12 * ref1
