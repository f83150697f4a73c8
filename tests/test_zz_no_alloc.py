"""talos_attn_bwd_noalloc_f32, the attention backward that allocates nothing (its scratch is a
static device array), against talos_attn_bwd_f32 on the same inputs: two calls in a row, the
second smaller, so a stale scratch from the first call would show in the second. Both entry points
run the same kernels in the same order, so the gradients must agree bit for bit."""
import ctypes

import numpy as np
import pytest

import talos_hip as th

DA = th.DeviceArray


def _case(B, S, H, dk, dv, causal, seed):
    rng = np.random.default_rng(seed)
    q, k = rng.normal(size=(B, S, H * dk)), rng.normal(size=(B, S, H * dk))
    v, g = rng.normal(size=(B, S, H * dv)), rng.normal(size=(B, S, H * dv))
    Q, K, V, G = (DA.from_numpy(a) for a in (q, k, v, g))
    O, L = DA.zeros((B, S, H * dv)), DA.zeros((B, H, S))
    scale = 1.0 / np.sqrt(dk)
    th.call("talos_attn_fwd_f32", B, S, H, dk, dv, scale, causal, Q.ptr, H * dk, K.ptr, H * dk, V.ptr, H * dv, O.ptr,
            H * dv, L.ptr, None)
    return (Q, K, V, O, L, G), scale


def _bwd(entry, B, S, H, dk, dv, causal, bufs, scale):
    Q, K, V, O, L, G = bufs
    dQ, dK, dV = DA.zeros((B, S, H * dk)), DA.zeros((B, S, H * dk)), DA.zeros((B, S, H * dv))
    th.call(entry, B, S, H, dk, dv, scale, causal, Q.ptr, H * dk, K.ptr, H * dk, V.ptr, H * dv, O.ptr, H * dv, L.ptr,
            G.ptr, H * dv, dQ.ptr, H * dk, dK.ptr, H * dk, dV.ptr, H * dv, None)
    return dQ.numpy(), dK.numpy(), dV.numpy()


@pytest.mark.gpu
def test_noalloc_attn_bwd_matches_attn_bwd():
    # seq > 32 takes the split dQ / dK-dV kernels, which keep D = rowsum(dO * O) in the scratch;
    # the second call is smaller (fewer rows, another head dim), the third takes the single-block
    # kernel of seq <= 32 (no scratch)
    cases = [(6, 200, 4, 64, 64, 1), (3, 77, 2, 32, 32, 0), (5, 32, 4, 32, 32, 1)]
    for i, (B, S, H, dk, dv, causal) in enumerate(cases):
        bufs, scale = _case(B, S, H, dk, dv, causal, 100 + i)
        got = _bwd("talos_attn_bwd_noalloc_f32", B, S, H, dk, dv, causal, bufs, scale)
        ref = _bwd("talos_attn_bwd_f32", B, S, H, dk, dv, causal, bufs, scale)
        for name, a, b in zip(("dq", "dk", "dv"), got, ref):
            assert np.all(np.isfinite(a)), f"case {i} {name}: non-finite"
            assert np.array_equal(a, b), f"case {i} {name}: max |diff| {np.abs(a - b).max():.3e}"


def test_noalloc_attn_bwd_rejects_more_rows_than_the_scratch():
    # checked on the host before any device call: runs without a GPU
    p = ctypes.c_void_p(256)
    args = [p, 64, p, 64, p, 64, p, 64, p, p, 64, p, 64, p, 64, p, 64, None]
    rc = th.lib().talos_attn_bwd_noalloc_f32(4096, 65, 4, 16, 16, ctypes.c_float(0.25), 1, *args)
    assert rc == th.ERR_UNSUPPORTED
    assert b"static scratch" in th.lib().talos_last_error()
    assert th.lib().talos_attn_bwd_noalloc_f32(2, 8, 4, 16, 16, ctypes.c_float(0.25), 1, None, *args[1:]) == th.ERR_NULL
