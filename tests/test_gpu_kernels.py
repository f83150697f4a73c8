"""GPU parity of the kernel-level entry points against the f64 oracle (and closed forms).

Comparison rule (north star): fp32 results within |got - ref| <= 1e-4 * |ref| + 1e-5 element-wise
against the f64 oracle run on the same fp32-rounded inputs; integer / index work (causal masks,
position tables) bit-exact.
"""
import ctypes
import math

import numpy as np
import pytest

import talos_hip as th
from common import FP32_ATOL, FP32_RTOL, check_close, f32, xavier

pytestmark = pytest.mark.gpu
DA = th.DeviceArray


def gemm(tA, tB, A, B, alpha=1.0, beta=0.0, C0=None):
    """Runs talos_gemm_f32 on host arrays (A, B stored as given; op applied by the flags)."""
    M = A.shape[1] if tA else A.shape[0]
    K = A.shape[0] if tA else A.shape[1]
    N = B.shape[0] if tB else B.shape[1]
    dA, dB = DA.from_numpy(A), DA.from_numpy(B)
    dC = DA.from_numpy(C0) if C0 is not None else DA.zeros((M, N))
    th.call("talos_gemm_f32", tA, tB, M, N, K, alpha, dA.ptr, A.shape[1], dB.ptr, B.shape[1], beta, dC.ptr, N, None)
    return dC.numpy()


def ref_gemm(tA, tB, A, B, alpha=1.0, beta=0.0, C0=None):
    a = f32(A).T if tA else f32(A)
    b = f32(B).T if tB else f32(B)
    r = alpha * (a @ b)
    if beta and C0 is not None:
        r = r + beta * f32(C0)
    return r


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (37, 5, 3), (128, 128, 32), (130, 257, 67), (256, 64, 64),
                                   (300, 129, 515)])
def test_gemm_layouts_and_ragged_shapes(tA, tB, M, N, K):
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    A = rng.normal(size=(K, M) if tA else (M, K)).astype(np.float32)
    B = rng.normal(size=(N, K) if tB else (K, N)).astype(np.float32)
    got = gemm(tA, tB, A, B)
    ref = ref_gemm(tA, tB, A, B)
    # dot products of length K in fp32: error ~ eps * sqrt(K) * |a||b|; bound it by the sum of |terms|
    a = np.abs(f32(A).T if tA else f32(A))
    b = np.abs(f32(B).T if tB else f32(B))
    bound = 1e-5 * (a @ b) + 1e-30
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


def test_gemm_alpha_beta_accumulate():
    rng = np.random.default_rng(3)
    A, B, C0 = (rng.normal(size=s).astype(np.float32) for s in ((200, 96), (96, 130), (200, 130)))
    got = gemm(0, 0, A, B, alpha=0.5, beta=1.0, C0=C0)
    check_close(got, ref_gemm(0, 0, A, B, 0.5, 1.0, C0), rtol=1e-5, atol=1e-4, name="alpha/beta")
    got = gemm(0, 0, A, B, alpha=1.0, beta=0.0, C0=np.full((200, 130), np.nan, np.float32))
    assert np.all(np.isfinite(got)), "beta = 0 must not read C"


def test_gemm_split_k_long_reduction():
    # dW = X^T dY over 65536 rows: the split-K path with f64 combination of partials
    rng = np.random.default_rng(4)
    X = rng.normal(size=(65536, 128)).astype(np.float32)
    G = rng.normal(size=(65536, 96)).astype(np.float32)
    got = gemm(1, 0, X, G)
    ref = f32(X).T @ f32(G)
    scale = np.abs(f32(X)).T @ np.abs(f32(G))
    err = np.abs(got - ref)
    assert np.all(err <= 1e-6 * scale + 1e-6), float(np.max(err / scale))


def test_bound_workspace_replaces_per_call_allocation():
    # A caller-owned workspace bound on this thread serves the scratch of the kernel-level entry
    # points: results equal the unbound calls' (the split-K product within its bound, since a
    # workspace too small for the library's split count makes it split K fewer times).
    rng = np.random.default_rng(6)
    ws_bytes = 1 << 20
    ws = DA.zeros(ws_bytes // 4)
    X = rng.normal(size=(65536, 64)).astype(np.float32)
    G = rng.normal(size=(65536, 64)).astype(np.float32)
    free = gemm(1, 0, X, G)
    x, dy = rng.normal(size=(5000, 96)), rng.normal(size=(5000, 96))
    w, rstd = rng.uniform(0.9, 1.1, 96), 1.0 / np.sqrt((x * x).mean(1) + 1e-6)
    Xd, Wd, Rd, DYd = (DA.from_numpy(a) for a in (x, w, rstd, dy))

    def norm_bwd():
        dx, dw = DA.zeros((5000, 96)), DA.zeros(96)
        th.call("talos_rmsnorm_bwd_f32", 5000, 96, Xd.ptr, Wd.ptr, Rd.ptr, DYd.ptr, 0.0, dx.ptr, 0.0, dw.ptr, None)
        s = DA.zeros(1)
        th.call("talos_reduce_sum_f32", 5000 * 96, 1.0, DYd.ptr, s.ptr, None)
        db = DA.zeros(96)
        th.call("talos_bias_grad_f32", 5000, 96, DYd.ptr, 0.0, db.ptr, None)
        return dx.numpy(), dw.numpy(), s.numpy(), db.numpy()

    ref = norm_bwd()
    th.call("talos_workspace_bind", ws.ptr, ws_bytes)
    try:
        bound = gemm(1, 0, X, G)
        got = norm_bwd()
        high = th.lib().talos_workspace_high_water()
    finally:
        th.call("talos_workspace_bind", None, 0)
    scale = np.abs(f32(X)).T @ np.abs(f32(G))
    assert np.all(np.abs(bound - free) <= 2e-6 * scale), "split-K product with the bound workspace"
    for a, b in zip(got, ref):
        assert np.array_equal(a, b)
    assert high > ws_bytes, "the split-K product asked for more than the bound workspace"


def test_gemm_batched_qk_pv():
    rng = np.random.default_rng(5)
    Bt, S, D = 6, 33, 20
    q, k, v = (rng.normal(size=(Bt, S, D)).astype(np.float32) for _ in range(3))
    dq, dk, dv = DA.from_numpy(q), DA.from_numpy(k), DA.from_numpy(v)
    sc = DA.zeros((Bt, S, S))
    th.call("talos_gemm_batched_f32", 0, 1, S, S, D, 1.0, dq.ptr, D, S * D, dk.ptr, D, S * D, 0.0, sc.ptr, S, S * S,
            Bt, None)
    ref = np.einsum("bid,bjd->bij", f32(q), f32(k))
    check_close(sc.numpy(), ref, rtol=1e-5, atol=1e-5, name="QK^T")
    o = DA.zeros((Bt, S, D))
    th.call("talos_gemm_batched_f32", 0, 0, S, D, S, 1.0, sc.ptr, S, S * S, dv.ptr, D, S * D, 0.0, o.ptr, D, S * D,
            Bt, None)
    check_close(o.numpy(), np.einsum("bij,bjd->bid", f32(sc.numpy()), f32(v)), rtol=1e-5, atol=1e-4, name="PV")


# --- C1: Linear [256,64] . [64,64] + MSE ------------------------------------------------
def test_c1_linear_mse_vs_oracle(oracle):
    rng = np.random.default_rng(100)
    X = f32(rng.normal(size=(256, 64)))
    W = f32(xavier(rng, 64, 64))
    b = np.zeros(64)
    T = f32(rng.normal(size=(256, 64)))
    loss_r, dx_r, dw_r, db_r = oracle.linear_mse(X, W, b, T)
    dX, dW, db, dT = DA.from_numpy(X), DA.from_numpy(W), DA.from_numpy(b), DA.from_numpy(T)
    Y, R, dY = DA.zeros((256, 64)), DA.zeros((256, 64)), DA.zeros((256, 64))
    gX, gW, gb, loss = DA.zeros((256, 64)), DA.zeros((64, 64)), DA.zeros(64), DA.zeros(1)
    n = 256 * 64
    th.call("talos_broadcast_rows_f32", 256, 64, db.ptr, Y.ptr, None)                        # y = broadcast(b)
    th.call("talos_gemm_f32", 0, 0, 256, 64, 64, 1.0, dX.ptr, 64, dW.ptr, 64, 1.0, Y.ptr, 64, None)  # y += X W
    th.call("talos_binary_fwd_f32", th.SUB, n, Y.ptr, dT.ptr, R.ptr, None)                   # r = y - t
    sq = DA.zeros((256, 64))
    th.call("talos_binary_fwd_f32", th.MUL, n, R.ptr, R.ptr, sq.ptr, None)
    th.call("talos_reduce_sum_f32", n, 1.0 / n, sq.ptr, loss.ptr, None)                       # mean
    th.call("talos_unary_fwd_f32", th.SCALE, n, 2.0 / n, 0.0, R.ptr, dY.ptr, None)           # dy = 2 r / N
    th.call("talos_gemm_f32", 0, 1, 256, 64, 64, 1.0, dY.ptr, 64, dW.ptr, 64, 1.0, gX.ptr, 64, None)  # dX += dY W^T
    th.call("talos_gemm_f32", 1, 0, 64, 64, 256, 1.0, dX.ptr, 64, dY.ptr, 64, 1.0, gW.ptr, 64, None)  # dW += X^T dY
    th.call("talos_bias_grad_f32", 256, 64, dY.ptr, 1.0, gb.ptr, None)                        # db += sum dY
    check_close(loss.numpy()[0], loss_r, name="loss")
    check_close(gX.numpy(), dx_r, name="dX")
    check_close(gW.numpy(), dw_r, name="dW")
    check_close(gb.numpy(), db_r, name="db")


# --- C2: row ops at [4096, 256] -----------------------------------------------------------
def test_c2_rmsnorm_fwd_bwd_vs_oracle(oracle):
    rng = np.random.default_rng(200)
    rows, dim, eps = 4096, 256, 1e-6
    x, g = f32(rng.normal(size=(rows, dim))), f32(rng.normal(size=(rows, dim)))
    w = f32(rng.uniform(0.9, 1.1, dim))
    y_r, dx_r, dw_r = oracle.rmsnorm_fwd_bwd(x, w, g, eps)
    dx_, dw_, dg_ = DA.from_numpy(x), DA.from_numpy(w), DA.from_numpy(g)
    y, rstd, dxo, dwo = DA.zeros((rows, dim)), DA.zeros(rows), DA.zeros((rows, dim)), DA.zeros(dim)
    th.call("talos_rmsnorm_fwd_f32", rows, dim, eps, dx_.ptr, dw_.ptr, y.ptr, rstd.ptr, None)
    th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 0.0, dxo.ptr, 0.0, dwo.ptr, None)
    check_close(y.numpy(), y_r, name="y")
    check_close(dxo.numpy(), dx_r, name="dx")
    check_close(dwo.numpy(), dw_r, name="dgain")
    # accumulate mode adds onto what is there
    th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 1.0, dxo.ptr, 1.0, dwo.ptr, None)
    check_close(dxo.numpy(), 2 * dx_r, name="dx accumulate")
    check_close(dwo.numpy(), 2 * dw_r, name="dgain accumulate")


# (rows, dim): 256 partial rows (C2), 34, 1024 (two rows a wave), 19, a single partial, and the
# generic kernel (dim 1000)
@pytest.mark.parametrize("rows,dim", [(4096, 256), (16 * 33 + 5, 128), (40000, 256), (300, 100), (7, 512),
                                      (37, 1000)])
def test_rmsnorm_bwd_workspace_deterministic(oracle, rows, dim):
    """talos_rmsnorm_bwd_f32 from a bound workspace (the C2 bench's mode): it matches the oracle,
    repeated calls give the same bits (the gain gradient's partial rows are added in a fixed
    order), and the accumulate mode adds onto dx and dgain."""
    from common import check_grad
    rng = np.random.default_rng(rows + dim)
    eps = 1e-6
    x, g = f32(rng.normal(size=(rows, dim))), f32(rng.normal(size=(rows, dim)))
    w = f32(rng.uniform(0.9, 1.1, dim))
    y_r, dx_r, dw_r = oracle.rmsnorm_fwd_bwd(x, w, g, eps)
    xh = x / np.sqrt((x * x).mean(1, keepdims=True) + eps)
    mag = np.abs(g * xh).sum(0)  # the gain gradient's magnitude sums
    ws = DA.zeros(1 << 20)
    th.call("talos_workspace_bind", ws.ptr, 4 << 20)
    try:
        dx_, dw_, dg_ = DA.from_numpy(x), DA.from_numpy(w), DA.from_numpy(g)
        y, rstd, dxo, dwo = DA.zeros((rows, dim)), DA.zeros(rows), DA.zeros((rows, dim)), DA.zeros(dim)
        th.call("talos_rmsnorm_fwd_f32", rows, dim, eps, dx_.ptr, dw_.ptr, y.ptr, rstd.ptr, None)
        th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 0.0, dxo.ptr, 0.0, dwo.ptr,
                None)
        first_dx, first_dw = dxo.numpy(), dwo.numpy()
        check_close(first_dx, dx_r, name="dx")
        check_grad(first_dw, dw_r, mag, name="dgain")
        for _ in range(3):
            th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 0.0, dxo.ptr, 0.0,
                    dwo.ptr, None)
            assert np.array_equal(dwo.numpy(), first_dw) and np.array_equal(dxo.numpy(), first_dx)
        th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 1.0, dxo.ptr, 1.0, dwo.ptr,
                None)
        check_close(dxo.numpy(), 2 * dx_r, name="dx accumulate")
        check_grad(dwo.numpy(), 2 * dw_r, 2 * mag, name="dgain accumulate")
    finally:
        th.call("talos_workspace_bind", None, 0)
        ws.free()


@pytest.mark.parametrize("dim", [8, 100, 128, 512, 1000])
def test_rmsnorm_dims(oracle, dim):
    rng = np.random.default_rng(dim)
    rows = 37
    x, g = f32(rng.normal(size=(rows, dim))), f32(rng.normal(size=(rows, dim)))
    w = f32(rng.uniform(0.9, 1.1, dim))
    y_r, dx_r, dw_r = oracle.rmsnorm_fwd_bwd(x, w, g, 1e-5)
    dx_, dw_, dg_ = DA.from_numpy(x), DA.from_numpy(w), DA.from_numpy(g)
    y, rstd, dxo, dwo = DA.zeros((rows, dim)), DA.zeros(rows), DA.zeros((rows, dim)), DA.zeros(dim)
    th.call("talos_rmsnorm_fwd_f32", rows, dim, 1e-5, dx_.ptr, dw_.ptr, y.ptr, rstd.ptr, None)
    th.call("talos_rmsnorm_bwd_f32", rows, dim, dx_.ptr, dw_.ptr, rstd.ptr, dg_.ptr, 0.0, dxo.ptr, 0.0, dwo.ptr, None)
    check_close(y.numpy(), y_r, name="y")
    check_close(dxo.numpy(), dx_r, name="dx")
    check_close(dwo.numpy(), dw_r, name="dgain")


@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("rows,cols", [(4096, 256), (50, 7), (64, 64)])
def test_c2_softmax_fwd_bwd_vs_oracle(oracle, causal, rows, cols):
    rng = np.random.default_rng(300 + cols + causal)
    x, g = f32(rng.normal(size=(rows, cols))), f32(rng.normal(size=(rows, cols)))
    y_r, dx_r = oracle.softmax_fwd_bwd(x, g, causal)
    dxi, dgi = DA.from_numpy(x), DA.from_numpy(g)
    y, dx = DA.zeros((rows, cols)), DA.from_numpy(np.full((rows, cols), 7.0, np.float32))
    th.call("talos_softmax_fwd_f32", rows, cols, causal, dxi.ptr, y.ptr, None)
    th.call("talos_softmax_bwd_f32", rows, cols, causal, y.ptr, dgi.ptr, 0.0, dx.ptr, None)
    yg, dxg = y.numpy(), dx.numpy()
    check_close(yg, y_r, name="y")
    check_close(dxg, dx_r, name="dx")
    if causal:
        q = np.arange(rows)[:, None] % cols
        mask = np.arange(cols)[None, :] > q
        # masked entries are exactly zero (bit-exact), in the forward and the backward
        assert np.all(yg[mask] == 0.0) and np.all(dxg[mask] == 0.0)
        assert np.all(dxg[q[:, 0] == 0] == 0.0)  # a row with a single key has zero gradient


def test_c2_rope_bwd_vs_oracle(oracle):
    rng = np.random.default_rng(400)
    n_seq, seq, heads, dim, base = 64, 64, 4, 64, 10000.0
    x, g = f32(rng.normal(size=(n_seq, seq, heads, dim))), f32(rng.normal(size=(n_seq, seq, heads, dim)))
    y_r, dx_r = oracle.rope_fwd_bwd(x, g, base)
    dxi, dgi = DA.from_numpy(x), DA.from_numpy(g)
    y, dx = DA.zeros(x.shape), DA.zeros(x.shape)
    th.call("talos_rope_fwd_f32", n_seq, seq, heads, dim, 0, base, dxi.ptr, y.ptr, None)
    th.call("talos_rope_bwd_f32", n_seq, seq, heads, dim, 0, base, dgi.ptr, 0.0, dx.ptr, None)
    check_close(y.numpy(), y_r, name="rope fwd")
    check_close(dx.numpy(), dx_r, name="rope bwd")
    # position 0 is the identity, bit-exact
    assert np.array_equal(dx.numpy()[:, 0], g[:, 0].astype(np.float32))


def test_rope_table_bit_exact(oracle):
    max_len, dim = 256, 32
    c_r, s_r = oracle.rope_table(max_len, dim, 10000.0)
    c, s = DA.zeros((max_len, dim // 2)), DA.zeros((max_len, dim // 2))
    th.call("talos_rope_table_f32", max_len, dim, 10000.0, c.ptr, s.ptr, None)
    assert np.array_equal(c.numpy(), c_r.astype(np.float32))
    assert np.array_equal(s.numpy(), s_r.astype(np.float32))


def test_rope_start_pos_and_accumulate(oracle):
    rng = np.random.default_rng(401)
    x = f32(rng.normal(size=(3, 5, 2, 8)))
    g = f32(rng.normal(size=x.shape))
    y_r, dx_r = oracle.rope_fwd_bwd(x, g, 500.0, start_pos=7)
    dxi, dgi = DA.from_numpy(x), DA.from_numpy(g)
    y, dx = DA.zeros(x.shape), DA.from_numpy(g)
    th.call("talos_rope_fwd_f32", 3, 5, 2, 8, 7, 500.0, dxi.ptr, y.ptr, None)
    th.call("talos_rope_bwd_f32", 3, 5, 2, 8, 7, 500.0, dgi.ptr, 1.0, dx.ptr, None)
    check_close(y.numpy(), y_r, name="y")
    check_close(dx.numpy(), dx_r + g, name="dx (+ existing)")


# --- attention ----------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [0, 1])
# 32 < seq <= 64 at head dims 32: the four-block backward (33 and 47 leave a partial second block)
@pytest.mark.parametrize("B,S,H,dk,dv", [(2, 7, 3, 5, 4), (3, 32, 4, 32, 32), (2, 64, 4, 32, 32),
                                         (3, 33, 2, 32, 32), (2, 47, 3, 32, 32),
                                         (1, 200, 2, 96, 64), (2, 300, 1, 16, 16),
                                         # seq <= 32: the single-block backward at every head-dim class
                                         (2, 20, 3, 64, 64), (2, 32, 2, 96, 64), (1, 17, 2, 128, 128),
                                         (2, 31, 3, 40, 24), (5, 1, 2, 32, 32)])
def test_attention_fwd_bwd_vs_oracle(oracle, causal, B, S, H, dk, dv):
    rng = np.random.default_rng(500 + S + dk + causal)
    q, k = f32(rng.normal(size=(B, S, H, dk))), f32(rng.normal(size=(B, S, H, dk)))
    v, g = f32(rng.normal(size=(B, S, H, dv))), f32(rng.normal(size=(B, S, H, dv)))
    scale = 1.0 / math.sqrt(dk)
    o_r, dq_r, dk_r, dv_r = oracle.attention_fwd_bwd(q, k, v, g, scale, causal)
    Q, K, V, G = (DA.from_numpy(a) for a in (q, k, v, g))
    O, L = DA.zeros((B, S, H, dv)), DA.zeros((B, H, S))
    dQ, dK, dV = DA.zeros(q.shape), DA.zeros(k.shape), DA.zeros(v.shape)
    hk, hv = H * dk, H * dv
    th.call("talos_attn_fwd_f32", B, S, H, dk, dv, scale, causal, Q.ptr, hk, K.ptr, hk, V.ptr, hv, O.ptr, hv, L.ptr,
            None)
    th.call("talos_attn_bwd_f32", B, S, H, dk, dv, scale, causal, Q.ptr, hk, K.ptr, hk, V.ptr, hv, O.ptr, hv, L.ptr,
            G.ptr, hv, dQ.ptr, hk, dK.ptr, hk, dV.ptr, hv, None)
    check_close(O.numpy(), o_r, name="o")
    check_close(dQ.numpy(), dq_r, name="dq")
    check_close(dK.numpy(), dk_r, name="dk")
    check_close(dV.numpy(), dv_r, name="dv")
    # lse matches the f64 log-sum-exp of the scaled (masked) scores
    s = np.einsum("bihd,bjhd->bhij", q, k) * scale
    if causal:
        s = np.where(np.triu(np.ones((S, S), bool), 1), -np.inf, s)
    mx = s.max(-1, keepdims=True)
    lse = (np.log(np.exp(s - mx).sum(-1, keepdims=True)) + mx)[..., 0]
    check_close(L.numpy(), lse, name="lse")


# --- element-wise / layout ops --------------------------------------------------------------
@pytest.mark.parametrize("op,fwd,dfn,lo,hi", [
    (th.RELU, lambda x: np.maximum(x, 0), lambda x: (x > 0) * 1.0, -2, 2),
    (th.EXP, np.exp, np.exp, -2, 2),
    (th.LOG, np.log, lambda x: 1 / x, 0.1, 3),
    (th.SIN, np.sin, np.cos, -3, 3),
    (th.COS, np.cos, lambda x: -np.sin(x), -3, 3),
    (th.SQRT, np.sqrt, lambda x: 0.5 / np.sqrt(x), 0.1, 3),
    (th.NEG, lambda x: -x, lambda x: -np.ones_like(x), -2, 2),
])
def test_unary_ops(op, fwd, dfn, lo, hi):
    rng = np.random.default_rng(op)
    x = f32(rng.uniform(lo, hi, 5000))
    g = f32(rng.normal(size=5000))
    dx0 = f32(rng.normal(size=5000))
    X, G, Y, DX = DA.from_numpy(x), DA.from_numpy(g), DA.zeros(5000), DA.from_numpy(dx0)
    th.call("talos_unary_fwd_f32", op, 5000, 0.0, 0.0, X.ptr, Y.ptr, None)
    th.call("talos_unary_bwd_f32", op, 5000, 0.0, 0.0, X.ptr, G.ptr, DX.ptr, None)
    check_close(Y.numpy(), fwd(x), rtol=2e-6, atol=1e-6, name="fwd")
    check_close(DX.numpy(), dx0 + dfn(x) * g, rtol=2e-6, atol=1e-6, name="bwd")


def test_gelu_clip_scale(oracle):
    rng = np.random.default_rng(9)
    x = f32(rng.normal(size=4096) * 3)
    X, Y, G, DX = DA.from_numpy(x), DA.zeros(4096), DA.from_numpy(np.ones(4096)), DA.zeros(4096)
    t = oracle.T.new(x, [4096])
    gt = t.gelu()
    gt.sum().backward()
    th.call("talos_unary_fwd_f32", th.GELU, 4096, 0.0, 0.0, X.ptr, Y.ptr, None)
    th.call("talos_unary_bwd_f32", th.GELU, 4096, 0.0, 0.0, X.ptr, G.ptr, DX.ptr, None)
    check_close(Y.numpy(), gt.data, name="gelu")
    check_close(DX.numpy(), t.grad, name="gelu'")
    th.call("talos_unary_fwd_f32", th.CLIP, 4096, -1.0, 1.5, X.ptr, Y.ptr, None)
    assert np.array_equal(Y.numpy(), np.clip(x, -1.0, 1.5).astype(np.float32))


def test_binary_ops_and_alias():
    rng = np.random.default_rng(10)
    a, b, g = (f32(rng.uniform(0.5, 2, 3000)) for _ in range(3))
    A, Bv, G = DA.from_numpy(a), DA.from_numpy(b), DA.from_numpy(g)
    for op, f, da, db in [(th.ADD, a + b, g, g), (th.SUB, a - b, g, -g), (th.MUL, a * b, g * b, g * a),
                          (th.DIV, a / b, g / b, -g * a / b ** 2)]:
        Y, DAo, DBo = DA.zeros(3000), DA.zeros(3000), DA.zeros(3000)
        th.call("talos_binary_fwd_f32", op, 3000, A.ptr, Bv.ptr, Y.ptr, None)
        th.call("talos_binary_bwd_f32", op, 3000, A.ptr, Bv.ptr, G.ptr, DAo.ptr, DBo.ptr, None)
        check_close(Y.numpy(), f, rtol=1e-6, atol=1e-7)
        check_close(DAo.numpy(), da, rtol=1e-6, atol=1e-7)
        check_close(DBo.numpy(), db, rtol=1e-6, atol=1e-7)
    # x * x with both operands the same tensor: d/dx = 2 x g accumulated once (src/autograd.rs:1729-1737)
    DX = DA.zeros(3000)
    th.call("talos_binary_bwd_f32", th.MUL, 3000, A.ptr, A.ptr, G.ptr, DX.ptr, DX.ptr, None)
    check_close(DX.numpy(), 2 * a * g, rtol=1e-6, atol=1e-7)


def test_reduce_transpose_concat_broadcast():
    rng = np.random.default_rng(11)
    x = f32(rng.normal(size=(3, 4, 5, 6)))
    X = DA.from_numpy(x)
    out = DA.zeros(1)
    th.call("talos_reduce_sum_f32", x.size, 0.5, X.ptr, out.ptr, None)
    check_close(out.numpy()[0], 0.5 * x.sum(), rtol=1e-6)
    shape = (ctypes.c_longlong * 4)(*x.shape)
    Y = DA.zeros((3, 5, 4, 6))
    th.call("talos_transpose_f32", 4, shape, 1, 2, X.ptr, Y.ptr, 0, None)
    assert np.array_equal(Y.numpy(), np.swapaxes(x, 1, 2).astype(np.float32))
    a, b = f32(rng.normal(size=(10, 3))), f32(rng.normal(size=(10, 5)))
    Ad, Bd, C = DA.from_numpy(a), DA.from_numpy(b), DA.zeros((10, 8))
    th.call("talos_concat_last_f32", 10, 3, 5, Ad.ptr, Bd.ptr, C.ptr, None)
    assert np.array_equal(C.numpy(), np.concatenate([a, b], 1).astype(np.float32))
    ga, gb = DA.zeros((10, 3)), DA.zeros((10, 5))
    th.call("talos_concat_last_bwd_f32", 10, 3, 5, C.ptr, ga.ptr, gb.ptr, None)
    assert np.array_equal(ga.numpy(), a.astype(np.float32)) and np.array_equal(gb.numpy(), b.astype(np.float32))
    v = DA.from_numpy(np.arange(7.0))
    o = DA.zeros((4, 7))
    th.call("talos_broadcast_rows_f32", 4, 7, v.ptr, o.ptr, None)
    assert np.array_equal(o.numpy(), np.tile(np.arange(7.0), (4, 1)).astype(np.float32))
    g = DA.from_numpy(np.array([2.0]))
    dx = DA.zeros(9)
    th.call("talos_fill_add_f32", 9, 0.25, g.ptr, dx.ptr, None)
    assert np.array_equal(dx.numpy(), np.full(9, 0.5, np.float32))
    db = DA.from_numpy(np.ones(6))
    ones = DA.from_numpy(np.ones((1000, 6)))  # held: a temporary would be freed before the launch
    th.call("talos_bias_grad_f32", 1000, 6, ones.ptr, 1.0, db.ptr, None)
    assert np.array_equal(db.numpy(), np.full(6, 1001.0, np.float32))


def test_empty_inputs_are_noops():
    p = DA.zeros(4)
    th.call("talos_gemm_f32", 0, 0, 0, 4, 4, 1.0, p.ptr, 4, p.ptr, 4, 0.0, p.ptr, 4, None)
    th.call("talos_rmsnorm_fwd_f32", 0, 4, 1e-6, p.ptr, p.ptr, p.ptr, p.ptr, None)
    th.call("talos_softmax_fwd_f32", 0, 4, 1, p.ptr, p.ptr, None)
    th.call("talos_unary_fwd_f32", th.EXP, 0, 0.0, 0.0, p.ptr, p.ptr, None)
    th.sync()
    # K = 0: C = beta * C
    C = DA.from_numpy(np.full((2, 4), 3.0))
    th.call("talos_gemm_f32", 0, 0, 2, 4, 0, 1.0, p.ptr, 1, p.ptr, 4, 1.0, C.ptr, 4, None)
    assert np.array_equal(C.numpy(), np.full((2, 4), 3.0, np.float32))
    th.call("talos_gemm_f32", 0, 0, 2, 4, 0, 1.0, p.ptr, 1, p.ptr, 4, 0.0, C.ptr, 4, None)
    assert np.array_equal(C.numpy(), np.zeros((2, 4), np.float32))


def bf16_round(a):
    """Round-to-nearest-even fp32 -> bf16 (kept in fp32), the rounding the bf16 GEMM applies."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("tA,tB", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (37, 5, 3), (130, 257, 67), (256, 128, 128), (300, 129, 515)])
def test_gemm_bf16acc_layouts(tA, tB, M, N, K):
    # bf16 x bf16 products are exact in fp32, so against an f64 product of the bf16-rounded inputs
    # only the fp32 accumulation error remains
    rng = np.random.default_rng(7 * M + N + K)
    A = rng.normal(size=(K, M) if tA else (M, K)).astype(np.float32)
    B = rng.normal(size=(N, K) if tB else (K, N)).astype(np.float32)
    dA, dB, dC = DA.from_numpy(A), DA.from_numpy(B), DA.zeros((M, N))
    th.call("talos_gemm_bf16acc_f32", tA, tB, M, N, K, 1.0, dA.ptr, A.shape[1], dB.ptr, B.shape[1], 0.0, dC.ptr, N,
            None)
    got = dC.numpy()
    Ab, Bb = bf16_round(A).astype(np.float64), bf16_round(B).astype(np.float64)
    a, b = (Ab.T if tA else Ab), (Bb.T if tB else Bb)
    ref = a @ b
    bound = 1e-5 * (np.abs(a) @ np.abs(b)) + 1e-30
    assert np.all(np.abs(got - ref) <= bound), np.max(np.abs(got - ref) / bound)


def test_gemm_bf16acc_split_k():
    rng = np.random.default_rng(8)
    X = rng.normal(size=(40000, 128)).astype(np.float32)
    G = rng.normal(size=(40000, 64)).astype(np.float32)
    dX, dG, dC = DA.from_numpy(X), DA.from_numpy(G), DA.zeros((128, 64))
    th.call("talos_gemm_bf16acc_f32", 1, 0, 128, 64, 40000, 1.0, dX.ptr, 128, dG.ptr, 64, 0.0, dC.ptr, 64, None)
    Xb, Gb = bf16_round(X).astype(np.float64), bf16_round(G).astype(np.float64)
    ref = Xb.T @ Gb
    scale = np.abs(Xb).T @ np.abs(Gb)
    assert np.all(np.abs(dC.numpy() - ref) <= 1e-6 * scale + 1e-6)


@pytest.mark.parametrize("n,off", [(1 << 16, 0), (4097, 0), (4096, 1)])
def test_gelu_entries(oracle, n, off):
    """talos_gelu_{fwd,bwd}_f32 against the oracle's gelu and its gradient, on the float4 path
    (n % 4 == 0, aligned) and the one-element path (ragged n, or pointers offset by one element),
    and bit-exact against the TALOS_GELU op of the unary entries (the same device function)."""
    rng = np.random.default_rng(31 + n + off)
    x, g, d0 = (f32(rng.normal(size=n) * s) for s in (3.0, 1.0, 1.0))
    t = oracle.T.new(x, [n])
    y = t.gelu()
    y.sum().backward()
    dref = np.asarray(t.grad)  # gelu'(x) in f64
    bufs = [DA.zeros(n + off) for _ in range(5)]
    X, G, Y, DX, DU = (b.offset(off) for b in bufs)
    for buf, a in ((bufs[0], x), (bufs[1], g), (bufs[3], d0)):
        buf.upload(np.concatenate([np.zeros(off, np.float32), a]))
    th.call("talos_gelu_fwd_f32", n, X, Y, None)
    check_close(bufs[2].numpy()[off:], y.data, name="gelu")
    th.call("talos_gelu_bwd_f32", n, X, G, 1.0, DX, None)  # accumulate into d0
    check_close(bufs[3].numpy()[off:], d0.astype(np.float64) + dref * g, name="gelu' (beta 1)")
    th.call("talos_gelu_bwd_f32", n, X, G, 0.0, DX, None)  # overwrite
    got = bufs[3].numpy()[off:]
    check_close(got, dref * g, name="gelu' (beta 0)")
    th.call("talos_unary_fwd_f32", th.GELU, n, 0.0, 0.0, X, DU, None)
    assert np.array_equal(bufs[4].numpy()[off:], bufs[2].numpy()[off:])
    bufs[4].upload(np.zeros(n + off, np.float32))
    th.call("talos_unary_bwd_f32", th.GELU, n, 0.0, 0.0, X, G, DU, None)
    assert np.array_equal(bufs[4].numpy()[off:], got)


def test_gelu_entries_c3_size():
    """At the MLP activation size of C3 ([32768, 512]) the float4 entries equal the unary op bit
    for bit (the oracle-checked function); every output is finite."""
    n = 32768 * 512
    rng = np.random.default_rng(5)
    x = f32(rng.normal(size=n) * 2)
    X, Y, U = DA.from_numpy(x), DA.zeros(n), DA.zeros(n)
    th.call("talos_gelu_fwd_f32", n, X.ptr, Y.ptr, None)
    th.call("talos_unary_fwd_f32", th.GELU, n, 0.0, 0.0, X.ptr, U.ptr, None)
    y, u = Y.numpy(), U.numpy()
    assert np.isfinite(y).all() and np.array_equal(y, u)


def _log_softmax(z):
    z = z.astype(np.float64)
    m = z.max(axis=1, keepdims=True)
    return z - m - np.log(np.exp(z - m).sum(axis=1, keepdims=True))


@pytest.mark.parametrize("n,A", [(1000, 3), (257, 7), (64, 40), (1, 1)])
def test_ppo_head_loss_entries(oracle, n, A):
    """talos_ppo_head_loss_{fwd,bwd}_f32 against the oracle's batched PPO loss graph (pinned
    against the per-sample graph of ppo.rs:702-749): loss, dlogits and dvalues; old log-probs
    spread so that samples fall inside and outside the clip range; stats sums add up to the loss
    and accumulate on a second call."""
    rng = np.random.default_rng(7 * n + A)
    logits = f32(rng.normal(size=(n, A)) * 1.5)
    values, ret, adv = (f32(rng.normal(size=n)) for _ in range(3))
    actions = rng.integers(0, A, n).astype(np.int32)
    lp = _log_softmax(logits)[np.arange(n), actions]
    old = f32(lp + rng.normal(scale=0.3, size=n))
    clip, cv, ce = 0.2, 0.5, 0.01
    cfg = oracle.PpoCfg(n, 1, 1, 1, 0, 1, 1, 1, A, 0, 0, 1e-5, 1e4, clip, cv, ce)
    ref_loss, ref_dl, ref_dv = oracle.ppo_batched_loss(cfg, logits, values, actions, old, adv, ret)
    Z, V, Ad, R, O = (DA.from_numpy(a) for a in (logits, values, adv, ret, old))
    Ac = DA.from_numpy(actions, np.int32)
    loss, stats = DA.zeros(1), DA.zeros(5, np.float64)
    th.call("talos_ppo_head_loss_fwd_f32", n, A, clip, cv, ce, Z.ptr, V.ptr, Ac.ptr, Ad.ptr, R.ptr, O.ptr,
            loss.ptr, stats.ptr, 0, None)
    check_close(loss.numpy(), [ref_loss], name="loss")
    st = stats.numpy()
    assert st[4] == n
    assert abs((-st[1] + cv * st[2] - ce * st[3]) / n - ref_loss) <= 1e-9 * max(1.0, abs(ref_loss))
    th.call("talos_ppo_head_loss_fwd_f32", n, A, clip, cv, ce, Z.ptr, V.ptr, Ac.ptr, Ad.ptr, R.ptr, O.ptr,
            None, stats.ptr, 1, None)
    assert np.allclose(stats.numpy(), 2 * st, rtol=1e-12, atol=0)
    DZ, DV, loss2 = DA.from_numpy(np.full((n, A), 7.0)), DA.from_numpy(np.full(n, 7.0)), DA.zeros(1)
    th.call("talos_ppo_head_loss_bwd_f32", n, A, clip, cv, ce, Z.ptr, V.ptr, Ac.ptr, Ad.ptr, R.ptr, O.ptr,
            DZ.ptr, DV.ptr, loss2.ptr, None)
    check_close(DZ.numpy(), ref_dl, name="dlogits")
    check_close(DV.numpy(), ref_dv, name="dvalues")
    assert loss2.numpy()[0] == loss.numpy()[0]


def test_ppo_head_loss_ratio_one_closed_form():
    """With old_logp equal to the current log-probability the ratio is exactly 1, both surrogates
    equal adv, and the loss reduces to mean(-adv + cv (v - ret)^2 - ce H)."""
    n, A = 48, 3
    rng = np.random.default_rng(2)
    logits = f32(rng.normal(size=(n, A)))
    values, ret, adv = (f32(rng.normal(size=n)) for _ in range(3))
    actions = (np.arange(n) % A).astype(np.int32)
    old = f32(_log_softmax(logits)[np.arange(n), actions])  # ratio 1 for every sample
    Z, V, Ad, R, O = (DA.from_numpy(a) for a in (logits, values, adv, ret, old))
    Ac = DA.from_numpy(actions, np.int32)
    loss = DA.zeros(1)
    th.call("talos_ppo_head_loss_fwd_f32", n, A, 0.2, 0.5, 0.01, Z.ptr, V.ptr, Ac.ptr, Ad.ptr, R.ptr, O.ptr,
            loss.ptr, None, 0, None)
    # ratio == 1: the surrogate is adv (both branches), so the loss has a closed form
    z = _log_softmax(logits)
    ent = -(np.exp(z) * z).sum(axis=1)
    closed = np.mean(-adv.astype(np.float64) + 0.5 * (values.astype(np.float64) - ret) ** 2 - 0.01 * ent)
    check_close(loss.numpy(), [closed], name="loss at ratio 1")


def test_async_mode_gives_the_same_results():
    """The asynchronous completion mode (talos_set_async(1)) enqueues the same work: a GEMM chain
    run in it and read after talos_stream_sync equals the default synchronous run bit for bit."""
    rng = np.random.default_rng(12)
    a, b = f32(rng.normal(size=(300, 200))), f32(rng.normal(size=(200, 130)))
    A, B = DA.from_numpy(a), DA.from_numpy(b)
    outs = []
    for mode in (0, 1):
        C, D = DA.zeros((300, 130)), DA.zeros((300, 130))
        th.call("talos_set_async", mode)
        try:
            th.call("talos_gemm_f32", 0, 0, 300, 130, 200, 1.0, A.ptr, 200, B.ptr, 130, 0.0, C.ptr, 130, None)
            th.call("talos_gelu_fwd_f32", 300 * 130, C.ptr, D.ptr, None)
            th.call("talos_stream_sync", None)
        finally:
            th.call("talos_set_async", 0)
        outs.append(D.numpy())
    assert np.array_equal(outs[0], outs[1])
    check_close(outs[0], np.asarray(oracle_free_gelu(ref_gemm(0, 0, a, b))), rtol=1e-4, atol=1e-4, name="gelu(AB)")


def oracle_free_gelu(v):
    from scipy.special import erf
    v = np.asarray(v, np.float64)
    return 0.5 * v * (1.0 + erf(v / np.sqrt(2.0)))


def test_graph_capture_of_entries_replays_exactly():
    """The kernel entries captured into a HIP graph in the asynchronous mode (with a bound
    workspace, so nothing allocates) replay to the eager results bit for bit, three times, with
    eager work that scribbles over the outputs between the replays; the captured entries record
    fill kernels, not memset nodes."""
    rng = np.random.default_rng(21)
    R, C = 2048, 256
    x, dy = f32(rng.normal(size=(R, C))), f32(rng.normal(size=(R, C)))
    w = f32(rng.uniform(0.9, 1.1, C))
    rstd = f32(1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + 1e-6))
    sm = np.exp(rng.normal(size=(R, C)))
    sm = f32(sm / sm.sum(1, keepdims=True))
    a, b = f32(rng.normal(size=(4096, 96))), f32(rng.normal(size=(4096, 80)))
    X, DY, W, RS, SM, A, B = (DA.from_numpy(v) for v in (x, dy, w, rstd, sm, a, b))
    DX, DW, DS, G, WG = DA.zeros((R, C)), DA.zeros(C), DA.zeros((R, C)), DA.zeros((R, C)), DA.zeros((96, 80))
    outs = (DX, DW, DS, G, WG)
    ws = DA.zeros(1 << 20)
    stream = th.stream_create()

    def work():
        th.call("talos_rmsnorm_bwd_f32", R, C, X.ptr, W.ptr, RS.ptr, DY.ptr, 0.0, DX.ptr, 0.0, DW.ptr, stream)
        th.call("talos_softmax_bwd_f32", R, C, 1, SM.ptr, DY.ptr, 0.0, DS.ptr, stream)
        th.call("talos_gelu_fwd_f32", R * C, DX.ptr, G.ptr, stream)
        # a weight-gradient product over 4096 rows (split over K, partials in the workspace)
        th.call("talos_gemm_f32", 1, 0, 96, 80, 4096, 1.0, A.ptr, 96, B.ptr, 80, 0.0, WG.ptr, 80, stream)

    th.call("talos_workspace_bind", ws.ptr, 4 << 20)
    try:
        work()
        th.call("talos_stream_sync", stream)
        eager = [o.numpy() for o in outs]
        graph = th.Graph(stream, work)
        for rep in range(3):
            for o in outs:  # eager work between the replays
                o.upload(np.full(o.shape, np.nan, np.float32))
            graph.launch()
            th.call("talos_stream_sync", stream)
            for o, e in zip(outs, eager):
                assert np.array_equal(o.numpy(), e), f"replay {rep}"
        del graph
    finally:
        th.call("talos_workspace_bind", None, 0)
        th.stream_destroy(stream)
    check_close(eager[4], ref_gemm(1, 0, a, b), rtol=1e-4, atol=1e-3, name="captured wgrad")


@pytest.mark.parametrize("rows,ca,cb", [(1000, 64, 32), (7, 4, 8), (33, 12, 0)])
def test_concat_split_float4_path(rows, ca, cb):
    """concat_last / its backward on widths that are multiples of 4 (the float4 kernels MLA's q / k
    concatenation uses) equal numpy bit for bit; the backward accumulates into da / db."""
    rng = np.random.default_rng(rows + ca)
    a, b = f32(rng.normal(size=(rows, ca))), f32(rng.normal(size=(rows, cb)))
    Ad, Bd, C = DA.from_numpy(a if ca else np.zeros((rows, 1))), DA.from_numpy(b if cb else np.zeros((rows, 1))), \
        DA.zeros((rows, ca + cb))
    th.call("talos_concat_last_f32", rows, ca, cb, Ad.ptr, Bd.ptr, C.ptr, None)
    cat = np.concatenate([a, b], 1)
    assert np.array_equal(C.numpy(), cat)
    ga0, gb0 = f32(rng.normal(size=(rows, ca))), f32(rng.normal(size=(rows, cb)))
    ga = DA.from_numpy(ga0 if ca else np.zeros((rows, 1)))
    gb = DA.from_numpy(gb0 if cb else np.zeros((rows, 1)))
    th.call("talos_concat_last_bwd_f32", rows, ca, cb, C.ptr, ga.ptr, gb.ptr, None)
    # the kernels add in fp32
    if ca:
        assert np.array_equal(ga.numpy(), ga0.astype(np.float32) + a.astype(np.float32))
    if cb:
        assert np.array_equal(gb.numpy(), gb0.astype(np.float32) + b.astype(np.float32))
