"""ctypes wrapper of the f64 oracle (liboracle.so built from talos_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker of the HIP path or as the reported CPU baseline.
The product (talos-xii_amd/) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
SRC = os.path.join(HERE, "talos_oracle.cpp")

_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)


def build(force=False):
    """Compiles liboracle.so with g++ (x86-64-v3: AVX2 + FMA, the reference's SIMD level)."""
    if not force and os.path.exists(LIB_PATH) and os.path.getmtime(LIB_PATH) >= os.path.getmtime(SRC):
        return LIB_PATH
    tmp = LIB_PATH + ".tmp"
    cmd = ["g++", "-O3", "-mavx2", "-mfma", "-fPIC", "-shared", "-pthread", "-std=c++17", SRC, "-o", tmp]
    subprocess.check_call(cmd)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


class BlockCfg(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int), ("seq", ctypes.c_int), ("d_model", ctypes.c_int),
                ("n_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("ffn_dim", ctypes.c_int),
                ("causal", ctypes.c_int), ("activation", ctypes.c_int), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("attention", ctypes.c_int), ("kv_latent", ctypes.c_int),
                ("rope_dim", ctypes.c_int), ("v_dim", ctypes.c_int)]


class PpoCfg(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int), ("seq", ctypes.c_int), ("in_dim", ctypes.c_int),
                ("d_model", ctypes.c_int), ("n_layers", ctypes.c_int), ("n_heads", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("ffn_dim", ctypes.c_int), ("n_actions", ctypes.c_int),
                ("causal", ctypes.c_int), ("activation", ctypes.c_int), ("eps", ctypes.c_float),
                ("rope_base", ctypes.c_float), ("clip_eps", ctypes.c_float), ("value_coef", ctypes.c_float),
                ("entropy_coef", ctypes.c_float), ("attention", ctypes.c_int), ("kv_latent", ctypes.c_int),
                ("rope_dim", ctypes.c_int), ("v_dim", ctypes.c_int)]


_lib = None


def lib():
    """Loads the prebuilt liboracle.so (__graft_entry__.build() compiles it). It is never compiled
    here: a process that has initialised the GPU must not start the compiler."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() (or pyoracle.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        L.orc_last_error.restype = ctypes.c_char_p
        for name in ["orc_tensor_new", "orc_tensor_new_len", "orc_tensor_rand", "orc_relu", "orc_log", "orc_exp",
                     "orc_sin", "orc_cos", "orc_sqrt", "orc_neg", "orc_sum", "orc_mean", "orc_gelu", "orc_detach",
                     "orc_matmul", "orc_add", "orc_sub", "orc_mul", "orc_div", "orc_mse_loss", "orc_clip",
                     "orc_scale", "orc_broadcast", "orc_broadcast_to_batch", "orc_transpose", "orc_reshape",
                     "orc_softmax", "orc_rmsnorm", "orc_rope", "orc_bmm_qt_k", "orc_bmm_p_v", "orc_concat_last",
                     "orc_last_token", "orc_tensor_numel"]:
            getattr(L, name).restype = ctypes.c_int64
        L.orc_tensor_new.argtypes = [_f64p, _i64p, ctypes.c_int]
        L.orc_tensor_new_len.argtypes = [_f64p, ctypes.c_int64, _i64p, ctypes.c_int]
        L.orc_tensor_rand.argtypes = [_i64p, ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_uint64]
        for name in ["orc_relu", "orc_log", "orc_exp", "orc_sin", "orc_cos", "orc_sqrt", "orc_neg", "orc_sum",
                     "orc_mean", "orc_gelu", "orc_detach", "orc_tensor_numel", "orc_tensor_rank",
                     "orc_tensor_has_ctx", "orc_backward", "orc_zero_grad", "orc_tensor_free"]:
            getattr(L, name).argtypes = [ctypes.c_int64]
        for name in ["orc_matmul", "orc_add", "orc_sub", "orc_mul", "orc_div", "orc_mse_loss", "orc_bmm_qt_k",
                     "orc_bmm_p_v", "orc_concat_last"]:
            getattr(L, name).argtypes = [ctypes.c_int64, ctypes.c_int64]
        L.orc_clip.argtypes = [ctypes.c_int64, ctypes.c_double, ctypes.c_double]
        L.orc_scale.argtypes = [ctypes.c_int64, ctypes.c_double]
        L.orc_broadcast.argtypes = [ctypes.c_int64, _i64p, ctypes.c_int]
        L.orc_broadcast_to_batch.argtypes = [ctypes.c_int64, ctypes.c_int64]
        L.orc_transpose.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int]
        L.orc_reshape.argtypes = [ctypes.c_int64, _i64p, ctypes.c_int]
        L.orc_softmax.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.orc_rmsnorm.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_double]
        L.orc_rope.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_double, ctypes.c_int64]
        L.orc_last_token.argtypes = [ctypes.c_int64, ctypes.c_int]
        L.orc_tensor_shape.argtypes = [ctypes.c_int64, _i64p]
        L.orc_tensor_data.argtypes = [ctypes.c_int64, _f64p]
        L.orc_tensor_grad.argtypes = [ctypes.c_int64, _f64p]
        L.orc_rope_table.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_double, _f64p, _f64p]
        L.orc_lcg_rand.argtypes = [ctypes.c_int64, ctypes.c_double, ctypes.c_double, ctypes.c_uint64, _f64p]
        L.orc_ppo_param_count.restype = ctypes.c_size_t
        L.orc_ppo_param_count.argtypes = [ctypes.POINTER(PpoCfg)]
        L.orc_block_param_count.restype = ctypes.c_size_t
        L.orc_block_param_count.argtypes = [ctypes.POINTER(BlockCfg)]
        L.orc_mla_param_count.restype = ctypes.c_size_t
        L.orc_mla_param_count.argtypes = [_i32p]
        L.orc_adam_step.restype = None
        L.orc_adam_step.argtypes = [ctypes.c_int64, _f64p, _f64p, _f64p, _f64p, ctypes.c_int, ctypes.c_double,
                                    ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double]
        L.orc_ppo_gae.restype = None
        L.orc_ppo_gae.argtypes = [ctypes.c_int64, _f64p, _f64p, ctypes.POINTER(ctypes.c_uint8), ctypes.c_double,
                                  ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double, _f64p, _f64p,
                                  _f64p]
        L.orc_decoder_new.restype = ctypes.c_void_p
        L.orc_decoder_new.argtypes = [ctypes.POINTER(PpoCfg), _f64p, ctypes.c_int64, ctypes.c_int64]
        L.orc_decoder_free.restype = None
        L.orc_decoder_free.argtypes = [ctypes.c_void_p]
        L.orc_decoder_step.argtypes = [ctypes.c_void_p, ctypes.c_int64, _f64p, ctypes.c_int64, _f64p, _f64p, _f64p]
        L.orc_decoder_prune.restype = None
        L.orc_decoder_prune.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        L.orc_decoder_clear.restype = None
        L.orc_decoder_clear.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.orc_decoder_cache.restype = ctypes.c_int64
        L.orc_decoder_cache.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, _f64p, _f64p]
        L.orc_sample_action.restype = ctypes.c_int
        L.orc_sample_action.argtypes = [_f64p, ctypes.c_int64, ctypes.c_double, _f64p]
        L.orc_threads.restype = ctypes.c_int
        L.orc_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(_f64p)


def _i64(a):
    a = np.ascontiguousarray(a, dtype=np.int64)
    return a, a.ctypes.data_as(_i64p)


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib().orc_last_error().decode())


def _f64(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64))


def threads():
    return lib().orc_threads()


def track_mag(on):
    """Leaves created while on carry gradient magnitude sums (T.mag)."""
    lib().orc_set_track_mag(int(bool(on)))


def set_threads(n):
    lib().orc_set_threads(int(n))


# ---------------------------------------------------------------------------
# Tape-level handle API (mirrors the reference Tensor; used by the KAT tests)
# ---------------------------------------------------------------------------
class T:
    """A handle to an oracle Tensor (src/autograd.rs:14-20)."""

    def __init__(self, h):
        if h == 0:
            raise RuntimeError(lib().orc_last_error().decode())
        self.h = h

    @staticmethod
    def new(data, shape):
        d = _f64(data).ravel()
        s, sp = _i64(shape)
        return T(lib().orc_tensor_new_len(_p(d), d.size, sp, len(shape)))

    @staticmethod
    def rand(shape, mn, mx, seed):
        s, sp = _i64(shape)
        return T(lib().orc_tensor_rand(sp, len(shape), mn, mx, seed))

    @property
    def shape(self):
        r = lib().orc_tensor_rank(self.h)
        out = np.zeros(r, np.int64)
        lib().orc_tensor_shape(self.h, out.ctypes.data_as(_i64p))
        return tuple(int(v) for v in out)

    @property
    def data(self):
        out = np.zeros(lib().orc_tensor_numel(self.h))
        lib().orc_tensor_data(self.h, _p(out))
        return out.reshape(self.shape)

    @property
    def grad(self):
        out = np.zeros(lib().orc_tensor_numel(self.h))
        lib().orc_tensor_grad(self.h, _p(out))
        return out.reshape(self.shape)

    @property
    def mag(self):
        """Gradient magnitude sums of a leaf created under track_mag(True) (zeros otherwise)."""
        out = np.zeros(lib().orc_tensor_numel(self.h))
        lib().orc_tensor_mag(self.h, _p(out))
        return out.reshape(self.shape)

    @property
    def has_ctx(self):
        return bool(lib().orc_tensor_has_ctx(self.h))

    def backward(self):
        _check(lib().orc_backward(self.h))

    def zero_grad(self):
        _check(lib().orc_zero_grad(self.h))

    def matmul(self, o):
        return T(lib().orc_matmul(self.h, o.h))

    def relu(self):
        return T(lib().orc_relu(self.h))

    def log(self):
        return T(lib().orc_log(self.h))

    def exp(self):
        return T(lib().orc_exp(self.h))

    def sin(self):
        return T(lib().orc_sin(self.h))

    def cos(self):
        return T(lib().orc_cos(self.h))

    def sqrt(self):
        return T(lib().orc_sqrt(self.h))

    def sum(self):
        return T(lib().orc_sum(self.h))

    def mean(self):
        return T(lib().orc_mean(self.h))

    def gelu(self):
        return T(lib().orc_gelu(self.h))

    def detach(self):
        return T(lib().orc_detach(self.h))

    def clip(self, mn, mx):
        return T(lib().orc_clip(self.h, mn, mx))

    def scale(self, s):
        return T(lib().orc_scale(self.h, s))

    def broadcast(self, shape):
        s, sp = _i64(shape)
        return T(lib().orc_broadcast(self.h, sp, len(shape)))

    def broadcast_to_batch(self, b):
        return T(lib().orc_broadcast_to_batch(self.h, b))

    def transpose(self, a, b):
        return T(lib().orc_transpose(self.h, a, b))

    def reshape(self, shape):
        s, sp = _i64(shape)
        return T(lib().orc_reshape(self.h, sp, len(shape)))

    def softmax(self, seq_len, causal=False):
        return T(lib().orc_softmax(self.h, seq_len, int(causal)))

    def rmsnorm(self, w, eps):
        return T(lib().orc_rmsnorm(self.h, w.h, eps))

    def rope(self, max_len, base=10000.0, start_pos=0):
        return T(lib().orc_rope(self.h, max_len, base, start_pos))

    def mse_loss(self, o):
        return T(lib().orc_mse_loss(self.h, o.h))

    def last_token(self, differentiable=True):
        return T(lib().orc_last_token(self.h, int(differentiable)))

    def __add__(self, o):
        return T(lib().orc_add(self.h, o.h))

    def __sub__(self, o):
        return T(lib().orc_sub(self.h, o.h))

    def __mul__(self, o):
        return T(lib().orc_mul(self.h, o.h))

    def __truediv__(self, o):
        return T(lib().orc_div(self.h, o.h))

    def __neg__(self):
        return T(lib().orc_neg(self.h))


def bmm_qt_k(q, k):
    return T(lib().orc_bmm_qt_k(q.h, k.h))


def bmm_p_v(p, v):
    return T(lib().orc_bmm_p_v(p.h, v.h))


def concat_last(a, b):
    return T(lib().orc_concat_last(a.h, b.h))


def free_all():
    lib().orc_free_all()


def rope_table(max_len, dim, base=10000.0):
    c = np.zeros(max_len * (dim // 2))
    s = np.zeros_like(c)
    lib().orc_rope_table(max_len, dim, base, _p(c), _p(s))
    return c.reshape(max_len, dim // 2), s.reshape(max_len, dim // 2)


def lcg_rand(n, mn, mx, seed):
    out = np.zeros(n)
    lib().orc_lcg_rand(n, mn, mx, seed, _p(out))
    return out


# ---------------------------------------------------------------------------
# Op- and model-level oracles
# ---------------------------------------------------------------------------
def linear_mse(x, w, b, y):
    x, w, b, y = map(_f64, (x, w, b, y))
    rows, in_f = x.shape
    out_f = w.shape[1]
    loss = ctypes.c_double()
    dx, dw, db = np.zeros_like(x), np.zeros_like(w), np.zeros_like(b)
    _check(lib().orc_linear_mse(ctypes.c_int64(rows), ctypes.c_int64(in_f), ctypes.c_int64(out_f), _p(x), _p(w),
                                _p(b), _p(y), ctypes.byref(loss), _p(dx), _p(dw), _p(db)))
    return loss.value, dx, dw, db


def rmsnorm_fwd_bwd(x, w, dy, eps):
    x, w, dy = map(_f64, (x, w, dy))
    rows, dim = x.shape
    y, dx, dw = np.zeros_like(x), np.zeros_like(x), np.zeros_like(w)
    _check(lib().orc_rmsnorm_fwd_bwd(ctypes.c_int64(rows), ctypes.c_int64(dim), ctypes.c_double(eps), _p(x), _p(w),
                                     _p(dy), _p(y), _p(dx), _p(dw)))
    return y, dx, dw


def softmax_fwd_bwd(x, dy, causal):
    x, dy = map(_f64, (x, dy))
    rows, cols = x.shape
    y, dx = np.zeros_like(x), np.zeros_like(x)
    _check(lib().orc_softmax_fwd_bwd(ctypes.c_int64(rows), ctypes.c_int64(cols), ctypes.c_int(int(causal)), _p(x),
                                     _p(dy), _p(y), _p(dx)))
    return y, dx


def rope_fwd_bwd(x, dy, base=10000.0, start_pos=0):
    """x, dy: [n_seq, seq, heads, dim]; position = start_pos + sequence index."""
    x, dy = map(_f64, (x, dy))
    n, s, h, d = x.shape
    y, dx = np.zeros_like(x), np.zeros_like(x)
    _check(lib().orc_rope_fwd_bwd(ctypes.c_int64(n), ctypes.c_int64(s), ctypes.c_int64(h), ctypes.c_int64(d),
                                  ctypes.c_double(base), ctypes.c_int64(start_pos), _p(x), _p(dy), _p(y), _p(dx)))
    return y, dx


def attention_fwd_bwd(q, k, v, dout, scale, causal):
    """q, k: [B,S,H,dk]; v, dout: [B,S,H,dv]."""
    q, k, v, dout = map(_f64, (q, k, v, dout))
    B, S, H, dk = q.shape
    dv = v.shape[3]
    o = np.zeros_like(v)
    dq, dkk, dvv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    _check(lib().orc_attention_fwd_bwd(*[ctypes.c_int64(t) for t in (B, S, H, dk, dv)], ctypes.c_double(scale),
                                       ctypes.c_int(int(causal)), _p(q), _p(k), _p(v), _p(dout), _p(o), _p(dq),
                                       _p(dkk), _p(dvv)))
    return o, dq, dkk, dvv


def block_param_count(cfg):
    return int(lib().orc_block_param_count(ctypes.byref(cfg)))


def _mag_out(params, mag):
    """The magnitude output of a model call: an array like params when asked for, else NULL."""
    return np.zeros_like(params) if mag else None


def _pm(a):
    return _p(a) if a is not None else None


def block_fwd_bwd(cfg, params, x, gout, mag=False):
    """out, dparams, dx (and with mag=True the parameter-gradient magnitude sums, Tensor::mag)."""
    params, x, gout = map(_f64, (params, x, gout))
    out, dparams, dx = np.zeros_like(x), np.zeros_like(params), np.zeros_like(x)
    dmag = _mag_out(params, mag)
    _check(lib().orc_block_fwd_bwd(ctypes.byref(cfg), _p(params), _p(x), _p(gout), _p(out), _p(dparams), _p(dx),
                                   _pm(dmag)))
    return (out, dparams, dx, dmag) if mag else (out, dparams, dx)


def ppo_param_count(cfg):
    return int(lib().orc_ppo_param_count(ctypes.byref(cfg)))


def ppo_fwd_bwd(cfg, params, states, actions, adv, ret, old_logp, mag=False):
    """loss, logits, values, dparams (and with mag=True the parameter-gradient magnitude sums)."""
    params, states, adv, ret, old_logp = map(_f64, (params, states, adv, ret, old_logp))
    actions = np.ascontiguousarray(actions, dtype=np.int32)
    B = cfg.batch
    loss = ctypes.c_double()
    logits = np.zeros((B, cfg.n_actions))
    values = np.zeros(B)
    dparams = np.zeros_like(params)
    dmag = _mag_out(params, mag)
    _check(lib().orc_ppo_fwd_bwd(ctypes.byref(cfg), _p(params), _p(states), actions.ctypes.data_as(_i32p), _p(adv),
                                 _p(ret), _p(old_logp), ctypes.byref(loss), _p(logits), _p(values), _p(dparams),
                                 _pm(dmag)))
    return (loss.value, logits, values, dparams, dmag) if mag else (loss.value, logits, values, dparams)


def ppo_fwd_bwd_per_sample(cfg, params, states, actions, adv, ret, old_logp, diff_last=True, mag=False):
    params, states, adv, ret, old_logp = map(_f64, (params, states, adv, ret, old_logp))
    actions = np.ascontiguousarray(actions, dtype=np.int32)
    loss = ctypes.c_double()
    dparams = np.zeros_like(params)
    dmag = _mag_out(params, mag)
    _check(lib().orc_ppo_fwd_bwd_per_sample(ctypes.byref(cfg), _p(params), _p(states), actions.ctypes.data_as(_i32p),
                                            _p(adv), _p(ret), _p(old_logp), ctypes.c_int(int(diff_last)),
                                            ctypes.byref(loss), _p(dparams), _pm(dmag)))
    return (loss.value, dparams, dmag) if mag else (loss.value, dparams)


def ppo_sample_loss(cfg, logits, value, action, old_logp, adv, ret):
    logits = _f64(logits)
    loss, dvalue = ctypes.c_double(), ctypes.c_double()
    dl = np.zeros_like(logits)
    _check(lib().orc_ppo_sample_loss(ctypes.byref(cfg), _p(logits), ctypes.c_double(value), ctypes.c_int(action),
                                     ctypes.c_double(old_logp), ctypes.c_double(adv), ctypes.c_double(ret),
                                     ctypes.byref(loss), _p(dl), ctypes.byref(dvalue)))
    return loss.value, dl, dvalue.value


def ppo_batched_loss(cfg, logits, values, actions, old_logp, adv, ret):
    logits, values, old_logp, adv, ret = map(_f64, (logits, values, old_logp, adv, ret))
    actions = np.ascontiguousarray(actions, dtype=np.int32)
    B = logits.shape[0]
    loss = ctypes.c_double()
    dl, dv = np.zeros_like(logits), np.zeros_like(values)
    _check(lib().orc_ppo_batched_loss(ctypes.byref(cfg), ctypes.c_int64(B), _p(logits), _p(values),
                                      actions.ctypes.data_as(_i32p), _p(old_logp), _p(adv), _p(ret),
                                      ctypes.byref(loss), _p(dl), _p(dv)))
    return loss.value, dl, dv


def mla_param_count(ci):
    ci = np.ascontiguousarray(ci, dtype=np.int32)
    return int(lib().orc_mla_param_count(ci.ctypes.data_as(_i32p)))


def mla_fwd_bwd(ci, eps, base, params, x, gout, mag=False):
    """ci = [batch, seq, d_model, n_heads, kv_latent, rope_dim, head_dim, v_dim, causal, literal_rope].
    out, dparams, dx (and with mag=True the parameter-gradient magnitude sums)."""
    ci = np.ascontiguousarray(ci, dtype=np.int32)
    params, x, gout = map(_f64, (params, x, gout))
    out, dparams, dx = np.zeros_like(x), np.zeros_like(params), np.zeros_like(x)
    dmag = _mag_out(params, mag)
    _check(lib().orc_mla_fwd_bwd(ci.ctypes.data_as(_i32p), ctypes.c_double(eps), ctypes.c_double(base), _p(params),
                                 _p(x), _p(gout), _p(out), _p(dparams), _p(dx), _pm(dmag)))
    return (out, dparams, dx, dmag) if mag else (out, dparams, dx)


def adam_step(p, g, m, v, t, lr, beta1=0.9, beta2=0.999, eps=1e-8, max_norm=0.0):
    """One Adam step in f64 (src/ppo.rs:519-533); max_norm > 0 adds the DQN global-norm clip
    (src/dqn.rs:207-226). Updates p, m, v (float64 arrays) in place."""
    for a in (p, m, v):
        assert a.dtype == np.float64 and a.flags.c_contiguous
    g = _f64(g)
    assert p.size == g.size == m.size == v.size
    lib().orc_adam_step(p.size, _p(p), _p(g), _p(m), _p(v), int(t), float(lr), float(beta1), float(beta2),
                        float(eps), float(max_norm))


def ppo_gae(rewards, values, terminals, r_mean=0.0, r_var=1.0, r_clip=10.0, gamma=0.99, lam=0.95):
    """PPO::update's advantage prologue in f64 (src/ppo.rs:650-676). Returns (adv_raw, returns,
    adv_norm)."""
    r, v = _f64(rewards), _f64(values)
    d = np.ascontiguousarray(np.asarray(terminals, dtype=np.uint8))
    n = r.size
    assert v.size == n and d.size == n and n > 0
    a, ret, an = np.empty(n), np.empty(n), np.empty(n)
    lib().orc_ppo_gae(n, _p(r), _p(v), d.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), float(r_mean), float(r_var),
                      float(r_clip), float(gamma), float(lam), _p(a), _p(ret), _p(an))
    return a, ret, an


class Decoder:
    """Rollout inference with the KV cache in f64 (forward_inference_step and
    forward_inference_cached, src/transformer.rs:157-196, 688-805; prune_kv_cache, :807-840),
    one cache per environment and layer."""

    def __init__(self, cfg, params, max_seq_len=256, n_envs=1):
        self.cfg = cfg
        self._p = _f64(params)
        self.h = lib().orc_decoder_new(ctypes.byref(cfg), _p(self._p), int(max_seq_len), int(n_envs))

    def step(self, env, token, start_pos):
        """Returns (logits [A], value, hidden [d]) for one token of env at start_pos."""
        token = _f64(token)
        lg, v, hid = np.zeros(self.cfg.n_actions), ctypes.c_double(), np.zeros(self.cfg.d_model)
        _check(lib().orc_decoder_step(self.h, int(env), _p(token), int(start_pos), _p(lg), ctypes.byref(v), _p(hid)))
        return lg, v.value, hid

    def prune(self, env, max_len):
        lib().orc_decoder_prune(self.h, int(env), int(max_len))

    def clear(self, env):
        lib().orc_decoder_clear(self.h, int(env))

    def cache(self, env, layer=0):
        """(k [len, H, dk], v [len, H, dv]) of env's cache at layer, oldest row first."""
        c = self.cfg
        mla = c.attention == 1
        dk, dv = c.head_dim + (c.rope_dim if mla else 0), (c.v_dim if mla else c.head_dim)
        n = lib().orc_decoder_cache(self.h, int(env), int(layer), None, None)
        k, v = np.zeros((n, c.n_heads, dk)), np.zeros((n, c.n_heads, dv))
        lib().orc_decoder_cache(self.h, int(env), int(layer), _p(k), _p(v))
        return k, v

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_decoder_free(self.h)
            self.h = None


def sample_action(logits, r):
    """The action choice of ActorCritic::step_inference_cached (src/ppo.rs:401-432) for the
    uniform draw r; returns (action, log-probability of the action)."""
    logits = _f64(logits)
    lp = ctypes.c_double()
    a = lib().orc_sample_action(_p(logits), logits.size, float(r), ctypes.byref(lp))
    return a, lp.value
