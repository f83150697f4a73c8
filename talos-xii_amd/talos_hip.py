"""ctypes binding of libtalos_hip.so (include/talos_hip.h) with a small device-buffer helper.

This is the Python side of the C ABI used by the tests and bench.py. It loads the in-tree
library built by build_lib.py and fails loudly when it is missing: there is no CPU fallback.
Device memory comes from the library's own allocator (talos_malloc), so a process using this
module needs no other GPU runtime.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtalos_hip.so")

# status codes (enum talos_status)
(OK, ERR_SHAPE, ERR_NULL, ERR_DTYPE, ERR_NO_DEVICE, ERR_HIP, ERR_ALLOC, ERR_HANDLE, ERR_UNSUPPORTED, ERR_IO,
 ERR_FORMAT) = range(11)
CKPT_BINCODE, CKPT_JSON = 0, 1  # enum talos_checkpoint_format
# enum talos_unary_op / talos_binary_op / talos_activation
RELU, LOG, EXP, SIN, COS, SQRT, NEG, SCALE, CLIP, GELU, COPY = range(11)
ADD, SUB, MUL, DIV = range(4)
ACT_GELU, ACT_RELU = 0, 1

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_d = ctypes.c_double
_ll = ctypes.c_longlong


class TalosError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"talos status {code}: {msg}")
        self.code = code


class BlockCfg(ctypes.Structure):
    _fields_ = [("batch", _i), ("seq", _i), ("d_model", _i), ("n_heads", _i), ("head_dim", _i), ("ffn_dim", _i),
                ("causal", _i), ("activation", _i), ("eps", _f), ("rope_base", _f), ("attention", _i),
                ("kv_latent", _i), ("rope_dim", _i), ("v_dim", _i)]


class PpoCfg(ctypes.Structure):
    _fields_ = [("batch", _i), ("seq", _i), ("in_dim", _i), ("d_model", _i), ("n_layers", _i), ("n_heads", _i),
                ("head_dim", _i), ("ffn_dim", _i), ("n_actions", _i), ("causal", _i), ("activation", _i),
                ("eps", _f), ("rope_base", _f), ("clip_eps", _f), ("value_coef", _f), ("entropy_coef", _f),
                ("attention", _i), ("kv_latent", _i), ("rope_dim", _i), ("v_dim", _i)]


ATTN_MHA, ATTN_MLA = 0, 1


class PpoUpdateArgs(ctypes.Structure):
    """talos_ppo_update_args (device pointers as integers)."""
    _fields_ = [("n", _i), ("states", _vp), ("lengths", _vp), ("actions", _vp), ("old_logp", _vp),
                ("rewards", _vp), ("values", _vp), ("terminals", _vp), ("reward_mean", _d), ("reward_var", _d),
                ("reward_clip", _d), ("gamma", _d), ("lambda_", _d), ("target_kl", _d), ("k_epochs", _i),
                ("lr", _d), ("params", _vp), ("adam_m", _vp), ("adam_v", _vp), ("adam_t", _i), ("work", _vp)]


class PpoUpdateResult(ctypes.Structure):
    _fields_ = [("epochs_run", _i), ("stopped_early", _i), ("approx_kl", _d), ("mean_loss", _d)]


PPO_NSTATS = 5
STAT_KL, STAT_POLICY, STAT_VALUE, STAT_ENTROPY, STAT_COUNT = range(5)


class MlaCfg(ctypes.Structure):
    _fields_ = [("batch", _i), ("seq", _i), ("d_model", _i), ("n_heads", _i), ("kv_latent", _i), ("rope_dim", _i),
                ("head_dim", _i), ("v_dim", _i), ("causal", _i), ("precision", _i), ("eps", _f), ("rope_base", _f)]


PREC_FP32, PREC_BF16 = 0, 1

# name -> argtypes (restype int unless listed in _RESTYPE)
_SIGS = {
    "talos_last_error": [],
    "talos_workspace_bind": [_vp, _sz],
    "talos_workspace_high_water": [],
    "talos_workspace_bytes": [],
    "talos_version": [],
    "talos_init": [],
    "talos_device_count": [ctypes.POINTER(_i)],
    "talos_malloc": [ctypes.POINTER(_vp), _sz],
    "talos_free": [_vp],
    "talos_memcpy_h2d": [_vp, _vp, _sz, _vp],
    "talos_memcpy_d2h": [_vp, _vp, _sz, _vp],
    "talos_memcpy_d2d": [_vp, _vp, _sz, _vp],
    "talos_memcpy_h2d_f64": [_vp, _vp, _sz, _vp],
    "talos_memcpy_d2h_f64": [_vp, _vp, _sz, _vp],
    "talos_fill_zero": [_vp, _sz, _vp],
    "talos_stream_sync": [_vp],
    "talos_set_async": [_i],
    "talos_get_async": [],
    "talos_stream_create": [ctypes.POINTER(_vp)],
    "talos_stream_destroy": [_vp],
    "talos_event_create": [ctypes.POINTER(_vp)],
    "talos_event_destroy": [_vp],
    "talos_event_record": [_vp, _vp],
    "talos_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(_f)],
    "talos_device_info": [ctypes.c_char_p, _sz, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_sz)],
    "talos_gemm_f32": [_i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _f, _vp, _i, _vp],
    "talos_gemm_bf16acc_f32": [_i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _f, _vp, _i, _vp],
    "talos_gemm_batched_f32":[_i, _i, _i, _i, _i, _f, _vp, _i, _ll, _vp, _i, _ll, _f, _vp, _i, _ll, _i, _vp],
    "talos_bias_grad_f32": [_i, _i, _vp, _f, _vp, _vp],
    "talos_rmsnorm_fwd_f32": [_i, _i, _f, _vp, _vp, _vp, _vp, _vp],
    "talos_rmsnorm_bwd_f32": [_i, _i, _vp, _vp, _vp, _vp, _f, _vp, _f, _vp, _vp],
    "talos_softmax_fwd_f32": [_i, _i, _i, _vp, _vp, _vp],
    "talos_softmax_bwd_f32": [_i, _i, _i, _vp, _vp, _f, _vp, _vp],
    "talos_rope_fwd_f32": [_i, _i, _i, _i, _i, _f, _vp, _vp, _vp],
    "talos_rope_bwd_f32": [_i, _i, _i, _i, _i, _f, _vp, _f, _vp, _vp],
    "talos_rope_table_f32": [_i, _i, _f, _vp, _vp, _vp],
    "talos_attn_fwd_f32": [_i, _i, _i, _i, _i, _f, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp],
    "talos_attn_bwd_f32": [_i, _i, _i, _i, _i, _f, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i,
                           _vp, _i, _vp, _i, _vp],
    "talos_attn_bwd_noalloc_f32": [_i, _i, _i, _i, _i, _f, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp,
                                   _i, _vp, _i, _vp, _i, _vp],
    "talos_unary_fwd_f32": [_i, _sz, _f, _f, _vp, _vp, _vp],
    "talos_unary_bwd_f32": [_i, _sz, _f, _f, _vp, _vp, _vp, _vp],
    "talos_gelu_fwd_f32": [_sz, _vp, _vp, _vp],
    "talos_gelu_bwd_f32": [_sz, _vp, _vp, _f, _vp, _vp],
    "talos_binary_fwd_f32": [_i, _sz, _vp, _vp, _vp, _vp],
    "talos_binary_bwd_f32": [_i, _sz, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_reduce_sum_f32": [_sz, _f, _vp, _vp, _vp],
    "talos_fill_add_f32": [_sz, _f, _vp, _vp, _vp],
    "talos_transpose_f32": [_i, ctypes.POINTER(_ll), _i, _i, _vp, _vp, _i, _vp],
    "talos_concat_last_f32": [_sz, _i, _i, _vp, _vp, _vp, _vp],
    "talos_concat_last_bwd_f32": [_sz, _i, _i, _vp, _vp, _vp, _vp],
    "talos_broadcast_rows_f32": [_sz, _i, _vp, _vp, _vp],
    "talos_grad_sumsq_workspace_bytes": [],
    "talos_grad_sumsq_f32": [_sz, _vp, _i, _vp, _vp, _vp],
    "talos_adam_step_f32": [_sz, _vp, _vp, _vp, _vp, _i, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                            ctypes.c_double, _vp, ctypes.c_double, _vp],
    "talos_block_param_count": [ctypes.POINTER(BlockCfg)],
    "talos_ppo_param_count": [ctypes.POINTER(PpoCfg)],
    "talos_block_plan_create": [ctypes.POINTER(BlockCfg), ctypes.POINTER(_vp)],
    "talos_block_fwd_bwd_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_plan_create": [ctypes.POINTER(PpoCfg), ctypes.POINTER(_vp)],
    "talos_ppo_fwd_bwd_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_forward_f32": [_vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_forward_n_f32": [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_minibatch_f32": [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp],
    "talos_ppo_head_loss_fwd_f32": [_i, _i, _f, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp],
    "talos_ppo_head_loss_bwd_f32": [_i, _i, _f, _f, _f, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_gae_f64": [_i, _vp, _vp, _vp, _d, _d, _d, _d, _d, _vp, _vp, _vp, _vp],
    "talos_ppo_update_work_bytes": [_vp, _i],
    "talos_ppo_update_f32": [_vp, ctypes.c_void_p, ctypes.c_void_p, _vp],
    "talos_mla_param_count": [ctypes.POINTER(MlaCfg)],
    "talos_mla_plan_create": [ctypes.POINTER(MlaCfg), ctypes.POINTER(_vp)],
    "talos_mla_fwd_bwd_f32": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_plan_destroy": [_vp],
    "talos_ppo_decoder_create": [ctypes.POINTER(PpoCfg), _i, _i, _i, ctypes.POINTER(_vp)],
    "talos_ppo_decoder_step_f32": [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    "talos_ppo_decoder_read_cache": [_vp, _i, _i, _vp, _vp, ctypes.POINTER(_i)],
    "talos_ppo_decoder_destroy": [_vp],
    "talos_ppo_checkpoint_encode": [ctypes.POINTER(PpoCfg), _vp, _i, _i, _vp, _sz, ctypes.POINTER(_sz)],
    "talos_ppo_checkpoint_decode": [ctypes.POINTER(PpoCfg), _vp, _sz, _i, _vp],
    "talos_ppo_checkpoint_save": [ctypes.POINTER(PpoCfg), _vp, _i, ctypes.c_char_p],
    "talos_ppo_checkpoint_load": [ctypes.POINTER(PpoCfg), ctypes.c_char_p, _vp],
    "talos_plan_profiler": [_vp, ctypes.POINTER(_vp)],
    "talos_profiler_enable": [_vp, _i, ctypes.c_char_p],
    "talos_profiler_read": [_vp, _vp, _i, ctypes.POINTER(_i)],
}


class ProfRecord(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 64), ("flops", ctypes.c_double), ("bytes", ctypes.c_double),
                ("ms", ctypes.c_float)]
_RESTYPE = {"talos_last_error": ctypes.c_char_p, "talos_version": ctypes.c_char_p, "talos_workspace_high_water": _sz,
            "talos_workspace_bytes": _sz, "talos_grad_sumsq_workspace_bytes": _sz, "talos_ppo_update_work_bytes": _sz, "talos_block_param_count": _sz, "talos_ppo_param_count": _sz, "talos_mla_param_count": _sz}

_lib = None


def lib():
    """Loads libtalos_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with talos-xii_amd/build_lib.py "
                               "(or __graft_entry__.build()); there is no fallback path")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, _i)
        _lib = L
    return _lib


def check(rc):
    if rc != OK:
        raise TalosError(rc, lib().talos_last_error().decode())
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args))


def device_count():
    n = _i(0)
    call("talos_device_count", ctypes.byref(n))
    return n.value


def device_info():
    name = ctypes.create_string_buffer(256)
    cu, clk, mem = _i(), _i(), _sz()
    call("talos_device_info", name, 256, ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(mem))
    return {"name": name.value.decode(), "cu_count": cu.value, "clock_khz": clk.value, "total_mem": mem.value}


def _host_params(cfg, params):
    p = np.ascontiguousarray(params, dtype=np.float32)
    n = lib().talos_ppo_param_count(ctypes.byref(cfg))
    if p.size != n:
        raise TalosError(ERR_SHAPE, f"{p.size} parameters, the configuration has {n}")
    return p


def checkpoint_encode(cfg, params, fmt=CKPT_BINCODE, max_seq_len=0):
    """The reference's ActorCritic checkpoint bytes (bincode or JSON) of host fp32 params."""
    p = _host_params(cfg, params)
    size = _sz()
    call("talos_ppo_checkpoint_encode", ctypes.byref(cfg), p.ctypes.data, max_seq_len, fmt, None, 0,
         ctypes.byref(size))
    buf = ctypes.create_string_buffer(size.value)
    call("talos_ppo_checkpoint_encode", ctypes.byref(cfg), p.ctypes.data, max_seq_len, fmt, buf, size.value,
         ctypes.byref(size))
    return buf.raw[:size.value]


def checkpoint_decode(cfg, data, fmt=CKPT_BINCODE):
    """Host fp32 params from checkpoint bytes."""
    out = np.zeros(lib().talos_ppo_param_count(ctypes.byref(cfg)), np.float32)
    call("talos_ppo_checkpoint_decode", ctypes.byref(cfg), data, len(data), fmt, out.ctypes.data)
    return out


def save_ppo_model(cfg, params, path, max_seq_len=0):
    """Writes "<path>.bin" and "<path>" as the reference's save_ppo_model does."""
    p = _host_params(cfg, params)
    call("talos_ppo_checkpoint_save", ctypes.byref(cfg), p.ctypes.data, max_seq_len, os.fsencode(path))


def load_ppo_model(cfg, path):
    """Host fp32 params from "<path>.bin", or from "<path>" as the reference's load_ppo_model does."""
    out = np.zeros(lib().talos_ppo_param_count(ctypes.byref(cfg)), np.float32)
    call("talos_ppo_checkpoint_load", ctypes.byref(cfg), os.fsencode(path), out.ctypes.data)
    return out


class Decoder:
    """A rollout decoder (talos_ppo_decoder_*): KV caches for n_envs environments."""

    def __init__(self, cfg, n_envs, context_len, max_seq_len=0):
        self.cfg = cfg
        self.h = _vp()
        call("talos_ppo_decoder_create", ctypes.byref(cfg), n_envs, context_len, max_seq_len, ctypes.byref(self.h))

    def step(self, n, params, tokens, positions, reset=None, uniforms=None, logits=None, values=None,
             actions=None, logp=None, stream=None):
        """All arguments are DeviceArray (or None). The parameters are kept alive: cache() of a
        latent cache expands its rows with the last step's weights."""
        ptr = lambda a: None if a is None else a.ptr  # noqa: E731
        call("talos_ppo_decoder_step_f32", self.h, n, ptr(params), ptr(tokens), ptr(positions), ptr(reset),
             ptr(uniforms), ptr(logits), ptr(values), ptr(actions), ptr(logp), stream)
        self._params = params

    def cache(self, layer, env):
        """(k [len, H, dk], v [len, H, dv]) of env's cache at layer, oldest row first."""
        c = self.cfg
        mla = c.attention == ATTN_MLA
        dk, dv = c.head_dim + (c.rope_dim if mla else 0), (c.v_dim if mla else c.head_dim)
        n = _i()
        call("talos_ppo_decoder_read_cache", self.h, layer, env, None, None, ctypes.byref(n))
        k = np.zeros((n.value, c.n_heads, dk), np.float32)
        v = np.zeros((n.value, c.n_heads, dv), np.float32)
        call("talos_ppo_decoder_read_cache", self.h, layer, env, k.ctypes.data, v.ctypes.data, ctypes.byref(n))
        return k, v

    def destroy(self):
        if self.h:
            call("talos_ppo_decoder_destroy", self.h)
            self.h = _vp()


class DeviceArray:
    """A device buffer of a numpy dtype (float32 or int32) owned by talos_malloc."""

    def __init__(self, shape, dtype=np.float32):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        p = _vp()
        call("talos_malloc", ctypes.byref(p), max(self.nbytes, 4))
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a, dtype=np.float32):
        a = np.ascontiguousarray(np.asarray(a, dtype=dtype))
        d = cls(a.shape, dtype)
        if a.nbytes:
            call("talos_memcpy_h2d", d.ptr, a.ctypes.data, a.nbytes, None)
        return d

    @classmethod
    def zeros(cls, shape, dtype=np.float32):
        d = cls(shape, dtype)
        call("talos_fill_zero", d.ptr, max(d.nbytes, 4), None)
        return d

    def numpy(self):
        call("talos_stream_sync", None)
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("talos_memcpy_d2h", out.ctypes.data, self.ptr, self.nbytes, None)
        return out

    def upload(self, a):
        a = np.ascontiguousarray(np.asarray(a, dtype=self.dtype))
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        call("talos_memcpy_h2d", self.ptr, a.ctypes.data, a.nbytes, None)

    def offset(self, n_elems):
        """Raw device pointer n_elems elements into the buffer."""
        return self.ptr + int(n_elems) * self.dtype.itemsize

    def free(self):
        if self.ptr:
            lib().talos_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            if getattr(self, "ptr", None) and _lib is not None:
                _lib.talos_free(self.ptr)
        except Exception:
            pass


def sync():
    call("talos_stream_sync", None)


class async_mode:
    """Context manager: the calling thread's kernel entries return once their work is enqueued
    (talos_set_async(1)) inside the block; the previous mode is restored on exit. The default
    mode is synchronous."""

    def __enter__(self):
        self.prev = lib().talos_get_async()
        call("talos_set_async", 1)
        return self

    def __exit__(self, *exc):
        call("talos_set_async", self.prev)
        return False


class Plan:
    """Owns a talos_plan (block or ppo)."""

    def __init__(self, kind, cfg):
        self.cfg = cfg
        self.kind = kind
        h = _vp()
        if kind == "block":
            call("talos_block_plan_create", ctypes.byref(cfg), ctypes.byref(h))
            self.n_params = lib().talos_block_param_count(ctypes.byref(cfg))
        elif kind == "mla":
            call("talos_mla_plan_create", ctypes.byref(cfg), ctypes.byref(h))
            self.n_params = lib().talos_mla_param_count(ctypes.byref(cfg))
        else:
            call("talos_ppo_plan_create", ctypes.byref(cfg), ctypes.byref(h))
            self.n_params = lib().talos_ppo_param_count(ctypes.byref(cfg))
        self.h = h.value

    def profile(self, enable=True, kernel_filter=None):
        """Switches per-launch event profiling of this plan on (clearing old records) or off."""
        prof = _vp()
        call("talos_plan_profiler", self.h, ctypes.byref(prof))
        call("talos_profiler_enable", prof, int(enable), kernel_filter.encode() if kernel_filter else None)

    def profile_records(self):
        """[(kernel, flops, bytes, ms)] of the profiled launches so far."""
        prof = _vp()
        call("talos_plan_profiler", self.h, ctypes.byref(prof))
        n = _i()
        call("talos_profiler_read", prof, None, 0, ctypes.byref(n))
        recs = (ProfRecord * max(1, n.value))()
        call("talos_profiler_read", prof, ctypes.cast(recs, _vp), n.value, ctypes.byref(n))
        return [(r.kernel.decode(), r.flops, r.bytes, r.ms) for r in recs[:n.value]]

    def destroy(self):
        if self.h:
            lib().talos_plan_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            if getattr(self, "h", None) and _lib is not None:
                _lib.talos_plan_destroy(self.h)
        except Exception:
            pass


_hip = None


def hip_runtime():
    """The HIP runtime library the extension is linked against (for graph capture)."""
    global _hip
    if _hip is None:
        lib()  # loads libamdhip64 as a dependency of the extension
        H = ctypes.CDLL("libamdhip64.so", mode=ctypes.RTLD_GLOBAL)
        for name, args in {"hipStreamBeginCapture": [_vp, _i], "hipStreamEndCapture": [_vp, ctypes.POINTER(_vp)],
                           "hipGraphInstantiate": [ctypes.POINTER(_vp), _vp, _vp, _vp, _sz],
                           "hipGraphLaunch": [_vp, _vp], "hipGraphExecDestroy": [_vp], "hipGraphDestroy": [_vp],
                           "hipMemcpyAsync": [_vp, _vp, _sz, _i, _vp]}.items():
            fn = getattr(H, name)
            fn.argtypes = args
            fn.restype = _i
        _hip = H
    return _hip


def _hip_check(rc, what):
    if rc != 0:
        raise TalosError(ERR_HIP, f"{what} failed with hipError_t {rc}")


def stream_create():
    """A non-blocking stream at the default priority (talos_stream_create); free it with
    stream_destroy."""
    h = _vp()
    call("talos_stream_create", ctypes.byref(h))
    return h.value


def stream_destroy(h):
    call("talos_stream_destroy", h)


class Graph:
    """A HIP graph captured from the work fn() enqueues on `stream` (a talos_stream_create
    stream). The library's entries are captured in their asynchronous mode (synchronous entries
    would wait on a capturing stream); fn must not allocate, so a caller-owned workspace should
    be bound (talos_workspace_bind) for entries that need scratch memory."""

    def __init__(self, stream, fn):
        H = hip_runtime()
        self.stream = stream
        self.exec = None
        with async_mode():
            _hip_check(H.hipStreamBeginCapture(stream, 1), "hipStreamBeginCapture")  # thread-local mode
            try:
                fn()
            finally:
                g = _vp()
                rc = H.hipStreamEndCapture(stream, ctypes.byref(g))
            _hip_check(rc, "hipStreamEndCapture")
        self.graph = g.value
        e = _vp()
        _hip_check(H.hipGraphInstantiate(ctypes.byref(e), self.graph, None, None, 0), "hipGraphInstantiate")
        self.exec = e.value

    def launch(self):
        _hip_check(hip_runtime().hipGraphLaunch(self.exec, self.stream), "hipGraphLaunch")

    def __del__(self):
        try:
            if _hip is not None:
                if self.exec:
                    _hip.hipGraphExecDestroy(self.exec)
                if getattr(self, "graph", None):
                    _hip.hipGraphDestroy(self.graph)
        except Exception:
            pass


class Timer:
    """HIP events on a stream (the stream the measured kernels are launched on)."""

    def __init__(self, stream=None):
        self.stream = stream
        a, b = _vp(), _vp()
        call("talos_event_create", ctypes.byref(a))
        call("talos_event_create", ctypes.byref(b))
        self.a, self.b = a.value, b.value

    def start(self):
        call("talos_event_record", self.a, self.stream)

    def stop_ms(self):
        call("talos_event_record", self.b, self.stream)
        ms = _f()
        call("talos_event_elapsed_ms", self.a, self.b, ctypes.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if _lib is not None:
                _lib.talos_event_destroy(self.a)
                _lib.talos_event_destroy(self.b)
        except Exception:
            pass
