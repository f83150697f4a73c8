"""CPU-side tests of the C ABI: the library loads, exports every function include/talos_hip.h
declares, and rejects bad arguments on the host before any device work (the reference panics via
assert! on the same conditions, src/autograd.rs:96-100, 209; src/nn.rs:187)."""
import ctypes
import os
import re

import numpy as np
import pytest

import talos_hip as th

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "talos_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t|void)\s+(talos_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def L():
    return th.lib()


def test_header_symbols_exported(L):
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in talos_hip.h but not exported: {missing}"
    # and the binding's signature table covers exactly the header
    assert sorted(th._SIGS) == names


def test_version_and_device_count(L):
    assert b"gfx950" in L.talos_version()
    assert th.device_count() >= 0


def _null():
    return ctypes.c_void_p(0)


def test_gemm_argument_errors(L):
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert L.talos_gemm_f32(0, 0, 4, 4, 4, 1.0, None, 4, p, 4, 0.0, p, 4, None) == th.ERR_NULL
    assert L.talos_gemm_f32(0, 0, -1, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, None) == th.ERR_SHAPE
    assert L.talos_gemm_f32(0, 0, 4, 4, 8, 1.0, p, 4, p, 4, 0.0, p, 4, None) == th.ERR_SHAPE  # lda < K
    assert L.talos_gemm_f32(1, 0, 8, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, None) == th.ERR_SHAPE  # lda < M (transA)
    assert L.talos_gemm_f32(0, 1, 4, 4, 8, 1.0, p, 8, p, 4, 0.0, p, 4, None) == th.ERR_SHAPE  # ldb < K (transB)
    assert L.talos_gemm_f32(0, 0, 4, 8, 4, 1.0, p, 4, p, 8, 0.0, p, 4, None) == th.ERR_SHAPE  # ldc < N
    assert L.talos_gemm_f32(2, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, None) == th.ERR_DTYPE
    assert L.talos_gemm_f32(0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.5, p, 4, None) == th.ERR_UNSUPPORTED
    assert b"beta" in L.talos_last_error()


def test_row_op_argument_errors(L):
    p = ctypes.c_void_p(16)
    assert L.talos_rmsnorm_fwd_f32(4, 0, 1e-6, p, p, p, p, None) == th.ERR_SHAPE
    assert L.talos_rmsnorm_fwd_f32(4, 8, 1e-6, None, p, p, p, None) == th.ERR_NULL
    assert L.talos_rmsnorm_bwd_f32(4, 8, p, p, p, p, 2.0, p, 0.0, p, None) == th.ERR_UNSUPPORTED
    assert L.talos_softmax_fwd_f32(4, 8, 3, p, p, None) == th.ERR_DTYPE
    assert L.talos_rope_fwd_f32(1, 4, 2, 7, 0, 1e4, p, p, None) == th.ERR_SHAPE  # odd dim
    assert L.talos_rope_fwd_f32(1, 4, 2, 8, -1, 1e4, p, p, None) == th.ERR_SHAPE
    assert L.talos_unary_fwd_f32(99, 4, 0.0, 0.0, p, p, None) == th.ERR_DTYPE
    assert L.talos_binary_fwd_f32(7, 4, p, p, p, None) == th.ERR_DTYPE
    shape = (ctypes.c_longlong * 2)(2, 3)
    assert L.talos_transpose_f32(2, shape, 0, 2, p, p, 0, None) == th.ERR_SHAPE
    assert L.talos_transpose_f32(7, shape, 0, 1, p, p, 0, None) == th.ERR_SHAPE


def test_attention_argument_errors(L):
    p = ctypes.c_void_p(16)
    args = [p, 96, p, 96, p, 96, p, 32, p, None]
    assert L.talos_attn_fwd_f32(2, 8, 4, 200, 32, 0.1, 1, *args) == th.ERR_UNSUPPORTED  # head dim > 128
    assert L.talos_attn_fwd_f32(2, 8, 4, 32, 32, 0.1, 2, *args) == th.ERR_DTYPE
    assert L.talos_attn_fwd_f32(2, 8, 4, 32, 32, 0.1, 1, p, 64, p, 96, p, 96, p, 32, p, None) == th.ERR_SHAPE


def test_plan_config_errors(L):
    cfg = th.BlockCfg(2, 8, 30, 4, 8, 64, 1, 0, 1e-6, 1e4)  # 4 * 8 != 30
    h = ctypes.c_void_p()
    assert L.talos_block_plan_create(ctypes.byref(cfg), ctypes.byref(h)) == th.ERR_SHAPE
    cfg = th.BlockCfg(2, 8, 32, 4, 8, 64, 1, 7, 1e-6, 1e4)  # bad activation
    assert L.talos_block_plan_create(ctypes.byref(cfg), ctypes.byref(h)) == th.ERR_DTYPE
    assert L.talos_block_fwd_bwd_f32(None, *([ctypes.c_void_p(16)] * 6), None) == th.ERR_HANDLE
    pc = th.PpoCfg(4, 8, 8, 32, 2, 4, 8, 64, 0, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)  # 0 actions
    assert L.talos_ppo_plan_create(ctypes.byref(pc), ctypes.byref(h)) == th.ERR_SHAPE
    # latent attention: unknown kind, odd RoPE width, missing latent, too-wide heads
    for bad, code in (((2, 0, 0, 0), th.ERR_DTYPE), ((1, 32, 5, 16), th.ERR_SHAPE), ((1, 0, 16, 16), th.ERR_SHAPE),
                      ((1, 32, 116, 16), th.ERR_UNSUPPORTED)):
        cfg = th.BlockCfg(2, 8, 64, 4, 16, 128, 0, 1, 1e-5, 1e4, *bad)
        assert L.talos_block_plan_create(ctypes.byref(cfg), ctypes.byref(h)) == code, bad


def test_param_counts_match_oracle(oracle):
    import common
    bc = th.BlockCfg(4, 64, 128, 4, 32, 512, 1, 0, 1e-6, 1e4)
    assert th.lib().talos_block_param_count(ctypes.byref(bc)) == 128 + 3 * 128 * 128 + 128 * 128 + 128 + 2 * 128 * 512 + 512 + 128
    pc = th.PpoCfg(8, 32, 8, 128, 2, 4, 32, 512, 3, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)
    opc = oracle.PpoCfg(8, 32, 8, 128, 2, 4, 32, 512, 3, 1, 0, 1e-5, 1e4, 0.2, 0.5, 0.01)
    n = th.lib().talos_ppo_param_count(ctypes.byref(pc))
    assert n == oracle.ppo_param_count(opc)
    assert n == common.ppo_params(np.random.default_rng(0), opc).size


def test_decoder_argument_errors_without_a_device(L):
    import workload
    cfg = th.PpoCfg(1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    h = ctypes.c_void_p()
    for n_envs, ctx, code in ((0, 8, th.ERR_SHAPE), (4, 0, th.ERR_UNSUPPORTED), (4, 1024, th.ERR_UNSUPPORTED)):
        assert L.talos_ppo_decoder_create(ctypes.byref(cfg), n_envs, ctx, 256, ctypes.byref(h)) == code
    bad = th.PpoCfg(1, 16, *workload.REFERENCE_ACTOR_CRITIC)
    bad.attention = 3
    assert L.talos_ppo_decoder_create(ctypes.byref(bad), 4, 8, 256, ctypes.byref(h)) == th.ERR_DTYPE
    p = ctypes.c_void_p(16)
    assert L.talos_ppo_decoder_step_f32(None, 1, p, p, p, None, None, None, None, None, None, None) == th.ERR_HANDLE
    assert L.talos_ppo_decoder_destroy(None) == th.OK


def test_reference_actor_critic_param_count(oracle):
    """The reference ActorCritic's parameter count, summed from the shapes of ActorCritic::new
    (src/ppo.rs:254-258) and LuckTransformer::new (src/transformer.rs:48-69): embed 8x64+64,
    norm_1 64, MLA w_dkv 64x32, w_uk / w_uv 32x64, w_q 64x64, w_kr / w_qr 64x64, w_o 64x64, norm_2
    64, ffn_1 64x128+128, ffn_2 128x64+64, norm_final 64, out_proj 64x64+64, actor 64x5+5, critic
    64x1+1."""
    import workload
    want = (8 * 64 + 64) + 64 + (64 * 32 + 2 * 32 * 64 + 64 * 64 + 2 * 64 * 64 + 64 * 64) + 64 + (64 * 128 + 128) + \
        (128 * 64 + 64) + 64 + (64 * 64 + 64) + (64 * 5 + 5) + (64 + 1)
    pc = th.PpoCfg(16, 16, *workload.REFERENCE_ACTOR_CRITIC)
    opc = oracle.PpoCfg(16, 16, *workload.REFERENCE_ACTOR_CRITIC)
    assert th.lib().talos_ppo_param_count(ctypes.byref(pc)) == want
    assert oracle.ppo_param_count(opc) == want
    assert workload.ppo_params(np.random.default_rng(0), opc).size == want
    bc = th.BlockCfg(16, 16, 64, 4, 16, 128, 0, 1, 1e-5, 1e4, th.ATTN_MLA, 32, 16, 16)
    obc = oracle.BlockCfg(16, 16, 64, 4, 16, 128, 0, 1, 1e-5, 1e4, th.ATTN_MLA, 32, 16, 16)
    nb = th.lib().talos_block_param_count(ctypes.byref(bc))
    assert nb == oracle.block_param_count(obc) == workload.mla_block_params(np.random.default_rng(0), obc).size


def test_no_device_is_a_clean_error(L):
    if th.device_count() > 0:
        pytest.skip("a GPU is present")
    p = ctypes.c_void_p()
    assert L.talos_malloc(ctypes.byref(p), 64) == th.ERR_NO_DEVICE
    assert L.talos_init() == th.ERR_NO_DEVICE
    assert b"GPU" in L.talos_last_error()


def test_optimizer_argument_errors(L):
    p = ctypes.c_void_p(16)
    args = (0.9, 0.999, 1e-8)
    assert L.talos_adam_step_f32(4, p, p, p, p, 0, 1e-3, *args, None, 0.0, None) == th.ERR_SHAPE  # t < 1
    assert L.talos_adam_step_f32(4, p, p, p, p, 1, 1e-3, 1.0, 0.999, 1e-8, None, 0.0, None) == th.ERR_SHAPE
    assert L.talos_adam_step_f32(4, p, p, p, p, 1, 1e-3, *args, p, 0.0, None) == th.ERR_SHAPE  # max_norm
    assert L.talos_adam_step_f32(4, None, p, p, p, 1, 1e-3, *args, None, 0.0, None) == th.ERR_NULL
    assert L.talos_adam_step_f32(0, None, None, None, None, 1, 1e-3, *args, None, 0.0, None) == th.OK
    assert L.talos_grad_sumsq_f32(4, p, 0, None, None, None) == th.ERR_NULL
    assert L.talos_grad_sumsq_f32(4, None, 0, p, None, None) == th.ERR_NULL
    assert L.talos_grad_sumsq_workspace_bytes() >= 8


def test_workspace_bind_validation():
    L = th.lib()
    assert L.talos_workspace_bind(None, 0) == th.OK
    assert L.talos_workspace_bind(None, 4096) == th.ERR_NULL
    assert L.talos_workspace_bind(ctypes.c_void_p(4096 + 16), 4096) == th.ERR_SHAPE
    assert L.talos_workspace_bind(ctypes.c_void_p(4096), 4096) == th.OK
    assert L.talos_workspace_high_water() == 0
    assert L.talos_workspace_bytes() == 4096
    assert L.talos_workspace_bind(None, 0) == th.OK
    assert L.talos_workspace_bytes() == 0


def test_completion_mode_switch():
    # synchronous by default (the reference's ops return finished results); per thread
    L = th.lib()
    assert L.talos_get_async() == 0
    assert L.talos_set_async(2) == th.ERR_SHAPE
    with th.async_mode():
        assert L.talos_get_async() == 1
        seen = []
        import threading
        t = threading.Thread(target=lambda: seen.append(L.talos_get_async()))
        t.start()
        t.join()
        assert seen == [0]  # another thread keeps its own (default) mode
    assert L.talos_get_async() == 0


def test_gelu_and_head_loss_argument_errors(L):
    p = ctypes.c_void_p(16)
    assert L.talos_gelu_fwd_f32(4, None, p, None) == th.ERR_NULL
    assert L.talos_gelu_bwd_f32(4, p, p, 0.5, p, None) == th.ERR_UNSUPPORTED
    assert L.talos_gelu_bwd_f32(4, p, None, 0.0, p, None) == th.ERR_NULL
    args = (0.2, 0.5, 0.01, p, p, p, p, p, p)
    assert L.talos_ppo_head_loss_fwd_f32(4, 3, *args, None, None, 0, None) == th.ERR_NULL  # no output
    assert L.talos_ppo_head_loss_fwd_f32(-1, 3, *args, p, None, 0, None) == th.ERR_SHAPE
    assert L.talos_ppo_head_loss_fwd_f32(4, 0, *args, p, None, 0, None) == th.ERR_SHAPE
    assert L.talos_ppo_head_loss_fwd_f32(4, 3, -0.1, 0.5, 0.01, p, p, p, p, p, p, p, None, 0, None) == th.ERR_SHAPE
    assert L.talos_ppo_head_loss_fwd_f32(4, 3, *args, p, None, 2, None) == th.ERR_SHAPE
    assert L.talos_ppo_head_loss_fwd_f32(4, 3, 0.2, 0.5, 0.01, p, None, p, p, p, p, p, None, 0, None) == th.ERR_NULL
    assert L.talos_ppo_head_loss_bwd_f32(4, 3, *args, None, p, None, None) == th.ERR_NULL
    assert L.talos_ppo_head_loss_bwd_f32(4, 3, *args, p, None, None, None) == th.ERR_NULL
