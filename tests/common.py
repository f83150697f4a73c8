"""Shared input generators and the comparison rule of the parity tests."""
import math
import os

import numpy as np

# Tolerances of the north star: fp32 within 1e-4 relative with a 1e-5 absolute floor,
# bf16-input MFMA variants within 2e-2 relative (floor scaled the same way).
FP32_RTOL, FP32_ATOL = 1e-4, 1e-5
BF16_RTOL, BF16_ATOL = 2e-2, 2e-3


def f32(a):
    """Rounds to fp32 and back to f64: the exact values the GPU path sees."""
    return np.asarray(a, dtype=np.float32).astype(np.float64)


# Parameter gradients that are sums over many token rows (dW = X^T dY, dgain, db) with an
# unscaled loss hold elements that cancel to a tiny fraction of the tensor's scale; there the
# fp32 rounding of the inputs alone exceeds 1e-5 absolute (torch's own fp32 CPU autograd fails
# the plain rule on the C3 block: 118 of 197504 parameter-gradient elements at batch 64). For
# those tensors the absolute floor is raised to 1e-6 of the tensor's largest |ref| (16 fp32 ulps
# of its largest element); everything else uses the plain floor.
GRAD_SCALE_FLOOR = 1e-6


# One record per check_close call that was given a scale floor: which tensor, the absolute floor
# it got, and how many of its elements pass only because of that floor (they would fail the plain
# rtol * |ref| + atol rule). conftest.py prints the records with a non-zero count at the end of
# the session and writes all of them to $TALOS_TOLERANCE_AUDIT (a JSON file) when that is set.
FLOOR_AUDIT = []


def check_close(got, ref, rtol=FP32_RTOL, atol=FP32_ATOL, name="", scale_floor=0.0):
    """Element-wise |got - ref| <= rtol * |ref| + max(atol, scale_floor * max|ref|); reports the
    worst element. With a scale floor, the elements that need it are counted in FLOOR_AUDIT."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    err = np.abs(got - ref)
    if scale_floor and ref.size:
        plain = err > rtol * np.abs(ref) + atol
        floor = max(atol, scale_floor * float(np.abs(ref).max()))
        FLOOR_AUDIT.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "tensor": name,
                            "size": int(ref.size), "floor": floor, "plain_atol": atol,
                            "max_abs_ref": float(np.abs(ref).max()), "needs_floor": int(plain.sum()),
                            "worst_err_over_plain": float(np.max(err / np.maximum(rtol * np.abs(ref) + atol, 1e-300)))})
        atol = floor
    bound = rtol * np.abs(ref) + atol
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{name}: {int(bad.sum())}/{err.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} err {err[i]:.3e} bound {bound[i]:.3e}")
    return float((err / (np.abs(ref) + atol)).max()) if err.size else 0.0


from workload import block_params, gacha_states, log_softmax, mla_params, ppo_params, xavier  # noqa: E402,F401


def reference_init_actor_critic(oracle, seed=12345):
    """The parameters ActorCritic::new(seed) builds (src/ppo.rs:254-258 with LuckTransformer::new,
    src/transformer.rs:48-69, and MultiHeadLatentAttention::new, :400-460): every Linear weight is
    Tensor::rand([in, out], -l, l, seed') with l = sqrt(6 / (in + out)) (src/nn.rs:20-35; the
    generator is the oracle's bit-exact LCG, src/autograd.rs:114-124), biases zero, RMSNorm gains
    one. Seeds: embed seed, MLA seed + 10 + {0..6}, ffn_1 seed + 20, ffn_2 seed + 30, out_proj
    seed + 40, actor seed + 100, critic seed + 200. Layout: workload.REFERENCE_ACTOR_CRITIC."""
    def lin(fin, fout, s, bias):
        lim = math.sqrt(6.0 / (fin + fout))
        w = oracle.lcg_rand(fin * fout, -lim, lim, s)
        return [w] + ([np.zeros(fout)] if bias else [])

    d, L, H, r, vd, F, A = 64, 32, 4, 16, 16, 128, 5
    parts = lin(8, d, seed, True) + [np.ones(d)]
    m = seed + 10
    parts += lin(d, L, m, False) + lin(L, H * vd, m + 1, False) + lin(L, H * vd, m + 2, False)
    parts += lin(d, H * vd, m + 3, False) + lin(d, H * r, m + 4, False) + lin(d, H * r, m + 5, False)
    parts += lin(H * vd, d, m + 6, False)
    parts += [np.ones(d)] + lin(d, F, seed + 20, True) + lin(F, d, seed + 30, True) + [np.ones(d)]
    parts += lin(d, d, seed + 40, True) + lin(d, A, seed + 100, True) + lin(d, 1, seed + 200, True)
    return np.concatenate(parts)
