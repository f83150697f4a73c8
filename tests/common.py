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


# Parameter gradients (dW = X^T G, an RMSNorm gain's sum_r g x_hat, a bias's sum_r g) are sums
# over many token rows. Where such a sum cancels to a small fraction of its terms, the fp32
# rounding of its terms and of the accumulation alone exceeds the plain 1e-5 absolute floor (torch's
# own fp32 CPU autograd of the C3 block fails the plain rule on 257 elements at batch 128). The
# bound for those elements is derived from the sum itself: the oracle returns, for every
# parameter-gradient element, the f64 magnitude sum M of its terms ((|X|^T |G|)_ij, sum_r |g x_hat|,
# sum_r |g|; pyoracle's mag=True), and
#     |got - ref| <= 1e-4 |ref| + max(1e-5, GRAD_KAPPA * 2^-24 * M).
# GRAD_KAPPA = 32 is the probabilistic rounding-error constant of the device's accumulation: a
# weight-gradient element is a chain of at most 256 fp32 multiply-adds per 512-row split (the
# splits are combined in f64), whose rounding error is ~sqrt(256) u M = 16 u M (Higham & Mary,
# "A new approach to probabilistic rounding error analysis", 2019), plus the relative error of
# the fp32 operands X and G themselves (a few u). A missing, doubled or misplaced row changes the
# element by a whole term, |x_ri g_rj|, which for the configurations' 2048..131072-row sums is
# M / rows on average: 8 to 500 times the allowance GRAD_KAPPA u M.
U32 = 2.0 ** -24
GRAD_KAPPA = 32.0
# The bf16-in / fp32-accumulate variant (north star: within 2e-2 relative) gets the same form with
# bf16's unit roundoff: |got - ref| <= 2e-2 |ref| + max(1e-5, BF16_KAPPA * 2^-8 * M). Rounding
# both operands of the final product to bf16 changes each term by at most 2 u |x g| (2 u M in
# all); the operands themselves come from bf16-in products upstream (the attention's gradients,
# the latent), whose own errors add to that. Measured on the bf16 MLA tests (56 tensors, seq 37
# to 256 and C5 at full size): at most 1.80 u M; BF16_KAPPA = 4 keeps about twice that. (About a
# fifth of the elements fail the plain 2e-2 |ref| + 1e-5 rule: their sums cancel below 2^-8 of
# their terms.) At this allowance a dropped row is invisible, so the bf16 paths are also pinned
# bit for bit: tests/test_gpu_models.py::test_mla_bf16_copies_bit_identical against the plan that
# rounds at staging, and that GEMM against f64 products of bf16-rounded operands (test_gpu_kernels).
U_BF16 = 2.0 ** -8
BF16_KAPPA = 4.0


# One record per check_grad call: which tensor, how many of its elements needed the magnitude
# allowance (they fail the plain rtol * |ref| + atol rule), and the kappa each tensor needed at
# most. conftest.py prints the records with a non-zero count at the end of the session and
# writes all of them to $TALOS_TOLERANCE_AUDIT (a JSON file) when that is set.
GRAD_AUDIT = []


def check_close(got, ref, rtol=FP32_RTOL, atol=FP32_ATOL, name=""):
    """Element-wise |got - ref| <= rtol * |ref| + atol; reports the worst element."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    err = np.abs(got - ref)
    return _report(got, ref, err, rtol * np.abs(ref) + atol, name, atol)


def check_grad(got, ref, mag, name="", kappa=GRAD_KAPPA, rtol=FP32_RTOL, atol=FP32_ATOL, audit=True, unit=U32):
    """A parameter gradient against the oracle with the magnitude-derived bound
    |got - ref| <= rtol |ref| + max(atol, kappa unit mag), mag the oracle's magnitude sums, unit
    2^-24 (fp32) or 2^-8 (check_grad_bf16) (audit=False keeps a deliberately wrong input out of
    the audit)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    mag = np.asarray(mag, dtype=np.float64)
    assert got.shape == ref.shape == mag.shape, f"{name}: shape {got.shape} vs {ref.shape} vs {mag.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    assert np.all(mag >= np.abs(ref) * (1 - 1e-12)), f"{name}: magnitude sums below |ref|"
    err = np.abs(got - ref)
    if ref.size and audit:
        plain = err > rtol * np.abs(ref) + atol
        need = np.where(plain, (err - rtol * np.abs(ref)) / (unit * np.maximum(mag, 1e-300)), 0.0)
        GRAD_AUDIT.append({"test": os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "tensor": name,
                           "rule": "bf16" if unit == U_BF16 else "fp32", "rtol": rtol,
                           "size": int(ref.size), "kappa": kappa, "needs_mag": int(plain.sum()),
                           "kappa_needed": float(need.max()), "max_abs_ref": float(np.abs(ref).max()),
                           "worst_err_over_plain": float(np.max(err / (rtol * np.abs(ref) + atol)))})
    return _report(got, ref, err, rtol * np.abs(ref) + np.maximum(atol, kappa * unit * mag), name, atol)


def check_grad_bf16(got, ref, mag, name="", kappa=BF16_KAPPA):
    """check_grad for the bf16-in variant: 2e-2 relative, 1e-5 absolute, BF16_KAPPA 2^-8 mag."""
    return check_grad(got, ref, mag, name, kappa=kappa, rtol=BF16_RTOL, atol=FP32_ATOL, unit=U_BF16)


def _report(got, ref, err, bound, name, atol):
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{name}: {int(bad.sum())}/{err.size} elements out of tolerance; worst at {i}: "
                             f"got {got[i]!r} ref {ref[i]!r} err {err[i]:.3e} bound {bound[i]:.3e}")
    return float((err / np.maximum(np.abs(ref) + atol, 1e-300)).max()) if err.size else 0.0


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
