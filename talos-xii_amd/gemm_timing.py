"""Single-GEMM timings through the C ABI.

Times `talos_gemm_f32` and `talos_gemm_bf16acc_f32` (include/talos_hip.h) on the product shapes of
the C4 step (M = 131072 token rows) and of the C5 MLA block (M = 16384), plus a long-K square
product, so the per-launch cost of the GEMM kernels can be read apart from the fused plans. The
library runs in its asynchronous mode and each shape is launched `--reps` times back to back
between two HIP events on the library's stream; the printed time is per launch (launch gaps
included, a few microseconds at most).

    python talos-xii_amd/gemm_timing.py [--set c4|c5|long|all] [--reps 20]

Each line: the shape (transA, transB, M, N, K), the dtype path, microseconds per launch and
TFLOP/s of the 2 M N K product flops. Operands are seeded normal values; outputs are not checked
here (tests/test_gpu_kernels.py checks the same entry points against the oracle).
"""
import argparse
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import talos_hip as th  # noqa: E402

SETS = {
    # C4: the d = 128 dX / QKV products, the MLP products (N = 512, K = 128) over all rows and
    # over 1/2 and 3/4 of them (output past / inside the Infinity Cache), a split-K weight gradient
    "c4": [(0, 1, 131072, 128, 512, "f32"), (0, 0, 131072, 128, 512, "f32"), (0, 0, 131072, 384, 128, "f32"),
           (0, 0, 131072, 512, 128, "f32"), (0, 0, 98304, 512, 128, "f32"), (0, 0, 65536, 512, 128, "f32"),
           (1, 0, 128, 512, 131072, "f32")],
    # C5: the MLA projections (forward, input gradient, weight gradient) in both paths
    "c5": [(0, 0, 16384, 512, 512, "f32"), (0, 0, 16384, 512, 512, "bf16"), (0, 1, 16384, 512, 512, "f32"),
           (0, 1, 16384, 512, 512, "bf16"), (1, 0, 512, 512, 16384, "f32"), (1, 0, 512, 512, 16384, "bf16")],
    # long K: the main loop without prologue / epilogue weight
    "long": [(0, 0, 4096, 4096, 8192, "f32"), (0, 0, 4096, 4096, 4096, "bf16")],
}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--set", default="all", choices=list(SETS) + ["all"])
    ap.add_argument("--reps", type=int, default=20)
    args = ap.parse_args()
    shapes = [s for k in (SETS if args.set == "all" else [args.set]) for s in SETS[k]]
    most_a = max(m * k for _, _, m, n, k, _ in shapes)
    most_b = max(k * n for _, _, m, n, k, _ in shapes)
    most_c = max(m * n for _, _, m, n, k, _ in shapes)
    rng = np.random.default_rng(0)
    A = th.DeviceArray.from_numpy(rng.standard_normal(most_a, dtype=np.float32))
    B = th.DeviceArray.from_numpy(rng.standard_normal(most_b, dtype=np.float32))
    C = th.DeviceArray.zeros(most_c)
    timer = th.Timer(None)
    print(f"device: {th.device_info()}", flush=True)
    with th.async_mode():
        for tA, tB, m, n, k, path in shapes:
            assert m * k <= most_a and k * n <= most_b and m * n <= most_c  # operands inside the buffers
            lda = m if tA else k
            ldb = k if tB else n
            fn = "talos_gemm_bf16acc_f32" if path == "bf16" else "talos_gemm_f32"
            call_args = (tA, tB, m, n, k, 1.0, A.ptr, lda, B.ptr, ldb, 0.0, C.ptr, n, None)
            th.call(fn, *call_args)  # warm-up (and the split-K workspace)
            th.sync()
            timer.start()
            for _ in range(args.reps):
                th.call(fn, *call_args)
            ms = timer.stop_ms() / args.reps
            print(f"({tA},{tB},{m},{n},{k}) {path}: {ms * 1e3:.1f} us  {2.0 * m * n * k / ms / 1e9:.1f} TFLOP/s",
                  flush=True)


if __name__ == "__main__":
    main()
