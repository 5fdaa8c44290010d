"""Parity checks run in a child process by tests/test_gpu_process_knobs.py,
so that the tuning variables the library reads once per process take effect
(GGQ_GEMV_U, GGQ_GEMV_PREFETCH, GGQ_GEMV_MAXLPR, GGQ_GEMV_BLOCKS,
GGQ_GEMM_TILE, GGQ_GEMM_PF).  Exits 0 when every check meets the bar
(rel-L2 <= 1e-4 against the fp64 oracle), 1 with the failing case otherwise."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import ggnpu_amd.lib as gl  # noqa: E402
from oracle import oracle as orc  # noqa: E402
from tests import test_gpu_parity as t  # noqa: E402

TOL = 1e-4


def main():
    import torch
    # torch's bundled HIP runtime is initialized before the library's context
    # (the other order leaves torch without devices).
    if not torch.cuda.is_available():
        print("no GPU")
        return 1
    orc.lib()
    ctx = gl.Context(0)
    try:
        rng = np.random.default_rng(0)
        # GEMV, one row and two rows (FMA kernels: GGQ_GEMV_MFMA=0 is set by the parent),
        # pieces per thread by K (2048, 4096, 8192) and the threads-per-row setting.
        for ty, N, K, M in ((12, 777, 2048, 1), (14, 300, 8192, 2), (8, 130, 8192, 1), (23, 65, 4096, 3)):
            raw = t.weights(ty, N, K, seed=N)
            A = rng.standard_normal((M, K)).astype(np.float32)
            err = orc.rel_l2(t.run_mm(ctx, ty, raw, N, K, A, 0), orc.mul_mat_f64(ty, raw, N, K, A, 0))
            if not err < TOL:
                print("gemv", ty, N, K, M, err)
                return 1
        # Prefill GEMM (per-row int8 activations, M > 8).
        for ty, N, K, M in ((8, 320, 1536, 96), (12, 200, 2048, 40), (20, 130, 1024, 64)):
            raw = t.weights(ty, N, K, seed=K)
            A = rng.standard_normal((M, K)).astype(np.float32)
            err = orc.rel_l2(t.run_mm(ctx, ty, raw, N, K, A, 1), orc.mul_mat_f64(ty, raw, N, K, A, 1))
            if not err < TOL:
                print("gemm", ty, N, K, M, err)
                return 1
    finally:
        ctx.close()
    print("ok")
    return 0


if __name__ == "__main__":
    sys.exit(main())
