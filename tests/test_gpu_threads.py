"""Host threads calling the synchronous entry point concurrently (ctypes
releases the GIL during the call): on one shared context, whose calls
serialize on its mutex and share its weight cache and staging buffers, and
on one context per thread.  Every result meets the parity bar."""
import ctypes
import threading

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests import test_gpu_parity as t

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _work(orc, ctx, seed, errors, reps=6):
    try:
        rng = np.random.default_rng(seed)
        ty = (12, 14, 8, 23)[seed % 4]
        N, K, M = 300 + 7 * seed, 2048, 1 + seed % 3
        raw = t.weights(ty, N, K, seed=seed)
        ref_in = [rng.standard_normal((M, K)).astype(np.float32) for _ in range(reps)]
        for A in ref_in:
            C = np.full((M, N), np.nan, np.float32)
            p = gl.MulMatParams()
            p.A, p.B, p.C = A.ctypes.data, raw.ctypes.data, C.ctypes.data
            p.M, p.N, p.K, p.lda, p.ldb, p.ldc, p.n_batches, p.B_type = M, N, K, K, K, N, 1, ty
            st = ctx.lib.ggq_mul_mat_q(ctx.h, ctypes.byref(p), 0)
            if st != 0:
                errors.append((seed, "status", st))
                return
            err = orc.rel_l2(C, orc.mul_mat_f64(ty, raw, N, K, A, 0))
            if not err < TOL:
                errors.append((seed, "err", err))
                return
    except Exception as e:  # reported by the main thread
        errors.append((seed, "exception", repr(e)))


@pytest.mark.parametrize("shared", [True, False])
def test_threads_host_api(orc, shared):
    import torch
    assert torch.cuda.is_available()
    n = 6
    ctxs = [gl.Context(0)] if shared else [gl.Context(0) for _ in range(n)]
    errors = []
    ths = [threading.Thread(target=_work, args=(orc, ctxs[0] if shared else ctxs[i], i, errors)) for i in range(n)]
    for th in ths:
        th.start()
    for th in ths:
        th.join(timeout=100)
    for c in ctxs:
        c.close()
    assert not any(th.is_alive() for th in ths)
    assert not errors, errors
