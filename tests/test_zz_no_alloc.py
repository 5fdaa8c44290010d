"""ggq_mul_mat_noalloc_dev: the allocation-free variant of ggq_mul_mat_dev
(scratch in one fixed per-GPU region).  Its output equals ggq_mul_mat_dev's
bit for bit, in every activation mode and on every scratch-using path (int8
GEMM with split-K partials, the M <= 8 per-row int8 path that the int8 GEMV
does not take, block32), on two calls in
a row with the second smaller (the region keeps the first call's contents);
a call needing more scratch than the region holds is refused before any
work is queued."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests.gpu_util import dev, host, stream_handle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    c = gl.Context(0)
    yield c
    c.close()


def call(ctx, fn, dW, t, N, K, x, M, mode, ldc=None):
    import torch
    ldc = ldc or N
    y = torch.full((M, ldc), float("nan"), device="cuda")
    st = fn(ctx.h, ctypes.c_void_p(dW.data_ptr()), t, N, K, ctypes.c_void_p(x.data_ptr()), K,
            ctypes.c_void_p(y.data_ptr()), ldc, M, mode, stream_handle())
    ctx.check(st, fn.__name__)
    return host(y)


# (type, N, K, M first, M second, act mode)
CASES = [(8, 1536, 1536, 512, 64, 1),     # int8 GEMM, then a smaller one
         (8, 384, 8960, 96, 16, 1),       # split-K partials
         (12, 2048, 2048, 8, 3, 1),       # M <= 8 per-row int8: the int8 GEMV, no scratch
         (8, 640, 1568, 7, 2, 1),         # M <= 8 per-row int8 with K not a multiple of 256:
                                          # codes and effective activations in the region,
                                          # then the fp32 GEMV
         (14, 512, 2048, 6, 2, 2),        # block32 activations
         (12, 4096, 2048, 1, 1, 0),       # fp32: no scratch at all
         (13, 1000, 3072, 64, 4, 1)]      # int8 GEMM, then M = 4 on the int8 GEMV


@pytest.mark.parametrize("t,N,K,M1,M2,mode", CASES)
def test_noalloc_matches_mul_mat_dev(ctx, orc, t, N, K, M1, M2, mode):
    import torch
    rng = np.random.default_rng(N + K + M1)
    raw = gl.encode(t, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    dW = dev(raw)
    for M in (M1, M2):
        A = rng.standard_normal((M, K)).astype(np.float32)
        x = torch.from_numpy(A).cuda()
        got = call(ctx, ctx.lib.ggq_mul_mat_noalloc_dev, dW, t, N, K, x, M, mode)
        exp = call(ctx, ctx.lib.ggq_mul_mat_dev, dW, t, N, K, x, M, mode)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (t, N, K, M, mode)
        if M <= 64:
            assert orc.rel_l2(got, orc.mul_mat_f64(t, raw, N, K, A, mode)) < 1e-4


def test_noalloc_rejects_oversized_scratch(ctx):
    import torch
    t, N, K, M = 8, 256, 8192, 4608  # 37.7 MB of int8 activations > the 32 MiB region
    raw = gl.encode(t, np.zeros((N, K), np.float32))
    dW = dev(raw)
    x = torch.zeros((M, K), device="cuda")
    y = torch.full((M, N), 7.0, device="cuda")
    st = ctx.lib.ggq_mul_mat_noalloc_dev(ctx.h, ctypes.c_void_p(dW.data_ptr()), t, N, K, ctypes.c_void_p(x.data_ptr()),
                                         K, ctypes.c_void_p(y.data_ptr()), N, M, 1, stream_handle())
    assert st == int(gl.Status.INVALID_PARAM)
    assert b"scratch" in ctx.lib.ggq_last_error_message(ctx.h)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())  # nothing was queued


def test_noalloc_refuses_overlap_on_another_stream(ctx):
    """A call whose region is still in use by an unfinished call on another
    stream is refused (nothing queued); once that work is done, or on the
    same stream, the call goes through."""
    import torch
    t, N, K, M = 8, 256, 1536, 64
    rng = np.random.default_rng(5)
    raw = gl.encode(t, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    dW = dev(raw)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda()
    y1 = torch.full((M, N), 3.0, device="cuda")
    y2 = torch.full((M, N), 7.0, device="cuda")
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()

    def go(y, s):
        return ctx.lib.ggq_mul_mat_noalloc_dev(ctx.h, ctypes.c_void_p(dW.data_ptr()), t, N, K,
                                               ctypes.c_void_p(x.data_ptr()), K, ctypes.c_void_p(y.data_ptr()), N, M,
                                               1, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        torch.cuda._sleep(50_000_000)  # keeps stream A busy (tens of ms to a second)
    ctx.check(go(y1, sa), "first call")
    assert go(y2, sb) == int(gl.Status.ERROR)
    assert b"in use" in ctx.lib.ggq_last_error_message(ctx.h)
    ctx.check(go(y1, sa), "same stream")  # ordered behind the first: accepted
    torch.cuda.synchronize()
    assert bool((y2 == 7.0).all())  # the refused call queued nothing
    ctx.check(go(y2, sb), "after the first finished")
    torch.cuda.synchronize()
    assert np.array_equal(host(y1), host(y2))
