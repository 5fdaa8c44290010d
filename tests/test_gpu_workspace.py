"""Workspace contract of the device entry points (include/ggq.h): a call being
captured into a HIP graph never allocates (it fails with a clear message
when its workspace is too small), ggq_reserve sizes the workspace ahead of a
capture, and a graph captured before the workspace grows stays valid after
the growth (outgrown buffers are kept until ggq_destroy)."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests import test_gpu_parity as t
from tests.gpu_util import dev

pytestmark = pytest.mark.gpu


def q8_call(c, dW, N, K, x, y, M, stream):
    return c.lib.ggq_mul_mat_dev(c.h, ctypes.c_void_p(dW.data_ptr()), 8, N, K, ctypes.c_void_p(x.data_ptr()), K,
                                 ctypes.c_void_p(y.data_ptr()), N, M, int(gl.ActMode.Q8_ROW), stream)


def test_capture_refuses_growth_then_reserve(orc):
    import torch
    c = gl.Context(0)
    try:
        N, K, M = 512, 4096, 64  # K > 2048: quantized into the workspace, split-K partials
        raw = t.weights(8, N, K, seed=3)
        dW = dev(raw)
        A = np.random.default_rng(3).standard_normal((M, K)).astype(np.float32)
        x = torch.from_numpy(A).cuda()
        y = torch.zeros((M, N), device="cuda")
        s = torch.cuda.Stream()
        sh = ctypes.c_void_p(s.cuda_stream)
        torch.cuda.synchronize()
        # fresh context: no workspace yet, so the captured call is refused
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                st = q8_call(c, dW, N, K, x, y, M, sh)
        assert st == int(gl.Status.ERROR)
        assert b"captured" in c.lib.ggq_last_error_message(c.h)
        del g
        torch.cuda.synchronize()
        # reserve, then the same capture works and replays match the oracle
        c.check(c.lib.ggq_reserve(c.h, 64 << 20), "reserve")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                c.check(q8_call(c, dW, N, K, x, y, M, sh), "captured q8")
        ref = orc.mul_mat_f64(8, raw, N, K, A, 1)
        for _ in range(3):
            y.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert orc.rel_l2(y.cpu().numpy(), ref) < t.TOL
    finally:
        c.close()


def test_graph_survives_workspace_growth(orc):
    """Capture with a small workspace, grow it with a larger eager call, then
    replay: the graph still reads the (kept) old buffer and is correct."""
    import torch
    c = gl.Context(0)
    try:
        N, K = 384, 4096  # the workspace path (K > 2048)
        raw = t.weights(8, N, K, seed=4)
        dW = dev(raw)
        rng = np.random.default_rng(4)
        A1 = rng.standard_normal((16, K)).astype(np.float32)
        A2 = rng.standard_normal((256, K)).astype(np.float32)
        x1, x2 = torch.from_numpy(A1).cuda(), torch.from_numpy(A2).cuda()
        y1, y2 = torch.zeros((16, N), device="cuda"), torch.zeros((256, N), device="cuda")
        s = torch.cuda.Stream()
        sh = ctypes.c_void_p(s.cuda_stream)
        with torch.cuda.stream(s):
            c.check(q8_call(c, dW, N, K, x1, y1, 16, sh), "warm-up")
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                c.check(q8_call(c, dW, N, K, x1, y1, 16, sh), "captured")
        with torch.cuda.stream(s):
            c.check(q8_call(c, dW, N, K, x2, y2, 256, sh), "growing call")
        torch.cuda.synchronize()
        assert orc.rel_l2(y2.cpu().numpy(), orc.mul_mat_f64(8, raw, N, K, A2, 1)) < t.TOL
        ref1 = orc.mul_mat_f64(8, raw, N, K, A1, 1)
        for _ in range(3):
            y1.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert orc.rel_l2(y1.cpu().numpy(), ref1) < t.TOL
    finally:
        c.close()


def test_capture_needs_no_workspace_on_the_panel_gemm(orc):
    """K <= 2048: the prefill GEMM quantizes the rows inside its own launch
    and uses no workspace, so a fresh context captures it without
    ggq_reserve; replays on fresh inputs match the oracle."""
    import torch
    c = gl.Context(0)
    try:
        N, K, M = 640, 1536, 96
        raw = t.weights(8, N, K, seed=5)
        dW = dev(raw)
        rng = np.random.default_rng(5)
        x = torch.zeros((M, K), device="cuda")
        y = torch.zeros((M, N), device="cuda")
        s = torch.cuda.Stream()
        sh = ctypes.c_void_p(s.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                c.check(q8_call(c, dW, N, K, x, y, M, sh), "captured panel GEMM")
        for _ in range(3):
            A = rng.standard_normal((M, K)).astype(np.float32)
            x.copy_(torch.from_numpy(A))
            y.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert orc.rel_l2(y.cpu().numpy(), orc.mul_mat_f64(8, raw, N, K, A, 1)) < t.TOL
    finally:
        c.close()
