"""Device entry points captured into one HIP graph (torch.cuda.graph on a
side stream) after an eager warm-up that sizes every workspace: a single-row
GEMV, a 4-row matrix-core GEMV, the per-row int8 GEMM with split-K, decode
attention with a span merge, and an MoE layer (routing, grouping, grouped
GEMVs, SwiGLU, combine).  The graph is replayed several times on fresh
inputs written between replays, with eager work in between; every replay
equals the eager result bit for bit (the kernels are deterministic), and the
eager results meet the parity bar against the oracle."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests import test_gpu_parity as t
from tests.gpu_util import dev

pytestmark = pytest.mark.gpu
ctx = t.ctx


def test_graph_replays_match_eager(ctx, orc):
    import torch
    lib = ctx.lib
    rng = np.random.default_rng(5)
    s = torch.cuda.Stream()
    sh = ctypes.c_void_p(s.cuda_stream)

    # weights and fixed inputs
    K, N = 2048, 700
    raw = t.weights(12, N, K, seed=1)
    dW = dev(raw)
    K8, N8, M8 = 1536, 1536, 64          # split-K GEMM shape (N small, K long)
    raw8 = t.weights(8, N8, K8, seed=2)
    dW8 = dev(raw8)
    n_head, n_kv, hd, ctx_len = 32, 8, 64, 900
    Kc = dev(rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32))
    Vc = dev(rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32))
    T, H, F, E, k = 16, 512, 256, 32, 4
    Wg = dev(gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32)))
    Wu = dev(gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32)))
    Wd = dev(gl.encode(14, (rng.standard_normal((E * H, F)) * 0.02).astype(np.float32)))

    # inputs (rewritten before every replay) and outputs
    x1 = torch.empty((1, K), device="cuda")
    x4 = torch.empty((4, K), device="cuda")
    x8 = torch.empty((M8, K8), device="cuda")
    q = torch.empty((1, n_head, hd), device="cuda")
    mx = torch.empty((T, H), device="cuda")
    ml = torch.empty((T, E), device="cuda")
    outs = {n: torch.empty(shape, device="cuda") for n, shape in
            (("y1", (1, N)), ("y4", (4, N)), ("y8", (M8, N8)), ("att", (1, n_head, hd)), ("moe", (T, H)))}
    moe = gl.MoeParams()
    moe.T, moe.H, moe.F, moe.E, moe.top_k = T, H, F, E, k
    moe.x, moe.router_logits = mx.data_ptr(), ml.data_ptr()
    moe.gate_type, moe.up_type, moe.down_type = 12, 12, 14
    moe.gate_exps, moe.up_exps, moe.down_exps = Wg.data_ptr(), Wu.data_ptr(), Wd.data_ptr()
    moe.out = outs["moe"].data_ptr()

    def work(stream):
        ctx.check(lib.ggq_mul_mat_dev(ctx.h, dW.data_ptr(), 12, N, K, x1.data_ptr(), K, outs["y1"].data_ptr(), N, 1,
                                      0, stream), "gemv")
        ctx.check(lib.ggq_mul_mat_dev(ctx.h, dW.data_ptr(), 12, N, K, x4.data_ptr(), K, outs["y4"].data_ptr(), N, 4,
                                      0, stream), "gemv4")
        ctx.check(lib.ggq_mul_mat_dev(ctx.h, dW8.data_ptr(), 8, N8, K8, x8.data_ptr(), K8, outs["y8"].data_ptr(), N8,
                                      M8, 1, stream), "gemm")
        ctx.check(lib.ggq_attention_decode_dev(ctx.h, q.data_ptr(), Kc.data_ptr(), Vc.data_ptr(), 1, n_head, n_kv, hd,
                                               ctx_len, ctx_len - 1, outs["att"].data_ptr(), stream), "attention")
        ctx.check(lib.ggq_moe_ffn_dev(ctx.h, ctypes.byref(moe), stream), "moe")

    def fill(seed):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        for a in (x1, x4, x8, q, mx, ml):
            a.copy_(torch.randn(a.shape, device="cuda", generator=g))

    with torch.cuda.stream(s):
        fill(0)
        work(sh)            # eager warm-up: every workspace is sized here
        work(sh)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        work(sh)
    torch.cuda.synchronize()

    for rep in range(4):
        fill(100 + rep)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = {n: o.clone() for n, o in outs.items()}
        with torch.cuda.stream(s):
            work(sh)        # eager on the same inputs
        torch.cuda.synchronize()
        for n, o in outs.items():
            assert torch.equal(got[n].view(torch.int32), o.view(torch.int32)), (rep, n)
        if rep == 0:        # the eager results themselves meet the bar
            a1 = x1.cpu().numpy()
            assert orc.rel_l2(got["y1"].cpu().numpy(), orc.mul_mat_f64(12, raw, N, K, a1, 0)) < 1e-4
            a4 = x4.cpu().numpy()
            assert orc.rel_l2(got["y4"].cpu().numpy(), orc.mul_mat_f64(12, raw, N, K, a4, 0)) < 1e-4
            a8 = x8.cpu().numpy()
            assert orc.rel_l2(got["y8"].cpu().numpy(), orc.mul_mat_f64(8, raw8, N8, K8, a8, 1)) < 1e-4
