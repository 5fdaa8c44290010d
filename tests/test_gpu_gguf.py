"""Weights read from a GGUF file (include/ggq_gguf.h) and uploaded unchanged
with ggq_gguf_upload, then multiplied on the GPU: same results as the
oracle on the bytes the file holds.  The expert tensor [K][N][E] arrives as
E matrices back to back (checked through the bit-exact dequant)."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from ggnpu_amd import gguf_writer as gw
from tests.gpu_util import empty, host, stream_handle

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    import torch
    # torch (its own HIP runtime) must see the device before this library's
    # runtime initializes it in the same process.
    assert torch.cuda.is_available()
    c = gl.Context(0)
    yield c
    c.close()


def _enc(t, N, K, seed):
    rng = np.random.default_rng(seed)
    return gl.encode(t, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))


def test_gguf_upload_and_matmul(ctx, orc, tmp_path):
    import torch
    K, E = 1024, 4
    tensors = [("blk.0.attn_q.weight", 12, [K, 96]), ("blk.0.ffn_down.weight", 14, [K, 64]),
               ("blk.0.attn_v.weight", 8, [K, 40]), ("blk.0.attn_k.weight", 23, [K, 33]),
               ("blk.0.ffn_up_exps.weight", 20, [K, 16, E])]
    raws = {}
    entries = []
    for i, (name, t, dims) in enumerate(tensors):
        N = int(np.prod(dims[1:]))
        raws[name] = _enc(t, N, K, seed=i + 3)
        entries.append((name, t, dims, raws[name].tobytes()))
    entries.append(("blk.0.attn_norm.weight", 0, [K], np.ones(K, np.float32).tobytes()))
    path = tmp_path / "w.gguf"
    gw.write(path, [("general.architecture", gw.STRING, "llama")], entries, alignment=64)
    A = np.random.default_rng(1).standard_normal((3, K)).astype(np.float32)
    with gl.GgufFile(path) as g:
        for name, t, dims in tensors:
            N = int(np.prod(dims[1:]))
            w = ctypes.c_void_p()
            ctx.check(g.lib.ggq_gguf_upload(ctx.h, g.h, name.encode(), ctypes.byref(w)), name)
            for mode in (gl.ActMode.F32, gl.ActMode.Q8_ROW):
                C = np.zeros((3, N), np.float32)
                ctx.check(ctx.lib.ggq_mul_mat(ctx.h, w, A.ctypes.data, K, C.ctypes.data, N, 3, int(mode)), name)
                assert orc.rel_l2(C, orc.mul_mat_f64(t, raws[name], N, K, A, int(mode))) < TOL, (name, mode)
            if len(dims) == 3:
                nb = N * K // gl.BLOCK[gl.GgmlType(t)][0]
                out = empty(N * K, torch.float32)
                ctx.check(ctx.lib.ggq_dequant_dev(ctx.h, ctx.lib.ggq_weight_device_ptr(w), t, nb,
                                                  ctypes.c_void_p(out.data_ptr()), stream_handle()), "deq")
                exp = orc.dequant(t, raws[name])
                assert np.array_equal(host(out).view(np.uint32), exp.view(np.uint32))
            ctx.check(ctx.lib.ggq_weight_free(ctx.h, w), "free")
        w = ctypes.c_void_p()
        assert g.lib.ggq_gguf_upload(ctx.h, g.h, b"blk.0.attn_norm.weight", ctypes.byref(w)) == gl.Status.INVALID_PARAM
        assert g.lib.ggq_gguf_upload(ctx.h, g.h, b"missing", ctypes.byref(w)) == gl.Status.NOT_FOUND
