"""Seeded randomized parity sweep over the device entry points: shapes and
options that the targeted tests do not enumerate (odd N, K at and around
block boundaries, ragged batch rows, padded strides, mixed formats in one
level, MoE with unequal gate/up formats, attention shapes), each against the
fp64 oracle with the bar of the targeted tests (rel-L2 <= 1e-4, same
activation treatment)."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests import test_gpu_parity as t
from tests.gpu_util import dev, empty, host, ptr, stream_handle

pytestmark = pytest.mark.gpu
ctx = t.ctx
TOL = 1e-4
KQ = (12, 13, 14)          # Q4_K, Q5_K, Q6_K: K a multiple of 256
SMALL = (8, 20, 23)        # Q8_0, IQ4_NL (K % 32), IQ4_XS (K % 256)


def _rand_k(rng, ty):
    if ty in (8, 20):
        return int(32 * rng.integers(1, 100))   # includes odd block counts (simple kernel)
    return int(256 * rng.integers(1, 33))


@pytest.mark.parametrize("seed", range(48))
def test_sweep_mul_mat(ctx, orc, seed):
    rng = np.random.default_rng(1000 + seed)
    ty = int(rng.choice(KQ + SMALL))
    K = _rand_k(rng, ty)
    N = int(rng.integers(1, 300))
    M = int(rng.integers(1, 10))
    mode = int(rng.integers(0, 3)) if K % 32 == 0 else 0
    lda = K + int(rng.integers(0, 3)) * 4
    ldc = N + int(rng.integers(0, 4))
    raw = t.weights(ty, N, K, seed=seed)
    A = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10)).astype(np.float32)
    got = t.run_mm(ctx, ty, raw, N, K, A, mode, lda=lda, ldc=ldc)
    err = orc.rel_l2(got, orc.mul_mat_f64(ty, raw, N, K, A, mode))
    assert err < TOL, (ty, N, K, M, mode, lda, ldc, err)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_batched_level(ctx, orc, seed):
    """ggq_mul_mat_batch_dev with 2-5 matrices sharing one input; every
    third case uses only Q4_K / Q6_K (the level kernel compiled for those)."""
    import torch
    rng = np.random.default_rng(2000 + seed)
    n = int(rng.integers(2, 6))
    K = int(256 * rng.integers(1, 17))
    types = [int(rng.choice((12, 14))) if seed % 3 == 0 else int(rng.choice(KQ + (23,))) for _ in range(n)]
    A = rng.standard_normal((1, K)).astype(np.float32)
    dA = dev(A)
    descs = (gl.GemvDesc * n)()
    keep, outs, raws = [], [], []
    for i, ty in enumerate(types):
        N = int(rng.integers(1, 600))
        raw = t.weights(ty, N, K, seed=seed * 10 + i)
        dW = dev(raw)
        C = torch.full((1, N), float("nan"), device="cuda")
        keep.append(dW)
        outs.append(C)
        raws.append((ty, N, raw))
        descs[i].W, descs[i].type, descs[i].N, descs[i].K = dW.data_ptr(), ty, N, K
        descs[i].A, descs[i].C = dA.data_ptr(), C.data_ptr()
    ctx.check(ctx.lib.ggq_mul_mat_batch_dev(ctx.h, descs, n, stream_handle()), "batch")
    for (ty, N, raw), C in zip(raws, outs):
        err = orc.rel_l2(host(C), orc.mul_mat_f64(ty, raw, N, K, A, 0))
        assert err < TOL, (types, ty, N, K, err)


@pytest.mark.parametrize("seed", range(12))
def test_sweep_batch_act(ctx, orc, seed):
    """ggq_mul_mat_batch_act_dev over 1-5 matrices sharing one input of 1-8
    rows, fp32 or per-row int8 activations: the single-row int8 rows
    quantized inside the fp32 kernels (staged or in registers), the int8
    matrix-core GEMV, the matrix-core GEMV for several fp32 rows."""
    import torch
    rng = np.random.default_rng(4000 + seed)
    n = int(rng.integers(1, 6))
    K = int(256 * rng.integers(1, 33))
    M = 1 if seed % 2 == 0 else int(rng.integers(1, 9))
    mode = int(rng.integers(0, 2))
    A = (rng.standard_normal((M, K)) * rng.uniform(0.01, 100)).astype(np.float32)
    dA = dev(A)
    descs = (gl.GemvDesc * n)()
    keep, outs, raws = [], [], []
    for i in range(n):
        ty = int(rng.choice(KQ + SMALL))
        N = int(rng.integers(1, 500))
        raw = t.weights(ty, N, K, seed=seed * 10 + i)
        dW = dev(raw)
        C = torch.full((M, N), float("nan"), device="cuda")
        keep.append(dW)
        outs.append(C)
        raws.append((ty, N, raw))
        descs[i].W, descs[i].type, descs[i].N, descs[i].K = dW.data_ptr(), ty, N, K
        descs[i].A, descs[i].C = dA.data_ptr(), C.data_ptr()
    ctx.check(ctx.lib.ggq_mul_mat_batch_act_dev(ctx.h, descs, n, M, mode, stream_handle()), "batch act")
    for (ty, N, raw), C in zip(raws, outs):
        err = orc.rel_l2(host(C), orc.mul_mat_f64(ty, raw, N, K, A, mode))
        assert err < TOL, (ty, N, K, M, mode, err)


@pytest.mark.parametrize("seed", range(8))
def test_sweep_moe(ctx, orc, seed):
    """Random token counts, expert counts and top-k; gate / up formats equal
    (one paired launch) or different (two launches); with and without the
    shared expert."""
    rng = np.random.default_rng(3000 + seed)
    T = int(rng.integers(1, 21))
    E = int(rng.choice((8, 16, 32)))
    k = int(rng.integers(1, 5))
    H = int(rng.choice((256, 512)))
    F = int(rng.choice((256, 512)))
    tg = int(rng.choice((12, 13)))
    tu = tg if seed % 2 == 0 else int(rng.choice((12, 13, 14)))
    td = int(rng.choice((12, 14)))
    shared = bool(seed % 3)
    (out, sel, wsel), (x, logits, Wg, Wu, Wd, Sg, Su, Sd, sw) = t.run_moe(ctx, T, H, F, E, k, shared, seed=seed,
                                                                            tg=tg, tu=tu, td=td)
    ref, rsel, rw = orc.moe_ffn_f64(x, logits, H, F, E, k, tg, Wg, tu, Wu, td, Wd, Sg, Su, Sd, sw)
    assert np.array_equal(sel, rsel)
    assert np.allclose(wsel, rw, rtol=1e-6)
    assert orc.rel_l2(out, ref) < TOL, (T, E, k, H, F, tg, tu, td, shared)


@pytest.mark.parametrize("seed", range(10))
def test_sweep_attention(ctx, orc, seed):
    import torch
    rng = np.random.default_rng(4000 + seed)
    n_kv = int(rng.choice((1, 2, 4, 8)))
    G = int(rng.choice((1, 2, 4, 8)))
    n_head = n_kv * G
    hd = int(rng.choice((64, 128)))
    ctx_len = int(rng.integers(1, 1500))
    n_tok = int(rng.integers(1, 5))
    pos0 = int(rng.integers(0, ctx_len + 3))
    q = rng.standard_normal((n_tok, n_head, hd)).astype(np.float32)
    Kc = rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32)
    Vc = rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32)
    out = empty((n_tok, n_head, hd), torch.float32)
    dq, dk, dv = dev(q), dev(Kc), dev(Vc)
    ctx.check(ctx.lib.ggq_attention_decode_dev(ctx.h, ptr(dq), ptr(dk), ptr(dv), n_tok, n_head, n_kv, hd, ctx_len,
                                               pos0, ptr(out), stream_handle()), "attention")
    got = host(out)
    exp = orc.flash_attn(q, Kc, Vc, n_head, [pos0 + i for i in range(n_tok)], f64=True)
    for i in range(n_tok):
        for h in range(n_head):
            assert orc.rel_l2(got[i, h], exp[i, h]) <= TOL, (seed, i, h)
