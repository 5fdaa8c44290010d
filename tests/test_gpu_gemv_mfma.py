"""The matrix-core GEMV (several fp32 activation rows): each lane's decoded
codes (exact fp16 integers) against activations split into fp16 hi + lo
parts under a per-(row, piece) power-of-two scale, v_mfma_f32_4x4x4_16b_f16,
run scale and bias in fp32.  Checked against the fp64 oracle with the bar of
the other GEMV tests (rel-L2 <= 1e-4, GGQ_ACT_F32 treatment) over every
format, the three slot layouts (K/32 <= 16, <= 32, <= 64 pieces per row),
two pieces per lane (K/32 in 65..128), the fallback beyond that, row counts
that leave partial row sets, activation rows of very different magnitudes,
and against the fp32 FMA kernels (GGQ_GEMV_MFMA=0)."""
import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests import test_gpu_parity as t
from tests.gpu_util import dev, empty, host, ptr, stream_handle

pytestmark = pytest.mark.gpu
ctx = t.ctx
TOL = 1e-4
TYPES = (8, 12, 13, 14, 20, 23)


def _k_for(ty, pieces):
    be = 256 if ty in (12, 13, 14, 23) else 32
    k = pieces * 32
    return ((k + be - 1) // be) * be


@pytest.mark.parametrize("ty", TYPES)
@pytest.mark.parametrize("pieces", [8, 24, 64, 96, 200])
@pytest.mark.parametrize("M", [2, 4, 5, 8, 16, 64])
def test_mfma_gemv_matches_oracle(ctx, orc, ty, pieces, M):
    K = _k_for(ty, pieces)
    N = 4 * 37 + 3  # rows that leave a partial group of 4
    raw = t.weights(ty, N, K, seed=ty * 100 + pieces + M)
    A = np.random.default_rng(M + pieces).standard_normal((M, K)).astype(np.float32)
    got = t.run_mm(ctx, ty, raw, N, K, A, 0)
    err = orc.rel_l2(got, orc.mul_mat_f64(ty, raw, N, K, A, 0))
    assert err < TOL, (ty, K, M, err)


@pytest.mark.parametrize("ty", [12, 14, 8])
def test_mfma_gemv_row_magnitudes(ctx, orc, ty):
    """Rows scaled by 1e-30 .. 1e30 and a row with one large value among
    tiny ones: per row the result meets the bar (the split's scale follows
    each row and piece)."""
    K, N, M = 2048, 260, 6
    raw = t.weights(ty, N, K, seed=7)
    rng = np.random.default_rng(3)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[0] *= 1e-30
    A[1] *= 1e30
    A[2] *= 1e-3
    A[3, :] = rng.standard_normal(K).astype(np.float32) * 1e-6
    A[3, 100] = 1e4
    A[4] = 0.0
    got = t.run_mm(ctx, ty, raw, N, K, A, 0)
    ref = orc.mul_mat_f64(ty, raw, N, K, A, 0)
    for m in range(M):
        if m == 4:
            assert np.all(got[m] == 0.0)
            continue
        assert orc.rel_l2(got[m], ref[m]) < TOL, m


def test_mfma_gemv_same_as_fma_path(ctx, orc, monkeypatch):
    """Both formulations meet the bar on the same problem and agree with each
    other to the bar."""
    K, N, M = 3072, 1000, 8
    for ty in (12, 23, 13):
        raw = t.weights(ty, N, K, seed=ty)
        A = np.random.default_rng(ty).standard_normal((M, K)).astype(np.float32)
        got = t.run_mm(ctx, ty, raw, N, K, A, 0)
        monkeypatch.setenv("GGQ_GEMV_MFMA", "0")
        fma = t.run_mm(ctx, ty, raw, N, K, A, 0)
        monkeypatch.delenv("GGQ_GEMV_MFMA")
        ref = orc.mul_mat_f64(ty, raw, N, K, A, 0)
        assert orc.rel_l2(got, ref) < TOL and orc.rel_l2(fma, ref) < TOL
        assert orc.rel_l2(got, fma) < TOL


@pytest.mark.parametrize("M", [2, 4, 8])
def test_mfma_batch_rows_mixed_types(ctx, orc, M):
    """ggq_mul_mat_batch_rows_dev with mixed formats in one matrix-core launch
    (configs[3] pattern: IQ4_NL / IQ4_XS / Q5_K)."""
    import torch
    rng = np.random.default_rng(M)
    shapes = [(20, 2048, 1024), (23, 1024, 1024), (13, 1024, 1024)]
    descs = (gl.GemvDesc * len(shapes))()
    keep, refs = [], []
    for i, (ty, N, K) in enumerate(shapes):
        raw = t.weights(ty, N, K, seed=i + 50 * M)
        A = rng.standard_normal((M, K)).astype(np.float32)
        dW, dA = dev(raw), dev(A)
        dC = torch.full((M, N), float("nan"), device="cuda")
        keep += [dW, dA, dC]
        descs[i].W, descs[i].type, descs[i].N, descs[i].K = dW.data_ptr(), ty, N, K
        descs[i].A, descs[i].C = dA.data_ptr(), dC.data_ptr()
        refs.append((dC, orc.mul_mat_f64(ty, raw, N, K, A, 0)))
    ctx.check(ctx.lib.ggq_mul_mat_batch_rows_dev(ctx.h, descs, len(shapes), M, stream_handle()), "batch rows")
    for dC, ref in refs:
        assert orc.rel_l2(host(dC), ref) < TOL


@pytest.mark.parametrize("ty", [12, 20, 14])
@pytest.mark.parametrize("lda_pad,ldc_pad", [(3, 1), (1, 0)])
def test_mfma_gemv_odd_strides(ctx, orc, ty, lda_pad, ldc_pad):
    """Activation rows at a stride that is not a multiple of 4 floats (the
    kernel's scalar activation loads) and padded output rows."""
    K, N, M = 1024 if ty != 14 else 2048, 200, 6
    raw = t.weights(ty, N, K, seed=lda_pad + ty)
    A = np.random.default_rng(ty).standard_normal((M, K)).astype(np.float32)
    got = t.run_mm(ctx, ty, raw, N, K, A, 0, lda=K + lda_pad, ldc=N + ldc_pad)
    assert orc.rel_l2(got, orc.mul_mat_f64(ty, raw, N, K, A, 0)) < TOL
