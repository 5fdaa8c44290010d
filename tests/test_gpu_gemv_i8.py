"""The decode GEMV on the int8 matrix cores (ggq_gemv_i8.hip), reached
through the C ABI for 1..8 activation rows and K a multiple of 256:

* fp32 activations (exact 3-digit fixed point): every format, 1..4 rows,
  ragged N, long K, strided and unaligned activation rows, extreme and mixed
  magnitudes, against the fp64 oracle (rel-L2 <= 1e-4);
* GGQ_ACT_Q8_ROW (codes quantized per row inside the kernel) and the
  pre-quantized entry point (ggq_mul_mat_q8_dev), 1..8 rows: the two agree
  bit for bit and meet the bar against the oracle's Q8_ROW treatment;
* several problems of mixed formats in one launch (ggq_mul_mat_batch_dev);
* every split of a tile's K over wavefronts (GGQ_I8_KW, read per launch);
* the fused options (RMSNorm prologue, product input, silu epilogue,
  residual add) through ggq_mul_mat_fused_dev.
"""
import ctypes
import os

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests.gpu_util import dev, empty, host, ptr, stream_handle
from tests.test_gpu_parity import TYPES, TOL, ctx, run_mm, weights  # noqa: F401

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _every_size(monkeypatch):
    # fp32 launches of any size take the matrix-core path here
    monkeypatch.setenv("GGQ_I8_MIN_BYTES", "0")


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_i8_gemv_f32_all_formats(ctx, orc, name, M):
    t = TYPES[name]
    for N, K in ((700, 256), (33, 2048), (16, 1024)):
        raw = weights(t, N, K, seed=N + K + t)
        A = np.random.default_rng(M * 7 + t).standard_normal((M, K)).astype(np.float32)
        got = run_mm(ctx, t, raw, N, K, A, 0)
        err = orc.rel_l2(got, orc.mul_mat_f64(t, raw, N, K, A, 0))
        assert err < TOL, (name, M, N, K, err)


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q8_0"])
def test_i8_gemv_long_k_and_strides(ctx, orc, name):
    t = TYPES[name]
    N, K = 300, 8960 if name == "Q8_0" else 8192
    raw = weights(t, N, K, seed=3 + t)
    A = np.random.default_rng(t).standard_normal((2, K)).astype(np.float32)
    for lda, ldc in ((K, N), (K + 3, N + 5)):  # unaligned rows take the scalar loads
        got = run_mm(ctx, t, raw, N, K, A, 0, lda=lda, ldc=ldc)
        assert orc.rel_l2(got, orc.mul_mat_f64(t, raw, N, K, A, 0)) < TOL, (lda, ldc)


@pytest.mark.parametrize("name", list(TYPES))
def test_i8_gemv_magnitudes(ctx, orc, name):
    """Rows of 1e-30, 1e30, mixed magnitudes inside one row, a zero row and a
    row with one non-zero value: the per-row power of two keeps 22 bits
    relative to the row maximum."""
    t = TYPES[name]
    N, K = 64, 512
    raw = weights(t, N, K, seed=9)
    rng = np.random.default_rng(9)
    rows = [rng.standard_normal(K) * 1e-30, rng.standard_normal(K) * 1e30,
            rng.standard_normal(K) * np.where(rng.random(K) < 0.5, 1e-3, 1e3), np.zeros(K)]
    one = np.zeros(K); one[77] = -3.5
    rows.append(one)
    for r in rows:
        A = r[None, :].astype(np.float32)
        got = run_mm(ctx, t, raw, N, K, A, 0)
        ref = orc.mul_mat_f64(t, raw, N, K, A, 0)
        if not np.any(ref):
            assert not np.any(got)
        else:
            assert orc.rel_l2(got, ref) < TOL


@pytest.mark.parametrize("name", list(TYPES))
@pytest.mark.parametrize("M", [1, 2, 5, 8])
def test_i8_gemv_q8_row_and_prequantized(ctx, orc, name, M):
    import torch
    t = TYPES[name]
    if t == 14 and M > 4:
        pytest.skip("Q6_K: up to 4 rows per launch on this path (more take the fp32 route)")
    N, K = 200, 1536 if name in ("Q8_0", "IQ4_NL") else 2048
    raw = weights(t, N, K, seed=M + t)
    A = np.random.default_rng(M + 100 * t).standard_normal((M, K)).astype(np.float32)
    got = run_mm(ctx, t, raw, N, K, A, 1)
    assert orc.rel_l2(got, orc.mul_mat_f64(t, raw, N, K, A, 1)) < TOL
    # quantize, then the pre-quantized entry point: the same codes, the same sums
    dA, dW = dev(A), dev(raw)
    q = empty((M, K), torch.int8)
    sa = empty((M,), torch.float32)
    ctx.check(ctx.lib.ggq_quantize_act_dev(ctx.h, ptr(dA), K, M, K, 1, ptr(q), ptr(sa), stream_handle()), "quant")
    C = empty((M, N), torch.float32)
    ctx.check(ctx.lib.ggq_mul_mat_q8_dev(ctx.h, ptr(dW), t, N, K, ptr(q), ptr(sa), M, ptr(C), N, stream_handle()),
              "q8_dev")
    assert np.array_equal(host(C).view(np.uint32), got.view(np.uint32))


def test_i8_gemv_batch_mixed_formats(ctx, orc):
    """One launch over problems of different formats, K and N (the decode
    step's q/k/v level shape, plus IQ4 / Q5_K / Q8_0 members)."""
    import torch
    specs = [(12, 2048, 2048), (12, 512, 2048), (14, 512, 2048), (23, 100, 1024), (13, 70, 512), (8, 333, 1536)]
    for M in (1, 2):
        rng = np.random.default_rng(M)
        keep, descs, ref = [], (gl.GemvDesc * len(specs))(), []
        for i, (t, N, K) in enumerate(specs):
            raw = weights(t, N, K, seed=50 + i)
            A = rng.standard_normal((M, K)).astype(np.float32)
            dW, dA = dev(raw), dev(A)
            dC = torch.full((M, N), float("nan"), device="cuda")
            keep += [dW, dA, dC]
            descs[i].W, descs[i].type, descs[i].N, descs[i].K = dW.data_ptr(), t, N, K
            descs[i].A, descs[i].C = dA.data_ptr(), dC.data_ptr()
            ref.append((t, raw, N, K, A, dC))
        ctx.check(ctx.lib.ggq_mul_mat_batch_rows_dev(ctx.h, descs, len(specs), M, stream_handle()), "batch")
        for t, raw, N, K, A, dC in ref:
            assert orc.rel_l2(host(dC), orc.mul_mat_f64(t, raw, N, K, A, 0)) < TOL, (t, N, K, M)


@pytest.mark.parametrize("kw", ["1", "2", "4", "16"])
def test_i8_gemv_k_splits(ctx, orc, kw, monkeypatch):
    monkeypatch.setenv("GGQ_I8_KW", kw)
    for t, N, K in ((12, 2048, 8192), (14, 96, 4096), (8, 40, 2560)):
        raw = weights(t, N, K, seed=int(kw) + t)
        A = np.random.default_rng(int(kw)).standard_normal((2, K)).astype(np.float32)
        for mode in (0, 1):
            got = run_mm(ctx, t, raw, N, K, A, mode)
            assert orc.rel_l2(got, orc.mul_mat_f64(t, raw, N, K, A, mode)) < TOL, (kw, t, mode)


@pytest.mark.parametrize("M", [1, 3, 8])
def test_batch_act_q8_row(ctx, orc, M):
    """ggq_mul_mat_batch_act_dev in GGQ_ACT_Q8_ROW: each entry meets the bar
    against the oracle's per-row int8 treatment, whether the level runs as
    one int8 launch or (a Q6_K entry above 4 rows, K not a multiple of 256)
    entry by entry; and it equals ggq_mul_mat_batch_rows_dev in GGQ_ACT_F32."""
    import torch
    specs = [(12, 2048, 2048), (14, 512, 2048), (20, 300, 1024), (8, 96, 96)]
    rng = np.random.default_rng(M)
    keep, descs, ref = [], (gl.GemvDesc * len(specs))(), []
    for i, (t, N, K) in enumerate(specs):
        raw = weights(t, N, K, seed=70 + i)
        A = rng.standard_normal((M, K)).astype(np.float32)
        dW, dA = dev(raw), dev(A)
        dC = torch.full((M, N), float("nan"), device="cuda")
        keep += [dW, dA, dC]
        descs[i].W, descs[i].type, descs[i].N, descs[i].K = dW.data_ptr(), t, N, K
        descs[i].A, descs[i].C = dA.data_ptr(), dC.data_ptr()
        ref.append((t, raw, N, K, A, dC))
    for mode in (1, 0):
        ctx.check(ctx.lib.ggq_mul_mat_batch_act_dev(ctx.h, descs, len(specs), M, mode, stream_handle()), "batch act")
        for t, raw, N, K, A, dC in ref:
            assert orc.rel_l2(host(dC), orc.mul_mat_f64(t, raw, N, K, A, mode)) < TOL, (t, N, K, M, mode)
    f32 = [host(r[5]).copy() for r in ref]
    ctx.check(ctx.lib.ggq_mul_mat_batch_rows_dev(ctx.h, descs, len(specs), M, stream_handle()), "batch rows")
    for r, y in zip(ref, f32):
        assert np.array_equal(host(r[5]).view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("M", [1, 2, 3])
@pytest.mark.parametrize("K", [1024, 2048, 8192])
def test_i8_fused_rmsnorm_and_residual(ctx, orc, M, K):
    """The fused options on the int8 matrix-core GEMV (every launch of any
    size takes it here): RMSNorm prologue (one row's sum of squares over the
    workgroup) on q/k/v-like entries and a residual add in place."""
    from tests.test_gpu_parity import test_fused_rmsnorm_qkv_and_residual
    test_fused_rmsnorm_qkv_and_residual(ctx, orc, M, K)


@pytest.mark.parametrize("t,K", [(14, 8192), (23, 1024), (13, 3072), (12, 2048)])
def test_i8_fused_swiglu(ctx, orc, t, K):
    """silu epilogue next to a plain entry, then the product input with and
    without the residual, on the int8 matrix-core GEMV."""
    from tests.test_gpu_parity import test_fused_swiglu
    test_fused_swiglu(ctx, orc, t, K)


def test_i8_fused_unaligned_and_default_norm(ctx, orc):
    """RMSNorm without weights (norm_w null) and with weights, on activation
    rows that are not 16-byte aligned (the scalar loads), against the
    oracle."""
    import torch
    from tests.test_gpu_parity import _fused_ref
    M, N, K = 2, 200, 2048
    rng = np.random.default_rng(5)
    A = (rng.standard_normal((M, K)) * 3.0).astype(np.float32)
    raw = weights(12, N, K, seed=5)
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    dW = dev(raw)
    Abuf = torch.zeros(M * K + 1, device="cuda")
    Av = Abuf[1:].view(M, K)
    Av.copy_(torch.from_numpy(A))
    nbuf = torch.from_numpy(nw).cuda()
    for norm in (None, nbuf):
        d = (gl.GemvFusedDesc * 1)()
        C = torch.full((M, N), float("nan"), device="cuda")
        d[0].W, d[0].type, d[0].N, d[0].K = dW.data_ptr(), 12, N, K
        d[0].A, d[0].C = Av.data_ptr(), C.data_ptr()
        d[0].rms_norm, d[0].rms_eps = 1, 1e-5
        if norm is not None:
            d[0].rms_w = norm.data_ptr()
        ctx.check(ctx.lib.ggq_mul_mat_fused_dev(ctx.h, d, 1, M, stream_handle()), "fused")
        ref = _fused_ref(orc, dict(A=A, type=12, W=raw, N=N, K=K, rms=True, eps=1e-5,
                                   rms_w=None if norm is None else nw), M)
        assert orc.rel_l2(host(C), ref) < TOL


def test_i8_gemv_f32_fixed_point_bound(ctx, orc, monkeypatch):
    """The worst case of the fixed point that carries fp32 activations on
    the int8 matrix cores: X = rint(x 2^e) with the row's largest magnitude
    in [2^21, 2^22), so |x - X 2^-e| <= 2^-22 max|x| for every value and
    |y_n - y_n(exact)| <= 2^-22 max|x| sum_k |w_nk| per output (plus fp32
    rounding).  The case: one 1e4 outlier whose weight column is zero and
    1e-3 values elsewhere, so the outputs rest entirely on values below the
    fixed-point step; the int8 path stays within that bound (and, as the
    bound allows, far from these small outputs).  The fp32 FMA kernel that
    launches of this size take by default folds each block's code bias into
    a run sum (a sum(x u) + b sum(x), Q8_0: b = -128 d), so its rounding is
    relative to sum |x| (|w| + 128 d) over the row: the same case costs it
    precision too, within that bound (2^-21 covers the two sums' roundings)."""
    t, N, K, j = TYPES["Q8_0"], 64, 4096, 777
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[:, j] = 0.0
    raw = gl.encode(t, w)
    x = (rng.standard_normal((1, K)) * 1e-3).astype(np.float32)
    x[0, j] = 1e4
    ref = orc.mul_mat_f64(t, raw, N, K, x, 0)
    wd = orc.dequant(t, raw).reshape(N, K).astype(np.float64)
    assert np.all(wd[:, j] == 0.0)
    slack = 1e-6 * np.abs(ref[0])
    bound_i8 = 2.0 ** -22 * 1e4 * np.abs(wd).sum(axis=1) + slack
    got = run_mm(ctx, t, raw, N, K, x, 0)  # GGQ_I8_MIN_BYTES=0: the int8 matrix cores
    assert np.all(np.abs(got[0] - ref[0]) <= bound_i8), np.max(np.abs(got[0] - ref[0]) / bound_i8)
    scales = np.frombuffer(raw.reshape(N, K // 32, 34)[:, :, :2].tobytes(), dtype=np.float16).astype(np.float64)
    bias = 128.0 * np.abs(np.repeat(scales.reshape(N, K // 32), 32, axis=1))
    bound_fma = 2.0 ** -21 * (np.abs(x[0]).astype(np.float64) * (np.abs(wd) + bias)).sum(axis=1) + slack
    monkeypatch.setenv("GGQ_I8_MIN_BYTES", str(16 << 20))  # the default: the fp32 FMA kernel
    got = run_mm(ctx, t, raw, N, K, x, 0)
    assert np.all(np.abs(got[0] - ref[0]) <= bound_fma), np.max(np.abs(got[0] - ref[0]) / bound_fma)
