"""Parity of the GEMV variants that the default launch configuration does
not select: the fp32 FMA kernels for several rows (GGQ_GEMV_MFMA=0) with
GGQ_GEMV_MBCAP 2 / 4; GGQ_MOE_MB 1 / 4 (the grouped default being 2); the
matrix-core kernel with 8 rows per pass (GGQ_GEMV_MFMA_MS=2) and for a
single row (GGQ_GEMV_MFMA1=1); its fp16 hi + lo products for plain batches
and fp32 products for expert groups (GGQ_GEMV_MFMA32=0 / 1), and its
activation rows read per wavefront instead of staged in LDS
(GGQ_GEMV_MFMA_XL=0); per-row int8 decode without the int8
matrix-core GEMV (GGQ_GEMV_I8=0: quantize, dequantize, fp32 kernel) and
fp32 launches of every size on it (GGQ_I8_MIN_BYTES=0); single per-row
int8 rows on it rather than quantized in the fp32 kernel's staging
(GGQ_GEMV_Q8XL=0).  The
library reads these knobs at each multi-row / grouped launch, so the checks
set them in this process and restore them afterwards."""
import os

import pytest

from tests import test_gpu_parity as t

pytestmark = pytest.mark.gpu

ctx = t.ctx  # module-scoped context fixture


def _set_env(values):
    old = {k: os.environ.get(k) for k in values}
    os.environ.update(values)
    return old


def _restore(old):
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


@pytest.fixture
def wide_rows(request):
    old = _set_env({"GGQ_GEMV_MBCAP": request.param, "GGQ_MOE_MB": request.param, "GGQ_GEMV_MFMA": "0"})
    yield request.param
    _restore(old)


@pytest.fixture
def mfma_knob(request):
    name, value = request.param
    old = _set_env({name: value})
    yield request.param
    _restore(old)


@pytest.mark.parametrize("wide_rows", ["2", "4"], indirect=True)
@pytest.mark.parametrize("M", [2, 3, 4, 8])
def test_batched_rows_wide(ctx, orc, wide_rows, M):
    t.test_batched_rows_gemv(ctx, orc, M)


@pytest.mark.parametrize("wide_rows", ["1", "2", "4"], indirect=True)
def test_moe_wide(ctx, orc, wide_rows):
    t.test_moe_small_vs_oracle(ctx, orc, True)
    t.test_moe_qwen35moe_shape_vs_oracle(ctx, orc)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_MFMA_MS", "2")], indirect=True)
@pytest.mark.parametrize("M", [5, 8, 9, 16])
def test_mfma_eight_rows_per_pass(ctx, orc, mfma_knob, M):
    t.test_batched_rows_gemv(ctx, orc, M)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_MFMA32", "0"), ("GGQ_GEMV_MFMA_XL", "0")],
                         indirect=True)
@pytest.mark.parametrize("M", [2, 5, 8, 16])
def test_mfma_product_and_staging(ctx, orc, mfma_knob, M):
    t.test_batched_rows_gemv(ctx, orc, M)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_MFMA32", "1")], indirect=True)
def test_moe_fp32_products(ctx, orc, mfma_knob):
    t.test_moe_small_vs_oracle(ctx, orc, True)
    t.test_moe_qwen35moe_shape_vs_oracle(ctx, orc)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_MFMA1", "1")], indirect=True)
@pytest.mark.parametrize("ty", [8, 12, 13, 14, 20, 23])
def test_mfma_single_row(ctx, orc, mfma_knob, ty):
    """One activation row through the matrix-core kernel (one and two pieces
    per lane) against the fp64 oracle."""
    import numpy as np
    for K in (1024, 4096):
        N = 333
        raw = t.weights(ty, N, K, seed=ty + K)
        A = np.random.default_rng(K).standard_normal((1, K)).astype(np.float32)
        got = t.run_mm(ctx, ty, raw, N, K, A, 0)
        assert orc.rel_l2(got, orc.mul_mat_f64(ty, raw, N, K, A, 0)) < t.TOL, (ty, K)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_MFMA", "0")], indirect=True)
@pytest.mark.parametrize("ty", [12, 14, 20])
def test_fma_path_batch_invariant(ctx, orc, mfma_knob, ty):
    """On the FMA kernels every row of a batch equals the same row computed
    alone, bit for bit."""
    import numpy as np
    K, N = 2048, 300
    raw = t.weights(ty, N, K, seed=ty)
    A = np.random.default_rng(ty).standard_normal((8, K)).astype(np.float32)
    for M in (4, 8):
        batch = t.run_mm(ctx, ty, raw, N, K, A[:M], 0)
        for m in range(M):
            alone = t.run_mm(ctx, ty, raw, N, K, A[m:m + 1], 0)
            assert np.array_equal(batch[m].view(np.uint32), alone[0].view(np.uint32)), (M, m)


@pytest.mark.parametrize("mfma_knob", [("GGQ_GEMV_I8", "0"), ("GGQ_I8_MIN_BYTES", "0"), ("GGQ_GEMV_Q8XL", "0")],
                         indirect=True)
@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q8_0", "IQ4_XS"])
def test_i8_gemv_switches(ctx, orc, mfma_knob, name):
    for M in (1, 3):
        t.test_gemv_f32_vs_oracle(ctx, orc, name, M)
    t.test_gemv_q8_act_vs_oracle(ctx, orc, name, 1)
