"""Parity of the kernel routes that the default launch configuration does not
select at the tests' shapes, reached through the library's remaining
path-selection variables (read at every launch, so the checks set them in
this process and restore them afterwards):

  GGQ_GEMV_MFMA=0      several activation rows on the fp32 FMA kernels (one
                       row per pass; the route of fused launches and of
                       K > 4096) instead of the matrix-core GEMV, plain and
                       expert-grouped;
  GGQ_I8_MIN_BYTES=0   fp32 and per-row int8 decode launches of every size on
                       the int8 matrix-core GEMV (by default only launches of
                       16 MB or more of weights).

GGQ_MOE_I8, GGQ_MOE_I8_GX, GGQ_MOE_I8_KW and GGQ_I8_KW (grouped int8 GEMV
decompositions) are exercised in test_gpu_parity.py, GGQ_MOE_GEMV_MAX_AVG in
test_gpu_parity.py and test_gpu_moe_stages.py, GGQ_ATTN_SPANS in
test_gpu_attention.py."""
import os

import pytest

from tests import test_gpu_parity as t

pytestmark = pytest.mark.gpu

ctx = t.ctx  # module-scoped context fixture


@pytest.fixture
def knob(request):
    name, value = request.param
    old = os.environ.get(name)
    os.environ[name] = value
    yield request.param
    if old is None:
        os.environ.pop(name, None)
    else:
        os.environ[name] = old


@pytest.mark.parametrize("knob", [("GGQ_GEMV_MFMA", "0")], indirect=True)
@pytest.mark.parametrize("M", [2, 3, 4, 8])
def test_batched_rows_fma(ctx, orc, knob, M):
    t.test_batched_rows_gemv(ctx, orc, M)


@pytest.mark.parametrize("knob", [("GGQ_GEMV_MFMA", "0")], indirect=True)
def test_moe_fma(ctx, orc, knob, monkeypatch):
    monkeypatch.setenv("GGQ_MOE_GEMV_MAX_AVG", "100000")
    t.test_moe_small_vs_oracle(ctx, orc, True)
    t.test_moe_qwen35moe_shape_vs_oracle(ctx, orc)


@pytest.mark.parametrize("knob", [("GGQ_GEMV_MFMA", "0")], indirect=True)
@pytest.mark.parametrize("ty", [12, 14, 20])
def test_fma_path_batch_invariant(ctx, orc, knob, ty):
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


@pytest.mark.parametrize("knob", [("GGQ_I8_MIN_BYTES", "0")], indirect=True)
@pytest.mark.parametrize("name", ["Q4_K", "Q6_K", "Q8_0", "IQ4_XS"])
def test_i8_gemv_all_sizes(ctx, orc, knob, name):
    for M in (1, 3):
        t.test_gemv_f32_vs_oracle(ctx, orc, name, M)
    t.test_gemv_q8_act_vs_oracle(ctx, orc, name, 1)
