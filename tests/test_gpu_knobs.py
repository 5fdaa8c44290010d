"""Parity of the rows-per-pass GEMV variants that the default launch
configuration does not select (GGQ_GEMV_MBCAP 2 / 4; GGQ_MOE_MB 1 / 4, the
grouped default being 2).  The
library reads these knobs at each multi-row / grouped launch, so the checks
set them in this process and restore them afterwards."""
import os

import pytest

from tests import test_gpu_parity as t

pytestmark = pytest.mark.gpu

ctx = t.ctx  # module-scoped context fixture


@pytest.fixture
def wide_rows(request):
    old = {k: os.environ.get(k) for k in ("GGQ_GEMV_MBCAP", "GGQ_MOE_MB")}
    os.environ["GGQ_GEMV_MBCAP"] = os.environ["GGQ_MOE_MB"] = request.param
    yield request.param
    for k, v in old.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


@pytest.mark.parametrize("wide_rows", ["2", "4"], indirect=True)
@pytest.mark.parametrize("M", [2, 3, 4, 8])
def test_batched_rows_wide(ctx, orc, wide_rows, M):
    t.test_batched_rows_gemv(ctx, orc, M)


@pytest.mark.parametrize("wide_rows", ["1", "2", "4"], indirect=True)
def test_moe_wide(ctx, orc, wide_rows):
    t.test_moe_small_vs_oracle(ctx, orc, True)
    t.test_moe_qwen35moe_shape_vs_oracle(ctx, orc)
