"""Tuning variables read once per process (GGQ_GEMV_U, GGQ_GEMV_PREFETCH,
GGQ_GEMV_MAXLPR, GGQ_GEMV_BLOCKS, GGQ_GEMM_TILE, GGQ_GEMM_PF, GGQ_GEMV_XLDS): each setting
runs tests/knob_check.py (GEMV and prefill GEMM parity against the fp64
oracle) in one child process, one after another."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("env", [
    {"GGQ_GEMV_U": "2"}, {"GGQ_GEMV_U": "4"}, {"GGQ_GEMV_PREFETCH": "0"},
    {"GGQ_GEMV_MAXLPR": "64"}, {"GGQ_GEMV_MAXLPR": "128"}, {"GGQ_GEMV_BLOCKS": "37"},
    {"GGQ_GEMM_TILE": "128"}, {"GGQ_GEMM_PF": "1"}, {"GGQ_GEMM_PF": "4"}, {"GGQ_GEMV_XLDS": "0"},
], ids=lambda e: ",".join(f"{k}={v}" for k, v in e.items()))
def test_process_knob(env):
    full = dict(os.environ, GGQ_GEMV_MFMA="0", **env)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "knob_check.py")], env=full,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, (env, r.stdout[-2000:], r.stderr[-2000:])
