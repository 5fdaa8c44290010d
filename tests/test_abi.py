"""C ABI checks that need no GPU: the library loads, exports exactly what
include/ggq.h and include/ggq_gguf.h declare, rejects bad arguments, and the synthetic-data
encoder produces valid blocks."""
import os
import re

import numpy as np
import pytest

import ggnpu_amd.lib as gl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = set()
    for h in ("ggq.h", "ggq_gguf.h"):
        txt = open(os.path.join(ROOT, "include", h)).read()
        txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
        names |= set(re.findall(r"\b(ggq_[a-z0-9_]+)\s*\(", txt))
    return names


def test_library_exports_every_declared_symbol():
    lib = gl.load_library()
    declared = header_functions()
    assert declared == set(gl.SIGNATURES), declared ^ set(gl.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name)


def test_row_bytes_and_invalid_types():
    lib = gl.load_library()
    assert lib.ggq_row_bytes(12, 2048) == 8 * 144
    assert lib.ggq_row_bytes(14, 8192) == 32 * 210
    assert lib.ggq_row_bytes(8, 1536) == 48 * 34
    assert lib.ggq_row_bytes(12, 100) == 0      # not a multiple of 256
    assert lib.ggq_row_bytes(2, 256) == 0       # Q4_0 unsupported


def test_null_context_is_invalid_param():
    lib = gl.load_library()
    assert lib.ggq_sync(None) == gl.Status.INVALID_PARAM
    assert lib.ggq_mul_mat_dev(None, None, 12, 8, 256, None, 256, None, 8, 1, 0, None) == gl.Status.INVALID_PARAM


def test_encode_rejects_bad_shapes():
    lib = gl.load_library()
    x = np.zeros(100, np.float32)
    out = np.zeros(1000, np.uint8)
    assert lib.ggq_encode(12, x.ctypes.data, 1, 100, out.ctypes.data) == gl.Status.INVALID_PARAM
    assert lib.ggq_encode(3, x.ctypes.data, 1, 32, out.ctypes.data) == gl.Status.INVALID_PARAM


# Worst-case relative reconstruction error of the simple encoders on N(0,1)
# rows (a sanity bound, not a parity claim: parity is on the bytes).
ENC_BOUND = {8: 0.02, 12: 0.15, 13: 0.08, 14: 0.05, 20: 0.15, 23: 0.15}


@pytest.mark.parametrize("t", sorted(ENC_BOUND))
def test_encoder_roundtrip_and_field_ranges(orc, t):
    rng = np.random.default_rng(t)
    be, bb = gl.BLOCK[gl.GgmlType(t)]
    x = (rng.standard_normal((8, 1024)) * 0.02).astype(np.float32)
    raw = gl.encode(t, x)
    assert raw.size == 8 * (1024 // be) * bb
    y = orc.dequant(t, raw).reshape(8, 1024)
    assert np.all(np.isfinite(y))
    assert orc.rel_l2(y, x) < ENC_BOUND[t]
    # deterministic
    assert np.array_equal(gl.encode(t, x), raw)


def test_create_without_device_reports_unavailable():
    """On a host with no GPU ggq_create must fail cleanly (no crash)."""
    import ctypes
    lib = gl.load_library()
    h = ctypes.c_void_p()
    st = lib.ggq_create(9999, ctypes.byref(h))
    assert st == gl.Status.DEVICE_UNAVAILABLE and not h.value
