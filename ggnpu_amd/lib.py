"""ctypes binding of libggq_hip.so (include/ggq.h).

Loading fails loudly when the shared library has not been built: there is no
fallback implementation behind this module.
"""
import ctypes
import enum
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libggq_hip.so")


class Status(enum.IntEnum):
    """ggnpu Status (include/ggnpu/backend.h:12-19)."""
    OK = 0
    ERROR = 1
    NOT_FOUND = 2
    INVALID_PARAM = 3
    DEVICE_UNAVAILABLE = 4
    OUT_OF_MEMORY = 5


class GgmlType(enum.IntEnum):
    """GGML type ids (include/ggnpu/tensor.h:11-42) supported by the backend."""
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ4_NL = 20
    IQ4_XS = 23


class ActMode(enum.IntEnum):
    F32 = 0
    Q8_ROW = 1
    Q8_BLOCK32 = 2


# (values per block, bytes per block): src/gguf/tensor.cpp:18-38
BLOCK = {
    GgmlType.Q8_0: (32, 34),
    GgmlType.Q4_K: (256, 144),
    GgmlType.Q5_K: (256, 176),
    GgmlType.Q6_K: (256, 210),
    GgmlType.IQ4_NL: (32, 18),
    GgmlType.IQ4_XS: (256, 136),
}
GROUP_ELEMS = {t: (16 if t == GgmlType.Q6_K else 32) for t in BLOCK}


def row_bytes(t, K):
    be, bb = BLOCK[GgmlType(t)]
    return (K // be) * bb


class GgqError(RuntimeError):
    def __init__(self, status, message=""):
        self.status = Status(status)
        super().__init__(f"{self.status.name}: {message}")


class MoeParams(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_int), ("H", ctypes.c_int), ("F", ctypes.c_int), ("E", ctypes.c_int),
        ("top_k", ctypes.c_int),
        ("x", ctypes.c_void_p), ("router_logits", ctypes.c_void_p),
        ("gate_type", ctypes.c_uint32), ("up_type", ctypes.c_uint32), ("down_type", ctypes.c_uint32),
        ("gate_exps", ctypes.c_void_p), ("up_exps", ctypes.c_void_p), ("down_exps", ctypes.c_void_p),
        ("gate_shexp", ctypes.c_void_p), ("up_shexp", ctypes.c_void_p), ("down_shexp", ctypes.c_void_p),
        ("shared_w", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("sel_experts", ctypes.c_void_p), ("sel_weights", ctypes.c_void_p),
    ]


class GemvDesc(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("type", ctypes.c_uint32), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("A", ctypes.c_void_p), ("C", ctypes.c_void_p)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("N", ctypes.c_int64), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int)]


class MulMatParams(ctypes.Structure):
    """MulMatParams (include/ggnpu/backend.h:21-35)."""
    _fields_ = [
        ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("C", ctypes.c_void_p),
        ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int),
        ("lda", ctypes.c_int), ("ldb", ctypes.c_int), ("ldc", ctypes.c_int),
        ("n_batches", ctypes.c_int32), ("scales", ctypes.c_void_p),
        ("n_weight_scales", ctypes.c_int), ("B_type", ctypes.c_uint32),
    ]


_P, _I, _U32, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_int64

# Every function declared in include/ggq.h, with its ctypes signature.
SIGNATURES = {
    "ggq_create": (_I, [_I, ctypes.POINTER(_P)]),
    "ggq_destroy": (None, [_P]),
    "ggq_last_error": (_I, [_P]),
    "ggq_last_error_message": (ctypes.c_char_p, [_P]),
    "ggq_name": (ctypes.c_char_p, [_P]),
    "ggq_is_available": (_I, [_P]),
    "ggq_sync": (_I, [_P]),
    "ggq_mul_mat_q": (_I, [_P, ctypes.POINTER(MulMatParams), _I]),
    "ggq_weight_upload": (_I, [_P, _P, _U32, _I64, _I64, ctypes.POINTER(_P)]),
    "ggq_weight_free": (_I, [_P, _P]),
    "ggq_weight_device_ptr": (_P, [_P]),
    "ggq_mul_mat": (_I, [_P, _P, _P, _I, _P, _I, _I, _I]),
    "ggq_mul_mat_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _P, _I, _I, _I, _P]),
    "ggq_mul_mat_batch_dev": (_I, [_P, _P, _I, _P]),
    "ggq_mul_mat_batch_rows_dev": (_I, [_P, _P, _I, _I, _P]),
    "ggq_mul_mat_q8_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _P, _I, _P, _I, _P]),
    "ggq_mul_mat_q8_batch_dev": (_I, [_P, _P, _I, _U32, _I64, _P, _P, _I, _P]),
    "ggq_dequant_dev": (_I, [_P, _P, _U32, _I64, _P, _P]),
    "ggq_quantize_act_dev": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "ggq_block_dot_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _P, _P]),
    "ggq_moe_ffn_dev": (_I, [_P, ctypes.POINTER(MoeParams), _P]),
    "ggq_encode": (_I, [_U32, _P, _I64, _I64, _P]),
    "ggq_row_bytes": (_I64, [_U32, _I64]),
}

_lib = None


def load_library(path=LIB_PATH):
    """Load libggq_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None and path == LIB_PATH:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} not built: run `python -m ggnpu_amd.build`")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path == LIB_PATH:
        _lib = lib
    return lib


def encode(t, x):
    """Encode a float32 numpy array [rows][K] to raw GGUF blocks (numpy uint8)."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, K = x.shape
    out = np.empty(rows * row_bytes(t, K), dtype=np.uint8)
    st = load_library().ggq_encode(int(t), x.ctypes.data, rows, K, out.ctypes.data)
    if st != 0:
        raise GgqError(st, "ggq_encode")
    return out


class Context:
    """Owning handle of a ggq_ctx (one per device)."""

    def __init__(self, device=0):
        self.lib = load_library()
        h = ctypes.c_void_p()
        st = self.lib.ggq_create(device, ctypes.byref(h))
        if st != 0:
            raise GgqError(st, f"ggq_create(device={device})")
        self.h = h

    def close(self):
        if self.h:
            self.lib.ggq_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, st, what=""):
        if st != 0:
            msg = self.lib.ggq_last_error_message(self.h)
            raise GgqError(st, f"{what}: {msg.decode() if msg else ''}")

    def sync(self):
        self.check(self.lib.ggq_sync(self.h), "sync")
