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


class Producer(enum.IntEnum):
    RMS_NORM = 1
    SWIGLU = 2


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


class MoeTrace(ctypes.Structure):
    """ggq_moe_trace (include/ggq.h)."""
    _fields_ = [
        ("act_mode", ctypes.c_int), ("T", ctypes.c_int), ("H", ctypes.c_int), ("F", ctypes.c_int),
        ("E", ctypes.c_int), ("top_k", ctypes.c_int), ("rows", ctypes.c_int), ("shared", ctypes.c_int),
        ("grp", ctypes.c_void_p), ("tok", ctypes.c_void_p), ("pos", ctypes.c_void_p),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("h", ctypes.c_void_p),
        ("h_codes", ctypes.c_void_p), ("h_scales", ctypes.c_void_p),
        ("down", ctypes.c_void_p), ("down_shared", ctypes.c_void_p),
    ]


class GemvDesc(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("type", ctypes.c_uint32), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("A", ctypes.c_void_p), ("C", ctypes.c_void_p)]


class GemmDesc(ctypes.Structure):
    _fields_ = [("W", ctypes.c_void_p), ("N", ctypes.c_int64), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int)]


class GemvFusedDesc(ctypes.Structure):
    """ggq_gemv_fused_desc (include/ggq.h)."""
    _fields_ = [("W", ctypes.c_void_p), ("type", ctypes.c_uint32), ("N", ctypes.c_int64), ("K", ctypes.c_int64),
                ("A", ctypes.c_void_p), ("A_up", ctypes.c_void_p), ("C", ctypes.c_void_p),
                ("residual", ctypes.c_void_p), ("rms_w", ctypes.c_void_p), ("rms_norm", ctypes.c_int),
                ("rms_eps", ctypes.c_float), ("silu", ctypes.c_int)]


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
    "ggq_reserve": (_I, [_P, _I64]),
    "ggq_mul_mat_q": (_I, [_P, ctypes.POINTER(MulMatParams), _I]),
    "ggq_weight_upload": (_I, [_P, _P, _U32, _I64, _I64, ctypes.POINTER(_P)]),
    "ggq_weight_free": (_I, [_P, _P]),
    "ggq_weight_device_ptr": (_P, [_P]),
    "ggq_mul_mat": (_I, [_P, _P, _P, _I, _P, _I, _I, _I]),
    "ggq_mul_mat_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _P, _I, _I, _I, _P]),
    "ggq_mul_mat_noalloc_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _P, _I, _I, _I, _P]),
    "ggq_mul_mat_batch_dev": (_I, [_P, _P, _I, _P]),
    "ggq_mul_mat_batch_rows_dev": (_I, [_P, _P, _I, _I, _P]),
    "ggq_mul_mat_batch_act_dev": (_I, [_P, _P, _I, _I, _I, _P]),
    "ggq_mul_mat_fused_dev": (_I, [_P, _P, _I, _I, _P]),
    "ggq_mul_mat_q8_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _P, _I, _P, _I, _P]),
    "ggq_logits_argmax_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _I, _P, _P, _P, _P]),
    "ggq_attention_decode_dev": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I64, _I64, _P, _P]),
    "ggq_mul_mat_q8_batch_dev": (_I, [_P, _P, _I, _U32, _I64, _P, _P, _I, _P]),
    "ggq_dequant_dev": (_I, [_P, _P, _U32, _I64, _P, _P]),
    "ggq_quantize_act_dev": (_I, [_P, _P, _I, _I, _I, _I, _P, _P, _P]),
    "ggq_produce_quantize_act_dev": (_I, [_P, _I, _P, _P, _I, _I, _I, ctypes.c_float, _P, _P, _P]),
    "ggq_block_dot_dev": (_I, [_P, _P, _U32, _I64, _I64, _P, _I, _P, _P]),
    "ggq_moe_ffn_dev": (_I, [_P, ctypes.POINTER(MoeParams), _P]),
    "ggq_moe_ffn_act_dev": (_I, [_P, ctypes.POINTER(MoeParams), _I, _P]),
    "ggq_moe_trace_get": (_I, [_P, ctypes.POINTER(MoeTrace)]),
    "ggq_moe_trace_rows": (_I, [_P, _I]),
    "ggq_encode": (_I, [_U32, _P, _I64, _I64, _P]),
    "ggq_row_bytes": (_I64, [_U32, _I64]),
}


class GgufTensor(ctypes.Structure):
    """ggq_gguf_tensor (include/ggq_gguf.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_uint32), ("n_dims", ctypes.c_int32),
                ("dims", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


_U64, _PC = ctypes.c_uint64, ctypes.c_char_p
# Every function declared in include/ggq_gguf.h.
SIGNATURES.update({
    "ggq_gguf_open": (_I, [_PC, ctypes.POINTER(_P)]),
    "ggq_gguf_close": (None, [_P]),
    "ggq_gguf_last_error": (_PC, []),
    "ggq_gguf_version": (ctypes.c_uint32, [_P]),
    "ggq_gguf_alignment": (_U64, [_P]),
    "ggq_gguf_data_offset": (_U64, [_P]),
    "ggq_gguf_file_size": (_U64, [_P]),
    "ggq_gguf_n_tensors": (_I64, [_P]),
    "ggq_gguf_tensor_at": (_I, [_P, _I64, ctypes.POINTER(GgufTensor)]),
    "ggq_gguf_find_tensor": (_I64, [_P, _PC]),
    "ggq_gguf_n_kv": (_I64, [_P]),
    "ggq_gguf_kv_key": (_PC, [_P, _I64]),
    "ggq_gguf_find_kv": (_I64, [_P, _PC]),
    "ggq_gguf_kv_type": (ctypes.c_uint32, [_P, _I64]),
    "ggq_gguf_kv_int": (_I, [_P, _I64, ctypes.POINTER(_I64)]),
    "ggq_gguf_kv_uint": (_I, [_P, _I64, ctypes.POINTER(_U64)]),
    "ggq_gguf_kv_float": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_double)]),
    "ggq_gguf_kv_str": (_I, [_P, _I64, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    "ggq_gguf_kv_array": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64),
                               ctypes.POINTER(_P)]),
    "ggq_gguf_kv_array_str": (_I, [_P, _I64, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    "ggq_gguf_upload": (_I, [_P, _P, _PC, ctypes.POINTER(_P)]),
})

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


class GgufFile:
    """A GGUF v3 file opened through ggq_gguf_open (read in place from the
    mapping; no GPU needed).  `tensors` maps name -> dict(type, dims, offset,
    nbytes, data pointer); `kv(key)` returns a metadata value as Python data
    (ints, floats, str/bytes, lists for arrays)."""

    _NUMERIC = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "<u1",
                10: "<u8", 11: "<i8", 12: "<f8"}

    def __init__(self, path):
        self.lib = load_library()
        h = ctypes.c_void_p()
        st = self.lib.ggq_gguf_open(os.fsencode(path), ctypes.byref(h))
        if st != Status.OK:
            raise GgqError(Status(st), self.lib.ggq_gguf_last_error().decode())
        self.h = h

    def close(self):
        if self.h:
            self.lib.ggq_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def tensors(self):
        out = {}
        for i in range(self.lib.ggq_gguf_n_tensors(self.h)):
            t = GgufTensor()
            if self.lib.ggq_gguf_tensor_at(self.h, i, ctypes.byref(t)) != Status.OK:
                raise GgqError(Status.ERROR, f"tensor {i}")
            out[t.name.decode()] = {"type": t.type, "dims": list(t.dims[: t.n_dims]), "offset": t.offset,
                                    "nbytes": t.nbytes, "data": t.data, "index": i}
        return out

    def tensor_bytes(self, name):
        t = self.tensors[name]
        return ctypes.string_at(t["data"], t["nbytes"])

    def keys(self):
        return [self.lib.ggq_gguf_kv_key(self.h, i).decode() for i in range(self.lib.ggq_gguf_n_kv(self.h))]

    def kv(self, key):
        import numpy as np
        i = self.lib.ggq_gguf_find_kv(self.h, key.encode())
        if i < 0:
            raise KeyError(key)
        t = self.lib.ggq_gguf_kv_type(self.h, i)
        if t == 8:
            p, n = ctypes.c_void_p(), ctypes.c_uint64()
            self.lib.ggq_gguf_kv_str(self.h, i, ctypes.byref(p), ctypes.byref(n))
            return ctypes.string_at(p, n.value).decode("utf-8", "replace")
        if t in (6, 12):
            v = ctypes.c_double()
            self.lib.ggq_gguf_kv_float(self.h, i, ctypes.byref(v))
            return v.value
        if t == 9:
            et, n, p = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_void_p()
            self.lib.ggq_gguf_kv_array(self.h, i, ctypes.byref(et), ctypes.byref(n), ctypes.byref(p))
            if et.value == 8:
                out = []
                for j in range(n.value):
                    sp, sn = ctypes.c_void_p(), ctypes.c_uint64()
                    self.lib.ggq_gguf_kv_array_str(self.h, i, j, ctypes.byref(sp), ctypes.byref(sn))
                    out.append(ctypes.string_at(sp, sn.value).decode("utf-8", "replace"))
                return out
            dt = np.dtype(self._NUMERIC[et.value])
            return np.frombuffer(ctypes.string_at(p, n.value * dt.itemsize), dt).tolist()
        if t == 10:
            v = ctypes.c_uint64()
            self.lib.ggq_gguf_kv_uint(self.h, i, ctypes.byref(v))
            return v.value
        v = ctypes.c_int64()
        if self.lib.ggq_gguf_kv_int(self.h, i, ctypes.byref(v)) != Status.OK:
            raise GgqError(Status.INVALID_PARAM, f"{key}: type {t}")
        return bool(v.value) if t == 7 else v.value
