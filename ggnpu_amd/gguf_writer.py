"""Minimal GGUF v3 writer: header, typed metadata, tensor infos, padding to
the alignment, tensor data -- for synthetic models (the tests' files and the
benchmark's full-size decode model).  Written from the format description in
include/ggq_gguf.h; the reader is ggq_gguf_* (ggnpu_amd/csrc/ggq_gguf.cpp)."""
import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        if et == STRING:
            return out + b"".join(_str(x) for x in items)
        return out + b"".join(struct.pack(_FMT[et], x) for x in items)
    return struct.pack(_FMT[t], v)


def build(kvs, tensors, alignment=32, version=3, magic=b"GGUF"):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, dims, raw bytes)]
    with dims fastest first (dims[0] = K).  Tensor data is laid out in order,
    each padded to `alignment`.  Returns (file bytes, {name: offset})."""
    head = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = {}, 0
    for name, gt, dims, raw in tensors:
        offsets[name] = off
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, off)
        off += (len(raw) + alignment - 1) // alignment * alignment
    pad = (-len(head)) % alignment
    data = bytearray()
    for name, gt, dims, raw in tensors:
        data += raw
        data += b"\0" * ((-len(raw)) % alignment)
    return bytes(head) + b"\0" * pad + bytes(data), offsets


def write(path, kvs, tensors, **kw):
    blob, offsets = build(kvs, tensors, **kw)
    with open(path, "wb") as f:
        f.write(blob)
    return offsets


def write_stream(path, kvs, tensors, alignment=32):
    """The layout of build(), written tensor by tensor: tensors is a list of
    (name, ggml_type, dims, nbytes, produce) where produce() returns the
    tensor's bytes when its turn comes (large synthetic models never hold
    the whole file in memory)."""
    head = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kvs)))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    off = 0
    for name, gt, dims, nbytes, _ in tensors:
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gt, off)
        off += (nbytes + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(bytes(head) + b"\0" * ((-len(head)) % alignment))
        for name, gt, dims, nbytes, produce in tensors:
            raw = produce()
            assert len(raw) == nbytes, name
            f.write(raw)
            f.write(b"\0" * ((-nbytes) % alignment))


def raw_bytes(a):
    return np.ascontiguousarray(a).tobytes()
