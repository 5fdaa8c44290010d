"""GGUF v3 reader (include/ggq_gguf.h) on files written by ggnpu_amd/gguf_writer.py:
every metadata type, tensor infos and data read in place, alignment, and
malformed files rejected with a message.  CPU only.  The type table is
pinned by the reference's own table for the six path types (golden
`type_table`, from src/gguf/tensor.cpp via the compiled reference)."""
import numpy as np
import pytest

import ggnpu_amd.lib as gl
from ggnpu_amd import gguf_writer as gw

Q8, Q4K, Q6K, IQ4XS, F32, F16 = 8, 12, 14, 23, 0, 1


def _weights(t, N, K, seed):
    rng = np.random.default_rng(seed)
    return gl.encode(t, (rng.standard_normal((N, K)) * 0.02).astype(np.float32))


def _kvs():
    return [
        ("general.architecture", gw.STRING, "llama"),
        ("general.name", gw.STRING, "Ünïcode name"),
        ("general.empty", gw.STRING, ""),
        ("u8", gw.UINT8, 250), ("i8", gw.INT8, -5), ("u16", gw.UINT16, 65000), ("i16", gw.INT16, -30000),
        ("u32", gw.UINT32, 4000000000), ("i32", gw.INT32, -2000000000),
        ("u64", gw.UINT64, 2**63 + 5), ("i64", gw.INT64, -(2**62)),
        ("f32", gw.FLOAT32, 1e-5), ("f64", gw.FLOAT64, 500000.25), ("flag", gw.BOOL, 1),
        ("llama.block_count", gw.UINT32, 16),
        ("arr.u8", gw.ARRAY, (gw.UINT8, [1, 2, 255])),
        ("arr.i16", gw.ARRAY, (gw.INT16, [-1, 7])),
        ("arr.f32", gw.ARRAY, (gw.FLOAT32, [0.5, -2.0, 3.25])),
        ("arr.i64", gw.ARRAY, (gw.INT64, [-(2**40), 3])),
        ("arr.empty", gw.ARRAY, (gw.INT32, [])),
        ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["<s>", "", "▁Paris", "x" * 300])),
    ]


def _tensors():
    K, N, E = 512, 24, 3
    return [
        ("blk.0.attn_q.weight", Q4K, [K, N], _weights(Q4K, N, K, 1).tobytes()),
        ("blk.0.ffn_down.weight", Q6K, [K, 40], _weights(Q6K, 40, K, 2).tobytes()),
        ("blk.0.ffn_gate_exps.weight", IQ4XS, [K, N, E], _weights(IQ4XS, N * E, K, 3).tobytes()),
        ("output.weight", Q8, [96, 7], _weights(Q8, 7, 96, 4).tobytes()),
        ("blk.0.attn_norm.weight", F32, [K], np.arange(K, dtype=np.float32).tobytes()),
        ("token_embd.weight", F16, [K, 5], np.ones((5, K), np.float16).tobytes()),
    ]


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_roundtrip_metadata_and_tensors(tmp_path, alignment):
    path = tmp_path / "m.gguf"
    kvs = _kvs()
    if alignment != 32:
        kvs = kvs + [("general.alignment", gw.UINT32, alignment)]
    tens = _tensors()
    offsets = gw.write(path, kvs, tens, alignment=alignment)
    with gl.GgufFile(path) as g:
        lib = g.lib
        assert lib.ggq_gguf_version(g.h) == 3
        assert lib.ggq_gguf_alignment(g.h) == alignment
        off = lib.ggq_gguf_data_offset(g.h)
        assert off % alignment == 0
        assert g.keys() == [k for k, _, _ in kvs]
        exp = {"general.architecture": "llama", "general.name": "Ünïcode name", "general.empty": "",
               "u8": 250, "i8": -5, "u16": 65000, "i16": -30000, "u32": 4000000000, "i32": -2000000000,
               "u64": 2**63 + 5, "i64": -(2**62), "f64": 500000.25, "flag": True, "llama.block_count": 16,
               "arr.u8": [1, 2, 255], "arr.i16": [-1, 7], "arr.f32": [0.5, -2.0, 3.25],
               "arr.i64": [-(2**40), 3], "arr.empty": [],
               "tokenizer.ggml.tokens": ["<s>", "", "▁Paris", "x" * 300]}
        for k, v in exp.items():
            assert g.kv(k) == v, k
        assert g.kv("f32") == pytest.approx(1e-5, rel=1e-7)
        tinfo = g.tensors
        assert list(tinfo) == [t[0] for t in tens]
        for name, gt, dims, raw in tens:
            t = tinfo[name]
            assert t["type"] == gt and t["dims"] == dims and t["offset"] == offsets[name]
            assert t["nbytes"] == len(raw)
            assert g.tensor_bytes(name) == raw
            assert lib.ggq_gguf_find_tensor(g.h, name.encode()) == t["index"]
        assert lib.ggq_gguf_find_tensor(g.h, b"nope") == -1
        assert lib.ggq_gguf_find_kv(g.h, b"nope") == -1
        # typed getters refuse the wrong type
        import ctypes
        v = ctypes.c_int64()
        i = lib.ggq_gguf_find_kv(g.h, b"general.name")
        assert lib.ggq_gguf_kv_int(g.h, i, ctypes.byref(v)) == gl.Status.INVALID_PARAM
        d = ctypes.c_double()
        assert lib.ggq_gguf_kv_float(g.h, lib.ggq_gguf_find_kv(g.h, b"u8"), ctypes.byref(d)) == gl.Status.INVALID_PARAM
        u = ctypes.c_uint64()
        assert lib.ggq_gguf_kv_uint(g.h, lib.ggq_gguf_find_kv(g.h, b"i8"), ctypes.byref(u)) == gl.Status.INVALID_PARAM


def test_type_table_matches_reference_for_path_types(golden, tmp_path):
    """nbytes = elements / block * block bytes with the reference's block
    sizes (tensor.cpp:18-38) for Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, IQ4_XS."""
    for t, blck, size in golden["type_table"]:
        K, N = int(blck) * 4, 3
        raw = b"\x11" * (N * 4 * int(size))
        path = tmp_path / f"t{t}.gguf"
        gw.write(path, [], [("w", int(t), [K, N], raw)])
        with gl.GgufFile(path) as g:
            assert g.tensors["w"]["nbytes"] == N * (K // int(blck)) * int(size)


def _expect_invalid(path, fragment):
    with pytest.raises(gl.GgqError) as e:
        gl.GgufFile(path)
    assert e.value.status == gl.Status.INVALID_PARAM
    assert fragment in str(e.value), str(e.value)


def test_malformed_files(tmp_path):
    p = tmp_path / "x.gguf"
    good, _ = gw.build(_kvs(), _tensors())
    p.write_bytes(gw.build(_kvs(), _tensors(), magic=b"GGUG")[0])
    _expect_invalid(p, "magic")
    p.write_bytes(gw.build(_kvs(), _tensors(), version=2)[0])
    _expect_invalid(p, "version")
    p.write_bytes(good[:20])
    _expect_invalid(p, "too small")
    for cut in (40, 300, 900):  # inside the KVs / tensor infos
        p.write_bytes(good[:cut])
        with pytest.raises(gl.GgqError):
            gl.GgufFile(p)
    p.write_bytes(good[:-100])  # last tensor's data cut short
    _expect_invalid(p, "past the end")
    p.write_bytes(gw.build([("k" * 1025, gw.UINT8, 1)], [])[0])
    _expect_invalid(p, "bad key")
    p.write_bytes(gw.build([("general.alignment", gw.UINT32, 48)], [])[0])
    _expect_invalid(p, "power of two")
    t = _tensors()[0]
    p.write_bytes(gw.build([], [t, t])[0])
    _expect_invalid(p, "duplicate")
    p.write_bytes(gw.build([], [("w", Q4K, [100, 2], b"\0" * 4096)])[0])
    _expect_invalid(p, "multiple of the block")
    # one KV whose value type (42) does not exist
    p.write_bytes(b"GGUF" + (3).to_bytes(4, "little") + (0).to_bytes(8, "little") + (1).to_bytes(8, "little")
                  + (1).to_bytes(8, "little") + b"k" + (42).to_bytes(4, "little"))
    _expect_invalid(p, "bad value")
    with pytest.raises(gl.GgqError) as e:
        gl.GgufFile(tmp_path / "missing.gguf")
    assert e.value.status == gl.Status.NOT_FOUND


def test_upload_without_device_reports_errors(tmp_path):
    """ggq_gguf_upload needs a context; argument errors come first."""
    import ctypes
    p = tmp_path / "m.gguf"
    gw.write(p, [], _tensors())
    with gl.GgufFile(p) as g:
        w = ctypes.c_void_p()
        assert g.lib.ggq_gguf_upload(None, g.h, b"output.weight", ctypes.byref(w)) == gl.Status.INVALID_PARAM
