"""Writes tests/golden/ref_vectors.npz from the ggnpu reference sources.

Runs in the build container only (it needs /root/reference): oracle/Makefile
compiles the reference's own src/quant, src/gguf/tensor.cpp and
src/backends/cpu_ref sources into oracle/_ref/libggnpu_ref.so; this script
feeds them seeded random-but-valid blocks plus edge blocks and stores inputs
and outputs.  The committed .npz is data (inputs and expected outputs), used
by tests/test_oracle.py and tests/test_gpu_parity.py on machines without the
reference.

    make -C oracle && python tests/golden/make_golden.py
"""
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as orc  # noqa: E402

TYPES = {"Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23}
# Byte offsets of the fp16 scale fields inside each block format.
F16_FIELDS = {8: [0], 12: [0, 2], 13: [0, 2], 14: [208], 20: [0], 23: [0]}
BLOCK = {8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 20: (32, 18), 23: (256, 136)}


def random_blocks(rng, t, n):
    """Random bytes with finite fp16 scales (normal and subnormal)."""
    be, bb = BLOCK[t]
    raw = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    for off in F16_FIELDS[t]:
        exp = rng.integers(0, 24, size=n)            # 0 = subnormal; <= 2^8 magnitude
        man = rng.integers(0, 1024, size=n)
        sign = rng.integers(0, 2, size=n)
        h = (sign << 15) | (exp << 10) | man
        raw[:, off] = h & 0xFF
        raw[:, off + 1] = h >> 8
    return raw


def edge_blocks(t):
    """d = 0, subnormal d, all-ones payload, negative d, max 6-bit scales."""
    be, bb = BLOCK[t]
    out = []
    for fill in (0x00, 0xFF, 0x55, 0xAA):
        for h in (0x0000, 0x0001, 0x03FF, 0x3C00, 0xBC00, 0x7BFF & 0x5BFF):
            b = np.full(bb, fill, dtype=np.uint8)
            for off in F16_FIELDS[t]:
                b[off] = h & 0xFF
                b[off + 1] = h >> 8
            out.append(b)
    return np.stack(out)


def main():
    ref = orc.ref_lib()
    if ref is None:
        sys.exit("oracle/_ref/libggnpu_ref.so not built (make -C oracle)")
    rng = np.random.default_rng(20261201)
    data = {}
    for name, t in TYPES.items():
        be, bb = BLOCK[t]
        raw = np.concatenate([random_blocks(rng, t, 64), edge_blocks(t)])
        n = raw.shape[0]
        flat = np.ascontiguousarray(raw.reshape(-1))
        out = np.empty(n * be, dtype=np.float32)
        assert ref.ref_dequant_blocks(t, flat.ctypes.data, n, out.ctypes.data) == 0
        data[f"{name}_raw"] = flat
        data[f"{name}_deq"] = out
        # per-row int8 requant (decode_*_for_npu) of a 4-row matrix
        K = be * 4 if be == 256 else be * 16
        rows = 4
        wraw = np.ascontiguousarray(random_blocks(rng, t, rows * K // be).reshape(-1))
        q = np.empty(rows * K, dtype=np.int8)
        s = np.empty(rows, dtype=np.float32)
        assert ref.ref_decode_for_npu(t, wraw.ctypes.data, wraw.size, rows, K, q.ctypes.data, s.ctypes.data) == 0
        data[f"{name}_npu_raw"] = wraw
        data[f"{name}_npu_q"] = q
        data[f"{name}_npu_s"] = s
        data[f"{name}_npu_shape"] = np.array([rows, K], dtype=np.int64)
    # CpuRefBackend::mul_mat_q on raw Q4_K / Q6_K (the only valid types there)
    for name in ("Q4_K", "Q6_K"):
        t = TYPES[name]
        N, K, M = 24, 512, 3
        W = np.ascontiguousarray(random_blocks(rng, t, N * K // 256).reshape(-1))
        A = rng.standard_normal((M, K), dtype=np.float32)
        C = np.empty((M, N), dtype=np.float32)
        assert ref.ref_cpuref_mul_mat(t, W.ctypes.data, N, K, A.ctypes.data, M, C.ctypes.data) == 0
        data[f"cpuref_{name}_W"] = W
        data[f"cpuref_{name}_A"] = A
        data[f"cpuref_{name}_C"] = C
        data[f"cpuref_{name}_shape"] = np.array([M, N, K], dtype=np.int64)
    # fp16 -> fp32 over every finite/inf/nan bit pattern
    f = np.array([ref.ref_fp16_to_f32(h) for h in range(65536)], dtype=np.float32)
    data["fp16_all"] = f
    # 6-bit scale/min unpack for random 12-byte inputs
    sc12 = rng.integers(0, 256, size=(256, 12), dtype=np.uint8)
    smv = np.empty((256, 8, 2), dtype=np.uint8)
    a, b = ctypes.c_uint8(), ctypes.c_uint8()
    for i in range(256):
        row = np.ascontiguousarray(sc12[i])
        for j in range(8):
            ref.ref_q4k_scale_min(j, row.ctypes.data, ctypes.byref(a), ctypes.byref(b))
            smv[i, j] = (a.value, b.value)
    data["scale_min_in"] = sc12
    data["scale_min_out"] = smv
    # type table (src/gguf/tensor.cpp:18-38)
    data["type_table"] = np.array([[t, ref.ref_blck_size(t), ref.ref_type_size(t)] for t in TYPES.values()],
                                  dtype=np.int64)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")
    np.savez_compressed(path, **data)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
