"""ctypes access to the CPU oracle (liboracle.so) and, when built, to the
reference sources compiled into oracle/_ref/libggnpu_ref.so.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and only as a checker / CPU baseline.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libggnpu_ref.so")

_P, _I, _U32, _I64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_int64

_ORC_SIGS = {
    "orc_block_elems": (_I, [_U32]),
    "orc_block_bytes": (_I, [_U32]),
    "orc_groups_per_block": (_I, [_U32]),
    "orc_fp16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_q4k_scale_min": (None, [_I, _P, _P, _P]),
    "orc_dequant_blocks": (_I, [_U32, _P, _I64, _P]),
    "orc_block_codes": (_I, [_U32, _P, _P]),
    "orc_quant_act_row": (None, [_P, _I, _I, _I, _P, _P]),
    "orc_quant_act_block32": (None, [_P, _I, _I, _I, _P, _P]),
    "orc_block_dot": (_I, [_U32, _P, _I64, _I64, _P, _I, _P]),
    "orc_mul_mat_f64": (_I, [_U32, _P, _I64, _I64, _P, _I, _I, _I, _P, _I]),
    "orc_mul_mat_cpuref_f32": (_I, [_U32, _P, _I64, _I64, _P, _I, _I, _P, _I]),
    "orc_mul_mat_rowdot_f32": (_I, [_U32, _P, _I64, _I64, _P, _I, _I, _P, _I]),
    "orc_moe_ffn_f64": (_I, [_P, _P, _I, _I, _I, _I, _I, _U32, _P, _U32, _P, _U32, _P,
                             _P, _P, _P, _P, _P, _P, _P]),
    "orc_moe_ffn_act_f64": (_I, [_P, _P, _I, _I, _I, _I, _I, _U32, _P, _U32, _P, _U32, _P,
                                 _P, _P, _P, _P, _I, _P, _P, _P]),
    "orc_rms_norm": (None, [_P, _I, _P, ctypes.c_float, _P]),
    "orc_silu": (None, [_P, _I, _P]),
    "orc_flash_attn": (None, [_P, _P, _P, _I, _I, _I64, _I64, _P]),
    "orc_flash_attn_f64": (None, [_P, _P, _P, _I, _I, _I64, _I64, _P]),
}

_REF_SIGS = {
    "ref_fp16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "ref_q4k_scale_min": (None, [_I, _P, _P, _P]),
    "ref_dequant_blocks": (_I, [_U32, _P, _I64, _P]),
    "ref_type_size": (ctypes.c_uint64, [_U32]),
    "ref_blck_size": (ctypes.c_uint64, [_U32]),
    "ref_decode_for_npu": (_I, [_U32, _P, ctypes.c_uint64, _I64, _I64, _P, _P]),
    "ref_cpuref_mul_mat": (_I, [_U32, _P, _I, _I, _P, _I, _P]),
    "ref_rowdot_mul_mat": (_I, [_U32, _P, _I, _I, _P, _I, _P]),
    "ref_rms_norm": (_I, [_P, _I, _P, ctypes.c_float, _P]),
    "ref_silu": (_I, [_P, _I, _P]),
    "ref_flash_attn": (_I, [_P, _P, _P, _I, _I, _I64, _I64, _P]),
}


def _bind(path, sigs):
    lib = ctypes.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_orc = None


def build_oracle():
    subprocess.run(["make", "-s", "-C", HERE, "oracle"], check=True)


def lib():
    global _orc
    if _orc is None:
        if not os.path.exists(ORACLE_SO):
            build_oracle()
        _orc = _bind(ORACLE_SO, _ORC_SIGS)
    return _orc


def ref_lib():
    """The compiled reference sources, or None where they are not available."""
    if not os.path.exists(REF_SO):
        return None
    return _bind(REF_SO, _REF_SIGS)


def _ptr(a):
    return a.ctypes.data


def block_elems(t):
    return lib().orc_block_elems(int(t))


def block_bytes(t):
    return lib().orc_block_bytes(int(t))


def dequant(t, raw, n_blocks=None):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    nb = raw.size // block_bytes(t) if n_blocks is None else n_blocks
    out = np.empty(nb * block_elems(t), dtype=np.float32)
    assert lib().orc_dequant_blocks(int(t), _ptr(raw), nb, _ptr(out)) == 0
    return out


def codes(t, raw):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    nb = raw.size // block_bytes(t)
    be, bb = block_elems(t), block_bytes(t)
    out = np.empty(nb * be, dtype=np.int8)
    for i in range(nb):
        blk = np.ascontiguousarray(raw[i * bb:(i + 1) * bb])
        lib().orc_block_codes(int(t), _ptr(blk), _ptr(out[i * be:]))
    return out


def quant_act(A, mode):
    A = np.ascontiguousarray(A, dtype=np.float32)
    M, K = A.shape
    q = np.empty((M, K), dtype=np.int8)
    if mode == 1:
        s = np.empty(M, dtype=np.float32)
        lib().orc_quant_act_row(_ptr(A), K, M, K, _ptr(q), _ptr(s))
    else:
        s = np.empty((M, K // 32), dtype=np.float32)
        lib().orc_quant_act_block32(_ptr(A), K, M, K, _ptr(q), _ptr(s))
    return q, s


def block_dot(t, W, N, K, qa):
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    M = qa.shape[0]
    ge = 16 if int(t) == 14 else 32
    out = np.empty((M, N, K // ge), dtype=np.int32)
    assert lib().orc_block_dot(int(t), _ptr(W), N, K, _ptr(qa), M, _ptr(out)) == 0
    return out


def mul_mat_f64(t, W, N, K, A, act_mode=0):
    A = np.ascontiguousarray(A, dtype=np.float32)
    M = A.shape[0]
    C = np.empty((M, N), dtype=np.float64)
    assert lib().orc_mul_mat_f64(int(t), _ptr(W), N, K, _ptr(A), K, M, act_mode, _ptr(C), N) == 0
    return C


def mul_mat_cpuref_f32(t, W, N, K, A):
    A = np.ascontiguousarray(A, dtype=np.float32)
    M = A.shape[0]
    C = np.empty((M, N), dtype=np.float32)
    assert lib().orc_mul_mat_cpuref_f32(int(t), _ptr(W), N, K, _ptr(A), K, M, _ptr(C), N) == 0
    return C


def mul_mat_rowdot_f32(t, W, N, K, A):
    A = np.ascontiguousarray(A, dtype=np.float32)
    M = A.shape[0]
    C = np.empty((M, N), dtype=np.float32)
    assert lib().orc_mul_mat_rowdot_f32(int(t), _ptr(W), N, K, _ptr(A), K, M, _ptr(C), N) == 0
    return C


def moe_ffn_f64(x, logits, H, F, E, topk, tg, Wg, tu, Wu, td, Wd, Sg=None, Su=None, Sd=None,
                shared_w=None, act_mode=0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T = x.shape[0]
    out = np.empty((T, H), dtype=np.float64)
    sel = np.empty((T, topk), dtype=np.int32)
    wsel = np.empty((T, topk), dtype=np.float32)
    sw = None if shared_w is None else np.ascontiguousarray(shared_w, dtype=np.float32)
    st = lib().orc_moe_ffn_act_f64(_ptr(x), _ptr(logits), T, H, F, E, topk, int(tg), _ptr(Wg), int(tu), _ptr(Wu),
                                   int(td), _ptr(Wd),
                                   None if Sg is None else _ptr(Sg), None if Su is None else _ptr(Su),
                                   None if Sd is None else _ptr(Sd), None if sw is None else _ptr(sw),
                                   int(act_mode), _ptr(out), _ptr(sel), _ptr(wsel))
    assert st == 0
    return out, sel, wsel


def rel_l2(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def rms_norm(x, w=None, eps=1e-5):
    """Row-wise orc_rms_norm of a [M][K] (or [K]) fp32 array."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    wp = None if w is None else np.ascontiguousarray(w, np.float32)
    for m in range(rows.shape[0]):
        lib().orc_rms_norm(rows[m].ctypes.data, rows.shape[1], None if wp is None else wp.ctypes.data,
                           float(eps), out[m].ctypes.data)
    return out.reshape(x.shape)


def silu(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_silu(x.ctypes.data, x.size, out.ctypes.data)
    return out


def expand_kv(cache, n_head):
    """main.cpp:3358-3379: the [ctx][n_kv][hd] cache of one layer as head-major
    [n_head][ctx][hd] with query head h reading kv head h // (n_head / n_kv)."""
    ctx, n_kv, hd = cache.shape
    groups = n_head // n_kv
    return np.ascontiguousarray(np.stack([cache[:, h // groups, :] for h in range(n_head)]), np.float32)


def flash_attn(q, Kc, Vc, n_head, query_pos, f64=True):
    """Attention of query rows q [n_tok][n_head][hd] over cache slabs Kc, Vc
    [ctx][n_kv][hd]; row t uses query_pos[t]."""
    ctx, n_kv, hd = Kc.shape
    K, V = expand_kv(Kc, n_head), expand_kv(Vc, n_head)
    out = np.empty((q.shape[0], n_head, hd), np.float64 if f64 else np.float32)
    for t in range(q.shape[0]):
        qt = np.ascontiguousarray(q[t], np.float32)
        fn = lib().orc_flash_attn_f64 if f64 else lib().orc_flash_attn
        fn(qt.ctypes.data, K.ctypes.data, V.ctypes.data, n_head, hd, ctx, int(query_pos[t]), out[t].ctypes.data)
    return out
