"""Pins the CPU oracle (oracle/ggq_oracle.c) before anything is checked
against it.  CPU only.

Each oracle function is checked against at least one of:
  * the reference's own unit-test goldens (tests/test_quant.cpp:209-288)
  * vectors produced by the reference sources (tests/golden/ref_vectors.npz)
  * closed forms / brute force computed independently in numpy
"""
import numpy as np
import pytest

TYPES = {"Q8_0": 8, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "IQ4_NL": 20, "IQ4_XS": 23}
KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], dtype=np.int8)


def f16(v):
    return int(np.array(v, dtype=np.float16).view(np.uint16))


# ---------------------------------------------------------------- goldens
def test_q4_k_reference_golden(orc):
    # tests/test_quant.cpp:209-236: d=0.5, dmin=0.25, scales 2 / mins 1 for
    # groups 0..3, qs[0]=0x31 -> out[0]=0.75, out[1]=-0.25, out[32]=2.75
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16(0.5)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(f16(0.25)).tobytes(), np.uint8)
    b[4:8] = 2
    b[8:12] = 1
    b[16] = 0x31
    out = orc.dequant(12, b)
    assert out[0] == 0.75 and out[1] == -0.25 and out[32] == 2.75


def test_q6_k_reference_golden(orc):
    # tests/test_quant.cpp:251-275: d=0.25, sc[0]=4, sc[4]=2, ql[0]=0x21
    b = np.zeros(210, np.uint8)
    b[208:210] = np.frombuffer(np.uint16(f16(0.25)).tobytes(), np.uint8)
    b[192] = 4
    b[196] = 2
    b[0] = 0x21
    out = orc.dequant(14, b)
    assert out[0] == -31.0 and out[64] == -15.0 and out[1] == -32.0


def test_q8_0_reference_values(orc):
    # tests/test_quant.cpp:130-152: d=1.0, qs[0]=3, qs[31]=1
    b = np.zeros(34, np.uint8)
    b[0:2] = [0x00, 0x3C]
    b[2] = 3
    b[33] = 1
    out = orc.dequant(8, b)
    assert out[0] == 3.0 and out[31] == 1.0 and np.count_nonzero(out) == 2


def test_type_table(orc, golden):
    # src/gguf/tensor.cpp:18-38 via the compiled reference, and the sizes
    # asserted by tests/test_quant.cpp:194-207 / tests/test_gguf.cpp:42-73
    for t, be, bb in golden["type_table"]:
        assert orc.block_elems(int(t)) == be and orc.block_bytes(int(t)) == bb
    assert orc.block_bytes(12) == 144 and orc.block_bytes(14) == 210


# ------------------------------------------------------ reference vectors
@pytest.mark.parametrize("name", list(TYPES))
def test_dequant_matches_reference_bitexact(orc, golden, name):
    t = TYPES[name]
    got = orc.dequant(t, golden[f"{name}_raw"])
    exp = golden[f"{name}_deq"]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_fp16_all_patterns(orc, golden):
    got = np.array([orc.lib().orc_fp16_to_f32(h) for h in range(65536)], dtype=np.float32)
    ref = golden["fp16_all"]
    finite = np.isfinite(ref) | np.isinf(ref)
    assert np.array_equal(got.view(np.uint32)[finite], ref.view(np.uint32)[finite])
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    # closed form: numpy's IEEE half conversion
    halves = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ok = ~np.isnan(halves)
    assert np.array_equal(got.view(np.uint32)[ok], halves.view(np.uint32)[ok])


def test_scale_min_unpack(orc, golden):
    import ctypes
    a, b = ctypes.c_uint8(), ctypes.c_uint8()
    for i, row in enumerate(golden["scale_min_in"]):
        row = np.ascontiguousarray(row)
        for j in range(8):
            orc.lib().orc_q4k_scale_min(j, row.ctypes.data, ctypes.byref(a), ctypes.byref(b))
            assert (a.value, b.value) == tuple(golden["scale_min_out"][i, j])


@pytest.mark.parametrize("name", ["Q4_K", "Q6_K"])
def test_f64_oracle_vs_reference_cpuref(orc, golden, name):
    """orc_mul_mat_f64 vs the compiled CpuRefBackend::mul_mat_q (fp32)."""
    M, N, K = golden[f"cpuref_{name}_shape"]
    W, A, C = golden[f"cpuref_{name}_W"], golden[f"cpuref_{name}_A"], golden[f"cpuref_{name}_C"]
    got = orc.mul_mat_f64(TYPES[name], W, int(N), int(K), A)
    assert orc.rel_l2(got, C) < 1e-5
    # the fp32 restatement reproduces the reference's own summation order
    got32 = orc.mul_mat_cpuref_f32(TYPES[name], W, int(N), int(K), A)
    assert np.array_equal(got32, C)


@pytest.mark.parametrize("name", list(TYPES))
def test_rowdot_oracle_pinned(orc, golden, name):
    """orc_mul_mat_rowdot_f32 (main.cpp:317-326): a running fp32 sum over the
    dequantized row -- bitwise a numpy float32 sequential cumsum, bitwise the
    reference decoders + loop where oracle/_ref is built, and not equal to a
    per-block partial-sum order."""
    t = TYPES[name]
    raw = golden[f"{name}_raw"]
    be, bb = orc.block_elems(t), orc.block_bytes(t)
    K = 512 if be == 256 else 128
    N = raw.size // bb // (K // be)
    W = np.ascontiguousarray(raw[: N * (K // be) * bb])
    A = np.random.default_rng(t).standard_normal((3, K)).astype(np.float32)
    got = orc.mul_mat_rowdot_f32(t, W, N, K, A)
    rows = orc.dequant(t, W).reshape(N, K)
    exp = np.cumsum(A[:, None, :] * rows[None, :, :], axis=2, dtype=np.float32)[:, :, -1]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    blockwise = np.zeros((3, N), np.float32)
    for b in range(K // be):
        sl = slice(b * be, (b + 1) * be)
        blockwise += np.cumsum(A[:, None, sl] * rows[None, :, sl], axis=2, dtype=np.float32)[:, :, -1]
    assert not np.array_equal(got, blockwise)
    ref = orc.ref_lib()
    if ref is not None:
        out = np.empty((3, N), np.float32)
        assert ref.ref_rowdot_mul_mat(t, W.ctypes.data, N, K, A.ctypes.data, 3, out.ctypes.data) == 0
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32))


# ------------------------------------------------------------ closed forms
def test_iq4_nl_closed_form(orc, golden):
    raw = golden["IQ4_NL_raw"].reshape(-1, 18)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    lo, hi = raw[:, 2:] & 15, raw[:, 2:] >> 4
    exp = np.concatenate([d * KV[lo].astype(np.float32), d * KV[hi].astype(np.float32)], axis=1)
    assert np.array_equal(orc.dequant(20, raw.reshape(-1)).reshape(-1, 32), exp)


def test_q8_0_closed_form(orc, golden):
    raw = golden["Q8_0_raw"].reshape(-1, 34)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1, 1)
    exp = raw[:, 2:].view(np.int8).astype(np.float32) * d
    assert np.array_equal(orc.dequant(8, raw.reshape(-1)).reshape(-1, 32), exp)


@pytest.mark.parametrize("name", list(TYPES))
def test_codes_times_scale_is_dequant(orc, golden, name):
    """Integer codes (the MFMA/dot operands) reproduce the dequant values:
    for formats without a min, value == scale * code with a per-group scale,
    so value/code is constant within each group."""
    t = TYPES[name]
    raw = golden[f"{name}_raw"][: 64 * orc.block_bytes(t)]
    q = orc.codes(t, raw).astype(np.float64)
    v = orc.dequant(t, raw).astype(np.float64)
    ge = 16 if t == 14 else 32
    q, v = q.reshape(-1, ge), v.reshape(-1, ge)
    if t in (12, 13):
        # affine: v = dl*q - ml -> dl = slope, check linearity within a group
        for g in range(q.shape[0]):
            if np.ptp(q[g]) == 0:
                continue
            A = np.stack([q[g], np.ones(ge)], 1)
            sol, *_ = np.linalg.lstsq(A, v[g], rcond=None)
            assert np.allclose(A @ sol, v[g], rtol=1e-6, atol=1e-6 * np.abs(v[g]).max())
    else:
        for g in range(q.shape[0]):
            nz = q[g] != 0
            assert np.all(v[g][~nz] == 0)
            if nz.any():
                r = v[g][nz] / q[g][nz]
                assert np.allclose(r, r[0], rtol=1e-6)


def test_quant_act_row_closed_form(orc):
    rng = np.random.default_rng(1)
    A = rng.standard_normal((5, 300)).astype(np.float32)
    A[1] = 0.0                              # zero row -> scale 1, all zero
    A[2, 7] = 0.5 * (np.abs(A[2]).max() / 127.0) * 3  # near a rounding tie
    q, s = orc.quant_act(A, 1)
    amax = np.abs(A).max(axis=1)
    s_exp = np.where(amax > 0, (amax / np.float32(127.0)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    assert np.array_equal(s, s_exp)
    inv = (np.float32(1.0) / s_exp).astype(np.float32)
    q_exp = np.clip(np.rint((A * inv[:, None]).astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(q, q_exp)
    assert np.all(q[1] == 0) and s[1] == 1.0
    # the row maximum maps to +-127
    assert np.all(np.abs(q[[0, 2, 3, 4]]).max(axis=1) == 127)


def test_quant_act_block32_closed_form(orc):
    rng = np.random.default_rng(2)
    A = rng.standard_normal((3, 128)).astype(np.float32)
    A[0, :32] = 0
    q, s = orc.quant_act(A, 2)
    blk = A.reshape(3, 4, 32)
    amax = np.abs(blk).max(axis=2)
    s_exp = np.where(amax > 0, (amax / np.float32(127.0)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    assert np.array_equal(s, s_exp)
    inv = (np.float32(1.0) / s_exp).astype(np.float32)
    q_exp = np.clip(np.rint((blk * inv[:, :, None]).astype(np.float32)), -128, 127).astype(np.int8)
    assert np.array_equal(q, q_exp.reshape(3, 128))


def test_quant_act_rounding_rules_pinned(orc):
    """Exact ties (half to even, not half away) and rows where dividing by
    the scale rounds differently from multiplying by its fp32 reciprocal
    (amd_xdna.cpp:598-603, 633-639, 762-766).  Expected codes come from exact
    rational arithmetic with explicit fp32 rounding; each wrong variant is
    shown to disagree, so either mistake in the oracle fails this test."""
    from tests import quant_rows as qr
    K = 64
    A = np.vstack([qr.tie_row(K), qr.reciprocal_rows(3, K, seed=11)])
    q, s = orc.quant_act(A, 1)
    for m in range(A.shape[0]):
        eq, es = qr.expected_codes(A[m])
        assert np.array_equal(q[m], eq), m
        assert s[m] == es
    assert q[0, :10].tolist() == [127, 0, 0, 2, -2, 2, -2, 4, -4, 4]
    assert q[0, 10:13].tolist() == [126, -126, -127]
    away = qr.variant_codes(A, divide=False, away=True)
    div = qr.variant_codes(A, divide=True, away=False)
    assert not np.array_equal(away[0], q[0])
    for m in range(1, A.shape[0]):
        assert (div[m] != q[m]).sum() >= K // 4, m
    # block32 mode: the same rows cut into 32-value blocks, each with its own
    # amax (the tie block's amax is 127, so its scale is exactly 1)
    B = np.vstack([np.concatenate([qr.tie_row(32), qr.reciprocal_rows(1, 32, seed=12)[0]]),
                   qr.reciprocal_rows(2, 32, seed=13).reshape(1, 64)])
    qb, sb = orc.quant_act(B, 2)
    for m in range(B.shape[0]):
        for b in range(2):
            eq, es = qr.expected_codes(B[m, 32 * b: 32 * b + 32])
            assert np.array_equal(qb[m, 32 * b: 32 * b + 32], eq), (m, b)
            assert sb[m, b] == es
    assert not np.array_equal(qr.variant_codes(B, False, True, block=32), qb)
    assert not np.array_equal(qr.variant_codes(B, True, False, block=32), qb)


@pytest.mark.parametrize("name", list(TYPES))
def test_block_dot_brute_force(orc, golden, name):
    t = TYPES[name]
    be, bb = orc.block_elems(t), orc.block_bytes(t)
    K = 256 if be == 256 else 64
    N = 3
    raw = golden[f"{name}_raw"][: N * (K // be) * bb]
    rng = np.random.default_rng(3)
    qa = rng.integers(-128, 128, size=(2, K), dtype=np.int8)
    got = orc.block_dot(t, raw, N, K, qa)
    codes = orc.codes(t, raw).astype(np.int64).reshape(N, K)
    ge = 16 if t == 14 else 32
    exp = (qa.astype(np.int64)[:, None, :] * codes[None, :, :]).reshape(2, N, K // ge, ge).sum(-1)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_f64_oracle_vs_numpy(orc, golden, mode):
    t = 23
    be, bb = 256, 136
    N, K = 5, 512
    raw = golden["IQ4_XS_raw"][: N * (K // be) * bb]
    rng = np.random.default_rng(4)
    A = rng.standard_normal((3, K)).astype(np.float32)
    W = orc.dequant(t, raw).astype(np.float64).reshape(N, K)
    if mode == 0:
        Ae = A.astype(np.float64)
    else:
        q, s = orc.quant_act(A, mode)
        Ae = q.astype(np.float64) * (s[:, None] if mode == 1 else np.repeat(s, 32, axis=1))
    assert orc.rel_l2(orc.mul_mat_f64(t, raw, N, K, A, mode), Ae @ W.T) < 1e-13


def test_moe_oracle_vs_numpy_loop(orc):
    """orc_moe_ffn_f64 vs a numpy restatement of main.cpp:3110-3193."""
    import ggnpu_amd.lib as gl
    rng = np.random.default_rng(5)
    T, H, F, E, k = 3, 256, 256, 6, 2
    Wg = gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wu = gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wd = gl.encode(14, (rng.standard_normal((E * H, F)) * 0.02).astype(np.float32))
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    out, sel, wsel = orc.moe_ffn_f64(x, logits, H, F, E, k, 12, Wg, 12, Wu, 14, Wd)
    dg = orc.dequant(12, Wg).astype(np.float64).reshape(E, F, H)
    du = orc.dequant(12, Wu).astype(np.float64).reshape(E, F, H)
    dd = orc.dequant(14, Wd).astype(np.float64).reshape(E, H, F)
    for t in range(T):
        order = np.argsort(-logits[t], kind="stable")[:k]
        assert list(sel[t]) == list(order)
        w = np.exp(logits[t, order].astype(np.float64) - logits[t, order[0]])
        w /= w.sum()
        ref = np.zeros(H)
        for j, e in enumerate(order):
            g, u = dg[e] @ x[t], du[e] @ x[t]
            h = (g / (1 + np.exp(-g)) * u).astype(np.float32).astype(np.float64)
            ref += w[j] * (dd[e] @ h)
        assert orc.rel_l2(out[t], ref) < 1e-12


def test_moe_oracle_q8_row_vs_numpy_loop(orc):
    """orc_moe_ffn_act_f64 in GGQ_ACT_Q8_ROW: each expert matmul quantizes
    its own input row (the token row for gate / up, the fp32 SwiGLU row for
    down) with the pinned per-row quantizer, and the result differs from the
    fp32-activation layer (so the mode is not silently ignored)."""
    import ggnpu_amd.lib as gl
    rng = np.random.default_rng(6)
    T, H, F, E, k = 3, 256, 256, 6, 2
    Wg = gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wu = gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wd = gl.encode(14, (rng.standard_normal((E * H, F)) * 0.02).astype(np.float32))
    Sg = gl.encode(12, (rng.standard_normal((F, H)) * 0.02).astype(np.float32))
    Su = gl.encode(12, (rng.standard_normal((F, H)) * 0.02).astype(np.float32))
    Sd = gl.encode(14, (rng.standard_normal((H, F)) * 0.02).astype(np.float32))
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    sw = rng.random(T).astype(np.float32)
    out, sel, _ = orc.moe_ffn_f64(x, logits, H, F, E, k, 12, Wg, 12, Wu, 14, Wd, Sg, Su, Sd, sw, act_mode=1)
    out32, _, _ = orc.moe_ffn_f64(x, logits, H, F, E, k, 12, Wg, 12, Wu, 14, Wd, Sg, Su, Sd, sw, act_mode=0)
    dg = orc.dequant(12, Wg).astype(np.float64).reshape(E, F, H)
    du = orc.dequant(12, Wu).astype(np.float64).reshape(E, F, H)
    dd = orc.dequant(14, Wd).astype(np.float64).reshape(E, H, F)
    sg = orc.dequant(12, Sg).astype(np.float64).reshape(F, H)
    su = orc.dequant(12, Su).astype(np.float64).reshape(F, H)
    sd = orc.dequant(14, Sd).astype(np.float64).reshape(H, F)

    def q8(row):
        q, s = orc.quant_act(row[None, :].astype(np.float32), 1)
        return q[0].astype(np.float64) * float(s[0])

    for t in range(T):
        order = np.argsort(-logits[t], kind="stable")[:k]
        assert list(sel[t]) == list(order)
        w = np.exp(logits[t, order].astype(np.float64) - logits[t, order[0]])
        w /= w.sum()
        xa = q8(x[t])
        ref = np.zeros(H)
        for wj, (G, U, D) in [(w[j], (dg[e], du[e], dd[e])) for j, e in enumerate(order)] + [(float(sw[t]), (sg, su, sd))]:
            g, u = G @ xa, U @ xa
            h = (g / (1 + np.exp(-g)) * u).astype(np.float32)
            ref += wj * (D @ q8(h))
        assert orc.rel_l2(out[t], ref) < 1e-12
    assert orc.rel_l2(out, out32) > 1e-4


def test_moe_oracle_routing_ties_and_nan(orc):
    """Routing rule beyond the reference's defined cases: ties go to the
    lower expert id (the reference's partial_sort leaves them unordered) and
    NaN ranks with -inf, so selections are always valid ids.  Distinct finite
    logits are ordered as std::partial_sort with `>` orders them."""
    import ggnpu_amd.lib as gl
    rng = np.random.default_rng(9)
    T, H, F, E, k = 5, 256, 256, 8, 3
    Wg = gl.encode(12, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wd = gl.encode(14, (rng.standard_normal((E * H, F)) * 0.02).astype(np.float32))
    x = rng.standard_normal((T, H)).astype(np.float32)
    lg = np.array([[0.1, 0.9, 0.9, 0.2, 0.9, 0.0, -1.0, 0.3],        # ties at 0.9
                   [np.nan] * 8,                                     # all NaN
                   [np.nan, -1, np.nan, 2, np.nan, np.nan, np.nan, np.nan],
                   [-np.inf, -np.inf, -np.inf, -np.inf, 5, -np.inf, -np.inf, np.nan],
                   [3, 1, 4, 1.5, 9, 2.6, 5.3, 5.8]], np.float32)
    _, sel, w = orc.moe_ffn_f64(x, lg, H, F, E, k, 12, Wg, 12, Wg, 14, Wd)
    assert sel.tolist() == [[1, 2, 4], [0, 1, 2], [3, 1, 0], [4, 0, 1], [4, 7, 6]]
    assert np.allclose(w[0], 1 / 3) and np.all(np.isnan(w[1]))
    assert np.all(np.isnan(w[2]))  # a NaN among the selected makes the softmax NaN
    assert np.allclose(w[3], [1, 0, 0])
    e = np.exp(np.float64([9, 5.8, 5.3]) - 9)
    assert np.allclose(w[4], e / e.sum(), rtol=1e-6)


# ------------------------------------------- RMSNorm / silu (fused GEMV)
@pytest.mark.parametrize("n,with_w,eps", [(2048, True, 1e-5), (1001, False, 1e-6), (64, True, 0.0)])
def test_rms_norm_matches_reference_and_closed_form(orc, n, with_w, eps):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32) * 3.0
    w = rng.standard_normal(n).astype(np.float32) if with_w else None
    got = orc.rms_norm(x, w, eps)
    ref = orc.ref_lib()
    if ref is not None:  # the compiled CpuRefBackend::rms_norm, bit for bit
        out = np.empty_like(x)
        assert ref.ref_rms_norm(x.ctypes.data, n, None if w is None else w.ctypes.data, eps, out.ctypes.data) == 0
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32))
    # closed form in fp64
    xd = x.astype(np.float64)
    exp = xd / np.sqrt(np.mean(xd * xd) + eps) * (1.0 if w is None else w.astype(np.float64))
    assert np.allclose(got, exp, rtol=3e-6, atol=1e-6)


def test_rms_norm_special_cases(orc):
    c = np.full(256, -2.5, np.float32)
    assert np.allclose(orc.rms_norm(c, None, 0.0), -1.0, rtol=2e-7, atol=0)  # constant row: sign
    z = np.zeros(64, np.float32)
    assert np.array_equal(orc.rms_norm(z, None, 1e-5), z)  # zero row stays zero (eps keeps it finite)


def test_silu_matches_reference_and_closed_form(orc):
    x = np.concatenate([np.linspace(-30, 30, 601), [0.0, -0.0, 1e-30, 88.0, -88.0]]).astype(np.float32)
    got = orc.silu(x)
    ref = orc.ref_lib()
    if ref is not None:
        out = np.empty_like(x)
        assert ref.ref_silu(x.ctypes.data, x.size, out.ctypes.data) == 0
        assert np.array_equal(got.view(np.uint32), out.view(np.uint32))
    xd = x.astype(np.float64)
    assert np.allclose(got, xd / (1.0 + np.exp(-xd)), rtol=2e-6, atol=1e-30)
    assert got[601] == 0.0 and got[605] == pytest.approx(-88.0 * np.exp(-88.0), rel=1e-3, abs=1e-36)


# ------------------------------------------------------- decode attention
@pytest.mark.parametrize("n_head,n_kv,hd,ctx,qpos", [(8, 2, 64, 300, 299), (4, 4, 128, 70, 40), (6, 1, 64, 33, 0)])
def test_flash_attn_matches_reference_and_f64(orc, n_head, n_kv, hd, ctx, qpos):
    rng = np.random.default_rng(ctx)
    q = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    Kc = rng.standard_normal((ctx, n_kv, hd)).astype(np.float32)
    Vc = rng.standard_normal((ctx, n_kv, hd)).astype(np.float32)
    got32 = orc.flash_attn(q, Kc, Vc, n_head, [qpos], f64=False)
    ref = orc.ref_lib()
    if ref is not None:  # the compiled CpuRefBackend::flash_attn on the expanded K/V, bit for bit
        K, V = orc.expand_kv(Kc, n_head), orc.expand_kv(Vc, n_head)
        out = np.empty((n_head, hd), np.float32)
        assert ref.ref_flash_attn(q[0].ctypes.data, K.ctypes.data, V.ctypes.data, n_head, hd, ctx, qpos,
                                  out.ctypes.data) == 0
        assert np.array_equal(got32[0].view(np.uint32), out.view(np.uint32))
    got64 = orc.flash_attn(q, Kc, Vc, n_head, [qpos])
    assert orc.rel_l2(got32, got64) < 1e-5
    # closed form in numpy (fp64), positions past qpos masked
    K, V = orc.expand_kv(Kc, n_head).astype(np.float64), orc.expand_kv(Vc, n_head).astype(np.float64)
    s = np.einsum("hd,hjd->hj", q[0].astype(np.float64), K[:, : qpos + 1]) / np.sqrt(hd)
    w = np.exp(s - s.max(axis=1, keepdims=True))
    w /= w.sum(axis=1, keepdims=True)
    assert np.allclose(got64[0], np.einsum("hj,hjd->hd", w, V[:, : qpos + 1]), rtol=1e-10, atol=1e-12)
    if qpos == 0:  # one visible position: the output is V[0] of each head's kv head
        assert np.allclose(got64[0], V[:, 0], rtol=0, atol=1e-15)


@pytest.mark.parametrize("name", list(TYPES))
def test_per_row_weight_requant_vs_reference_vectors(orc, golden, name):
    """A11, the XDNA host's per-row weight requantization (decode_*_for_npu,
    q8_0.cpp:30-77, q4_k.cpp:43-91, q5_k.cpp, q6_k.cpp:41-89, iq4_nl.cpp:36-82,
    iq4_xs.cpp:41-87): dequantize the row, scale = max|x| / 127 (1 for an
    all-zero row), code = clamp(nearbyint(x * (1 / scale))).  The oracle's
    dequant followed by its per-row activation quantizer (the same rule,
    amd_xdna.cpp:598-603) reproduces the int8 codes and scales that the
    compiled reference wrote, bit for bit.  The weights are never requantized
    on the GPU path; this pins the CPU baseline's host-preparation step."""
    t = TYPES[name]
    raw = golden[f"{name}_npu_raw"]
    N, K = (int(v) for v in golden[f"{name}_npu_shape"])
    rows = orc.dequant(t, raw).reshape(N, K)
    q, s = orc.quant_act(rows, 1)
    assert np.array_equal(s.view(np.uint32), golden[f"{name}_npu_s"].astype(np.float32).view(np.uint32))
    assert np.array_equal(q.reshape(-1), golden[f"{name}_npu_q"].astype(np.int8))
