"""The MoE layer checked stage by stage against the oracle, at the full bar.

The layer (src/cli/main.cpp:3110-3193 per token) is route -> gate / up ->
SwiGLU -> down -> weighted combine.  With per-row int8 activations
(GGQ_ACT_Q8_ROW, amd_xdna.cpp:598-603 for every mul_mat_q of the loop) the
down projection quantizes the fp32 SwiGLU row, and a code of that row can
flip at a rounding tie between any two fp32 computations of the row; so
each stage is checked on the device's own input to it
(ggq_moe_trace_get):

  routing     selections equal a numpy top-k (ties to the lower expert id),
              the pair rows of every (token, slot) point back at them;
  gate / up   every pair row's outputs vs orc_mul_mat_f64 on the token row,
              same activation treatment, rel-L2 <= 1e-4 per row;
  SwiGLU      the device's fp32 rows equal silu(gate) * up of its own gate /
              up outputs (fp64, 1e-6), and their int8 codes and scales equal
              orc_quant_act_row of those rows bit for bit (Q8_ROW);
  down        every pair row's outputs vs orc_mul_mat_f64 on the device's
              SwiGLU row (quantized again by the pinned oracle quantizer in
              Q8_ROW mode, i.e. on the codes just checked), 1e-4 per row;
  combine     each token's output vs the fp64 weighted sum of the device's
              down rows in the reference's order, 1e-4 per token.

Shapes: the qwen35moe-A3B layer of the benchmark (H 2048, 256 experts of
FFN 512, top-8, shared expert, Q4_K gate / up, Q6_K down) at 64 tokens
(grouped int8 GEMV path) and 512 tokens (expert-grouped GEMM path), and
small layers with every format forced onto each path.
"""
import ctypes
import os

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

TOL = 1e-4
Q4K, Q6K = 12, 14


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    c = gl.Context(0)
    c.check(c.lib.ggq_moe_trace_rows(c.h, 1), "trace rows")
    yield c
    c.close()


def d2h(p, shape, dtype):
    """Copy `shape` elements of a device pointer (from the trace) to numpy."""
    import torch
    n = int(np.prod(shape))
    tdt = {np.float32: torch.float32, np.int32: torch.int32, np.int8: torch.int8}[dtype]
    buf = torch.empty(n, dtype=tdt, device="cuda")
    nbytes = n * np.dtype(dtype).itemsize
    # the HIP runtime torch and the library already share (never a second copy)
    hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    assert hip.hipMemcpy(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(p), ctypes.c_size_t(nbytes), 3) == 0
    return buf.cpu().numpy().reshape(shape)


def topk_ref(logits, k):
    """Top-k by descending logit, ties to the lower index; softmax over the
    selected (main.cpp:3126-3135)."""
    order = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    sel = np.take_along_axis(logits, order, axis=1).astype(np.float64)
    w = np.exp(sel - sel[:, :1])
    return order.astype(np.int32), w / w.sum(axis=1, keepdims=True)


def expert_rows(raw, t, n_rows, K, e):
    rb = gl.row_bytes(t, K)
    return np.ascontiguousarray(raw[e * n_rows * rb:(e + 1) * n_rows * rb])


def per_row_err(got, ref):
    num = np.linalg.norm(got.astype(np.float64) - ref, axis=1)
    den = np.linalg.norm(ref, axis=1)
    return num / np.where(den > 0, den, 1.0)


def run_layer(ctx, T, H, F, E, k, types, act_mode, seed, shared=True, hot=0):
    import torch
    tg, tu, td = types
    rng = np.random.default_rng(seed)
    Wg = gl.encode(tg, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wu = gl.encode(tu, (rng.standard_normal((E * F, H)) * 0.02).astype(np.float32))
    Wd = gl.encode(td, (rng.standard_normal((E * H, F)) * 0.02).astype(np.float32))
    S = [None] * 3
    sw = None
    if shared:
        S = [gl.encode(tg, (rng.standard_normal((F, H)) * 0.02).astype(np.float32)),
             gl.encode(tu, (rng.standard_normal((F, H)) * 0.02).astype(np.float32)),
             gl.encode(td, (rng.standard_normal((H, F)) * 0.02).astype(np.float32))]
        sw = (1.0 / (1.0 + np.exp(-rng.standard_normal(T)))).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if hot:  # the first `hot` experts take most tokens
        logits[:, :hot] += 3.0
    keep = [dev(a) for a in (x, logits, Wg, Wu, Wd)] + [dev(a) if a is not None else None for a in (*S, sw)]
    out = empty((T, H), torch.float32)
    sel = empty((T, k), torch.int32)
    wsel = empty((T, k), torch.float32)
    p = gl.MoeParams()
    p.T, p.H, p.F, p.E, p.top_k = T, H, F, E, k
    p.x, p.router_logits = keep[0].data_ptr(), keep[1].data_ptr()
    p.gate_type, p.up_type, p.down_type = tg, tu, td
    p.gate_exps, p.up_exps, p.down_exps = keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr()
    if shared:
        p.gate_shexp, p.up_shexp, p.down_shexp = keep[5].data_ptr(), keep[6].data_ptr(), keep[7].data_ptr()
        p.shared_w = keep[8].data_ptr()
    p.out, p.sel_experts, p.sel_weights = out.data_ptr(), sel.data_ptr(), wsel.data_ptr()
    ctx.check(ctx.lib.ggq_moe_ffn_act_dev(ctx.h, ctypes.byref(p), act_mode, None), "moe")
    torch.cuda.synchronize()
    tr = gl.MoeTrace()
    ctx.check(ctx.lib.ggq_moe_trace_get(ctx.h, ctypes.byref(tr)), "trace")
    assert tr.act_mode == act_mode and tr.T == T and tr.E == E and tr.shared == int(shared)
    return dict(x=x, logits=logits, Wg=Wg, Wu=Wu, Wd=Wd, S=S, sw=sw, out=host(out), sel=host(sel),
                wsel=host(wsel), tr=tr)


def check_stages(orc, L, T, H, F, E, k, types, act_mode, n_experts=None, n_shared=None, seed=0):
    tg, tu, td = types
    tr = L["tr"]
    nk = T * k
    rows = nk + (T if tr.shared else 0)
    assert tr.rows == rows
    grp = d2h(tr.grp, (E + 1,), np.int32)
    tok = d2h(tr.tok, (nk,), np.int32)
    pos = d2h(tr.pos, (T, k), np.int32)
    G = d2h(tr.gate, (rows, F), np.float32)
    U = d2h(tr.up, (rows, F), np.float32)
    assert tr.h, "fp32 SwiGLU rows not traced"
    Hh = d2h(tr.h, (rows, F), np.float32)
    D = d2h(tr.down, (nk, H), np.float32)
    Dsh = d2h(tr.down_shared, (T, H), np.float32) if tr.shared else None

    # routing
    rsel, rw = topk_ref(L["logits"], k)
    assert np.array_equal(L["sel"], rsel)
    assert np.allclose(L["wsel"], rw, rtol=1e-6)
    assert grp[0] == 0 and grp[E] == nk and np.all(np.diff(grp) >= 0)
    for t in range(T):
        for j in range(k):
            p, e = pos[t, j], rsel[t, j]
            assert grp[e] <= p < grp[e + 1] and tok[p] == t, (t, j)

    # gate / up per expert on the token rows
    rng = np.random.default_rng(seed)
    experts = np.arange(E) if n_experts is None or n_experts >= E else np.sort(rng.choice(E, n_experts, replace=False))
    worst = 0.0
    for e in experts:
        r0, r1 = grp[e], grp[e + 1]
        if r0 == r1:
            continue
        A = L["x"][tok[r0:r1]]
        for t, raw, Y in ((tg, L["Wg"], G), (tu, L["Wu"], U)):
            ref = orc.mul_mat_f64(t, expert_rows(raw, t, F, H, e), F, H, A, act_mode)
            err = per_row_err(Y[r0:r1], ref)
            worst = max(worst, err.max())
            assert err.max() < TOL, ("gate/up", e, err.max())
    sh_tok = None
    if tr.shared:
        sh_tok = np.arange(T) if n_shared is None or n_shared >= T else np.sort(rng.choice(T, n_shared, replace=False))
        for t, raw, Y in ((tg, L["S"][0], G), (tu, L["S"][1], U)):
            ref = orc.mul_mat_f64(t, raw, F, H, L["x"][sh_tok], act_mode)
            err = per_row_err(Y[nk + sh_tok], ref)
            worst = max(worst, err.max())
            assert err.max() < TOL, ("shared gate/up", err.max())

    # SwiGLU rows: silu(gate) * up of the device's own gate / up outputs
    Gd, Ud = G.astype(np.float64), U.astype(np.float64)
    assert orc.rel_l2(Hh, Gd / (1.0 + np.exp(-Gd)) * Ud) < 1e-6
    if act_mode == 1:
        qh = d2h(tr.h_codes, (rows, F), np.int8)
        sh = d2h(tr.h_scales, (rows,), np.float32)
        rq, rs = orc.quant_act(Hh, 1)
        assert np.array_equal(sh, rs), "SwiGLU row scales"
        assert np.array_equal(qh, rq), "SwiGLU row codes"

    # down per expert on the device's SwiGLU rows
    for e in experts:
        r0, r1 = grp[e], grp[e + 1]
        if r0 == r1:
            continue
        ref = orc.mul_mat_f64(td, expert_rows(L["Wd"], td, H, F, e), H, F, Hh[r0:r1], act_mode)
        err = per_row_err(D[r0:r1], ref)
        worst = max(worst, err.max())
        assert err.max() < TOL, ("down", e, err.max())
    if tr.shared:
        ref = orc.mul_mat_f64(td, L["S"][2], H, F, Hh[nk + sh_tok], act_mode)
        err = per_row_err(Dsh[sh_tok], ref)
        worst = max(worst, err.max())
        assert err.max() < TOL, ("shared down", err.max())

    # combine in the reference's order, fp64
    ref = np.zeros((T, H))
    for j in range(k):
        ref += L["wsel"][:, j:j + 1].astype(np.float64) * D[pos[:, j]].astype(np.float64)
    if tr.shared:
        ref += L["sw"][:, None].astype(np.float64) * Dsh.astype(np.float64)
    err = per_row_err(L["out"], ref)
    assert err.max() < TOL, ("combine", err.max())
    return worst


@pytest.mark.parametrize("T,act_mode", [(64, 1), (512, 1), (64, 0), (512, 0)])
def test_moe_stages_qwen35moe(ctx, orc, T, act_mode):
    """The benchmark's layer at 64 and 512 tokens, both
    activation treatments; 48 sampled experts (every row of each) and 64
    sampled tokens of the shared expert per stage."""
    H, F, E, k = 2048, 512, 256, 8
    types = (Q4K, Q4K, Q6K)
    L = run_layer(ctx, T, H, F, E, k, types, act_mode, seed=T + act_mode)
    worst = check_stages(orc, L, T, H, F, E, k, types, act_mode, n_experts=48, n_shared=64, seed=T)
    print(f"T={T} act_mode={act_mode}: worst per-row rel_l2 {worst:.2e}")


@pytest.mark.parametrize("types", [(12, 12, 14), (12, 13, 14), (8, 8, 23), (20, 20, 12), (13, 13, 8)])
@pytest.mark.parametrize("avg", ["100000", "0"])
def test_moe_stages_q8_row_both_paths(ctx, orc, monkeypatch, types, avg):
    """Per-row int8 MoE with every format, forced onto the grouped int8 GEMV
    (GGQ_MOE_GEMV_MAX_AVG large) and onto the expert-grouped GEMM
    (GGQ_MOE_GEMV_MAX_AVG=0), every stage of every expert checked."""
    monkeypatch.setenv("GGQ_MOE_GEMV_MAX_AVG", avg)
    T, H, F, E, k = 48, 512, 256, 16, 4
    for shared in (False, True):
        L = run_layer(ctx, T, H, F, E, k, types, 1, seed=sum(types) + shared, shared=shared)
        check_stages(orc, L, T, H, F, E, k, types, 1)


@pytest.mark.parametrize("types", [(12, 12, 14), (12, 13, 14), (8, 8, 23), (20, 20, 12), (13, 13, 8)])
def test_moe_stages_f32_gemm_formats(ctx, orc, monkeypatch, types):
    """fp32-activation MoE on the expert-grouped fp16 GEMM
    (GGQ_MOE_GEMV_MAX_AVG=0) with every format, paired and unpaired gate /
    up, groups of several 32-row tiles, every stage of every expert."""
    monkeypatch.setenv("GGQ_MOE_GEMV_MAX_AVG", "0")
    T, H, F, E, k = 96, 512, 256, 8, 4
    for shared in (False, True):
        L = run_layer(ctx, T, H, F, E, k, types, 0, seed=sum(types) + 7 * shared, shared=shared)
        check_stages(orc, L, T, H, F, E, k, types, 0)


@pytest.mark.parametrize("T", [1, 8, 16])
@pytest.mark.parametrize("act_mode", [0, 1])
def test_moe_stages_decode_batch(ctx, orc, T, act_mode):
    """Decode-sized batches (up to 16 tokens), where the grouping launch
    also routes the tokens and, with per-row int8 activations, quantizes
    their rows: selections, every stage of every expert and the layer
    output at the full bar."""
    H, F, E, k = 1024, 512, 32, 4
    types = (Q4K, Q4K, Q6K)
    L = run_layer(ctx, T, H, F, E, k, types, act_mode, seed=T + 100 * act_mode)
    check_stages(orc, L, T, H, F, E, k, types, act_mode)
    ref, rsel, _ = orc.moe_ffn_f64(L["x"], L["logits"], H, F, E, k, *types[:1], L["Wg"], types[1], L["Wu"],
                                   types[2], L["Wd"], *L["S"], L["sw"], act_mode=act_mode)
    assert np.array_equal(L["sel"], rsel)
    if act_mode == 0:
        assert orc.rel_l2(L["out"], ref) < TOL


@pytest.mark.parametrize("H,F,types", [(2048, 512, (Q4K, Q4K, Q6K)), (1024, 512, (Q6K, Q6K, Q6K))])
def test_moe_stages_q8_row_tiles_many_passes(ctx, orc, H, F, types):
    """Per-row int8 MoE with ~113 pair rows per expert on average (T = 384,
    16 experts, top-4 plus the shared expert), where the int8 row tiles run
    each group in several passes of 24 or 32 rows (no 32-row GEMM above a
    size bound); routing skewed so that a few experts take most rows; every
    stage of every expert at the full bar."""
    T, E, k = 384, 16, 4
    L = run_layer(ctx, T, H, F, E, k, types, 1, seed=H + 7 * F + sum(types), hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    assert int(grp[-1]) + T > 100 * (E + 1)
    assert np.diff(grp).max() > 4 * 32
    check_stages(orc, L, T, H, F, E, k, types, 1)


@pytest.mark.parametrize("H,F,T,E,types", [(1024, 256, 128, 16, (Q4K, Q4K, Q6K)), (1024, 768, 128, 16, (Q4K, Q4K, Q6K)),
                                           (1024, 512, 64, 32, (Q4K, Q4K, Q6K)), (1056, 1024, 64, 32, (8, 8, Q6K))])
def test_moe_stages_f32_down_f16_row_tiles(ctx, orc, monkeypatch, H, F, T, E, types):
    """fp32-activation MoE at prefill-sized batches (the fp16 GEMM path,
    GGQ_MOE_GEMV_MAX_AVG=0), where a Q6_K down projection runs on the row
    tiles with the SwiGLU rows as fp16 hi + lo planes: 32 rows a pass at
    K = 256, 16 at K = 512, 768 and 1024 (N = 1056: a partial 128-row
    tile); routing skewed so that a few experts take several passes; every
    stage of every expert."""
    monkeypatch.setenv("GGQ_MOE_GEMV_MAX_AVG", "0")
    k = 4
    L = run_layer(ctx, T, H, F, E, k, types, 0, seed=F + T + E, hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    assert np.diff(grp).max() > 32
    check_stages(orc, L, T, H, F, E, k, types, 0)


@pytest.mark.parametrize("E", [300, 1023])
@pytest.mark.parametrize("act_mode", [0, 1])
def test_moe_stages_many_experts_shared(ctx, orc, monkeypatch, E, act_mode):
    """More than 256 experts with a shared expert (E = 1023: 1024 groups with
    it), where the grouping launch is the chunked counting sort, which builds
    no chunk lists: the grouped int8 launches then build their own
    (i8_chunks_kernel), with the shared expert's rows written by that kernel
    in fp32 mode (GGQ_MOE_I8=1) and by the tile-list kernel in per-row int8
    mode (the grouped int8 GEMV forced by GGQ_MOE_GEMV_MAX_AVG)."""
    monkeypatch.setenv("GGQ_MOE_I8", "1")
    monkeypatch.setenv("GGQ_MOE_GEMV_MAX_AVG", "100000")
    T, H, F, k = 40, 256, 256, 4
    types = (Q4K, Q4K, Q6K)
    L = run_layer(ctx, T, H, F, E, k, types, act_mode, seed=E + act_mode)
    check_stages(orc, L, T, H, F, E, k, types, act_mode, n_experts=64, seed=E)
    ref, rsel, _ = orc.moe_ffn_f64(L["x"], L["logits"], H, F, E, k, *types[:1], L["Wg"], types[1], L["Wu"],
                                   types[2], L["Wd"], *L["S"], L["sw"], act_mode=act_mode)
    assert np.array_equal(L["sel"], rsel)
    if act_mode == 0:
        assert orc.rel_l2(L["out"], ref) < TOL


@pytest.mark.parametrize("H,F,types", [(2048, 512, (Q4K, Q4K, Q6K)), (1024, 256, (Q4K, Q4K, Q6K)),
                                       (1024, 768, (Q4K, Q4K, Q6K)), (1024, 1024, (Q4K, Q4K, Q6K)),
                                       (1056, 512, (8, 8, Q6K))])
def test_moe_stages_f32_down_row_tiles(ctx, orc, H, F, types):
    """fp32 MoE at decode-sized batches with a Q6_K down projection, which
    runs on the expert-grouped row tiles (4 pair rows per pass): K = F of
    1, 2, 3 and 4 Q6_K blocks, N = H a multiple of the 128-row tile or not
    (1056), and routing skewed so that a few experts take many rows (several
    passes over their weights) next to experts with none, plus the shared
    expert's rows (8 passes); every stage of every expert."""
    T, E, k = 32, 32, 4
    L = run_layer(ctx, T, H, F, E, k, types, 0, seed=H + F, hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    assert np.diff(grp).max() > 8 and (np.diff(grp) == 0).any()
    check_stages(orc, L, T, H, F, E, k, types, 0)


@pytest.mark.parametrize("H,F,types", [(1024, 512, (Q4K, Q4K, Q6K)), (1024, 512, (Q4K, Q4K, Q4K)),
                                       (1024, 768, (Q6K, Q6K, Q6K)), (2048, 256, (Q4K, Q4K, Q6K)),
                                       (1056, 512, (8, 8, Q6K))])
def test_moe_stages_q8_row_tiles(ctx, orc, H, F, types):
    """Per-row int8 MoE between 3 and 12 pair rows per expert on average,
    where Q4_K / Q6_K gate+up and down run on the int8 row tiles with 16
    rows of an expert per pass: K = 256..2048, N a multiple of the 128-row tile
    or not (1056), routing skewed so that a few experts take several passes
    next to experts with none; every stage of every expert at the full bar."""
    T, E, k = 64, 48, 4
    L = run_layer(ctx, T, H, F, E, k, types, 1, seed=H + 3 * F + sum(types), hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    assert np.diff(grp).max() > 16 and (np.diff(grp) == 0).any()
    check_stages(orc, L, T, H, F, E, k, types, 1)


@pytest.mark.parametrize("H,F,types", [(1024, 512, (Q4K, Q4K, Q6K)), (2048, 768, (Q6K, Q6K, Q4K)),
                                       (1056, 512, (8, 8, Q6K))])
def test_moe_stages_q8_row_tiles_narrow(ctx, orc, H, F, types):
    """Per-row int8 MoE between 1 and 4 pair rows per expert on average
    (T = 36, 64 experts, top-4 plus the shared expert: 2.8 rows per group),
    where Q4_K / Q6_K launches run on the int8 row tiles with 8 rows of an
    expert per pass (the Q8_0 gate / up of the last case on the grouped
    GEMV); routing skewed so that a few experts take several passes next
    to experts with none; every stage of every expert at the full bar."""
    T, E, k = 36, 64, 4
    L = run_layer(ctx, T, H, F, E, k, types, 1, seed=H + 11 * F + sum(types), hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    rows = int(grp[-1]) + T
    assert (E + 1) < rows <= 3 * (E + 1)
    assert np.diff(grp).max() > 8 and (np.diff(grp) == 0).any()
    check_stages(orc, L, T, H, F, E, k, types, 1)


@pytest.mark.parametrize("H,F,types", [(2048, 512, (Q4K, Q4K, Q6K)), (1024, 512, (Q4K, Q4K, Q4K)),
                                       (1024, 768, (Q6K, Q6K, Q6K)), (1056, 512, (8, 8, Q6K))])
def test_moe_stages_q8_row_tiles_wide(ctx, orc, H, F, types):
    """Per-row int8 MoE between 12 and 24 pair rows per expert on average
    (T = 128, 32 experts, top-4 plus the shared expert: 19 rows per group),
    where the int8 row tiles carry 24 or 32 rows of an expert per pass:
    Q4_K gate+up at K = 2048 with 24 rows and at K = 1024 with 32 (the min
    term on the f32 MFMA from the staged code sums), Q6_K gate+up at
    K = 1024 and Q4_K / Q6_K down with 32; routing skewed so that a few
    experts take several passes; every stage of every expert at the full
    bar."""
    T, E, k = 128, 32, 4
    L = run_layer(ctx, T, H, F, E, k, types, 1, seed=H + 5 * F + sum(types), hot=3)
    grp = d2h(L["tr"].grp, (E + 1,), np.int32)
    rows = int(grp[-1]) + T
    assert 12 * (E + 1) < rows <= 24 * (E + 1)
    assert np.diff(grp).max() > 32
    check_stages(orc, L, T, H, F, E, k, types, 1)
