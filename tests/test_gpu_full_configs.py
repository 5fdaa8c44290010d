"""Parity at the benchmark's own shapes, launched exactly as bench.py launches
them (same entry points, same grouping of weights per call), so that the
kernel variants chosen at those shapes (grid sizes, row slots, split-K
plans, second expert passes) carry parity evidence.  Each matrix is checked
on a seeded sample of its output rows (weight rows) against the fp64 oracle
(orc_mul_mat_f64, orc_moe_ffn_f64) with the same activation treatment;
relative L2 <= 1e-4.
"""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests.gpu_util import dev, empty, host, ptr, stream_handle

pytestmark = pytest.mark.gpu

TOL = 1e-4
Q4K, Q6K, Q8_0 = 12, 14, 8
LLAMA_LAYER = [("q", Q4K, 2048, 2048), ("k", Q4K, 512, 2048), ("v", Q6K, 512, 2048),
               ("o", Q4K, 2048, 2048), ("gate", Q4K, 8192, 2048), ("up", Q4K, 8192, 2048),
               ("down", Q6K, 2048, 8192)]
QWEN_LAYER = [("q", Q8_0, 1536, 1536), ("k", Q8_0, 256, 1536), ("v", Q8_0, 256, 1536),
              ("o", Q8_0, 1536, 1536), ("gate", Q8_0, 8960, 1536), ("up", Q8_0, 8960, 1536),
              ("down", Q8_0, 1536, 8960)]


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    c = gl.Context(0)
    yield c
    c.close()


def make(t, N, K, seed):
    """Seeded N(0, 0.02) weights (drawn on the device for speed) -> blocks."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = (torch.randn((N, K), generator=g, device="cuda") * 0.02).cpu().numpy()
    return gl.encode(t, x)


def rows_of(raw, t, N, K, idx):
    rb = gl.row_bytes(t, K)
    return np.ascontiguousarray(raw.reshape(N, rb)[idx]).reshape(-1)


def sample(N, n, seed):
    if N <= n:
        return np.arange(N)
    rng = np.random.default_rng(seed)
    idx = np.sort(rng.choice(N, n, replace=False))
    idx[0], idx[-1] = 0, N - 1  # both ends of the matrix
    return np.unique(idx)


def check_rows(orc, t, raw, N, K, A, C, mode, n_rows, seed, what):
    idx = sample(N, n_rows, seed)
    ref = orc.mul_mat_f64(t, rows_of(raw, t, N, K, idx), len(idx), K, A, mode)
    err = orc.rel_l2(C[:, idx], ref)
    assert err < TOL, (what, err)
    return err


def test_decode_step_levels_as_benchmarked(ctx, orc):
    """the 65-launch step (16 layers x {q+k+v batch, o, gate+up
    batch, down} + the 128256x2048 output projection), every matrix distinct,
    each with its own fp32 input as in bench.py; 128 sampled rows per layer
    matrix and 1024 of the output projection against the oracle."""
    import torch
    rng = np.random.default_rng(21)
    layers = []
    for li in range(16):
        mats = []
        for j, (name, t, N, K) in enumerate(LLAMA_LAYER):
            raw = make(t, N, K, 1000 + 7 * li + j)
            A = rng.standard_normal((1, K)).astype(np.float32)
            mats.append(dict(name=name, t=t, N=N, K=K, raw=raw, A=A, dW=dev(raw), dA=dev(A),
                             dC=torch.full((1, N), float("nan"), device="cuda")))
        layers.append(mats)
    t, N, K = Q4K, 128256, 2048
    raw = make(t, N, K, 77)
    A = rng.standard_normal((1, K)).astype(np.float32)
    out = dict(name="output", t=t, N=N, K=K, raw=raw, A=A, dW=dev(raw), dA=dev(A),
               dC=torch.full((1, N), float("nan"), device="cuda"))
    s = stream_handle()

    def single(m):
        ctx.check(ctx.lib.ggq_mul_mat_dev(ctx.h, ptr(m["dW"]), m["t"], m["N"], m["K"], ptr(m["dA"]), m["K"],
                                          ptr(m["dC"]), m["N"], 1, 0, s), m["name"])

    def batch(ms):
        d = (gl.GemvDesc * len(ms))()
        for i, m in enumerate(ms):
            d[i].W, d[i].type, d[i].N, d[i].K = m["dW"].data_ptr(), m["t"], m["N"], m["K"]
            d[i].A, d[i].C = m["dA"].data_ptr(), m["dC"].data_ptr()
        ctx.check(ctx.lib.ggq_mul_mat_batch_dev(ctx.h, d, len(ms), s), "batch")

    for q, k, v, o, g, u, dn in layers:
        batch([q, k, v])
        single(o)
        batch([g, u])
        single(dn)
    single(out)
    torch.cuda.synchronize()
    worst = 0.0
    for li, mats in enumerate(layers):
        for m in mats:
            C = host(m["dC"])
            assert not np.isnan(C).any(), (li, m["name"])
            worst = max(worst, check_rows(orc, m["t"], m["raw"], m["N"], m["K"], m["A"], C, 0, 128,
                                          li * 10 + len(m["name"]), f"layer {li} {m['name']}"))
    C = host(out["dC"])
    assert not np.isnan(C).any()
    worst = max(worst, check_rows(orc, t, raw, N, K, A, C, 0, 1024, 5, "output projection"))
    print(f"decode step: worst rel_l2 {worst:.2e}")


def test_prefill_layer_as_benchmarked(ctx, orc):
    """one Qwen2.5-1.5B layer on 512 tokens as bench.py runs it:
    per-level int8 row quantization (ggq_quantize_act_dev), q+k+v and gate+up
    as ggq_mul_mat_q8_batch_dev launches (the 280-tile gate+up GEMM), o and
    down as ggq_mul_mat_q8_dev.  1024 sampled columns per matrix x 128
    sampled token rows (16 from each 64-row tile) against the oracle in
    Q8_ROW mode."""
    import torch
    T = 512
    rng = np.random.default_rng(31)
    mats = {}
    for j, (name, t, N, K) in enumerate(QWEN_LAYER):
        raw = make(t, N, K, 2000 + j)
        mats[name] = dict(t=t, N=N, K=K, raw=raw, dW=dev(raw), dC=torch.full((T, N), float("nan"), device="cuda"))
    xin = {lv: rng.standard_normal((T, K)).astype(np.float32)
           for lv, K in (("qkv", 1536), ("o", 1536), ("gu", 1536), ("down", 8960))}
    s = stream_handle()
    qin = {}
    for lv, X in xin.items():
        dX = dev(X)
        q = empty((T, X.shape[1]), torch.int8)
        sc = empty((T,), torch.float32)
        ctx.check(ctx.lib.ggq_quantize_act_dev(ctx.h, ptr(dX), X.shape[1], T, X.shape[1], 1, ptr(q), ptr(sc), s),
                  "quantize")
        qin[lv] = (dX, q, sc)

    def batch(names, lv):
        ms = [mats[n] for n in names]
        _, q, sc = qin[lv]
        d = (gl.GemmDesc * len(ms))(*[gl.GemmDesc(m["dW"].data_ptr(), m["N"], m["dC"].data_ptr(), m["N"]) for m in ms])
        ctx.check(ctx.lib.ggq_mul_mat_q8_batch_dev(ctx.h, d, len(ms), ms[0]["t"], ms[0]["K"], ptr(q), ptr(sc), T, s),
                  "q8 batch")

    def single(name, lv):
        m = mats[name]
        _, q, sc = qin[lv]
        ctx.check(ctx.lib.ggq_mul_mat_q8_dev(ctx.h, ptr(m["dW"]), m["t"], m["N"], m["K"], ptr(q), ptr(sc), T,
                                             ptr(m["dC"]), m["N"], s), "q8")

    batch(["q", "k", "v"], "qkv")
    single("o", "o")
    batch(["gate", "up"], "gu")
    single("down", "down")
    torch.cuda.synchronize()
    level = {"q": "qkv", "k": "qkv", "v": "qkv", "o": "o", "gate": "gu", "up": "gu", "down": "down"}
    rows = np.concatenate([64 * b + np.sort(np.random.default_rng(b).choice(64, 16, replace=False)) for b in range(8)])
    for name, m in mats.items():
        C = host(m["dC"])
        assert not np.isnan(C).any(), name
        A = xin[level[name]][rows]
        check_rows(orc, m["t"], m["raw"], m["N"], m["K"], A, C[rows], 1, 1024, len(name), name)


@pytest.mark.parametrize("T,act_mode,n_check", [(64, 0, 64), (512, 1, 128), (64, 1, 64)])
def test_moe_layer_as_benchmarked(ctx, orc, T, act_mode, n_check):
    """the qwen35moe-A3B MoE layer at the benchmark's 64 tokens
    (E 256, FFN 512, top-8, Q4_K gate/up, Q6_K down, sigmoid-weighted shared
    expert), one ggq_moe_ffn_dev call, every token against the oracle; and
    the prefill-sized batch of 512 tokens with per-row int8 activations (the
    grouped int8 GEMM path), a seeded sample of its tokens against the
    oracle's per-token loop in the same mode (tokens are independent)."""
    import torch
    H, F, E, k = 2048, 512, 256, 8
    Wg, Wu, Wd = make(Q4K, E * F, H, 51), make(Q4K, E * F, H, 52), make(Q6K, E * H, F, 53)
    Sg, Su, Sd = make(Q4K, F, H, 54), make(Q4K, F, H, 55), make(Q6K, H, F, 56)
    rng = np.random.default_rng(57)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    sw = (1.0 / (1.0 + np.exp(-rng.standard_normal(T)))).astype(np.float32)
    keep = [dev(a) for a in (x, logits, Wg, Wu, Wd, Sg, Su, Sd, sw)]
    out = empty((T, H), torch.float32)
    sel = empty((T, k), torch.int32)
    p = gl.MoeParams()
    p.T, p.H, p.F, p.E, p.top_k = T, H, F, E, k
    p.x, p.router_logits = keep[0].data_ptr(), keep[1].data_ptr()
    p.gate_type, p.up_type, p.down_type = Q4K, Q4K, Q6K
    p.gate_exps, p.up_exps, p.down_exps = keep[2].data_ptr(), keep[3].data_ptr(), keep[4].data_ptr()
    p.gate_shexp, p.up_shexp, p.down_shexp = keep[5].data_ptr(), keep[6].data_ptr(), keep[7].data_ptr()
    p.shared_w, p.out, p.sel_experts = keep[8].data_ptr(), out.data_ptr(), sel.data_ptr()
    ctx.check(ctx.lib.ggq_moe_ffn_act_dev(ctx.h, ctypes.byref(p), act_mode, stream_handle()), "moe")
    got, gsel = host(out), host(sel)
    counts = np.bincount(gsel.reshape(-1), minlength=E)
    assert counts.max() > 4, "expected an expert with a second pass of token rows"
    rows = np.sort(np.random.default_rng(T).choice(T, n_check, replace=False))
    ref, rsel, _ = orc.moe_ffn_f64(x[rows], logits[rows], H, F, E, k, Q4K, Wg, Q4K, Wu, Q6K, Wd, Sg, Su, Sd, sw[rows],
                                   act_mode=act_mode)
    assert np.array_equal(gsel[rows], rsel)
    if act_mode == 1:  # two quantized stages: see assert_q8_moe_close
        from tests.test_gpu_parity import assert_q8_moe_close
        assert_q8_moe_close(orc, got[rows], ref)
        return
    err = orc.rel_l2(got[rows], ref)
    assert err < TOL, err
    for i, t in enumerate(rows):
        assert orc.rel_l2(got[t], ref[i]) < TOL, t


IQ4NL, IQ4XS, Q5K = 20, 23, 13
QWEN3_LAYER = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
               ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072)]


@pytest.mark.parametrize("M", [1, 4, 8])
def test_config4_layer_as_benchmarked(ctx, orc, M):
    """one Qwen3-0.6B layer (types [IQ4_NL, IQ4_XS, Q5_K][i % 3]
    over q, k, v, o, gate, up, down) with M = 1, 4 and 8 fp32 activation rows,
    one ggq_mul_mat_batch_rows_dev launch per dependency level (q+k+v, o,
    gate+up, down) exactly as bench.py's bench_config4 launches them (q/k/v
    sharing one input, gate/up another), eagerly and then as a captured HIP
    graph replayed on fresh inputs; 512 sampled weight rows of every matrix
    (all rows up to 512) against the fp64 oracle, every activation row."""
    import torch
    cycle = [IQ4NL, IQ4XS, Q5K]
    rng = np.random.default_rng(40 + M)
    mats = []
    for i, (name, N, K) in enumerate(QWEN3_LAYER):
        t = cycle[i % 3]
        raw = make(t, N, K, 4000 + 10 * M + i)
        mats.append(dict(name=name, t=t, N=N, K=K, raw=raw, dW=dev(raw),
                         dC=torch.full((M, N), float("nan"), device="cuda")))
    ins = {lv: torch.empty((M, K), device="cuda") for lv, K in (("attn", 1024), ("o", 2048), ("ffn", 1024),
                                                                 ("down", 3072))}
    which = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "ffn", "up": "ffn", "down": "down"}
    levels = [mats[0:3], mats[3:4], mats[4:6], mats[6:7]]
    descs = []
    for lv in levels:
        arr = (gl.GemvDesc * len(lv))()
        for i, m in enumerate(lv):
            arr[i].W, arr[i].type, arr[i].N, arr[i].K = m["dW"].data_ptr(), m["t"], m["N"], m["K"]
            arr[i].A, arr[i].C = ins[which[m["name"]]].data_ptr(), m["dC"].data_ptr()
        descs.append((arr, len(lv)))

    def run_on(s):
        for arr, n in descs:
            ctx.check(ctx.lib.ggq_mul_mat_batch_rows_dev(ctx.h, arr, n, M, s), "batch rows")

    def check(tag):
        torch.cuda.synchronize()
        for j, m in enumerate(mats):
            C = host(m["dC"])
            assert not np.isnan(C).any(), (tag, m["name"])
            A = host(ins[which[m["name"]]])
            check_rows(orc, m["t"], m["raw"], m["N"], m["K"], A, C, 0, 512, j, f"{tag} M={M} {m['name']}")
            m["dC"].fill_(float("nan"))

    for x in ins.values():
        x.copy_(torch.from_numpy(rng.standard_normal(tuple(x.shape)).astype(np.float32)))
    run_on(stream_handle())
    check("eager")
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run_on(ctypes.c_void_p(s.cuda_stream))
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            run_on(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for rep in range(2):
        for x in ins.values():
            x.copy_(torch.from_numpy(rng.standard_normal(tuple(x.shape)).astype(np.float32)))
        torch.cuda.synchronize()
        g.replay()
        check(f"graph replay {rep}")
    del g
