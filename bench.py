"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline workload: the matmuls of one Llama-3.2-1B
decode step in the Q4_K_M layout -- 16 layers x {q, k, v, o, gate, up, down}
(Q4_K, with attn_v and ffn_down in Q6_K) plus the 128256-row output projection
-- batch 1, fp32 activations.  One "step" = those 113 GEMVs over weights that
are resident in HBM (raw GGUF blocks, never re-quantized).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--graph] [--no-extra]

Prints one JSON line.  `value` is HBM GB/s over the algorithmic bytes of the
step (raw weight bytes + fp32 activation-in + fp32 output bytes).  Extra keys:
  roofline      the GEMV kernel's per-launch time measured with HIP events on
                the launch stream, vs the 8 TB/s HBM peak
  cpu_baseline  the single-core CPU restatement of the reference's
                CpuRefBackend::mul_mat_q on layer 0 of the same workload
  extra         config 1 (single Q4_K GEMV, weights rotated over 32 copies to
                defeat the 256 MB MALL) and config 3 (Qwen2.5-1.5B 512-token
                Q8_0 prefill, int8 TOPS on MFMA)
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import ggnpu_amd.lib as gl  # noqa: E402

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0

Q4K, Q6K, Q8_0 = int(gl.GgmlType.Q4_K), int(gl.GgmlType.Q6_K), int(gl.GgmlType.Q8_0)

# (name, type, N, K) per layer -- configs[1]
LLAMA_LAYER = [("q", Q4K, 2048, 2048), ("k", Q4K, 512, 2048), ("v", Q6K, 512, 2048),
               ("o", Q4K, 2048, 2048), ("gate", Q4K, 8192, 2048), ("up", Q4K, 8192, 2048),
               ("down", Q6K, 2048, 8192)]
LLAMA_LAYERS = 16
LLAMA_OUTPUT = ("output", Q4K, 128256, 2048)
# Qwen2.5-1.5B, hidden 1536, FFN 8960, 12 q / 2 kv heads of 128
QWEN_LAYER = [("q", Q8_0, 1536, 1536), ("k", Q8_0, 256, 1536), ("v", Q8_0, 256, 1536),
              ("o", Q8_0, 1536, 1536), ("gate", Q8_0, 8960, 1536), ("up", Q8_0, 8960, 1536),
              ("down", Q8_0, 1536, 8960)]
QWEN_LAYERS = 28
PREFILL_TOKENS = 512


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Mat:
    """One resident weight matrix plus its activation / output buffers."""

    def __init__(self, torch, name, t, N, K, raw_dev, M=1, x=None):
        self.name, self.t, self.N, self.K, self.M = name, t, N, K, M
        self.w = raw_dev
        self.x = x if x is not None else torch.randn((M, K), device="cuda", dtype=torch.float32)
        self.y = torch.empty((M, N), device="cuda", dtype=torch.float32)

    def bytes(self):
        return gl.row_bytes(self.t, self.K) * self.N + 4 * self.M * (self.K + self.N)


def make_weight(torch, gen, t, N, K):
    """Seeded N(0, 0.02) fp32 values -> GGUF blocks (host encoder) -> HBM."""
    x = (torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02).cpu().numpy()
    raw = gl.encode(t, x)
    dev = torch.zeros(raw.size + 256, dtype=torch.uint8, device="cuda")
    dev[: raw.size].copy_(torch.from_numpy(raw))
    return dev, raw


def launch_batch(ctx, ms, stream):
    """Independent M=1 matmuls of one dependency level in one call."""
    descs = (gl.GemvDesc * len(ms))()
    for i, m in enumerate(ms):
        descs[i].W, descs[i].type, descs[i].N, descs[i].K = m.w.data_ptr(), m.t, m.N, m.K
        descs[i].A, descs[i].C = m.x.data_ptr(), m.y.data_ptr()
    st = ctx.lib.ggq_mul_mat_batch_dev(ctx.h, descs, len(ms), stream)
    if st != 0:
        ctx.check(st, "mul_mat_batch_dev")


def launch(ctx, m, act_mode, stream):
    st = ctx.lib.ggq_mul_mat_dev(ctx.h, ctypes.c_void_p(m.w.data_ptr()), m.t, m.N, m.K,
                                 ctypes.c_void_p(m.x.data_ptr()), m.K, ctypes.c_void_p(m.y.data_ptr()), m.N,
                                 m.M, act_mode, stream)
    if st != 0:
        ctx.check(st, f"mul_mat_dev {m.name}")


def time_steps(torch, fn, steps, warmup, gpu_time=False):
    """Wall seconds per step over `steps` steps after `warmup` (synchronize
    on both sides).  With gpu_time, also the GPU seconds per step from HIP
    events recorded on the launch stream (torch's current stream) at the two
    ends of the same timed region."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    if gpu_time:
        return wall, e0.elapsed_time(e1) / 1e3 / steps
    return wall


def back_to_back_times(torch, fns, reps):
    """Mean GPU seconds per call of each callable, from HIP events around
    `reps` back-to-back calls queued behind a ~1 ms spin kernel, so that the
    queue is full when the first call starts and host submission time is not
    counted (repeated small weights are partly served from cache)."""
    out = []
    for fn in fns:
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(2_000_000)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / 1e3 / reps)
    return out


def bench_decode_step(torch, ctx, steps, warmup, use_graph, stream, fuse_levels=True, probe_levels=True):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    mats, host_layer0 = [], []
    t0 = time.time()
    for layer in range(LLAMA_LAYERS):
        # q/k/v read one normed input and gate/up another, as in a forward pass.
        shared = {n: torch.randn((1, 2048), device="cuda", dtype=torch.float32) for n in ("attn", "ffn")}
        for name, t, N, K in LLAMA_LAYER:
            dev, raw = make_weight(torch, gen, t, N, K)
            x = shared["attn"] if name in ("q", "k", "v") else shared["ffn"] if name in ("gate", "up") else None
            m = Mat(torch, f"blk{layer}.{name}", t, N, K, dev, x=x)
            mats.append(m)
            if layer == 0:
                host_layer0.append((m, raw))
    name, t, N, K = LLAMA_OUTPUT
    dev, _ = make_weight(torch, gen, t, N, K)
    mats.append(Mat(torch, name, t, N, K, dev))
    torch.cuda.synchronize()
    log(f"decode step: {len(mats)} matrices resident ({sum(m.bytes() for m in mats) / 1e6:.1f} MB) "
        f"in {time.time() - t0:.1f}s")

    # Dependency levels of a real decode step: q/k/v read the same normed
    # input, gate/up read the same normed residual; o, down and the output
    # projection each depend on the previous level.  One call per level.
    levels = []
    for layer in range(LLAMA_LAYERS):
        q, k, v, o, gate, up, down = mats[7 * layer: 7 * layer + 7]
        levels += [[q, k, v], [o], [gate, up], [down]]
    levels.append([mats[-1]])

    def step_levels(strm):
        for lv in levels:
            if len(lv) == 1 or not fuse_levels:
                for m in lv:
                    launch(ctx, m, 0, strm)
            else:
                launch_batch(ctx, lv, strm)

    def step():
        step_levels(stream)

    fn = step
    if use_graph:
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step_stream = ctypes.c_void_p(s.cuda_stream)
            step_levels(step_stream)  # warm the kernels outside capture
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                step_levels(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        fn = g.replay
    sec, gpu_sec = time_steps(torch, fn, steps, warmup, gpu_time=True)
    step_bytes = sum(m.bytes() for m in mats)

    def level_fn(lv):
        if len(lv) == 1 or not fuse_levels:
            return lambda: [launch(ctx, m, 0, stream) for m in lv]
        return lambda: launch_batch(ctx, lv, stream)

    # Per-level breakdown of layer 0 and the output projection (diagnostic).
    if not probe_levels:
        return levels, host_layer0, sec, gpu_sec, step_bytes, []
    probe = levels[:4] + [levels[-1]]
    kt = back_to_back_times(torch, [level_fn(lv) for lv in probe], reps=10)
    return levels, host_layer0, sec, gpu_sec, step_bytes, list(zip(probe, kt))


def bench_config1(torch, ctx, stream, reps=200, act_mode=0):
    """Single Q4_K GEMV 8192x2048; 32 distinct HBM copies rotated.  act_mode
    0 = fp32 activations, 1 = per-row int8 activations (GGQ_ACT_Q8_ROW)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    dev, _ = make_weight(torch, gen, Q4K, 8192, 2048)
    copies = [dev.clone() for _ in range(32)]
    x = torch.randn((1, 2048), device="cuda")
    mats = [Mat(torch, f"c1.{i}", Q4K, 8192, 2048, c, x=x) for i, c in enumerate(copies)]

    def run():
        for m in mats:
            launch(ctx, m, act_mode, stream)

    sec, gsec = time_steps(torch, run, max(1, reps // 32), 2, gpu_time=True)
    sec /= len(mats)
    kmean = gsec / len(mats)
    b = mats[0].bytes()
    act = "fp32" if act_mode == 0 else "per-row int8 (GGQ_ACT_Q8_ROW)"
    return {"workload": f"Q4_K GEMV 8192x2048 batch 1, {act} activations (32 rotated copies)", "bytes_per_call": b,
            "us_per_call_wall": sec * 1e6, "us_per_call_gpu_event": kmean * 1e6,
            "GBps": b / kmean / 1e9, "frac_hbm_peak": b / kmean / 1e9 / HBM_PEAK_GBS}


def bench_decode_levels(torch, ctx, levels, stream, act_mode, steps=30):
    """The decode step's levels again with another activation treatment:
    one ggq_mul_mat_batch_act_dev call per dependency level."""
    calls = []
    for lv in levels:
        descs = (gl.GemvDesc * len(lv))()
        for i, m in enumerate(lv):
            descs[i].W, descs[i].type, descs[i].N, descs[i].K = m.w.data_ptr(), m.t, m.N, m.K
            descs[i].A, descs[i].C = m.x.data_ptr(), m.y.data_ptr()
        calls.append((descs, len(lv)))

    def run():
        for descs, n in calls:
            st = ctx.lib.ggq_mul_mat_batch_act_dev(ctx.h, descs, n, 1, act_mode, stream)
            if st != 0:
                ctx.check(st, "mul_mat_batch_act_dev")

    sec, gsec = time_steps(torch, run, steps, 3, gpu_time=True)
    b = sum(m.bytes() for lv in levels for m in lv)
    return {"workload": "configs[1] decode step, per-row int8 activations (GGQ_ACT_Q8_ROW), one call per level",
            "ms_per_step": round(sec * 1e3, 4), "GBps": round(b / sec / 1e9, 1),
            "kernel_us_per_step": round(gsec * 1e6, 1), "frac_hbm_peak": round(b / gsec / 1e9 / HBM_PEAK_GBS, 4)}


def bench_decode_fused(torch, ctx, stream, steps=30):
    """configs[1]'s matmuls with their neighbours fused in (ggq_mul_mat_fused_dev):
    per layer RMSNorm + q/k/v (one launch), o + residual add, RMSNorm +
    gate (silu epilogue) / up (one launch), down reading silu(gate) * up +
    residual add; then
    RMSNorm + output projection.  65 launches, as the matmul-only step.  Attention is out of
    scope: o reads a synthetic attention output."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    H, F = 2048, 8192
    x = torch.randn((1, H), device="cuda", generator=gen)
    attn = torch.randn((1, H), device="cuda", generator=gen)
    gbuf = torch.empty((1, F), device="cuda")
    ubuf = torch.empty((1, F), device="cuda")
    nw = 1.0 + 0.1 * torch.randn((H,), device="cuda", generator=gen)
    q, k, v = (torch.empty((1, n), device="cuda") for n in (2048, 512, 512))
    logits = torch.empty((1, LLAMA_OUTPUT[2]), device="cuda")
    layers, total = [], 0
    for _ in range(LLAMA_LAYERS):
        ws = {}
        for name, t, N, K in LLAMA_LAYER:
            ws[name], raw = make_weight(torch, gen, t, N, K)
            total += raw.size
        layers.append(ws)
    wout, raw = make_weight(torch, gen, Q4K, LLAMA_OUTPUT[2], H)
    total += raw.size

    def desc(w, t, N, K, A, C, **kw):
        d = gl.GemvFusedDesc()
        d.W, d.type, d.N, d.K, d.A, d.C = w.data_ptr(), t, N, K, A.data_ptr(), C.data_ptr()
        if "up" in kw:
            d.A_up = kw["up"].data_ptr()
        d.silu = int(bool(kw.get("silu")))
        if kw.get("rms"):
            d.rms_norm, d.rms_eps, d.rms_w = 1, 1e-5, nw.data_ptr()
        if kw.get("res") is not None:
            d.residual = kw["res"].data_ptr()
        return d

    plan = []
    for ws in layers:
        plan.append([desc(ws["q"], Q4K, 2048, H, x, q, rms=True), desc(ws["k"], Q4K, 512, H, x, k, rms=True),
                     desc(ws["v"], Q6K, 512, H, x, v, rms=True)])
        plan.append([desc(ws["o"], Q4K, H, H, attn, x, res=x)])
        plan.append([desc(ws["gate"], Q4K, F, H, x, gbuf, rms=True, silu=True),
                     desc(ws["up"], Q4K, F, H, x, ubuf, rms=True)])
        plan.append([desc(ws["down"], Q6K, H, F, gbuf, x, up=ubuf, res=x)])
    plan.append([desc(wout, Q4K, LLAMA_OUTPUT[2], H, x, logits, rms=True)])
    arrays = [((gl.GemvFusedDesc * len(lv))(*lv), len(lv)) for lv in plan]

    def run():
        for arr, n in arrays:
            ctx.check(ctx.lib.ggq_mul_mat_fused_dev(ctx.h, arr, n, 1, stream), "fused")

    sec, gsec = time_steps(torch, run, steps, 3, gpu_time=True)
    return {"workload": "Llama-3.2-1B decode matmuls with RMSNorm / SwiGLU / residual fused in (65 launches)",
            "weight_bytes": total, "ms_per_step": round(sec * 1e3, 4), "gpu_ms_per_step": round(gsec * 1e3, 4),
            "GBps": round(total / gsec / 1e9, 1)}


def bench_launch_floor(torch, n=65, reps=20):
    """Per-launch floor of a step built from n dependent launches (the decode
    step has 65): a HIP graph of n one-element kernels, and of n copies of
    1 MB (1024 workgroups' worth), each launch depending on the previous one;
    GPU time per launch from events around graph replays (no CPU launch cost
    in the timed region)."""
    out = {}
    for name, nbytes in (("tiny", 4), ("copy_1MB", 1 << 20)):
        a = torch.zeros(nbytes // 4, device="cuda")
        b = torch.zeros_like(a)
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            for _ in range(3):
                for i in range(n):
                    (b if i % 2 else a).copy_(a if i % 2 else b)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                (b if i % 2 else a).copy_(a if i % 2 else b)
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(torch.cuda.current_stream())
        for _ in range(reps):
            g.replay()
        e1.record(torch.cuda.current_stream())
        e1.synchronize()
        out[name] = {"us_per_launch": round(e0.elapsed_time(e1) * 1e3 / (reps * n), 2)}
    out["workload"] = f"{n} dependent launches in a HIP graph: one-element copies and 1 MB copies"
    return out


def bench_logits(torch, ctx, stream, reps=50):
    """Output projection of configs[1] (128256x2048 Q4_K, batch 1) alone and
    with the device-side greedy token choice (ggq_logits_argmax_dev, logits
    not kept): GPU time per call from events around back-to-back calls."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    name, t, N, K = LLAMA_OUTPUT
    w, _ = make_weight(torch, gen, t, N, K)
    m = Mat(torch, name, t, N, K, w)
    tok = torch.empty((1,), dtype=torch.int32, device="cuda")

    def argmax():
        ctx.check(ctx.lib.ggq_logits_argmax_dev(ctx.h, ctypes.c_void_p(w.data_ptr()), t, N, K,
                                                ctypes.c_void_p(m.x.data_ptr()), 1, 0, None,
                                                ctypes.c_void_p(tok.data_ptr()), None, stream), "argmax")

    plain, fused = back_to_back_times(torch, [lambda: launch(ctx, m, 0, stream), argmax], reps)
    return {"workload": "128256x2048 Q4_K projection, batch 1", "gemv_us": round(plain * 1e6, 2),
            "gemv_argmax_us": round(fused * 1e6, 2), "GBps_with_argmax": round(m.bytes() / fused / 1e9, 1)}


def bench_attention(torch, ctx, stream, reps=50):
    """Decode attention of one token over a layer's KV cache
    (ggq_attention_decode_dev), Llama-3.2-1B heads (32 query heads, 8 kv
    heads, head_dim 64) at contexts 1024 / 4096 / 16384, and Llama-3-8B heads
    (head_dim 128) at 4096.  Algorithmic bytes: K and V of the visible
    positions once (2 * ctx * n_kv * head_dim * 4) plus q and out."""
    res = {}
    for tag, n_head, n_kv, hd, ctx_len in (("1b_ctx1024", 32, 8, 64, 1024), ("1b_ctx4096", 32, 8, 64, 4096),
                                           ("1b_ctx16384", 32, 8, 64, 16384), ("8b_ctx4096", 32, 8, 128, 4096)):
        q = torch.randn((1, n_head, hd), device="cuda")
        Kc = torch.randn((ctx_len, n_kv, hd), device="cuda")
        Vc = torch.randn((ctx_len, n_kv, hd), device="cuda")
        out = torch.empty_like(q)

        def run():
            ctx.check(ctx.lib.ggq_attention_decode_dev(ctx.h, ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(Kc.data_ptr()),
                                                       ctypes.c_void_p(Vc.data_ptr()), 1, n_head, n_kv, hd, ctx_len,
                                                       ctx_len - 1, ctypes.c_void_p(out.data_ptr()), stream), "attn")

        (sec,) = back_to_back_times(torch, [run], reps)
        nbytes = 2 * ctx_len * n_kv * hd * 4 + 2 * n_head * hd * 4
        res[tag] = {"us": round(sec * 1e6, 2), "GBps": round(nbytes / sec / 1e9, 1)}
    return {"workload": "decode attention, 1 token, fp32 KV cache", **res}


def bench_host_api(torch, ctx, stream, steps=5, warmup=2):
    """configs[1] through the drop-in entry point the reference's backend
    calls, ggq_mul_mat_q (MulMatParams with host A, B and C, synchronous):
    113 calls per step, one per matmul as main.cpp issues them.  B is the
    host copy of the raw blocks; the first call of each uploads it to HBM
    and later calls find it resident (keyed by pointer).  Each call copies
    A in and C out over PCIe and waits: this is the PCIe-inclusive rate, not
    the benchmark value."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    host = []
    for layer in range(LLAMA_LAYERS):
        for name, t, N, K in LLAMA_LAYER:
            x = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).cpu().numpy()
            host.append((t, N, K, gl.encode(t, x)))
    t, N, K = LLAMA_OUTPUT[1:]
    x = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).cpu().numpy()
    host.append((t, N, K, gl.encode(t, x)))
    rng = np.random.default_rng(5)
    acts = {K: rng.standard_normal(K).astype(np.float32) for K in {h[2] for h in host}}
    outs = [np.empty(N, np.float32) for _, N, _, _ in host]
    params = []
    for (t, N, K, raw), out in zip(host, outs):
        p = gl.MulMatParams()
        p.A, p.B, p.C = acts[K].ctypes.data, raw.ctypes.data, out.ctypes.data
        p.M, p.N, p.K, p.n_batches, p.B_type = 1, N, K, 1, t
        params.append(p)

    def step():
        for p in params:
            st = ctx.lib.ggq_mul_mat_q(ctx.h, ctypes.byref(p), 0)
            if st != 0:
                ctx.check(st, "mul_mat_q")

    for _ in range(warmup):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    sec_py = (time.perf_counter() - t0) / steps
    # The same calls from a C++ loop (the reference's caller is C++): the
    # driver gets the entry point of the library already loaded here.
    drv = ctypes.CDLL(os.path.join(os.path.dirname(gl.LIB_PATH), "libggq_host_bench.so"))
    drv.ggq_host_bench_run.restype = ctypes.c_int
    drv.ggq_host_bench_run.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    arr = (gl.MulMatParams * len(params))(*params)
    sec = ctypes.c_double(0.0)
    ctx.check(drv.ggq_host_bench_run(ctypes.cast(ctx.lib.ggq_mul_mat_q, ctypes.c_void_p), ctx.h, arr, len(params), 0,
                                     warmup, steps, ctypes.byref(sec)), "host bench")
    sec = sec.value
    nbytes = sum(gl.row_bytes(t, K) * N + 4 * (K + N) for t, N, K, _ in host)
    return {"workload": "configs[1] decode step as 113 synchronous ggq_mul_mat_q calls (host A/B/C, weights "
                        "resident after the first call), issued from a C++ loop",
            "ms_per_step": round(sec * 1e3, 3), "GBps": round(nbytes / sec / 1e9, 1),
            "us_per_call": round(sec * 1e6 / len(params), 2),
            "us_per_call_from_python": round(sec_py * 1e6 / len(params), 2)}


def bench_prefill(torch, ctx, stream, steps=3, fused=False):
    """28 layers of Q8_0 matmuls on 512 tokens, per-row int8
    activations (reference XDNA semantics).  Each layer quantizes its four
    distinct inputs once (q/k/v share one, gate/up share one; o and down
    have their own), as a forward pass would, and the quantization kernels
    are inside the timed region.  int8-MFMA GEMM; weights sharing an input
    run as one launch (ggq_mul_mat_q8_batch_dev).  fused=True instead calls
    ggq_mul_mat_batch_act_dev per level on the fp32 inputs (quantization
    inside the GEMM launch where K <= 2048)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2)
    layer = []
    for name, t, N, K in QWEN_LAYER:
        dev, _ = make_weight(torch, gen, t, N, K)
        layer.append((name, t, N, K, dev))
    T = PREFILL_TOKENS
    # four distinct fp32 inputs per layer and their int8 buffers
    xin = {lv: torch.randn((T, K), device="cuda") for lv, K in (("qkv", 1536), ("o", 1536), ("gu", 1536), ("down", 8960))}
    qin = {lv: (torch.empty((T, x.shape[1]), dtype=torch.int8, device="cuda"), torch.empty((T,), device="cuda"))
           for lv, x in xin.items()}
    qmode = int(gl.ActMode.Q8_ROW)
    mm_single = ctx.lib.ggq_mul_mat_q8_dev
    mm_multi = ctx.lib.ggq_mul_mat_q8_batch_dev
    level_of = {"q": "qkv", "k": "qkv", "v": "qkv", "o": "o", "gate": "gu", "up": "gu", "down": "down"}
    mats = []
    for li in range(QWEN_LAYERS):
        for name, t, N, K, dev in layer:
            w = dev if li == 0 else dev.clone()
            mats.append(Mat(torch, f"blk{li}.{name}", t, N, K, w, M=T, x=xin[level_of[name]]))

    def quant(lv):
        x = xin[lv]
        q, sc = qin[lv]
        st = ctx.lib.ggq_quantize_act_dev(ctx.h, ctypes.c_void_p(x.data_ptr()), x.shape[1], T, x.shape[1], qmode,
                                          ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(sc.data_ptr()), stream)
        ctx.check(st, "quantize_act")

    def mm(m):
        q, sc = qin[level_of[m.name.split(".")[1]]]
        st = mm_single(ctx.h, ctypes.c_void_p(m.w.data_ptr()), m.t, m.N, m.K,
                       ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(sc.data_ptr()), T,
                       ctypes.c_void_p(m.y.data_ptr()), m.N, stream)
        ctx.check(st, "mul_mat_q8(h)_dev")

    def mm_batch(ms):
        """Weights sharing one quantized input: one multi-weight launch."""
        q, sc = qin[level_of[ms[0].name.split(".")[1]]]
        descs = (gl.GemmDesc * len(ms))(*[gl.GemmDesc(m.w.data_ptr(), m.N, m.y.data_ptr(), m.N) for m in ms])
        st = mm_multi(ctx.h, descs, len(ms), ms[0].t, ms[0].K,
                      ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(sc.data_ptr()), T, stream)
        ctx.check(st, "mul_mat_q8(h)_batch_dev")

    def run_given_codes():
        for li in range(QWEN_LAYERS):
            lm = mats[7 * li: 7 * li + 7]
            quant("qkv")
            mm_batch(lm[:3])
            quant("o")
            mm(lm[3])
            quant("gu")
            mm_batch(lm[4:6])
            quant("down")
            mm(lm[6])

    # Each dependency level as one ggq_mul_mat_batch_act_dev call on the fp32
    # input (the reference's mul_mat_q quantizes inside the call).
    level_descs = []
    for li in range(QWEN_LAYERS):
        lm = mats[7 * li: 7 * li + 7]
        for ms in (lm[:3], lm[3:4], lm[4:6], lm[6:7]):
            arr = (gl.GemvDesc * len(ms))()
            for i, m in enumerate(ms):
                arr[i].W, arr[i].type, arr[i].N, arr[i].K = m.w.data_ptr(), m.t, m.N, m.K
                arr[i].A, arr[i].C = m.x.data_ptr(), m.y.data_ptr()
            level_descs.append((arr, len(ms)))

    def run_levels():
        for arr, n in level_descs:
            ctx.check(ctx.lib.ggq_mul_mat_batch_act_dev(ctx.h, arr, n, T, qmode, stream), "batch_act")

    run = run_levels if fused else run_given_codes
    sec = time_steps(torch, run, steps, 1)
    ops = sum(2 * m.M * m.N * m.K for m in mats)
    return {"workload": "Qwen2.5-1.5B Q8_0 prefill, 512 tokens x 28 layers, per-row int8 activations "
                        "(4 activation quantizations per layer included)",
            "int8_ops": ops, "ms_per_step": sec * 1e3, "TOPS": ops / sec / 1e12,
            "frac_int8_peak": ops / sec / 1e12 / INT8_PEAK_TOPS}


# Qwen3-0.6B, hidden 1024, FFN 3072, 16 q / 8 kv heads of 128, 28 layers;
# the type of tensor i (q, k, v, o, gate, up, down order) is [IQ4_NL, IQ4_XS, Q5_K][i % 3].
IQ4NL, IQ4XS, Q5K = int(gl.GgmlType.IQ4_NL), int(gl.GgmlType.IQ4_XS), int(gl.GgmlType.Q5_K)
QWEN3_SHAPES = [("q", 2048, 1024), ("k", 1024, 1024), ("v", 1024, 1024), ("o", 1024, 2048),
                ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072)]
QWEN3_LAYERS = 28


def bench_config4(torch, ctx, stream, steps=40):
    """28 Qwen3-0.6B layers of IQ4_NL / IQ4_XS / Q5_K matmuls with
    batch 1, 4 and 8 fp32 activation rows; one launch per dependency level
    (q/k/v, o, gate/up, down) through ggq_mul_mat_batch_rows_dev, called
    from Python per step ("us") and replayed as one captured HIP graph
    ("us_graph")."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    cycle = [IQ4NL, IQ4XS, Q5K]
    layer = []
    for i, (name, N, K) in enumerate(QWEN3_SHAPES):
        dev, _ = make_weight(torch, gen, cycle[i % 3], N, K)
        layer.append((name, cycle[i % 3], N, K, dev))
    weights = [[(n, t, N, K, d if li == 0 else d.clone()) for n, t, N, K, d in layer] for li in range(QWEN3_LAYERS)]
    res = {"workload": "Qwen3-0.6B shapes x 28 layers, types [IQ4_NL, IQ4_XS, Q5_K][i % 3] over q,k,v,o,gate,up,down",
           "types": {n: gl.GgmlType(t).name for n, t, _, _, _ in layer}}
    for M in (1, 4, 8):
        mats = []
        for li in range(QWEN3_LAYERS):
            # q/k/v share one input (K=1024), gate/up another, as in a forward pass.
            shared = {n: torch.randn((M, 1024), device="cuda", dtype=torch.float32) for n in ("attn", "ffn")}
            for n, t, N, K, d in weights[li]:
                x = shared["attn"] if n in ("q", "k", "v") else shared["ffn"] if n in ("gate", "up") else None
                mats.append(Mat(torch, f"b{M}.{li}.{n}", t, N, K, d, M=M, x=x))
        levels = []
        for li in range(QWEN3_LAYERS):
            q, k, v, o, g, u, dn = mats[7 * li: 7 * li + 7]
            levels += [[q, k, v], [o], [g, u], [dn]]
        descs = []
        for lv in levels:
            arr = (gl.GemvDesc * len(lv))()
            for i, m in enumerate(lv):
                arr[i].W, arr[i].type, arr[i].N, arr[i].K = m.w.data_ptr(), m.t, m.N, m.K
                arr[i].A, arr[i].C = m.x.data_ptr(), m.y.data_ptr()
            descs.append((arr, len(lv)))

        def run_on(st, M=M, descs=descs):
            for arr, n in descs:
                ctx.check(ctx.lib.ggq_mul_mat_batch_rows_dev(ctx.h, arr, n, M, st), "batch rows")

        sec = time_steps(torch, lambda: run_on(stream), steps, 2)
        # The same 112 launches captured once as a HIP graph and replayed
        # (no host enqueue per launch: batch 1 is close to host-bound from
        # Python otherwise).
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run_on(ctypes.c_void_p(s.cuda_stream))
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=s):
                run_on(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        gsec = time_steps(torch, g.replay, steps, 2)
        b = sum(m.bytes() for m in mats)
        res[f"batch{M}"] = {"bytes": b, "us": round(sec * 1e6, 1), "GBps": round(b / sec / 1e9, 1),
                            "frac_hbm_peak": round(b / sec / 1e9 / HBM_PEAK_GBS, 4),
                            "us_graph": round(gsec * 1e6, 1), "GBps_graph": round(b / gsec / 1e9, 1)}
        del g
    return res


def bench_config5(torch, ctx, stream, steps=50, T=64, act_mode=0):
    """one qwen35moe-A3B MoE FFN layer, 64 tokens (T), top-8 of
    256 experts (FFN 512, Q4_K gate/up, Q6_K down) + 1 shared expert, as one
    expert-grouped ggq_moe_ffn_act_dev call (act_mode 0: fp32 activations,
    1: per-row int8 activations), 50 calls timed after 5.  The launches the
    layer takes depend on the pair rows per expert: grouped GEMVs, int8 row
    tiles, expert-grouped GEMMs (fp16 hi + lo for fp32)."""
    H, F, E, k = 2048, 512, 256, 8
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    wg, _ = make_weight(torch, gen, Q4K, E * F, H)
    wu, _ = make_weight(torch, gen, Q4K, E * F, H)
    wd, _ = make_weight(torch, gen, Q6K, E * H, F)
    sg, _ = make_weight(torch, gen, Q4K, F, H)
    su, _ = make_weight(torch, gen, Q4K, F, H)
    sd, _ = make_weight(torch, gen, Q6K, H, F)
    x = torch.randn((T, H), device="cuda", generator=gen)
    logits = torch.randn((T, E), device="cuda", generator=gen)
    sw = torch.sigmoid(torch.randn((T,), device="cuda", generator=gen))
    out = torch.empty((T, H), device="cuda")
    sel = torch.empty((T, k), dtype=torch.int32, device="cuda")
    p = gl.MoeParams()
    p.T, p.H, p.F, p.E, p.top_k = T, H, F, E, k
    p.x, p.router_logits = x.data_ptr(), logits.data_ptr()
    p.gate_type, p.up_type, p.down_type = Q4K, Q4K, Q6K
    p.gate_exps, p.up_exps, p.down_exps = wg.data_ptr(), wu.data_ptr(), wd.data_ptr()
    p.gate_shexp, p.up_shexp, p.down_shexp = sg.data_ptr(), su.data_ptr(), sd.data_ptr()
    p.shared_w, p.out, p.sel_experts = sw.data_ptr(), out.data_ptr(), sel.data_ptr()

    def run():
        ctx.check(ctx.lib.ggq_moe_ffn_act_dev(ctx.h, ctypes.byref(p), act_mode, stream), "moe_ffn")

    sec = time_steps(torch, run, steps, 5)
    hit = int(torch.unique(sel).numel())
    per_expert = 2 * gl.row_bytes(Q4K, H) * F + gl.row_bytes(Q6K, F) * H
    b = (hit + 1) * per_expert + 4 * T * H * 2 + 4 * T * E
    act = "fp32" if act_mode == 0 else "per-row int8 (GGQ_ACT_Q8_ROW)"
    return {"workload": f"qwen35moe-A3B MoE FFN layer: {T} tokens, top-8 of 256 experts (FFN 512) + shared, "
                        f"Q4_K gate/up, Q6_K down, {act} activations, one grouped call", "experts_hit": hit,
            "bytes": b, "us": round(sec * 1e6, 1), "GBps": round(b / sec / 1e9, 1),
            "frac_hbm_peak": round(b / sec / 1e9 / HBM_PEAK_GBS, 4)}


def bench_decode_token(torch, ctx, stream, n_tok=24, start=512, n_ctx=1024):
    """A whole Llama-3.2-1B decode token (16 layers, hidden 2048, 32 q / 8 kv
    heads of 64, FFN 8192, vocab 128256) from a GGUF file: a synthetic
    Q4_K_M model (q/k/o/gate/up/output and the token embedding Q4_K, v and
    down Q6_K, F32 norms; seeded N(0, 0.02) weights, one matrix per shape
    repeated over the layers) is written to a temporary file, opened with
    ggq_gguf_open and uploaded unchanged with ggq_gguf_upload.  Per token:
    the embedding row decoded on the device (ggq_dequant_dev); per layer
    q/k/v with the attention RMSNorm fused in (v written straight into the
    layer's KV-cache slot), RoPE on q and k together by the caller (torch, as
    the reference keeps RoPE with its caller) and k copied into the cache,
    ggq_attention_decode_dev over the
    start + t positions, o with the residual, gate (silu) / up with the FFN
    norm, down on silu(gate) * up with the residual; then the output norm
    (torch) and ggq_logits_argmax_dev, whose token is read back and fed to
    the next token's embedding (one host round trip per token, as a decode
    loop has).  The cache holds `start` synthetic positions before the
    first timed token."""
    import tempfile
    from ggnpu_amd import gguf_writer as gw
    L, H, NH, NKV, HD, F, V = 16, 2048, 32, 8, 64, 8192, 128256
    EPS, BASE = 1e-5, 500000.0
    rng = np.random.default_rng(7)
    enc = {}

    def weight(t, N, K):
        key = (t, N, K)
        if key not in enc:
            enc[key] = gl.encode(t, (rng.standard_normal((N, K), dtype=np.float32) * 0.02)).tobytes()
        return enc[key]

    def norm_bytes():
        return (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32).tobytes()

    shapes = {"attn_q": (Q4K, NH * HD, H), "attn_k": (Q4K, NKV * HD, H), "attn_v": (Q6K, NKV * HD, H),
              "attn_output": (Q4K, H, NH * HD), "ffn_gate": (Q4K, F, H), "ffn_up": (Q4K, F, H),
              "ffn_down": (Q6K, H, F)}
    tensors = [("token_embd.weight", Q4K, [H, V], gl.row_bytes(Q4K, H) * V, lambda: weight(Q4K, V, H))]
    for li in range(L):
        tensors.append((f"blk.{li}.attn_norm.weight", 0, [H], 4 * H, norm_bytes))
        tensors.append((f"blk.{li}.ffn_norm.weight", 0, [H], 4 * H, norm_bytes))
        for name, (t, N, K) in shapes.items():
            tensors.append((f"blk.{li}.{name}.weight", t, [K, N], gl.row_bytes(t, K) * N,
                            (lambda t=t, N=N, K=K: weight(t, N, K))))
    tensors.append(("output_norm.weight", 0, [H], 4 * H, norm_bytes))
    tensors.append(("output.weight", Q4K, [H, V], gl.row_bytes(Q4K, H) * V, lambda: weight(Q4K, V, H)))
    kvs = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.UINT32, L),
           ("llama.embedding_length", gw.UINT32, H), ("llama.feed_forward_length", gw.UINT32, F),
           ("llama.attention.head_count", gw.UINT32, NH), ("llama.attention.head_count_kv", gw.UINT32, NKV),
           ("llama.attention.layer_norm_rms_epsilon", gw.FLOAT32, EPS), ("llama.rope.freq_base", gw.FLOAT32, BASE)]
    lib = ctx.lib
    t0 = time.time()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "llama-3.2-1b-synthetic-q4_k_m.gguf")
        gw.write_stream(path, kvs, tensors)
        fbytes = os.path.getsize(path)
        enc.clear()
        dev, handles = {}, []
        with gl.GgufFile(path) as g:
            assert (g.kv("llama.block_count"), g.kv("llama.attention.head_count_kv")) == (L, NKV)
            eps = g.kv("llama.attention.layer_norm_rms_epsilon")
            base = g.kv("llama.rope.freq_base")
            for name, info in g.tensors.items():
                if info["type"] == 0:
                    dev[name] = torch.from_numpy(np.frombuffer(g.tensor_bytes(name), np.float32).copy()).cuda()
                else:
                    w = ctypes.c_void_p()
                    ctx.check(g.lib.ggq_gguf_upload(ctx.h, g.h, name.encode(), ctypes.byref(w)), name)
                    handles.append(w)
                    dims = info["dims"]
                    dev[name] = (lib.ggq_weight_device_ptr(w), info["type"], int(np.prod(dims[1:])), dims[0])
    setup_s = time.time() - t0
    weight_bytes = sum(gl.row_bytes(v[1], v[3]) * v[2] for v in dev.values() if isinstance(v, tuple))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(8)
    Kc = torch.randn((L, n_ctx, NKV, HD), device="cuda", generator=gen)
    Vc = torch.randn((L, n_ctx, NKV, HD), device="cuda", generator=gen)
    half = HD // 2
    theta = torch.arange(n_ctx, dtype=torch.float64, device="cuda")[:, None] * \
        base ** (-2.0 * torch.arange(half, dtype=torch.float64, device="cuda") / HD)
    cos_t, sin_t = torch.cos(theta).float(), torch.sin(theta).float()
    qk = torch.empty((NH + NKV, HD), device="cuda")  # q and k next to each other: one RoPE for both
    q, kbuf = qk[:NH], qk[NH:]
    att = torch.empty((1, NH * HD), device="cuda")
    gb, ub = torch.empty((1, F), device="cuda"), torch.empty((1, F), device="cuda")
    x = torch.empty((1, H), device="cuda")
    logits = torch.empty((1, V), device="cuda")
    tok = torch.zeros((1,), dtype=torch.int32, device="cuda")
    emb = dev["token_embd.weight"]
    emb_row = gl.row_bytes(Q4K, H)

    def descs(entries):
        arr = (gl.GemvFusedDesc * len(entries))()
        for d, e in zip(arr, entries):
            d.W, d.type, d.N, d.K = dev[e["w"]]
            d.A, d.C = e["A"], e["C"]
            if "up" in e:
                d.A_up = e["up"]
            if e.get("res"):
                d.residual = e["C"]
            if "norm" in e:
                d.rms_norm, d.rms_eps, d.rms_w = 1, eps, dev[e["norm"]].data_ptr()
            d.silu = int(e.get("silu", False))
        return arr, len(entries)

    # the launches' descriptors, built once (per token only the k / v cache
    # slots of the q/k/v entries change)
    plan = []
    for li in range(L):
        p = f"blk.{li}."
        plan.append((descs([{"w": p + "attn_q.weight", "A": x.data_ptr(), "C": q.data_ptr(), "norm": p + "attn_norm.weight"},
                            {"w": p + "attn_k.weight", "A": x.data_ptr(), "C": kbuf.data_ptr(), "norm": p + "attn_norm.weight"},
                            {"w": p + "attn_v.weight", "A": x.data_ptr(), "C": 0, "norm": p + "attn_norm.weight"}]),
                     descs([{"w": p + "attn_output.weight", "A": att.data_ptr(), "C": x.data_ptr(), "res": True}]),
                     descs([{"w": p + "ffn_gate.weight", "A": x.data_ptr(), "C": gb.data_ptr(),
                             "norm": p + "ffn_norm.weight", "silu": True},
                            {"w": p + "ffn_up.weight", "A": x.data_ptr(), "C": ub.data_ptr(), "norm": p + "ffn_norm.weight"}]),
                     descs([{"w": p + "ffn_down.weight", "A": gb.data_ptr(), "up": ub.data_ptr(), "C": x.data_ptr(),
                             "res": True}])))

    def fused(dn):
        ctx.check(lib.ggq_mul_mat_fused_dev(ctx.h, dn[0], dn[1], 1, stream), "fused")

    def rope(v, n, pos):
        v = v.view(n, HD)
        a, b = v[:, :half].clone(), v[:, half:]
        c, s = cos_t[pos], sin_t[pos]
        v[:, :half] = a * c - b * s
        v[:, half:] = a * s + b * c

    def token(t, pos):
        ctx.check(lib.ggq_dequant_dev(ctx.h, ctypes.c_void_p(emb[0] + t * emb_row), Q4K, H // 256,
                                      ctypes.c_void_p(x.data_ptr()), stream), "embedding")
        for li in range(L):
            qkv, o, gu, down = plan[li]
            kslot, vslot = Kc[li, pos], Vc[li, pos]
            qkv[0][2].C = vslot.data_ptr()
            fused(qkv)
            rope(qk, NH + NKV, pos)
            kslot.copy_(kbuf)
            ctx.check(lib.ggq_attention_decode_dev(ctx.h, q.data_ptr(), Kc[li].data_ptr(), Vc[li].data_ptr(), 1, NH, NKV,
                                                   HD, pos + 1, pos, att.data_ptr(), stream), "attention")
            fused(o)
            fused(gu)
            fused(down)
        xo = x * torch.rsqrt((x * x).mean() + eps) * dev["output_norm.weight"]
        wo = dev["output.weight"]
        ctx.check(lib.ggq_logits_argmax_dev(ctx.h, wo[0], wo[1], wo[2], wo[3], xo.data_ptr(), 1, 0, logits.data_ptr(),
                                            tok.data_ptr(), None, stream), "logits")
        return int(tok.item())  # the decode loop's host round trip

    t = 1
    for i in range(4):  # warm-up tokens
        t = token(t, start - 4 + i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(n_tok):
        t = token(t, start + i)
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / n_tok
    for w in handles:
        ctx.check(lib.ggq_weight_free(ctx.h, w), "free")
    return {"workload": f"Llama-3.2-1B decode token from a GGUF file (synthetic Q4_K_M, {fbytes / 1e6:.0f} MB): 16 layers "
                        f"with RMSNorm / SwiGLU / residual fused, RoPE by the caller (torch), attention over "
                        f"{start}..{start + n_tok - 1} positions, output norm, logits + greedy token, token read back",
            "tokens": n_tok, "ms_per_token": round(sec * 1e3, 3), "tokens_per_s": round(1.0 / sec, 1),
            "weight_GBps": round(weight_bytes / sec / 1e9, 1), "setup_s": round(setup_s, 1)}


def host_cpu():
    """Host CPU model and core counts for the cpu_baseline records."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"host_cpu": model, "host_cores_total": os.cpu_count(),
            "host_cores_usable": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None}


class CpuPath:
    """The reference's CPU arithmetic, one core: the compiled reference
    sources (oracle/_ref, "reference") where present, else the oracle's
    bit-identical restatements ("port").
      cpuref(t, W, N, K, A)  CpuRefBackend::mul_mat_q (cpu_ref.cpp:87-117;
                             Q4_K / Q6_K, the types it takes)
      rowdot(t, W, N, K, A)  the CLI's dequantize-row + fp32 dot for weights
                             no backend takes (main.cpp:317-326, :1380-1386)"""

    def __init__(self):
        from oracle import oracle as orc
        self.orc = orc
        self.ref = orc.ref_lib()
        self.kind = "reference" if self.ref is not None else "port"

    def _run(self, fn_ref, fn_orc, t, W, N, K, A):
        A = np.ascontiguousarray(A, dtype=np.float32)
        if self.ref is None:
            return fn_orc(t, W, N, K, A)
        C = np.empty((A.shape[0], N), np.float32)
        st = fn_ref(t, W.ctypes.data, N, K, A.ctypes.data, A.shape[0], C.ctypes.data)
        assert st == 0, st
        return C

    def cpuref(self, t, W, N, K, A):
        return self._run(self.ref and self.ref.ref_cpuref_mul_mat, self.orc.mul_mat_cpuref_f32, t, W, N, K, A)

    def rowdot(self, t, W, N, K, A):
        return self._run(self.ref and self.ref.ref_rowdot_mul_mat, self.orc.mul_mat_rowdot_f32, t, W, N, K, A)

    def what(self, fn):
        src = {"cpuref": ("oracle/_ref CpuRefBackend::mul_mat_q (reference sources, -O3)",
                          "oracle/ggq_oracle.c orc_mul_mat_cpuref_f32"),
               "rowdot": ("oracle/_ref reference block decoders + main.cpp:317-326 row-dot loop",
                          "oracle/ggq_oracle.c orc_mul_mat_rowdot_f32")}[fn]
        return src[0] if self.ref is not None else src[1]


def _timed(budget_s, body):
    """Repeat body() until budget_s has passed; (passes, seconds)."""
    t0, n = time.perf_counter(), 0
    while True:
        body()
        n += 1
        el = time.perf_counter() - t0
        if el > budget_s:
            return n, el


def _host_weight(rng, t, N, K):
    return gl.encode(t, (rng.standard_normal((N, K), dtype=np.float32) * 0.02))


def _cpu_record(cp, value, unit, sample, **kw):
    return {"value": round(value, 4), "unit": unit, "cores": 1, "kind": cp.kind, "sample": sample, **host_cpu(), **kw}


def cpu_baseline(host_layer0, budget_s=6.0):
    """CpuRefBackend::mul_mat_q over layer 0 of the decode step."""
    cp = CpuPath()
    rng = np.random.default_rng(0)
    work = [(m.t, raw, m.N, m.K, rng.standard_normal((1, m.K)).astype(np.float32)) for m, raw in host_layer0]
    nbytes = sum(gl.row_bytes(t, K) * N + 4 * (K + N) for t, _, N, K, _ in work)
    reps, el = _timed(budget_s, lambda: [cp.cpuref(t, raw, N, K, A) for t, raw, N, K, A in work])
    return _cpu_record(cp, reps * nbytes / el / 1e9, "GB/s",
                       f"Llama-3.2-1B layer 0 (q,k,v,o,gate,up,down; {nbytes / 1e6:.1f} MB Q4_K/Q6_K), batch 1, "
                       f"{reps} passes in {el:.1f}s, {cp.what('cpuref')}")


def cpu_baseline_config0(budget_s=3.0):
    """CpuRefBackend::mul_mat_q on the 8192x2048 Q4_K GEMV."""
    cp = CpuPath()
    rng = np.random.default_rng(1)
    W = _host_weight(rng, Q4K, 8192, 2048)
    A = rng.standard_normal((1, 2048)).astype(np.float32)
    nbytes = W.size + 4 * (2048 + 8192)
    reps, el = _timed(budget_s, lambda: cp.cpuref(Q4K, W, 8192, 2048, A))
    return _cpu_record(cp, reps * nbytes / el / 1e9, "GB/s",
                       f"the whole workload (Q4_K 8192x2048, batch 1), {reps} calls in {el:.1f}s, {cp.what('cpuref')}",
                       us_per_call=round(el / reps * 1e6, 1))


def cpu_baseline_config2(budget_s=4.0, rows=32):
    """the reference on the CPU for Q8_0 weights is the
    dequantize-row + fp32 dot loop (CpuRefBackend takes no Q8_0,
    main.cpp:317-326); timed on the first `rows` rows of each layer-0 weight
    for all 512 tokens and scaled to the 28-layer step.  The accelerator
    route's host preparation is timed beside it: the per-row int8 activation
    quantization (amd_xdna.cpp:598-603, per step) and the per-row int8 weight
    requantization decode_q8_0_for_npu (q8_0.cpp:30-77, once per weight)."""
    cp = CpuPath()
    rng = np.random.default_rng(2)
    T = PREFILL_TOKENS
    mats = [(name, _host_weight(rng, Q8_0, rows, K), K) for name, _, _, K in QWEN_LAYER]
    acts = {K: rng.standard_normal((T, K)).astype(np.float32) for K in (1536, 8960)}
    sample_ops = sum(2 * T * rows * K for _, _, K in mats)
    reps, el = _timed(budget_s, lambda: [cp.rowdot(Q8_0, W, rows, K, acts[K]) for _, W, K in mats])
    sec_per_op = el / reps / sample_ops
    step_ops = QWEN_LAYERS * sum(2 * T * N * K for _, _, N, K in QWEN_LAYER)
    # host prep of the int8 route: four activation quantizations per layer
    # (port: the reference's quantizer lives in the accelerator backend) and
    # the weight requantization (reference decode_q8_0_for_npu where built)
    t0 = time.perf_counter()
    for K in (1536, 1536, 1536, 8960):
        cp.orc.quant_act(acts[K], 1)
    act_quant_ms = (time.perf_counter() - t0) * 1e3 * QWEN_LAYERS
    req_rows = sum(rows for _ in mats)
    t0 = time.perf_counter()
    for _, W, K in mats:
        if cp.ref is not None:
            q = np.empty((rows, K), np.int8)
            sc = np.empty(rows, np.float32)
            assert cp.ref.ref_decode_for_npu(Q8_0, W.ctypes.data, W.size, rows, K, q.ctypes.data, sc.ctypes.data) == 0
    req_s = time.perf_counter() - t0
    model_elems = QWEN_LAYERS * sum(N * K for _, _, N, K in QWEN_LAYER)
    req_elems = sum(rows * K for _, _, K in mats)
    step_s = sec_per_op * step_ops + act_quant_ms / 1e3
    out = _cpu_record(cp, step_ops / step_s / 1e12, "TOPS",
                      f"first {rows} rows of each Qwen2.5-1.5B layer-0 Q8_0 weight x {T} tokens ({reps} passes in "
                      f"{el:.1f}s, {cp.what('rowdot')}), scaled to the 28-layer step; plus the per-row int8 "
                      "activation quantization of the step's 112 inputs (oracle port, single core)",
                      ms_per_step=round(step_s * 1e3, 1), act_quant_ms_per_step=round(act_quant_ms, 1))
    if cp.ref is not None:
        out["weight_requant_s_once"] = round(req_s / req_elems * model_elems, 2)
        out["weight_requant_note"] = ("reference decode_q8_0_for_npu (q8_0.cpp:30-77) on the same rows, scaled to "
                                      "the model's 28 layers; paid once per weight (WeightCache), not per step")
    return out


def cpu_baseline_config3(budget_s=2.0):
    """IQ4_NL / IQ4_XS / Q5_K weights take the dequantize-row +
    fp32 dot loop (main.cpp:317-326) on the CPU; layer 0 at batch 1 and 8."""
    cp = CpuPath()
    rng = np.random.default_rng(3)
    cycle = [IQ4NL, IQ4XS, Q5K]
    mats = [(cycle[i % 3], _host_weight(rng, cycle[i % 3], N, K), N, K) for i, (_, N, K) in enumerate(QWEN3_SHAPES)]
    res = {}
    for M in (1, 8):
        acts = {K: rng.standard_normal((M, K)).astype(np.float32) for K in (1024, 2048, 3072)}
        nbytes = sum(W.size + 4 * M * (K + N) for _, W, N, K in mats)
        reps, el = _timed(budget_s, lambda: [cp.rowdot(t, W, N, K, acts[K]) for t, W, N, K in mats])
        res[M] = (reps * nbytes / el / 1e9, reps, el, el / reps * QWEN3_LAYERS * 1e6)
    g1, reps, el, us1 = res[1]
    return _cpu_record(cp, g1, "GB/s",
                       f"Qwen3-0.6B layer 0 (7 weights, IQ4_NL/IQ4_XS/Q5_K), batch 1: {reps} passes in {el:.1f}s, "
                       f"{cp.what('rowdot')}", us_per_step_batch1=round(us1, 1),
                       batch8={"GBps": round(res[8][0], 3), "us_per_step": round(res[8][3], 1)})


def cpu_baseline_config4(budget_s=6.0, T=64):
    """the reference's per-token MoE loop (main.cpp:3110-3193):
    per token top-8 of 256 router logits, softmax over the selected, then
    for each selected expert and the shared one gate / up (Q4_K 512x2048)
    and down (Q6_K 2048x512) through CpuRefBackend::mul_mat_q, silu(gate) *
    up, weighted sum.  The 256 experts occupy distinct host memory (16
    encoded experts copied over the 256 slots: the timing does not depend on
    the values)."""
    cp = CpuPath()
    H, F, E, k = 2048, 512, 256, 8
    rng = np.random.default_rng(5)
    pool = [(_host_weight(rng, Q4K, F, H), _host_weight(rng, Q4K, F, H), _host_weight(rng, Q6K, H, F)) for _ in range(16)]
    experts = [tuple(a.copy() for a in pool[e % 16]) for e in range(E)]
    shared = pool[0]
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    sw = 1.0 / (1.0 + np.exp(-rng.standard_normal(T).astype(np.float32)))

    def expert(ws, xt):
        g = cp.cpuref(Q4K, ws[0], F, H, xt)
        u = cp.cpuref(Q4K, ws[1], F, H, xt)
        a = (g / (1.0 + np.exp(-g))) * u
        return cp.cpuref(Q6K, ws[2], H, F, a)

    t0, done, hit = time.perf_counter(), 0, set()
    for t in range(T):
        xt = x[t: t + 1]
        sel = np.argsort(-logits[t], kind="stable")[:k]
        w = np.exp(logits[t, sel] - logits[t, sel[0]])
        w /= w.sum()
        out = np.zeros((1, H), np.float32)
        for e, we in zip(sel, w):
            out += we * expert(experts[e], xt)
            hit.add(int(e))
        out += sw[t] * expert(shared, xt)
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    el = time.perf_counter() - t0
    layer_s = el / done * T
    per_expert = 2 * gl.row_bytes(Q4K, H) * F + gl.row_bytes(Q6K, F) * H
    # the same algorithmic bytes as the GPU line (each hit expert once)
    sel_all = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    nbytes = (len(np.unique(sel_all)) + 1) * per_expert + 4 * T * H * 2 + 4 * T * E
    return _cpu_record(cp, nbytes / layer_s / 1e9, "GB/s",
                       f"{done} of {T} tokens through the per-token loop in {el:.1f}s, scaled to the {T}-token layer; "
                       f"GB/s over the GPU line's algorithmic bytes; {cp.what('cpuref')}",
                       us_per_layer=round(layer_s * 1e6, 1))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--graph", action="store_true", help="replay the step as a HIP graph")
    ap.add_argument("--no-extra", action="store_true", help="skip config 1 / config 3 / CPU baseline")
    ap.add_argument("--only", choices=["decode", "token", "config1", "config1_q8", "prefill", "config4", "moe", "logits", "fused", "attention", "host", "copy",
                                       "floor"],
                    default=None,
                    help="run one workload only and print its result (profiling aid)")
    ap.add_argument("--moe-tokens", type=int, default=64,
                    help="tokens of the MoE layer for --only moe (the bench line uses 64)")
    ap.add_argument("--moe-act", type=int, default=0, choices=[0, 1],
                    help="activation treatment of --only moe: 0 fp32, 1 per-row int8")
    ap.add_argument("--per-matmul", action="store_true",
                    help="one launch per matmul instead of one per dependency level")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the backend is a single-device hot path "
              "(multi-GPU sharding is a design note, not part of this build)", file=sys.stderr)
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ctx = gl.Context(0)
    # All work runs on one non-default stream: kernels are launched on it and
    # the HIP events are recorded on it (a null handle would select the
    # library's own stream, which the events would not see).
    side = torch.cuda.Stream()
    torch.cuda.set_stream(side)
    stream = ctypes.c_void_p(side.cuda_stream)
    assert stream.value, "expected a non-null stream handle"

    if args.only == "copy":
        # Known-size device copy: the calibration kernel for the HBM byte
        # counters (FETCH_SIZE / WRITE_SIZE) of the profiles.
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_per_copy": src.numel(), "copies": 4}), flush=True)
        return
    if args.only == "floor":
        print(json.dumps({"only": "floor", **bench_launch_floor(torch)}), flush=True)
        ctx.close()
        return
    if args.only in ("token", "config1", "config1_q8", "prefill", "config4", "moe", "logits", "fused", "attention", "host"):
        res = {"token": bench_decode_token, "config1": bench_config1, "config1_q8": lambda t, c, st: bench_config1(t, c, st, act_mode=1),
               "prefill": bench_prefill, "config4": bench_config4,
               "moe": lambda *a: bench_config5(*a, T=args.moe_tokens, act_mode=args.moe_act), "logits": bench_logits, "fused": bench_decode_fused,
               "attention": bench_attention, "host": bench_host_api}[args.only](
                   torch, ctx, stream)
        print(json.dumps({"only": args.only, **res}), flush=True)
        ctx.close()
        return
    levels, host_layer0, sec, gpu_sec, step_bytes, per_level = bench_decode_step(
        torch, ctx, args.steps, args.warmup, args.graph, stream, not args.per_matmul, args.only != "decode")
    value = step_bytes / sec / 1e9
    achieved = step_bytes / gpu_sec / 1e9
    out = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak); prefill int8 GEMM TOPS (% MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 activations x Q4_K/Q6_K raw blocks (fp32 accumulate)",
        "data": "synthetic: seeded N(0,0.02) weights encoded to GGUF blocks, N(0,1) activations",
        "config": {"workload": "Llama-3.2-1B decode step matmuls (configs[1]): 16 layers q/k/v/o/gate/up/down "
                               "Q4_K (v, down Q6_K) + 128256x2048 Q4_K output, batch 1",
                   "matmuls_per_step": sum(len(lv) for lv in levels), "launch_groups_per_step": len(levels),
                   "bytes_per_step": step_bytes,
                   "graph": bool(args.graph),
                   "launches": "one per dependency level (q/k/v, o, gate/up, down, output)"
                   if not args.per_matmul else "one per matmul"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode GEMV kernels: algorithmic bytes per step / GPU time per step from HIP "
                               "events on the launch stream around the timed steps (kernels back to back)",
                     "kernel_us_per_step": round(gpu_sec * 1e6, 1)},
    }
    # HBM bytes per step from the FETCH_SIZE / WRITE_SIZE profiles (scaled by
    # the copy-kernel calibration recorded with them).
    tpath = os.path.join(ROOT, "profiles", "decode_step_traffic.json")
    if os.path.exists(tpath) and not args.per_matmul:
        with open(tpath) as f:
            t = json.load(f)
        out["roofline"]["traffic"] = t.get("traffic_bytes_per_step")
        out["roofline"]["traffic_unit"] = "HBM bytes per step (rocprofv3 FETCH_SIZE + WRITE_SIZE, " + t["source"] + ")"
    if not args.no_extra and args.only != "decode":
        # Every BASELINE config beside the headline, each with its own CPU
        # baseline (configs[0] in both activation treatments; configs[1]'s
        # CPU baseline is the top-level one).
        out["extra"] = {}
        for key, fn, cpu in (
                ("config1", bench_config1, cpu_baseline_config0),
                ("config1_q8_row", lambda t, c, st: bench_config1(t, c, st, act_mode=1), None),
                ("config2_q8_row", lambda t, c, st: bench_decode_levels(t, c, levels, st, 1), None),
                ("config3_prefill", bench_prefill, cpu_baseline_config2),
                ("config4_iq4_q5k", bench_config4, cpu_baseline_config3),
                ("config5_moe", bench_config5, cpu_baseline_config4),
                ("config5_moe_q8_row", lambda t, c, st: bench_config5(t, c, st, act_mode=1), None),
                ("config5_moe_512", lambda t, c, st: bench_config5(t, c, st, steps=10, T=512, act_mode=0), None),
                ("config5_moe_512_q8_row", lambda t, c, st: bench_config5(t, c, st, steps=10, T=512, act_mode=1), None),
                ("logits_argmax", bench_logits, None), ("attention_decode", bench_attention, None),
                ("host_api_decode", bench_host_api, None), ("decode_fused", bench_decode_fused, None),
                ("decode_token_gguf", bench_decode_token, None)):
            try:
                out["extra"][key] = fn(torch, ctx, stream)
            except Exception as e:  # reported, never silently replaced
                out["extra"][key] = {"error": str(e)}
            if cpu is not None:
                out["extra"][key]["cpu_baseline"] = cpu()
        out["cpu_baseline"] = cpu_baseline(host_layer0)
    per = {"method": "HIP events around 10 back-to-back launches of the level (small weights partly cache-warm)"}
    for lv, d in per_level:
        key = "+".join(m.name.split(".")[-1] for m in lv)
        per[key] = {"us": round(d * 1e6, 2), "GBps": round(sum(m.bytes() for m in lv) / d / 1e9, 1)}
    out["per_level_layer0"] = per
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
