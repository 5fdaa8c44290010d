"""A few decode tokens of a small Llama-style model read from a GGUF file,
run through the device entry points only, against an fp64 restatement.

The file (ggnpu_amd/gguf_writer.py) carries the tensor names and metadata of a
llama GGUF: Q4_K q/k/o/gate/up/output, Q6_K v/down, F32 norms and
embedding.  The weights go to HBM with ggq_gguf_upload; per token and layer
the GPU path is
  ggq_mul_mat_fused_dev  q/k/v with the attention RMSNorm prologue
  (caller)               RoPE on q and k, K/V written into the layer's cache
  ggq_attention_decode_dev
  ggq_mul_mat_fused_dev  o with the residual add
  ggq_mul_mat_fused_dev  gate (silu) / up with the FFN RMSNorm prologue
  ggq_mul_mat_fused_dev  down on silu(gate) * up with the residual add
and per token the output norm (caller) and ggq_logits_argmax_dev.  The
order follows the reference's decode step (main.cpp:3236-3498); RoPE and the
cache write stay with the caller, as they do in the reference.  The
restatement uses the oracle's bit-exact dequantized weights in fp64, the
oracle's RMSNorm formula, the same RoPE and an exact softmax.  Bar: logits
and hidden state within rel-L2 1e-4 at every token; the greedy token equal
wherever the top two logits differ by more than 1e-3 relative."""
import ctypes

import numpy as np
import pytest

import ggnpu_amd.lib as gl
from ggnpu_amd import gguf_writer as gw

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, F, V = 256, 4, 2, 64, 512, 1024
EPS, ROPE_BASE = 1e-5, 10000.0
Q4K, Q6K, F32 = 12, 14, 0
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    c = gl.Context(0)
    yield c
    c.close()


def _model(L, seed=0):
    rng = np.random.default_rng(seed)
    mats = {}

    def q(name, t, N, K, scale=0.05):
        w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
        mats[name] = (t, N, K, gl.encode(t, w))

    norms = {}
    for li in range(L):
        q(f"blk.{li}.attn_q.weight", Q4K, NH * HD, H)
        q(f"blk.{li}.attn_k.weight", Q4K, NKV * HD, H)
        q(f"blk.{li}.attn_v.weight", Q6K, NKV * HD, H)
        q(f"blk.{li}.attn_output.weight", Q4K, H, NH * HD)
        q(f"blk.{li}.ffn_gate.weight", Q4K, F, H)
        q(f"blk.{li}.ffn_up.weight", Q4K, F, H)
        q(f"blk.{li}.ffn_down.weight", Q6K, H, F)
        norms[f"blk.{li}.attn_norm.weight"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        norms[f"blk.{li}.ffn_norm.weight"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    q("output.weight", Q4K, V, H)
    norms["output_norm.weight"] = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    embd = rng.standard_normal((V, H)).astype(np.float32)
    return mats, norms, embd


def _write(path, mats, norms, embd, L):
    kvs = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.UINT32, L),
           ("llama.embedding_length", gw.UINT32, H), ("llama.feed_forward_length", gw.UINT32, F),
           ("llama.attention.head_count", gw.UINT32, NH), ("llama.attention.head_count_kv", gw.UINT32, NKV),
           ("llama.attention.layer_norm_rms_epsilon", gw.FLOAT32, EPS), ("llama.rope.freq_base", gw.FLOAT32, ROPE_BASE)]
    tensors = [("token_embd.weight", F32, [H, V], embd.tobytes())]
    tensors += [(n, F32, [H], w.tobytes()) for n, w in norms.items()]
    tensors += [(n, t, [K, N], raw.tobytes()) for n, (t, N, K, raw) in mats.items()]
    gw.write(path, kvs, tensors, alignment=32)


def _rope_np(v, n_heads, pos):
    """NeoX-style rotation of each head's halves (main.cpp:3325-3343), fp64."""
    v = v.reshape(n_heads, HD).astype(np.float64)
    half = HD // 2
    theta = pos * ROPE_BASE ** (-2.0 * np.arange(half) / HD)
    c, s = np.cos(theta), np.sin(theta)
    a, b = v[:, :half].copy(), v[:, half:].copy()
    return np.concatenate([a * c - b * s, a * s + b * c], axis=1).reshape(-1)


def _rms_np(x, w):
    return x / np.sqrt(np.mean(x * x) + EPS) * w


def _reference(orc, mats, norms, embd, tokens, L):
    W = {n: orc.dequant(t, raw).reshape(N, K).astype(np.float64) for n, (t, N, K, raw) in mats.items()}
    nw = {n: w.astype(np.float64) for n, w in norms.items()}
    Kc = np.zeros((L, len(tokens), NKV, HD))
    Vc = np.zeros((L, len(tokens), NKV, HD))
    out = []
    for pos, tok in enumerate(tokens):
        x = embd[tok].astype(np.float64)
        for li in range(L):
            p = f"blk.{li}."
            xn = _rms_np(x, nw[p + "attn_norm.weight"])
            q = _rope_np(W[p + "attn_q.weight"] @ xn, NH, pos)
            k = _rope_np(W[p + "attn_k.weight"] @ xn, NKV, pos)
            Kc[li, pos] = k.reshape(NKV, HD)
            Vc[li, pos] = (W[p + "attn_v.weight"] @ xn).reshape(NKV, HD)
            att = np.empty(NH * HD)
            for h in range(NH):
                kv = h // (NH // NKV)
                sc = Kc[li, : pos + 1, kv] @ q[h * HD:(h + 1) * HD] / np.sqrt(HD)
                w = np.exp(sc - sc.max())
                att[h * HD:(h + 1) * HD] = (w / w.sum()) @ Vc[li, : pos + 1, kv]
            x = x + W[p + "attn_output.weight"] @ att
            xn = _rms_np(x, nw[p + "ffn_norm.weight"])
            g = W[p + "ffn_gate.weight"] @ xn
            u = W[p + "ffn_up.weight"] @ xn
            x = x + W[p + "ffn_down.weight"] @ (g / (1.0 + np.exp(-g)) * u)
        logits = W["output.weight"] @ _rms_np(x, nw["output_norm.weight"])
        out.append((x, logits))
    return out


@pytest.mark.parametrize("L", [2, 16])
def test_llama_decode_tokens_from_gguf(ctx, orc, tmp_path, L):
    """2 layers, and the 16 layers of Llama-3.2-1B (at small widths)."""
    import torch
    mats, norms, embd = _model(L)
    path = tmp_path / "tiny-llama.gguf"
    _write(path, mats, norms, embd, L)
    tokens = [3, 17, 999, 3, 512, 77]
    ref = _reference(orc, mats, norms, embd, tokens, L)

    lib = ctx.lib
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    with gl.GgufFile(path) as g:
        assert g.kv("general.architecture") == "llama"
        assert (g.kv("llama.block_count"), g.kv("llama.attention.head_count_kv")) == (L, NKV)
        eps = g.kv("llama.attention.layer_norm_rms_epsilon")
        dev = {}
        handles = []
        for name, info in g.tensors.items():
            if info["type"] == F32:
                arr = np.frombuffer(g.tensor_bytes(name), np.float32).reshape(list(reversed(info["dims"])))
                dev[name] = torch.from_numpy(arr.copy()).cuda()
            else:
                w = ctypes.c_void_p()
                ctx.check(g.lib.ggq_gguf_upload(ctx.h, g.h, name.encode(), ctypes.byref(w)), name)
                handles.append(w)
                dims = info["dims"]
                dev[name] = (lib.ggq_weight_device_ptr(w), info["type"], int(np.prod(dims[1:])), dims[0])

    def fused(entries):
        descs = (gl.GemvFusedDesc * len(entries))()
        for d, e in zip(descs, entries):
            d.W, d.type, d.N, d.K = dev[e["w"]]
            d.A, d.C = e["A"].data_ptr(), e["C"].data_ptr()
            if "up" in e:
                d.A_up = e["up"].data_ptr()
            if e.get("res"):
                d.residual = e["C"].data_ptr()  # in place: C = C + W.A
            if "norm" in e:
                d.rms_norm, d.rms_eps, d.rms_w = 1, eps, dev[e["norm"]].data_ptr()
            d.silu = int(e.get("silu", False))
        ctx.check(lib.ggq_mul_mat_fused_dev(ctx.h, descs, len(entries), 1, stream), "fused")

    def rope_t(v, n_heads, pos):
        v = v.view(n_heads, HD)
        half = HD // 2
        theta = pos * ROPE_BASE ** (-2.0 * torch.arange(half, dtype=torch.float64, device="cuda") / HD)
        c, s = torch.cos(theta).float(), torch.sin(theta).float()
        a, b = v[:, :half].clone(), v[:, half:].clone()
        v[:, :half] = a * c - b * s
        v[:, half:] = a * s + b * c

    n_ctx = len(tokens)
    Kc = torch.zeros((L, n_ctx, NKV, HD), device="cuda")
    Vc = torch.zeros((L, n_ctx, NKV, HD), device="cuda")
    buf = {k: torch.empty((1, n), device="cuda") for k, n in
           (("q", NH * HD), ("k", NKV * HD), ("v", NKV * HD), ("att", NH * HD), ("g", F), ("u", F))}
    logits = torch.empty((1, V), device="cuda")
    tok = torch.empty((1,), dtype=torch.int32, device="cuda")
    for pos, t in enumerate(tokens):
        x = dev["token_embd.weight"][t].reshape(1, H).clone()
        for li in range(L):
            p = f"blk.{li}."
            fused([{"w": p + "attn_q.weight", "A": x, "C": buf["q"], "norm": p + "attn_norm.weight"},
                   {"w": p + "attn_k.weight", "A": x, "C": buf["k"], "norm": p + "attn_norm.weight"},
                   {"w": p + "attn_v.weight", "A": x, "C": buf["v"], "norm": p + "attn_norm.weight"}])
            rope_t(buf["q"], NH, pos)
            rope_t(buf["k"], NKV, pos)
            Kc[li, pos] = buf["k"].view(NKV, HD)
            Vc[li, pos] = buf["v"].view(NKV, HD)
            ctx.check(lib.ggq_attention_decode_dev(ctx.h, buf["q"].data_ptr(), Kc[li].data_ptr(), Vc[li].data_ptr(),
                                                   1, NH, NKV, HD, pos + 1, pos, buf["att"].data_ptr(), stream),
                      "attention")
            fused([{"w": p + "attn_output.weight", "A": buf["att"], "C": x, "res": True}])
            fused([{"w": p + "ffn_gate.weight", "A": x, "C": buf["g"], "norm": p + "ffn_norm.weight", "silu": True},
                   {"w": p + "ffn_up.weight", "A": x, "C": buf["u"], "norm": p + "ffn_norm.weight"}])
            fused([{"w": p + "ffn_down.weight", "A": buf["g"], "up": buf["u"], "C": x, "res": True}])
        xo = x / torch.sqrt((x * x).mean() + eps) * dev["output_norm.weight"]
        w_out = dev["output.weight"]
        ctx.check(lib.ggq_logits_argmax_dev(ctx.h, w_out[0], w_out[1], w_out[2], w_out[3], xo.data_ptr(), 1, 0,
                                            logits.data_ptr(), tok.data_ptr(), None, stream), "logits")
        torch.cuda.synchronize()
        x_ref, l_ref = ref[pos]
        got_l = logits.cpu().numpy()[0]
        assert orc.rel_l2(x.cpu().numpy()[0], x_ref) <= TOL, pos
        assert orc.rel_l2(got_l, l_ref) <= TOL, pos
        top2 = np.sort(l_ref)[-2:]
        if top2[1] - top2[0] > 1e-3 * abs(top2[1]):
            assert int(tok.item()) == int(np.argmax(l_ref)), pos
    for w in handles:
        ctx.check(lib.ggq_weight_free(ctx.h, w), "free")
