"""Decode attention over the KV cache (ggq_attention_decode_dev) against the
oracle's restatement of CpuRefBackend::flash_attn (cpu_ref.cpp:223-280) over
the GQA-expanded cache (main.cpp:3358-3379), which is itself pinned bit-exact
to the compiled reference in test_oracle.py.  Bar: rel-L2 <= 1e-4 against the
fp64 oracle per (row, head), fp32 arithmetic on the GPU."""
import numpy as np
import pytest

import ggnpu_amd.lib as gl
from tests.gpu_util import dev, empty, host, ptr, stream_handle

pytestmark = pytest.mark.gpu
TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    import torch
    assert torch.cuda.is_available()
    c = gl.Context(0)
    yield c
    c.close()


def _case(seed, n_tok, n_head, n_kv, hd, ctx_len, qscale=1.0):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((n_tok, n_head, hd)) * qscale).astype(np.float32)
    Kc = rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32)
    Vc = rng.standard_normal((ctx_len, n_kv, hd)).astype(np.float32)
    return q, Kc, Vc


def _run(ctx, q, Kc, Vc, n_head, pos0):
    import torch
    n_tok, _, hd = q.shape
    ctx_len, n_kv, _ = Kc.shape
    out = empty((n_tok, n_head, hd), torch.float32)
    dq, dk, dv = dev(q), dev(Kc), dev(Vc)
    ctx.check(ctx.lib.ggq_attention_decode_dev(ctx.h, ptr(dq), ptr(dk), ptr(dv), n_tok, n_head, n_kv, hd, ctx_len,
                                               pos0, ptr(out), stream_handle()), "attention")
    return host(out)


def _check(orc, got, q, Kc, Vc, n_head, pos0):
    qp = [pos0 + t for t in range(q.shape[0])]
    exp = orc.flash_attn(q, Kc, Vc, n_head, qp, f64=True)
    for t in range(q.shape[0]):
        for h in range(n_head):
            err = orc.rel_l2(got[t, h], exp[t, h])
            assert err <= TOL, (t, h, err)


@pytest.mark.parametrize("n_tok,n_head,n_kv,hd,ctx_len,pos0", [
    (1, 32, 8, 64, 300, 299),     # Llama-3.2-1B decode, ctx not a multiple of the chunk
    (1, 32, 8, 128, 4100, 4099),  # Llama-3-8B heads, many chunks
    (3, 8, 8, 128, 1000, 997),    # G = 1, several rows
    (4, 4, 2, 64, 80, 10),        # G = 2, rows see a prefix; later chunks fully masked
    (2, 16, 2, 128, 1, 0),        # G = 8, one position
    (5, 8, 1, 64, 129, 60),       # rows straddling a chunk boundary (60..64)
    (2, 8, 2, 64, 50, 200),       # positions past ctx_len see the whole cache
])
def test_attention_matches_oracle(ctx, orc, n_tok, n_head, n_kv, hd, ctx_len, pos0):
    q, Kc, Vc = _case(n_tok * 7 + ctx_len, n_tok, n_head, n_kv, hd, ctx_len)
    got = _run(ctx, q, Kc, Vc, n_head, pos0)
    _check(orc, got, q, Kc, Vc, n_head, pos0)


def test_attention_peaked_scores_and_determinism(ctx, orc):
    """Large scores (softmax close to one-hot, exp underflows to 0 for most
    positions) and bitwise-repeatable output."""
    q, Kc, Vc = _case(11, 2, 32, 8, 64, 700, qscale=8.0)
    a = _run(ctx, q, Kc, Vc, 32, 698)
    b = _run(ctx, q, Kc, Vc, 32, 698)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    _check(orc, a, q, Kc, Vc, 32, 698)


def test_attention_rejects_bad_shapes(ctx):
    import torch
    buf = empty(4096, torch.float32)
    p, s = ptr(buf), stream_handle()
    lib = ctx.lib
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 1, 32, 8, 96, 4, 0, p, s) == gl.Status.INVALID_PARAM
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 1, 12, 4, 64, 4, 0, p, s) == gl.Status.INVALID_PARAM
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 1, 10, 4, 64, 4, 0, p, s) == gl.Status.INVALID_PARAM
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 1, 8, 8, 64, 0, 0, p, s) == gl.Status.INVALID_PARAM
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 1, 8, 8, 64, 4, -1, p, s) == gl.Status.INVALID_PARAM
    import ctypes
    mis = ctypes.c_void_p(buf.data_ptr() + 4)
    assert lib.ggq_attention_decode_dev(ctx.h, mis, p, p, 1, 8, 8, 64, 4, 0, p, s) == gl.Status.INVALID_PARAM
    assert lib.ggq_attention_decode_dev(ctx.h, p, p, p, 0, 8, 8, 64, 4, 0, p, s) == gl.Status.OK


@pytest.mark.parametrize("spans", ["1", "3", "7", "100000"])
def test_attention_span_counts(ctx, orc, monkeypatch, spans):
    """Same results for any split of the positions into spans (GGQ_ATTN_SPANS,
    read at every launch): one span (no merge), uneven spans, and one span
    per 64-position step; rows with later positions masked in some spans."""
    monkeypatch.setenv("GGQ_ATTN_SPANS", spans)
    q, Kc, Vc = _case(5, 3, 16, 4, 128, 1000, qscale=2.0)
    got = _run(ctx, q, Kc, Vc, 16, 640)
    _check(orc, got, q, Kc, Vc, 16, 640)
