"""q/k RMSNorm and RoPE on the GPU against the float64 oracle (tessery test_kernels.py:96-110,
256-286 shapes and tolerances), plus the fp16 k prologue and the fp32 unfused Qwen3 block."""

import numpy as np
import pytest

from oracle import attention as ref_attention
from oracle import norm_rope as ref
from tessery_amd import workloads
from tessery_amd.workloads import bf16_values, bf16_words
from tests.test_gpu_attention import check_f32, run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("unit_weight", [True, False])
def test_rms_norm(runtime, unit_weight):
    rng = np.random.default_rng(4)
    x = rng.normal(size=(2, 3, 64)).astype(np.float32)
    w = bf16_words(np.ones(64) if unit_weight else rng.uniform(0.5, 1.5, 64))
    got = run(runtime, "rms_norm", [x, w], x.shape, threads=6 * 32, group_size=32, cols=64,
              eps=1e-6)
    np.testing.assert_allclose(got, ref.rms_norm(x, bf16_values(w), 1e-6), atol=1e-6)


def test_rms_norm_in_place(runtime):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(37, 128)).astype(np.float32)
    w = bf16_words(rng.uniform(0.5, 1.5, 128))
    xb, wb = runtime.upload(x), runtime.upload(w)
    try:
        with runtime.command():
            runtime._dispatch("rms_norm", [xb, wb, xb], threads=37 * 32, group_size=32, cols=128,
                              eps=1e-6)
        got = runtime.read(xb, x.shape)
    finally:
        xb.close()
        wb.close()
    np.testing.assert_allclose(got, ref.rms_norm(x, bf16_values(w), 1e-6), atol=1e-6)


@pytest.mark.parametrize("rows,cols", [(9, 1030), (5, 66), (130, 1024), (3, 4)])
def test_rms_norm_widths(runtime, rows, cols):
    """Row widths that take the scalar path (cols % 4 != 0) and the float4 path (hidden 1024)."""
    rng = np.random.default_rng(cols)
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    w = bf16_words(rng.uniform(0.5, 1.5, cols))
    got = run(runtime, "rms_norm", [x, w], x.shape, threads=rows * 32, group_size=32, cols=cols,
              eps=1e-6)
    np.testing.assert_allclose(got, ref.rms_norm(x, bf16_values(w), 1e-6), atol=1e-6,
                               rtol=1e-6)


@pytest.mark.parametrize("shape,theta",[((2, 3, 4, 64), 10000.0), ((2, 512, 2, 128), 1e6)])
def test_rope(runtime, shape, theta):
    rng = np.random.default_rng(8)
    x = rng.normal(size=shape).astype(np.float32)
    buffer = runtime.upload(x)
    try:
        with runtime.command():
            runtime._dispatch("rope", [buffer], threads=x.size // 2, n=x.size // 2,
                              heads=shape[2], seq=shape[1], dim=shape[3], theta=theta)
        got = runtime.read(buffer, x.shape)
    finally:
        buffer.close()
    np.testing.assert_allclose(got, ref.rope(x, theta), atol=2e-6)


# (dim, heads): lanes per position = dim / 16 * heads = 16, 32, 64, 24 (does not divide 256),
# 256 (one position per pass), 40
@pytest.mark.parametrize("dim,heads", [(32, 8), (64, 8), (128, 8), (128, 3), (128, 32), (64, 5)])
def test_norm_rope_f16_prologue(runtime, dim, heads):
    check_norm_rope_f16(runtime, dim, heads, np.array([70, 0, 1, 33], np.uint32), seq=70)


def test_norm_rope_f16_many_rows(runtime):
    """More than 64 batch rows: the launcher's per-row grid (the compacted one scans at most 64)."""
    rng = np.random.default_rng(66)
    check_norm_rope_f16(runtime, 128, 8, rng.integers(0, 6, 66).astype(np.uint32), seq=5)


def check_norm_rope_f16(runtime, dim, heads, lengths, seq):
    shape = workloads.Shape(len(lengths), seq, 2 * heads, heads, dim, causal=True)
    t = workloads.qwen_layer(shape, 0, seed=dim + heads)
    sentinel = np.full((2,) + t["k"].shape, np.nan, np.float16)
    bufs = [runtime.upload(t["k"]), runtime.upload(t["k_norm"]), runtime.upload(lengths),
            runtime.upload(sentinel)]
    try:
        with runtime.command():
            runtime._dispatch("norm_rope_f16", bufs, threads=shape.tokens, group_size=256,
                              heads=shape.kv_heads, seq=shape.seq, dim=dim, eps=workloads.EPS,
                              theta=workloads.THETA, flags=1)
        got = runtime.read(bufs[3], sentinel.shape, np.float16).astype(np.float64)
    finally:
        for b in bufs:
            b.close()
    expected = ref.norm_rope(t["k"], bf16_values(t["k_norm"]), workloads.EPS, workloads.THETA)
    for b, length in enumerate(lengths):
        exp = expected[b, :length]
        assert np.all(np.abs(got[0, b, :length] - exp) <= 2.0**-11 * np.abs(exp) + 1e-7)
        # fp32 math: absolute error at the scale of the row (RoPE sums can cancel)
        assert np.all(np.abs(got[0, b, :length] + got[1, b, :length] - exp) <= 2e-6 * (np.abs(exp) + 1))
        assert np.isnan(got[:, b, length:]).all()  # padded rows are never written


def test_fp32_unfused_qwen_block(runtime):
    """tessery's op order (qwen3.py:216-245) in fp32: rms_norm + rope on q and on k, in place,
    then the attention route; against the float64 composition."""
    shape = workloads.Shape(2, 96, 4, 2, 128, causal=True)
    rng = np.random.default_rng(21)
    q = rng.normal(size=(2, 96, 4, 128)).astype(np.float32)
    k = rng.normal(size=(2, 96, 2, 128)).astype(np.float32)
    v = rng.normal(size=(2, 96, 2, 128)).astype(np.float32)
    gq, gk = bf16_words(rng.uniform(0.5, 1.5, 128)), bf16_words(rng.uniform(0.5, 1.5, 128))
    lengths = np.array([96, 41], np.uint32)
    bufs = {n: runtime.upload(a) for n, a in dict(q=q, k=k, v=v, gq=gq, gk=gk, lengths=lengths).items()}
    bufs["out"] = runtime.buffer(q.nbytes)
    tokens = shape.tokens
    try:
        with runtime.command():
            for name, heads, w in (("q", 4, "gq"), ("k", 2, "gk")):
                runtime._dispatch("rms_norm", [bufs[name], bufs[w], bufs[name]],
                                  threads=tokens * heads * 32, group_size=32, cols=128, eps=1e-6)
                count = tokens * heads * 64
                runtime._dispatch("rope", [bufs[name]], threads=count, n=count, heads=heads,
                                  seq=96, dim=128, theta=1e6)
            runtime._attention([bufs["q"], bufs["k"], bufs["v"], bufs["lengths"], bufs["out"]],
                               tokens=tokens, seq=96, heads=4, kv_heads=2, dim=128)
        got = runtime.read(bufs["out"], q.shape)
    finally:
        for b in bufs.values():
            b.close()
    qn = ref.norm_rope(q, bf16_values(gq), 1e-6, 1e6)
    kn = ref.norm_rope(k, bf16_values(gk), 1e-6, 1e6)
    check_f32(got, ref_attention.attention(qn, kn, v, lengths, bidirectional=False))


@pytest.mark.parametrize("tokens,heads,seq,dim", [(64, 16, 32, 128), (24, 8, 12, 64),
                                                  (10, 2, 5, 256), (9, 3, 3, 8), (6, 2, 3, 12)])
def test_rms_norm_then_rope_fused_in_one_command(runtime, tokens, heads, seq, dim):
    """rms_norm in place followed by rope on the same rows (qwen3.py:216-237) runs as one kernel
    when both sit in one command; the bits equal the two launches run in separate commands."""
    rng = np.random.default_rng(dim + heads)
    x = (3.0 * rng.normal(size=(tokens * heads, dim))).astype(np.float32)
    w = bf16_words(rng.uniform(0.5, 1.5, dim))
    theta, eps = 1e6, 1e-6
    count = tokens * heads * dim // 2

    def norm(buf, wb):
        runtime._dispatch("rms_norm", [buf, wb, buf], threads=tokens * heads * 32, group_size=32,
                          cols=dim, eps=eps)

    def rope(buf):
        runtime._dispatch("rope", [buf], threads=count, n=count, heads=heads, seq=seq, dim=dim,
                          theta=theta)

    results = []
    for fused in (True, False):
        xb, wb = runtime.upload(x), runtime.upload(w)
        try:
            if fused:
                with runtime.command():
                    norm(xb, wb)
                    rope(xb)
            else:
                with runtime.command():
                    norm(xb, wb)
                with runtime.command():
                    rope(xb)
            results.append(runtime.read(xb, x.shape))
        finally:
            xb.close()
            wb.close()
    np.testing.assert_array_equal(results[0], results[1])
    # rows are [batch, seq, heads] in order (tokens is a multiple of seq in every case)
    want = ref.norm_rope(x.reshape(-1, seq, heads, dim), bf16_values(w), eps, theta)
    np.testing.assert_allclose(results[0], want.reshape(x.shape), atol=2e-5, rtol=1e-5)


@pytest.mark.parametrize("rows,cols,in_place", [(130, 1024, False), (7, 64, False), (5, 1030, False),
                                                (33, 1024, True)])
def test_add_then_rms_norm_fused_in_one_command(runtime, rows, cols, in_place):
    """add(x, r -> x) followed by rms_norm(x -> y) (the residual and the next norm of
    qwen3.py:246-280) runs as one pass inside one command; x and y equal, bit for bit, the two
    launches run in separate commands (cols % 4 != 0 is not fused and must match too)."""
    rng = np.random.default_rng(rows + cols)
    x = rng.normal(size=(rows, cols)).astype(np.float32)
    r = (0.5 * rng.normal(size=(rows, cols))).astype(np.float32)
    w = bf16_words(rng.uniform(0.5, 1.5, cols))
    outs = []
    for fused in (True, False):
        xb, rb, wb = runtime.upload(x), runtime.upload(r), runtime.upload(w)
        yb = xb if in_place else runtime.buffer(x.nbytes)
        try:
            add = dict(threads=rows * cols, n=rows * cols)
            norm = dict(threads=rows * 32, group_size=32, cols=cols, eps=1e-6)
            if fused:
                with runtime.command():
                    runtime._dispatch("add", [xb, rb, xb], **add)
                    runtime._dispatch("rms_norm", [xb, wb, yb], **norm)
            else:
                with runtime.command():
                    runtime._dispatch("add", [xb, rb, xb], **add)
                with runtime.command():
                    runtime._dispatch("rms_norm", [xb, wb, yb], **norm)
            outs.append((runtime.read(xb, x.shape), runtime.read(yb, x.shape)))
        finally:
            for b in {id(b): b for b in (xb, rb, wb, yb)}.values():
                b.close()
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    want = ref.rms_norm(x.astype(np.float64) + r, bf16_values(w), 1e-6)
    np.testing.assert_allclose(outs[0][1], want, atol=2e-6, rtol=2e-6)
