"""fp32 projections and the elementwise kernels of tessery's BERT layer on the GPU
(test_kernels.py:299-353, 404-420, 600-640): float64 accuracy, the route partition seen in the
dispatch counts, rows outside a route's region untouched, and the BGE layer composed from these
routes (bert.py:186-230) against the float64 oracle."""

import math

import numpy as np
import pytest

from oracle import bert_block as ref
from tests.test_gpu_attention import run

pytestmark = pytest.mark.gpu


def test_layer_norm(runtime):
    rng = np.random.default_rng(37)
    x = rng.normal(size=(3, 67)).astype(np.float32)
    scale = rng.normal(size=67).astype(np.float32)
    bias = rng.normal(size=67).astype(np.float32)
    out = run(runtime, "layer_norm", [x, scale, bias], x.shape, threads=3 * 32, group_size=32,
              cols=67, eps=1e-12)
    np.testing.assert_allclose(out, ref.layer_norm(x, scale, bias, 1e-12), atol=1e-6, rtol=1e-5)
    # many rows, out aliasing x
    x = rng.normal(size=(203, 384)).astype(np.float32)
    w, b = rng.uniform(0.5, 1.5, 384).astype(np.float32), rng.normal(size=384).astype(np.float32)
    bufs = [runtime.upload(a) for a in (x, w, b)]
    try:
        with runtime.command():
            runtime._dispatch("layer_norm", [bufs[0], bufs[1], bufs[2], bufs[0]], threads=203 * 32,
                              group_size=32, cols=384, eps=1e-12)
        np.testing.assert_allclose(runtime.read(bufs[0], x.shape), ref.layer_norm(x, w, b, 1e-12),
                                   atol=1e-5, rtol=1e-5)
    finally:
        for bb in bufs:
            bb.close()


def test_gelu_erf_form_and_bias(runtime):
    x = np.linspace(-12, 12, 10001, dtype=np.float32)
    buffer = runtime.upload(x)
    try:
        with runtime.command():
            runtime._dispatch("gelu_f32", [buffer], threads=x.size, n=x.size)
        expected = np.array([0.5 * float(v) * (1 + math.erf(float(v) / math.sqrt(2))) for v in x])
        np.testing.assert_allclose(runtime.read(buffer, x.shape), expected, atol=2e-6, rtol=1e-6)
    finally:
        buffer.close()
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    bias = np.array([-2, -1, 1, 2], np.float32)
    a, b = runtime.upload(x), runtime.upload(bias)
    try:
        with runtime.command():
            runtime._dispatch("add_bias", [a, b], threads=x.size, n=x.size, cols=4)
        np.testing.assert_array_equal(runtime.read(a, x.shape), x + bias)
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize(
    "shape", [(8, 8, 32), (16, 384, 384), (32, 512, 384), (32, 1536, 384), (8, 65, 32), (9, 64, 32),
              (3, 7, 5), (40, 130, 200)])
def test_tiled_matmul_and_unaligned_fallback(runtime, shape):
    m, k, n = shape
    rng = np.random.default_rng(33)
    a = rng.normal(size=(m, k)).astype(np.float32)
    b = rng.normal(size=(k, n)).astype(np.float32)
    before = dict(runtime.diagnostics()["dispatches"])
    got = runtime.matmul(a, b)
    np.testing.assert_allclose(got, a.astype(np.float64) @ b.astype(np.float64), atol=5e-5, rtol=5e-5)
    tiled = m >= 8 and m % 8 == 0 and n % 32 == 0 and k % 8 == 0 and k <= 512
    name = "matmul_f32_tiled" if tiled else "matmul_f32"
    if m >= 8 and (n, k) in ((384, 384), (1536, 384), (384, 1536)):
        name = "matmul_f32_chunk32"
    after = runtime.diagnostics()["dispatches"]
    assert {key: after[key] - before.get(key, 0) for key in after if after[key] != before.get(key, 0)} == {name: 1}
    assert runtime.active_bytes == 0


@pytest.mark.parametrize("m", [8, 9, 10, 11, 12, 13, 14, 15, 128, 4096])
@pytest.mark.parametrize("n,k", [(384, 384), (1536, 384), (384, 1536)])
@pytest.mark.parametrize("pattern", ["random", "cancellation"])
def test_f32_chunked_projections_and_bounded_tail(runtime, m, n, k, pattern):
    rng = np.random.default_rng(2026 + m)
    x = rng.normal(size=(m, k)).astype(np.float32)
    w = rng.normal(size=(n, k)).astype(np.float32)
    if pattern == "cancellation":
        x[:, 1::2] = -x[:, ::2]
        w[:, 1::2] = w[:, ::2] + np.float32(2**-16)
    expected = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(runtime.matmul(x, np.ascontiguousarray(w.T)), expected, atol=5e-5,
                               rtol=5e-5)


@pytest.mark.parametrize("rows,cols,k", [(11000, 384, 1536), (2800, 1536, 384), (10944, 384, 384),
                                         (4000, 384, 384), (4096, 384, 1536)])
@pytest.mark.parametrize("pattern", ["random", "cancellation", "wide range"])
def test_large_projections_on_split_bf16_mfma(runtime, rows, cols, k, pattern):
    """Shapes with at least 64 tiles of 64 x 128 (K % 32 == 0, N % 128 == 0) run on bf16 MFMA with
    both operands split exactly into three bf16 terms and six products per fp32 product (below 512
    tiles with K split into partial sums added in order); the result keeps fp32 accuracy against a
    float64 product, through cancellation (pairs of columns that nearly cancel) and over a wide
    exponent range (bf16 keeps fp32's exponent)."""
    rng = np.random.default_rng(rows + cols + k)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    w = rng.normal(scale=k ** -0.5, size=(cols, k)).astype(np.float32)
    if pattern == "cancellation":
        x[:, 1::2] = -x[:, ::2]
        w[:, 1::2] = w[:, ::2] + np.float32(2**-16)
    elif pattern == "wide range":
        x *= np.exp2(rng.integers(-40, 40, size=(rows, 1))).astype(np.float32)
        w *= np.exp2(rng.integers(-20, 20, size=(1, k))).astype(np.float32)
    expected = x.astype(np.float64) @ w.astype(np.float64).T
    got = runtime.matmul(x, np.ascontiguousarray(w.T))
    scale = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    # fp32-grade: within a few units of 2^-24 of the sum of |products|
    assert np.max(np.abs(got - expected) / np.maximum(scale, 1e-300)) < 2e-6
    if pattern == "random":
        np.testing.assert_allclose(got, expected, atol=5e-5, rtol=5e-5)


@pytest.mark.parametrize("rows,cols,k", [(2800, 1536, 384), (11000, 384, 1536), (4000, 384, 1536)])
def test_large_fused_projection_gelu_matches_split(runtime, rows, cols, k):
    """The bias + GELU epilogue of the split-bf16 projection gives the bits of the projection
    followed by the gelu_f32 launch, and both match a float64 reference."""
    rng = np.random.default_rng(rows * 5 + k)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    w = rng.normal(scale=k ** -0.5, size=(cols, k)).astype(np.float32)
    bias = rng.normal(size=cols).astype(np.float32)

    def run(split):
        bufs = [runtime.upload(a) for a in (x, w, np.zeros((rows, cols), np.float32), bias)]
        try:
            steps = [lambda: runtime._matmul_bias_f32(bufs, rows=rows, cols=cols, k=k),
                     lambda: runtime._dispatch("gelu_f32", [bufs[2]], threads=rows * cols,
                                               n=rows * cols)]
            if split:
                for step in steps:
                    with runtime.command():
                        step()
            else:
                with runtime.command():
                    for step in steps:
                        step()
            return runtime.read(bufs[2], (rows, cols))
        finally:
            for b in bufs:
                b.close()

    fused, split = run(False), run(True)
    np.testing.assert_array_equal(fused, split)
    np.testing.assert_allclose(fused, ref.gelu(ref.linear(x, w, bias)), atol=5e-5, rtol=5e-5)


def test_f32_scalar_tail_does_not_touch_complete_rows(runtime):
    rng = np.random.default_rng(33)
    x = rng.normal(size=(15, 1536)).astype(np.float32)
    w = rng.normal(size=(384, 1536)).astype(np.float32)
    sentinel = np.full((15, 384), np.nan, np.float32)
    buffers = [runtime.upload(a) for a in (x, w, sentinel)]
    try:
        with runtime.command():
            runtime._dispatch("matmul_f32", buffers, threads=2 * 384 * 32, group_size=32, n=8,
                              rows=15, cols=384, k=1536)
        out = runtime.read(buffers[-1], (15, 384))
        assert np.isnan(out[:8]).all()
        np.testing.assert_allclose(out[8:], x[8:].astype(np.float64) @ w.astype(np.float64).T,
                                   atol=5e-5, rtol=5e-5)
    finally:
        for b in buffers:
            b.close()


@pytest.mark.parametrize("rows", [1, 7, 8, 13, 129])
@pytest.mark.parametrize("cols,k", [(384, 384), (1536, 384), (384, 1536), (385, 384)])
def test_affine_projection_routes(runtime, rows, cols, k):
    """_matmul_bias_f32 on every branch of its partition, against x W^T + b in float64."""
    rng = np.random.default_rng(rows + cols)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    w = rng.normal(scale=k ** -0.5, size=(cols, k)).astype(np.float32)
    bias = rng.normal(size=cols).astype(np.float32)
    bufs = [runtime.upload(x), runtime.upload(w), runtime.buffer(rows * cols * 4), runtime.upload(bias)]
    try:
        with runtime.command():
            runtime._matmul_bias_f32(bufs, rows=rows, cols=cols, k=k)
        np.testing.assert_allclose(runtime.read(bufs[2], (rows, cols)), ref.linear(x, w, bias),
                                   atol=5e-5, rtol=5e-5)
    finally:
        for b in bufs:
            b.close()


def bge_weights(rng, hidden, inter):
    w = {}
    for name, (n, k) in {"q": (hidden, hidden), "k": (hidden, hidden), "v": (hidden, hidden),
                         "o": (hidden, hidden), "i": (inter, hidden), "out": (hidden, inter)}.items():
        w[name] = rng.normal(scale=k ** -0.5, size=(n, k)).astype(np.float32)
        w[name + "_b"] = rng.normal(scale=0.1, size=n).astype(np.float32)
    for ln in ("ln1", "ln2"):
        w[ln + "_w"] = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
        w[ln + "_b"] = rng.normal(scale=0.1, size=hidden).astype(np.float32)
    return w


def bge_layer(runtime, x, lengths, w, heads, eps):
    """bert.py:186-230 on the runtime (one encoder layer, x updated in place)."""
    b, s, hidden = x.shape
    tokens, inter = b * s, w["i"].shape[0]
    bufs = {name: runtime.upload(a) for name, a in w.items()}
    bufs["x"] = runtime.upload(x.reshape(tokens, hidden))
    bufs["len"] = runtime.upload(lengths.astype(np.uint32))
    for name, width in (("q_", hidden), ("k_", hidden), ("v_", hidden), ("att", hidden),
                        ("proj", hidden), ("act", inter)):
        bufs[name] = runtime.buffer(tokens * width * 4)

    def linear(src, dst, name, outputs, inputs):
        runtime._matmul_bias_f32([bufs[src], bufs[name], bufs[dst], bufs[name + "_b"]], rows=tokens,
                                 cols=outputs, k=inputs)

    def norm(name):
        runtime._dispatch("layer_norm", [bufs["x"], bufs[name + "_w"], bufs[name + "_b"], bufs["x"]],
                          threads=tokens * 32, group_size=32, cols=hidden, eps=eps)

    try:
        with runtime.command():
            for target, name in (("q_", "q"), ("k_", "k"), ("v_", "v")):
                linear("x", target, name, hidden, hidden)
            runtime._attention([bufs["q_"], bufs["k_"], bufs["v_"], bufs["len"], bufs["att"]],
                               tokens=tokens, seq=s, heads=heads, kv_heads=heads,
                               dim=hidden // heads, bidirectional=True)
            linear("att", "proj", "o", hidden, hidden)
            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]], threads=tokens * hidden,
                              n=tokens * hidden)
            norm("ln1")
            linear("x", "act", "i", inter, hidden)
            runtime._dispatch("gelu_f32", [bufs["act"]], threads=tokens * inter, n=tokens * inter)
            linear("act", "proj", "out", hidden, inter)
            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]], threads=tokens * hidden,
                              n=tokens * hidden)
            norm("ln2")
        return runtime.read(bufs["x"], x.shape)
    finally:
        for bb in bufs.values():
            bb.close()


@pytest.mark.parametrize("batch,seq,lengths", [(2, 16, [16, 9]), (2, 64, [64, 23]),
                                               (3, 96, [96, 2, 71]), (1, 129, [100])])
def test_bge_layer_matches_oracle(runtime, batch, seq, lengths):
    """BGE-small widths (hidden 384, 12 heads x 32, intermediate 1536); S = 16 takes the scalar
    attention route, 64 and 96 the tiled one, 129 the tail route."""
    rng = np.random.default_rng(seq + batch)
    hidden, heads, inter, eps = 384, 12, 1536, 1e-12
    x = rng.normal(size=(batch, seq, hidden)).astype(np.float32)
    lengths = np.array(lengths, np.uint32)
    w = bge_weights(rng, hidden, inter)
    got = bge_layer(runtime, x, lengths, w, heads, eps)
    expected = ref.layer(x, lengths, w, heads=heads, eps=eps)
    np.testing.assert_allclose(got, expected, atol=5e-5, rtol=5e-5)


def test_bge_layer_at_32x512_matches_oracle_on_sampled_rows(runtime):
    """The layer at the bge_layer_32x512 size (16,384 tokens: every projection on the split-bf16
    kernel) against the float64 oracle on batch rows 0, 1 and 31 (rows are independent)."""
    rng = np.random.default_rng(3232)
    batch, seq, hidden, heads, inter, eps = 32, 512, 384, 12, 1536, 1e-12
    x = rng.normal(size=(batch, seq, hidden)).astype(np.float32)
    lengths = rng.integers(2, seq + 1, size=batch).astype(np.uint32)
    w = bge_weights(rng, hidden, inter)
    got = bge_layer(runtime, x, lengths, w, heads, eps)
    rows = [0, 1, 31]
    expected = ref.layer(x[rows], lengths[rows], w, heads=heads, eps=eps)
    np.testing.assert_allclose(got[rows], expected, atol=5e-5, rtol=5e-5)


@pytest.mark.parametrize("rows,cols,k", [(64, 1536, 384), (200, 384, 1536), (13, 96, 40)])
def test_fused_projection_gelu_and_residual_norm_are_bit_exact(runtime, rows, cols, k):
    """Within one command the runtime runs projection + gelu_f32 and add + layer_norm (in place)
    as single launches; split over two commands they run separately. Same bits either way."""
    rng = np.random.default_rng(rows * 3 + k)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    w = rng.normal(scale=k ** -0.5, size=(cols, k)).astype(np.float32)
    bias = rng.normal(size=cols).astype(np.float32)
    resid = rng.normal(size=(rows, cols)).astype(np.float32)
    lw, lb = rng.uniform(0.5, 1.5, cols).astype(np.float32), rng.normal(size=cols).astype(np.float32)

    def run_layer(split):
        bufs = [runtime.upload(a) for a in (x, w, np.zeros((rows, cols), np.float32), bias, resid, lw, lb)]
        xb, wb, yb, bb, rb, lwb, lbb = bufs
        try:
            steps = [
                lambda: runtime._matmul_bias_f32([xb, wb, yb, bb], rows=rows, cols=cols, k=k),
                lambda: runtime._dispatch("gelu_f32", [yb], threads=rows * cols, n=rows * cols),
                lambda: runtime._dispatch("add", [rb, yb, rb], threads=rows * cols, n=rows * cols),
                lambda: runtime._dispatch("layer_norm", [rb, lwb, lbb, rb], threads=rows * 32,
                                          group_size=32, cols=cols, eps=1e-12),
            ]
            if split:
                for s in steps:
                    with runtime.command():
                        s()
            else:
                with runtime.command():
                    for s in steps:
                        s()
            return runtime.read(yb, (rows, cols)), runtime.read(rb, (rows, cols))
        finally:
            for b in bufs:
                b.close()

    fused_y, fused_r = run_layer(False)
    split_y, split_r = run_layer(True)
    np.testing.assert_array_equal(fused_y, split_y)
    np.testing.assert_array_equal(fused_r, split_r)
    expected_y = ref.gelu(ref.linear(x, w, bias))
    np.testing.assert_allclose(fused_y, expected_y, atol=5e-5, rtol=5e-5)
    np.testing.assert_allclose(fused_r, ref.layer_norm(resid + expected_y, lw, lb, 1e-12),
                               atol=5e-5, rtol=5e-5)


def plan_replays(runtime, x, lengths, w, heads, eps, replays):
    """The BGE layer of bge_layer() captured once as a plan and replayed `replays` times over the
    same buffers; x is rewritten from the host before every replay (eager work between them).
    Returns the layer output of the capture run and of every replay."""
    b, s, hidden = x.shape
    tokens, inter = b * s, w["i"].shape[0]
    bufs = {name: runtime.upload(a) for name, a in w.items()}
    bufs["x"] = runtime.upload(x.reshape(tokens, hidden))
    bufs["len"] = runtime.upload(lengths.astype(np.uint32))
    for name, width in (("q_", hidden), ("k_", hidden), ("v_", hidden), ("att", hidden),
                        ("proj", hidden), ("act", inter)):
        bufs[name] = runtime.buffer(tokens * width * 4)
    order = sorted(bufs)
    outs = []

    def linear(src, dst, name, outputs, inputs):
        runtime._matmul_bias_f32([bufs[src], bufs[name], bufs[dst], bufs[name + "_b"]], rows=tokens,
                                 cols=outputs, k=inputs)

    def norm(name):
        runtime._dispatch("layer_norm", [bufs["x"], bufs[name + "_w"], bufs[name + "_b"], bufs["x"]],
                          threads=tokens * 32, group_size=32, cols=hidden, eps=eps)

    try:
        with runtime._workspace():
            for _ in range(replays + 1):
                runtime.write(bufs["x"], x.reshape(tokens, hidden))
                with runtime.command():
                    with runtime._execution_plan(("bge", b, s), [bufs[n] for n in order]) as replayed:
                        if not replayed:
                            for target, name in (("q_", "q"), ("k_", "k"), ("v_", "v")):
                                linear("x", target, name, hidden, hidden)
                            runtime._attention([bufs["q_"], bufs["k_"], bufs["v_"], bufs["len"],
                                                bufs["att"]], tokens=tokens, seq=s, heads=heads,
                                               kv_heads=heads, dim=hidden // heads, bidirectional=True)
                            linear("att", "proj", "o", hidden, hidden)
                            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]],
                                              threads=tokens * hidden, n=tokens * hidden)
                            norm("ln1")
                            linear("x", "act", "i", inter, hidden)
                            runtime._dispatch("gelu_f32", [bufs["act"]], threads=tokens * inter,
                                              n=tokens * inter)
                            linear("act", "proj", "out", hidden, inter)
                            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]],
                                              threads=tokens * hidden, n=tokens * hidden)
                            norm("ln2")
                outs.append(runtime.read(bufs["x"], x.shape))
        return outs
    finally:
        for bb in bufs.values():
            bb.close()


@pytest.mark.parametrize("graphs", ["1", "0"])
def test_plan_replay_graphs_match_eager(monkeypatch, graphs):
    """Plan replays run as cached HIP graphs (TESSERY_HIP_GRAPHS=0: launched one by one); every
    replay, with host writes and synchronizations between them, equals the eager capture run
    bit for bit, and that run matches the float64 oracle."""
    from tessery_amd import HipRuntime

    monkeypatch.setenv("TESSERY_HIP_GRAPHS", graphs)
    rng = np.random.default_rng(71)
    hidden, heads, inter, eps = 384, 12, 1536, 1e-12
    x = rng.normal(size=(2, 64, hidden)).astype(np.float32)
    lengths = np.array([64, 23], np.uint32)
    w = bge_weights(rng, hidden, inter)
    with HipRuntime() as rt:
        outs = plan_replays(rt, x, lengths, w, heads, eps, replays=5)
        diag = rt.diagnostics()
    assert diag["plan_builds"] == 1 and diag["plan_hits"] == 5
    assert (diag["graph_builds"], diag["graph_launches"]) == ((1, 5) if graphs == "1" else (0, 0))
    for out in outs[1:]:
        np.testing.assert_array_equal(out, outs[0])
    np.testing.assert_allclose(outs[0], ref.layer(x, lengths, w, heads=heads, eps=eps), atol=5e-5,
                               rtol=5e-5)
