"""Fused gate/up projection + SiLU on the GPU (tessery test_kernels.py:286-294, 780-857):
float64 accuracy at atol = rtol = 5e-5, the route selection, bit-identical results between the
fused routes and linear4 + linear4 + silu_gate, and rows outside a route's region untouched.
Also the Qwen3 layer tail composed from these routes (qwen3.py:246-280) against the oracle."""

import numpy as np
import pytest

from oracle import qwen_block
from oracle import quant4 as ref
from tessery_amd.workloads import bf16_values, bf16_words

pytestmark = pytest.mark.gpu


def test_silu_gate_elementwise(runtime):
    rng = np.random.default_rng(11)
    x = rng.normal(scale=3.0, size=(37, 65)).astype(np.float32)
    up = rng.normal(size=x.shape).astype(np.float32)
    a, b = runtime.upload(x), runtime.upload(up)
    try:
        with runtime.command():
            runtime._dispatch("silu_gate", [a, b], threads=x.size, n=x.size)
        np.testing.assert_allclose(runtime.read(a, x.shape), ref.silu_gate(x, up), atol=1e-6, rtol=1e-6)
        np.testing.assert_array_equal(runtime.read(b, up.shape), up)
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize(
    "rows", [8, 15, 16, 17, 23, 24, 25, 127, 128, 129, 159, 160, 161, 255, 256, 257, 511, 512, 513])
@pytest.mark.parametrize("cancellation", [False, True])
def test_selected_gated4_fallback_and_output_guard(runtime, rows, cancellation):
    rng = np.random.default_rng(2401)
    n, k = 3072, 1024
    x = (rng.integers(-4, 5, size=(rows, k)) / 8).astype(np.float32)
    arrays, sets = [], []
    for _ in range(2):
        codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
        if cancellation:
            codes[:, 1::2] = codes[:, ::2]
            x[:, ::2], x[:, 1::2] = 1.0, -1.0
        w = (ref.pack(codes), bf16_words(np.full((n, k // 64), 0.125)),
             bf16_words(np.full((n, k // 64), -1.0)))
        arrays.extend(w)
        sets.append(w)
    expected = ref.gated4(x, sets[0], sets[1])
    sentinel = np.full((rows + 2, n), np.nan, dtype=np.float32)
    buffers = [runtime.upload(a) for a in [x, *arrays, sentinel, sentinel]]
    try:
        before = runtime.diagnostics()["dispatches"]
        with runtime.command():
            runtime._gated4(buffers, rows=rows, cols=n, k=k)
        after = runtime.diagnostics()["dispatches"]
        fused = rows in (16, 24, 128, 160, 256, 512)
        assert after.get("gated4_16x32_k64", 0) - before.get("gated4_16x32_k64", 0) == int(fused)
        assert after.get("gated4_8x32", 0) - before.get("gated4_8x32", 0) == int(rows == 24)
        selected = runtime.read(buffers[7], sentinel.shape)
        assert np.isnan(selected[rows:]).all()
        np.testing.assert_allclose(selected[:rows], expected, atol=5e-5, rtol=5e-5)
        with runtime.command():
            runtime._linear4([*buffers[:4], buffers[7]], rows=rows, cols=n, k=k)
            runtime._linear4([buffers[0], *buffers[4:7], buffers[8]], rows=rows, cols=n, k=k)
            runtime._dispatch("silu_gate", buffers[7:], threads=rows * n, n=rows * n)
        baseline = runtime.read(buffers[7], sentinel.shape)
        np.testing.assert_array_equal(selected[:rows], baseline[:rows])
    finally:
        for b in buffers:
            b.close()
    assert runtime.active_bytes == 0


@pytest.mark.parametrize("offset", [0, 16])
def test_gated8_complete_tile_offset_and_output_guard(runtime, offset):
    """Ones x words 0x11111111, scale 1, bias 0: gate = up = 64 on the 8 rows of the tile."""
    n, k = 32, 64
    x = np.ones((offset + 8, k), dtype=np.float32)
    packed = np.full((n, k // 8), 0x11111111, dtype=np.uint32)
    scales, biases = bf16_words(np.ones((n, 1))), bf16_words(np.zeros((n, 1)))
    sentinel = np.full((offset + 10, n), np.nan, dtype=np.float32)
    buffers = [runtime.upload(a) for a in [x, packed, scales, biases, packed, scales, biases, sentinel]]
    try:
        with runtime.command():
            runtime._dispatch("gated4_8x32", buffers, threads=128, group_size=128, n=offset,
                              rows=offset + 8, cols=n, k=k)
        out = runtime.read(buffers[-1], sentinel.shape)
        assert np.isnan(out[:offset]).all() and np.isnan(out[offset + 8:]).all()
        np.testing.assert_allclose(out[offset:offset + 8], 64.0 / (1 + np.exp(-64.0)) * 64.0,
                                   rtol=5e-5, atol=5e-5)
    finally:
        for b in buffers:
            b.close()


@pytest.mark.parametrize("rows,cols,k", [(16, 96, 128), (40, 160, 192), (3, 64, 64)])
def test_gated4_other_shapes_match_oracle(runtime, rows, cols, k):
    """Shapes outside the fused table run linear4 twice and silu_gate."""
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    sets = [(ref.pack(rng.integers(0, 16, size=(cols, k), dtype=np.uint32)),
             bf16_words(rng.uniform(0.01, 0.2, size=(cols, k // 64))),
             bf16_words(rng.uniform(-1, 0.1, size=(cols, k // 64)))) for _ in range(2)]
    buffers = [runtime.upload(a) for a in [x, *sets[0], *sets[1]]]
    buffers += [runtime.buffer(rows * cols * 4), runtime.buffer(rows * cols * 4)]
    try:
        with runtime.command():
            runtime._gated4(buffers, rows=rows, cols=cols, k=k)
        got = runtime.read(buffers[7], (rows, cols))
        np.testing.assert_allclose(got, ref.gated4(x, sets[0], sets[1]), atol=5e-5, rtol=5e-5)
    finally:
        for b in buffers:
            b.close()


@pytest.mark.parametrize("rows,cols,k,fused", [(1024, 3072, 1024, True), (1040, 384, 512, True),
                                               (1029, 384, 512, False)])
def test_gated_mlp_on_fp16_mfma_runs_as_one_kernel_with_the_same_bits(runtime, rows, cols, k,
                                                                       fused):
    """From 1024 rows the projections run on fp16 MFMA (row-scaled hi + lo halves of x). When the
    reference's unfused gated form (linear4 gate, linear4 up, silu_gate) is queued with each
    projection in one launch over all rows, the runtime runs the three as one kernel that stages x
    once for both weight sets; it leaves the same bits in both outputs as the three launches in
    separate commands. At 1029 rows each projection is several launches and nothing is fused."""
    rng = np.random.default_rng(rows + cols + k)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    sets = [(ref.pack(rng.integers(0, 16, size=(cols, k), dtype=np.uint32)),
             bf16_words(rng.uniform(0.01, 0.2, size=(cols, k // 64))),
             bf16_words(rng.uniform(-1, 0.1, size=(cols, k // 64)))) for _ in range(2)]
    buffers = [runtime.upload(a) for a in [x, *sets[0], *sets[1]]]
    buffers += [runtime.buffer(rows * cols * 4) for _ in range(4)]
    try:
        before = runtime.diagnostics()["fused_gated"]
        with runtime.command():
            runtime._gated4(buffers[:9], rows=rows, cols=cols, k=k)
        assert runtime.diagnostics()["fused_gated"] == before + int(fused)
        g2, u2 = buffers[9], buffers[10]
        with runtime.command():
            runtime._linear4([*buffers[:4], g2], rows=rows, cols=cols, k=k)
        with runtime.command():
            runtime._linear4([buffers[0], *buffers[4:7], u2], rows=rows, cols=cols, k=k)
        with runtime.command():
            runtime._dispatch("silu_gate", [g2, u2], threads=rows * cols, n=rows * cols)
        assert runtime.diagnostics()["fused_gated"] == before + int(fused)
        got_g, got_u = (runtime.read(b, (rows, cols)) for b in buffers[7:9])
        np.testing.assert_array_equal(got_g, runtime.read(g2, (rows, cols)))
        np.testing.assert_array_equal(got_u, runtime.read(u2, (rows, cols)))
        # against float64: each projection within 2e-6 of sum_k |x| |w| of its element (the fp16
        # MFMA path's bound), carried through silu(g) * u (|silu'| < 1.1)
        xd = x.astype(np.float64)
        wg, wu = (ref.dequantize(*w, k) for w in sets)
        gate, up = xd @ wg.T, xd @ wu.T
        bg, bu = 2e-6 * (np.abs(xd) @ np.abs(wg).T), 2e-6 * (np.abs(xd) @ np.abs(wu).T)
        assert np.all(np.abs(got_u - up) <= bu)
        silu = gate / (1.0 + np.exp(-gate))
        bound = 1.1 * bg * (np.abs(up) + bu) + np.abs(silu) * bu + 1e-30
        assert np.all(np.abs(got_g - silu * up) <= bound), float((np.abs(got_g - silu * up) / bound).max())
    finally:
        for b in buffers:
            b.close()


def layer_tail_weights(rng, hidden, attn_width, inter):
    def weight_set(n, k, scale):
        return (ref.pack(rng.integers(0, 16, size=(n, k), dtype=np.uint32)),
                bf16_words(rng.uniform(0.2, 1.0, size=(n, k // 64)) * scale),
                bf16_words(rng.uniform(-7.5, -0.0, size=(n, k // 64)) * scale))
    return {"o": weight_set(hidden, attn_width, 0.02), "gate": weight_set(inter, hidden, 0.05),
            "up": weight_set(inter, hidden, 0.05), "down": weight_set(hidden, inter, 0.02)}


def layer_tail(runtime, x, attended, w, gamma_words, eps):
    """qwen3.py:246-280 on the runtime: o_proj, residual add, RMSNorm, gated4, down_proj,
    residual add. Returns the residual stream after the layer."""
    tokens, hidden = x.shape
    inter = w["gate"][0].shape[0]
    bufs = {"x": runtime.upload(x), "att": runtime.upload(attended),
            "gamma": runtime.upload(gamma_words), "proj": runtime.buffer(tokens * hidden * 4),
            "norm": runtime.buffer(tokens * hidden * 4), "gate": runtime.buffer(tokens * inter * 4),
            "up": runtime.buffer(tokens * inter * 4)}
    for name, arrays in w.items():
        bufs.update({f"{name}{i}": runtime.upload(a) for i, a in enumerate(arrays)})
    try:
        with runtime.command():
            runtime._linear4([bufs["att"], bufs["o0"], bufs["o1"], bufs["o2"], bufs["proj"]],
                             rows=tokens, cols=hidden, k=attended.shape[1])
            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]], threads=tokens * hidden,
                              n=tokens * hidden)
            runtime._dispatch("rms_norm", [bufs["x"], bufs["gamma"], bufs["norm"]],
                              threads=tokens * 32, group_size=32, cols=hidden, eps=eps)
            runtime._gated4([bufs["norm"], bufs["gate0"], bufs["gate1"], bufs["gate2"], bufs["up0"],
                             bufs["up1"], bufs["up2"], bufs["gate"], bufs["up"]],
                            rows=tokens, cols=inter, k=hidden)
            runtime._linear4([bufs["gate"], bufs["down0"], bufs["down1"], bufs["down2"], bufs["proj"]],
                             rows=tokens, cols=hidden, k=inter)
            runtime._dispatch("add", [bufs["x"], bufs["proj"], bufs["x"]], threads=tokens * hidden,
                              n=tokens * hidden)
        return runtime.read(bufs["x"], x.shape)
    finally:
        for b in bufs.values():
            b.close()


@pytest.mark.parametrize("tokens", [16, 24, 37, 128])
def test_qwen3_layer_tail_matches_oracle(runtime, tokens):
    """Qwen3-0.6B widths (hidden 1024, 16 x 128 attention, intermediate 3072); the fused gated
    route runs at 16, 24 and 128 tokens, the unfused one at 37."""
    rng = np.random.default_rng(5 + tokens)
    hidden, attn_width, inter, eps = 1024, 2048, 3072, 1e-6
    x = rng.normal(size=(tokens, hidden)).astype(np.float32)
    attended = rng.normal(scale=0.5, size=(tokens, attn_width)).astype(np.float32)
    w = layer_tail_weights(rng, hidden, attn_width, inter)
    gamma = bf16_words(rng.uniform(0.5, 1.5, hidden))
    got = layer_tail(runtime, x, attended, w, gamma, eps)
    expected = qwen_block.layer_tail(x, attended, w, bf16_values(gamma), eps=eps)
    scale = np.abs(expected).max()
    np.testing.assert_allclose(got, expected, atol=1e-5 * scale, rtol=1e-4)


@pytest.mark.parametrize("rows,cols,k,fused", [(4096, 1024, 1024, True), (1040, 256, 512, True),
                                               (1029, 256, 512, False)])
def test_two_projections_of_one_x_run_as_one_kernel_with_the_same_bits(runtime, rows, cols, k,
                                                                       fused):
    """Two uint4 projections of the same x with the same shape queued back to back (a Qwen3
    layer's k and v projections) run as one fp16-MFMA launch from 1024 rows, leaving the bits of
    the two launches in separate commands in both outputs; at 1029 rows each projection is
    several launches and nothing is fused."""
    rng = np.random.default_rng(7 * rows + cols + k)
    x = rng.normal(size=(rows, k)).astype(np.float32)
    sets = [(ref.pack(rng.integers(0, 16, size=(cols, k), dtype=np.uint32)),
             bf16_words(rng.uniform(0.01, 0.2, size=(cols, k // 64))),
             bf16_words(rng.uniform(-1, 0.1, size=(cols, k // 64)))) for _ in range(2)]
    buffers = [runtime.upload(a) for a in [x, *sets[0], *sets[1]]]
    outs = [runtime.buffer(rows * cols * 4) for _ in range(4)]
    try:
        before = runtime.diagnostics()["fused_pairs"]
        with runtime.command():
            runtime._linear4([*buffers[:4], outs[0]], rows=rows, cols=cols, k=k)
            runtime._linear4([buffers[0], *buffers[4:7], outs[1]], rows=rows, cols=cols, k=k)
        assert runtime.diagnostics()["fused_pairs"] == before + int(fused)
        with runtime.command():
            runtime._linear4([*buffers[:4], outs[2]], rows=rows, cols=cols, k=k)
        with runtime.command():
            runtime._linear4([buffers[0], *buffers[4:7], outs[3]], rows=rows, cols=cols, k=k)
        assert runtime.diagnostics()["fused_pairs"] == before + int(fused)
        got = [runtime.read(b, (rows, cols)) for b in outs]
        np.testing.assert_array_equal(got[0], got[2])
        np.testing.assert_array_equal(got[1], got[3])
        # and within the fp16 MFMA path's bound of float64 (2e-6 of sum_k |x| |w| per element)
        xd = x.astype(np.float64)
        for (packed, s, b), y in zip(sets, got[:2]):
            w = ref.dequantize(packed, s, b, k, "bf16")
            bound = 2e-6 * (np.abs(xd) @ np.abs(w).T) + 1e-30
            assert np.all(np.abs(y - xd @ w.T) <= bound)
    finally:
        for b in buffers + outs:
            b.close()
