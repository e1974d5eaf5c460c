"""Attention parity on the GPU through the C ABI (HipRuntime -> mi_dispatch), against the float64
oracle on identical seeded inputs.

fp32 routes use tessery's own tolerance (atol 2e-6, rtol 2e-5, test_kernels.py:157) and must
also stay within max-abs 1e-4. The plain fp16-operand route (fp32 accumulation) and every fp16
output use max-abs 2e-3 against the oracle evaluated in float64 on the same fp16 inputs. The fused
norm + RoPE route with fp32 output carries q, k and P as hi + lo fp16 pairs (about 22 bits) and is
held to the fp32 bar, max-abs 1e-4 (it measures about 1.5e-6): losing one of the splits measures
5.6e-4 or more and fails it. Masked / padded / GQA index mapping is
exercised by ragged lengths, padded query rows, head groups of 1, 2 and 4, and sentinel bytes
around the output."""

import numpy as np
import pytest

from oracle import attention as ref
from oracle import norm_rope
from tessery_amd import workloads
from tests.conftest import GOLDEN

pytestmark = pytest.mark.gpu

F32_ATOL, F32_RTOL, F32_MAX = 2e-6, 2e-5, 1e-4
F16_MAX = 2e-3
FUSED_F32_MAX = 1e-4  # attention_f16_norm_rope with fp32 output


def fused_bar(out_dtype):
    return FUSED_F32_MAX if out_dtype == "f32" else F16_MAX


def run(engine, kernel, inputs, shape, out_dtype=np.float32, **params):
    """Upload inputs, dispatch one route by name, read the output (test_kernels.py:26-39)."""
    buffers = []
    try:
        for array in inputs:
            buffers.append(engine.upload(array))
        out = engine.buffer(int(np.prod(shape)) * np.dtype(out_dtype).itemsize)
        buffers.append(out)
        with engine.command():
            engine._dispatch(kernel, buffers, **params)
        return engine.read(out, shape, out_dtype)
    finally:
        for b in buffers:
            b.close()


def attend(engine, q, k, v, lengths, *, bidirectional, precision="f32", out_dtype=None):
    b, s, h, d = q.shape
    buffers = [engine.upload(a) for a in (q, k, v, lengths.astype(np.uint32))]
    odt = np.float16 if out_dtype == "f16" else np.float32
    buffers.append(engine.buffer(q.size * np.dtype(odt).itemsize))
    try:
        with engine.command():
            engine._attention(buffers, tokens=b * s, seq=s, heads=h, kv_heads=k.shape[2], dim=d,
                              bidirectional=int(bidirectional), precision=precision,
                              out_dtype=out_dtype)
        return engine.read(buffers[-1], q.shape, odt)
    finally:
        for x in buffers:
            x.close()


def check_f32(got, expected):
    np.testing.assert_allclose(got, expected, atol=F32_ATOL, rtol=F32_RTOL)
    assert np.max(np.abs(got - expected)) <= F32_MAX


# ---- fp32: tessery's own cases ---------------------------------------------------------------


def test_scalar_causal_gqa_seed17(runtime):
    f = np.load(GOLDEN / "attention_cases.npz")
    q = f["s17_q"]
    got = run(runtime, "attention", [q, f["s17_k"], f["s17_v"], f["s17_lengths"]], q.shape,
              threads=2 * 5 * 4 * 32, group_size=32, seq=5, heads=4, kv_heads=2, dim=64,
              scale=64**-0.5)
    check_f32(got, f["s17_expected"])


def test_scalar_bidirectional_seed83(runtime):
    f = np.load(GOLDEN / "attention_cases.npz")
    q = f["s83_q"]
    got = run(runtime, "attention", [q, f["s83_k"], f["s83_v"], f["s83_lengths"]], q.shape,
              threads=2 * 5 * 3 * 32, group_size=32, seq=5, heads=3, kv_heads=3, dim=8,
              scale=8**-0.5, bidirectional=True)
    check_f32(got, f["s83_expected"])


def test_bge_small_c1_through_route(runtime):
    f = np.load(GOLDEN / "attention_cases.npz")
    got = attend(runtime, f["c1_q"], f["c1_k"], f["c1_v"], f["c1_lengths"], bidirectional=True)
    check_f32(got, f["c1_expected"])
    assert runtime.diagnostics()["dispatches"] == {"attention": 1}
    assert got.reshape(2, 16, 384).shape == (2, 16, 384)


@pytest.mark.parametrize("dim", [32, 128])
@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize(
    "seq,length_pair",
    [(64, (1, 33)), (65, (1, 65)), (71, (33, 71)), (95, (65, 95)), (127, (1, 127)),
     (128, (31, 32)), (129, (65, 129)), (136, (129, 136)), (255, (254, 255)), (511, (1, 511)),
     (512, (511, 512))],
)
def test_tiled_attention_ragged_f64(runtime, dim, bidirectional, seq, length_pair):
    """tessery test_kernels.py:160-210, same seed, shapes and kernel names."""
    rng = np.random.default_rng(393)
    heads, kv = 4, 2
    q = rng.normal(size=(2, seq, heads, dim)).astype(np.float32)
    k, v = [rng.normal(size=(2, seq, kv, dim)).astype(np.float32) for _ in range(2)]
    lengths = np.array(length_pair, np.uint32)
    got = run(runtime, f"attention_tail_{dim}" if seq % 32 else "attention_tiled",
              [q, k, v, lengths], q.shape, threads=2 * ((seq + 7) // 8) * heads * 128,
              group_size=128, seq=seq, heads=heads, kv_heads=kv, dim=dim, scale=dim**-0.5,
              bidirectional=bidirectional)
    check_f32(got, ref.attention(q, k, v, lengths, bidirectional=bidirectional))


@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize("pattern", ["alternating", "later_maximum", "uniform"])
@pytest.mark.parametrize("seq", [65, 128, 129, 511])
def test_extreme_logits_and_masked_blocks(runtime, bidirectional, pattern, seq):
    """tessery test_kernels.py:213-253: logits near +-1131, late maxima, V = 1e10 when masked."""
    rng = np.random.default_rng(718)
    heads, dim = 2, 128
    q = np.full((1, seq, heads, dim), 10, np.float32)
    k = q.copy()
    k[:, 1::2] *= -1
    if pattern == "later_maximum":
        k[:] = -10
        k[:, 32:64] = 10
    elif pattern == "uniform":
        k[:] = 0
    v = rng.normal(size=q.shape).astype(np.float32)
    length = 65 if pattern == "later_maximum" else 33
    v[:, length:] = 1e10
    got = run(runtime, f"attention_tail_{dim}" if seq % 32 else "attention_tiled",
              [q, k, v, np.array([length], np.uint32)], q.shape,
              threads=((seq + 7) // 8) * heads * 128, group_size=128, seq=seq, heads=heads,
              kv_heads=heads, dim=dim, scale=dim**-0.5, bidirectional=bidirectional)
    expected = np.empty(q.shape)
    for pos in range(seq):
        end = length if bidirectional else min(pos + 1, length)
        if pattern == "later_maximum":
            chosen = v[0, 32 : min(end, 64)] if end > 32 else v[0, :end]
        else:
            chosen = v[0, :end:2] if pattern == "alternating" else v[0, :end]
        expected[0, pos] = chosen.astype(np.float64).mean(axis=0)
    check_f32(got, expected)


def test_qwen3_8x512_fp32_route(runtime):
    """The fp32 route at the Qwen3 8x512 shape (bench.py --workload qwen3_8x512_f32, layer 0):
    q/k normalized and rotated in float64 and rounded to fp32, v N(0,1), lengths U{64..512}."""
    shape, lengths = workloads.qwen3_8x512()
    t = workloads.qwen_layer(shape, 0, seed=3)
    qn = workloads.bf16_values(t["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(t["k_norm"]).astype(np.float64)
    q = norm_rope.norm_rope(t["q"], qn, workloads.EPS, workloads.THETA).astype(np.float32)
    k = norm_rope.norm_rope(t["k"], kn, workloads.EPS, workloads.THETA).astype(np.float32)
    v = t["v"].astype(np.float32)
    got = attend(runtime, q, k, v, lengths, bidirectional=False)
    check_f32(got, ref.attention(q, k, v, lengths, bidirectional=False))


@pytest.mark.parametrize("heads,kv", [(8, 2), (16, 2), (12, 4)])
@pytest.mark.parametrize("bidirectional", [False, True])
def test_fp32_d128_head_groups(runtime, heads, kv, bidirectional):
    """fp32 D = 128 with 4, 8 and 3 query heads per kv head: 4 and 8 heads share a wavefront's
    rows, 3 does not divide 16 and gives one head per wavefront. Ragged lengths, S % 32 != 0."""
    rng = np.random.default_rng(577)
    q = rng.normal(size=(2, 200, heads, 128)).astype(np.float32)
    k, v = [rng.normal(size=(2, 200, kv, 128)).astype(np.float32) for _ in range(2)]
    lengths = np.array([137, 200], np.uint32)
    got = attend(runtime, q, k, v, lengths, bidirectional=bidirectional)
    check_f32(got, ref.attention(q, k, v, lengths, bidirectional=bidirectional))


@pytest.mark.parametrize("seq,name", [(16, "attention"), (64, "attention_tiled"),
                                      (100, "attention_tail_32"), (512, "attention_tiled")])
def test_route_dispatch_counts_and_output_guard(runtime, seq, name):
    """One dispatch of the expected route; nothing written past the output."""
    rng = np.random.default_rng(seq)
    b, h, d = 3, 6, 32
    q = rng.normal(size=(b, seq, h, d)).astype(np.float32)
    k, v = [rng.normal(size=(b, seq, h, d)).astype(np.float32) for _ in range(2)]
    lengths = np.array([seq, max(1, seq // 3), 1], np.uint32)
    bufs = [runtime.upload(a) for a in (q, k, v, lengths)]
    sentinel = np.full(q.size + 4096, np.nan, np.float32)
    bufs.append(runtime.upload(sentinel))
    try:
        # output buffer larger than needed: route validation uses sizes as lower bounds
        with runtime.command():
            runtime._attention(bufs, tokens=b * seq, seq=seq, heads=h, kv_heads=h, dim=d,
                               bidirectional=1)
        out = runtime.read(bufs[-1], sentinel.shape)
    finally:
        for x in bufs:
            x.close()
    assert runtime.diagnostics()["dispatches"] == {name: 1}
    assert np.isnan(out[q.size:]).all()
    check_f32(out[: q.size].reshape(q.shape), ref.attention(q, k, v, lengths, bidirectional=True))


def test_bge_small_32x512_layer0(runtime):
    shape, lengths = workloads.bge_small_32x512()
    t = workloads.bge_layer(shape, 0)
    got = attend(runtime, t["q"], t["k"], t["v"], lengths, bidirectional=True)
    check_f32(got, ref.attention(t["q"], t["k"], t["v"], lengths, bidirectional=True))


# ---- fp16 operands, fp32 accumulation ---------------------------------------------------------


def f16_inputs(seed, b, s, h, kv, d):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, s, h, d), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((b, s, kv, d), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((b, s, kv, d), dtype=np.float32).astype(np.float16)
    return q, k, v


@pytest.mark.parametrize("out_dtype", ["f32", "f16"])
@pytest.mark.parametrize("bidirectional", [False, True])
@pytest.mark.parametrize(
    "b,s,h,kv,d,lengths",
    [
        (2, 1, 4, 2, 128, (1, 1)),
        (2, 7, 4, 2, 128, (7, 3)),
        (2, 33, 8, 2, 64, (33, 1)),
        (3, 64, 4, 4, 64, (64, 63, 2)),
        (2, 40, 4, 2, 32, (40, 9)),
        (2, 100, 16, 8, 128, (100, 37)),
        (2, 129, 2, 1, 128, (129, 65)),
        (4, 464, 16, 8, 128, (464, 1, 230, 63)),
        (2, 512, 16, 8, 128, (512, 511)),
    ],
)
def test_f16_attention(runtime, b, s, h, kv, d, lengths, bidirectional, out_dtype):
    q, k, v = f16_inputs(b * 1000 + s, b, s, h, kv, d)
    lengths = np.array(lengths, np.uint32)
    got = attend(runtime, q, k, v, lengths, bidirectional=bidirectional, precision="f16",
                 out_dtype=out_dtype)
    expected = ref.attention(q, k, v, lengths, bidirectional=bidirectional)
    err = np.max(np.abs(got.astype(np.float64) - expected))
    assert err <= F16_MAX, err


@pytest.mark.parametrize("d", [8, 96])
def test_f16_scalar_route(runtime, d):
    q, k, v = f16_inputs(d, 2, 19, 4, 2, d)
    lengths = np.array([19, 5], np.uint32)
    got = attend(runtime, q, k, v, lengths, bidirectional=False, precision="f16", out_dtype="f32")
    assert runtime.diagnostics()["dispatches"] == {"attention_f16_scalar": 1}
    assert np.max(np.abs(got - ref.attention(q, k, v, lengths, bidirectional=False))) <= F16_MAX


def norm_rope_attend(engine, t, lengths, shape, out_dtype="f32"):
    b, s, h, kv, d = shape.batch, shape.seq, shape.heads, shape.kv_heads, shape.dim
    arrays = [t["q"], t["k"], t["v"], lengths.astype(np.uint32)]
    bufs = [engine.upload(a) for a in arrays]
    odt = np.float16 if out_dtype == "f16" else np.float32
    bufs.append(engine.buffer(t["q"].size * np.dtype(odt).itemsize))
    bufs += [engine.upload(t["q_norm"]), engine.upload(t["k_norm"]), engine.buffer(2 * t["k"].nbytes)]
    try:
        with engine.command():
            engine._attention_norm_rope(bufs, tokens=b * s, seq=s, heads=h, kv_heads=kv, dim=d,
                                        eps=workloads.EPS, theta=workloads.THETA,
                                        out_dtype=out_dtype)
        planes = engine.read(bufs[7], (2,) + t["k"].shape, np.float16)
        return engine.read(bufs[4], t["q"].shape, odt), planes
    finally:
        for x in bufs:
            x.close()


def oracle_norm_rope(t, lengths):
    qn = workloads.bf16_values(t["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(t["k_norm"]).astype(np.float64)
    q = norm_rope.norm_rope(t["q"], qn, workloads.EPS, workloads.THETA)
    k = norm_rope.norm_rope(t["k"], kn, workloads.EPS, workloads.THETA)
    return k, ref.attention(q, k, t["v"], lengths, bidirectional=False)


@pytest.mark.parametrize("out_dtype", ["f32", "f16"])
def test_qwen_norm_rope_fixture(runtime, out_dtype):
    f = np.load(GOLDEN / "qwen_small.npz")
    t = {name: f[name] for name in ("q", "k", "v", "q_norm", "k_norm")}
    shape = workloads.Shape(2, 40, 4, 2, 128, causal=True)
    out, planes = norm_rope_attend(runtime, t, f["lengths"], shape, out_dtype)
    err = np.max(np.abs(out.astype(np.float64) - f["expected"]))
    assert err <= fused_bar(out_dtype), err
    # the k prologue writes valid rows only: hi within fp16 rounding of the float64 value, and
    # hi + lo within fp32 rounding of it
    hi, lo = planes[0].astype(np.float64), planes[1].astype(np.float64)
    for bi, length in enumerate(f["lengths"]):
        exp = f["k_normed"][bi, :length]
        assert np.all(np.abs(hi[bi, :length] - exp) <= 2.0**-11 * np.abs(exp) + 1e-7)
        assert np.all(np.abs(hi[bi, :length] + lo[bi, :length] - exp) <= 2e-6 * (np.abs(exp) + 1))


@pytest.mark.parametrize("out_dtype", ["f32", "f16"])
def test_qwen3_8x512(runtime, out_dtype):
    shape, lengths = workloads.qwen3_8x512()
    t = workloads.qwen_layer(shape, 0, seed=3)
    out, _ = norm_rope_attend(runtime, t, lengths, shape, out_dtype)
    _, expected = oracle_norm_rope(t, lengths)
    err = np.max(np.abs(out.astype(np.float64) - expected))
    assert err <= fused_bar(out_dtype), err


@pytest.mark.parametrize("layer", [0, 27])
def test_qwen3_32x512(runtime, layer):
    """The benchmark workload itself (log-uniform lengths, execution width 464, fp32 output)."""
    shape, lengths = workloads.qwen3_32x512()
    t = workloads.qwen_layer(shape, layer, seed=4)
    out, _ = norm_rope_attend(runtime, t, lengths, shape, "f32")
    _, expected = oracle_norm_rope(t, lengths)
    err = np.max(np.abs(out.astype(np.float64) - expected))
    assert err <= FUSED_F32_MAX, err


def test_qwen3_32x512_full_length_f16_out(runtime):
    """Every length 512 with fp16 output (the headline shape at full length): the whole batch runs
    on the GPU, batch rows 0, 13 and 31 are checked against the float64 oracle at the fp16-output
    bar."""
    shape, lengths = workloads.qwen3_32x512_full()
    t = workloads.qwen_layer(shape, 0, seed=4)
    out, _ = norm_rope_attend(runtime, t, lengths, shape, "f16")
    rows = [0, 13, 31]
    sub = {name: (t[name][rows] if t[name].ndim == 4 else t[name]) for name in t}
    _, expected = oracle_norm_rope(sub, lengths[rows])
    err = np.max(np.abs(out[rows].astype(np.float64) - expected))
    assert err <= fused_bar("f16"), err


def layers_in_one_command(engine, layers, lengths, shape, out_dtype, shared_k_work):
    """Layers queued back to back in one command, each the fused route's k prologue then its
    attention; k planes per layer (the attention of layer i may then carry layer i + 1's
    prologue) or one shared k buffer (it may not). Returns outputs, k planes and the number of
    launch-time pairs that ran."""
    odt = np.float16 if out_dtype == "f16" else np.float32
    lens = engine.upload(lengths.astype(np.uint32))
    sets = []
    shared = engine.buffer(2 * layers[0]["k"].nbytes)
    for t in layers:
        s = {n: engine.upload(t[n]) for n in ("q", "k", "v", "q_norm", "k_norm")}
        s["out"] = engine.buffer(t["q"].size * np.dtype(odt).itemsize)
        s["kw"] = shared if shared_k_work else engine.buffer(2 * t["k"].nbytes)
        sets.append(s)
    before = engine.diagnostics()["fused_pairs"]
    b, sq, h, kv, d = shape.batch, shape.seq, shape.heads, shape.kv_heads, shape.dim
    with engine.command():
        for s in sets:
            engine._attention_norm_rope(
                [s["q"], s["k"], s["v"], lens, s["out"], s["q_norm"], s["k_norm"], s["kw"]],
                tokens=b * sq, seq=sq, heads=h, kv_heads=kv, dim=d, eps=workloads.EPS,
                theta=workloads.THETA, out_dtype=out_dtype)
    fused = engine.diagnostics()["fused_pairs"] - before
    outs = [engine.read(s["out"], t["q"].shape, odt) for s, t in zip(sets, layers)]
    planes = [engine.read(s["kw"], (2,) + t["k"].shape, np.float16) for s, t in zip(sets, layers)]
    return outs, planes, fused


@pytest.mark.parametrize("shape,lengths,out_dtype", [
    (workloads.Shape(8, 464, 16, 8, 128, causal=True), (464, 1, 300, 17, 464, 129, 64, 2), "f32"),
    (workloads.Shape(8, 256, 16, 8, 128, causal=True), (256, 256, 200, 3, 77, 128, 255, 1), "f16"),
    (workloads.Shape(16, 72, 8, 2, 128, causal=True), tuple(range(72, 56, -1)), "f32"),
    # the headline shape: blocks run in pairs (more than two rounds of workgroups)
    (workloads.Shape(32, 464, 16, 8, 128, causal=True),
     tuple(int(x) for x in workloads.lengths_loguniform(4, 32)), "f32"),
])
def test_attention_carries_next_layers_k_prologue(runtime, shape, lengths, out_dtype):
    """Three layers in one command with a k buffer per layer: attention of layers 0 and 1 carry
    the k prologues of layers 1 and 2 in extra workgroups of their launches. Outputs and k
    planes equal those of each layer run in a command of its own, bit for bit, and layer 0 is
    within the fused route's bar of the float64 oracle."""
    lengths = np.array(lengths, np.uint32)
    layers = [workloads.qwen_layer(shape, i, seed=70) for i in range(3)]
    outs, planes, fused = layers_in_one_command(runtime, layers, lengths, shape, out_dtype, False)
    assert fused == 2
    for i, t in enumerate(layers):
        alone, alone_planes = norm_rope_attend(runtime, t, lengths, shape, out_dtype)
        np.testing.assert_array_equal(outs[i], alone)
        for bi, length in enumerate(lengths):  # the prologue writes valid rows only
            np.testing.assert_array_equal(planes[i][:, bi, :length], alone_planes[:, bi, :length])
    _, expected = oracle_norm_rope(layers[0], lengths)
    assert np.max(np.abs(outs[0].astype(np.float64) - expected)) <= fused_bar(out_dtype)


def test_shared_k_buffer_is_not_carried(runtime):
    """With one k buffer for every layer, the next layer's prologue would overwrite the planes
    the attention still reads: no pair runs, and each layer's result equals its own command's."""
    shape = workloads.Shape(8, 128, 16, 8, 128, causal=True)
    lengths = np.array([128, 5, 64, 100, 1, 128, 33, 90], np.uint32)
    layers = [workloads.qwen_layer(shape, i, seed=71) for i in range(2)]
    outs, _, fused = layers_in_one_command(runtime, layers, lengths, shape, "f32", True)
    assert fused == 0
    for i, t in enumerate(layers):
        alone, _ = norm_rope_attend(runtime, t, lengths, shape, "f32")
        np.testing.assert_array_equal(outs[i], alone)


@pytest.mark.parametrize("aligned_first", [False, True])
def test_fused_late_maximum_moves_the_running_max(runtime, aligned_first):
    """Fused route, causal: keys 40-55 line up with every query of head 0 (logit 128 / sqrt(128)
    = 11.3, 16.3 in log2 units, past the lazy max's slack of 8) and point away from head 1's,
    whose rows share the wavefront. q and k sit in channel 63, whose RoPE angle stays below
    3e-4 rad up to position 200, so they stay aligned after the rotation. The running max of head
    0 rows past position 40 moves in the middle of the row (rescale and score shift) while the
    neighbouring lanes keep theirs. With aligned_first the aligned keys come first (0-15)
    and every later tile stays far below the max."""
    rng = np.random.default_rng(1234)
    b, s, h, kv, d = 2, 200, 4, 2, 128
    shape = workloads.Shape(b, s, h, kv, d, causal=True)
    lengths = np.array([200, 150], np.uint32)
    q = np.zeros((b, s, h, d), np.float16)
    q[:, :, 0::2, 63] = 4.0   # heads 0 and 2: towards the late keys
    q[:, :, 1::2, 63] = -4.0  # heads 1 and 3: away from them
    k = rng.normal(size=(b, s, kv, d)).astype(np.float16)
    late = slice(0, 16) if aligned_first else slice(40, 56)
    k[:, late] = 0
    k[:, late, :, 63] = 3.0
    v = rng.normal(size=(b, s, kv, d)).astype(np.float16)
    one = np.full(d, 0x3F80, np.uint16)  # bf16 1.0
    t = {"q": q, "k": k, "v": v, "q_norm": one, "k_norm": one}
    out, _ = norm_rope_attend(runtime, t, lengths, shape, "f32")
    _, expected = oracle_norm_rope(t, lengths)
    err = np.max(np.abs(out.astype(np.float64) - expected))
    assert err <= FUSED_F32_MAX, err


@pytest.mark.parametrize("route", ["fused", "plain"])
def test_f16_routes_are_deterministic(runtime, route):
    """The same launch on the same inputs gives the same bits. Full tiles skip the causal masking,
    so their row max reads the QK^T accumulators right after the MFMA chain; this pins that the
    read waits for the chain to finish (it once depended on timing)."""
    shape = workloads.Shape(4, 256, 16, 8, 128, causal=True)
    lengths = np.array([256, 200, 64, 17], np.uint32)
    if route == "fused":
        t = workloads.qwen_layer(shape, 0, seed=12)
        first, _ = norm_rope_attend(runtime, t, lengths, shape, "f32")
        second, _ = norm_rope_attend(runtime, t, lengths, shape, "f32")
    else:
        q, k, v = f16_inputs(12, 4, 256, 16, 8, 128)
        first = attend(runtime, q, k, v, lengths, bidirectional=False, precision="f16")
        second = attend(runtime, q, k, v, lengths, bidirectional=False, precision="f16")
    np.testing.assert_array_equal(first, second)
