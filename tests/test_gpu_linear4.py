"""uint4 group-64 projection routes on the GPU (tessery test_kernels.py:55-81, 421-516, 648-776):
float64 accuracy at atol = rtol = 5e-5, the expected route partition, bit-identical results
between routes over the same rows, and rows outside a route's region left untouched."""

import numpy as np
import pytest

from oracle import quant4 as ref
from tessery_amd.workloads import bf16_words
from tests.conftest import GOLDEN
from tests.test_gpu_attention import run

pytestmark = pytest.mark.gpu


def make(seed, m, n, k, cancellation=False):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    x = rng.normal(size=(m, k)).astype(np.float32)
    if cancellation:
        codes[:, 1::2] = codes[:, ::2]
        x[:, ::2], x[:, 1::2] = 1.0, -1.0
    scales = bf16_words(rng.uniform(0.01, 0.2, size=(n, k // 64)))
    biases = bf16_words(rng.uniform(-1, 0.1, size=(n, k // 64)))
    return x, ref.pack(codes), scales, biases


def project(engine, arrays, m, n, k, out=None):
    bufs = [engine.upload(a) for a in arrays]
    bufs.append(engine.upload(out) if out is not None else engine.buffer(m * n * 4))
    try:
        with engine.command():
            engine._linear4(bufs, rows=m, cols=n, k=k)
        shape = out.shape if out is not None else (m, n)
        return engine.read(bufs[-1], shape)
    finally:
        for b in bufs:
            b.close()


def test_fixture_and_known_answer(runtime):
    f = np.load(GOLDEN / "linear4_small.npz")
    got = project(runtime, [f["x"], f["packed"], f["scales"], f["biases"]], 7, 64, 128)
    np.testing.assert_allclose(got, f["expected"], atol=5e-5, rtol=5e-5)
    # scale 0.125 bias -0.5 (test_kernels.py:55-81) through the scalar route
    rng = np.random.default_rng(1)
    code = rng.integers(0, 16, size=(8, 128), dtype=np.uint32)
    x = rng.normal(size=(3, 128)).astype(np.float32)
    arrays = [x, ref.pack(code), bf16_words(np.full((8, 2), 0.125)), bf16_words(np.full((8, 2), -0.5))]
    got = run(runtime, "linear4", arrays, (3, 8), threads=8 * 32, group_size=32, rows=3, cols=8, k=128)
    np.testing.assert_allclose(got, x @ (code * 0.125 - 0.5).T, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("m,n,k", [(m, 64, k) for m in (1, 2, 7, 8, 9, 12, 15, 16, 17, 31)
                                   for k in (64, 1024, 3072)] + [(7, 33, 128)])
def test_tiled_accuracy_and_route(runtime, m, n, k):
    x, packed, scales, biases = make(417, m, n, k)
    got = project(runtime, [x, packed, scales, biases], m, n, k)
    np.testing.assert_allclose(got, ref.linear4(x, packed, scales, biases), atol=5e-5, rtol=5e-5)
    expected = {"linear4": 1}
    if m >= 5 and n % 32 == 0:
        expected = {}
        if m >= 8:
            expected["linear4_tiled"] = 1
        if m % 8:
            expected["linear4" if m % 8 <= 4 else "linear4_tail"] = 1
    assert runtime.diagnostics()["dispatches"] == expected


@pytest.mark.parametrize("m,n,k", [(16, 1024, 1024), (32, 2048, 1024), (16, 3072, 1024),
                                   (32, 1024, 2048), (32, 1024, 3072), (4096, 1024, 1024)])
@pytest.mark.parametrize("pattern", ["random", "cancellation"])
def test_large_tiles_f64_and_bitwise_between_routes(runtime, m, n, k, pattern):
    arrays = list(make(821, m, n, k, pattern == "cancellation"))
    previous = run(runtime, "linear4_tiled", arrays, (m, n), threads=(m // 8) * (n // 32) * 128,
                   group_size=128, rows=m, cols=n, k=k)
    actual = run(runtime, "linear4_16x32_k64", arrays, (m, n), threads=(m // 16) * (n // 32) * 256,
                 group_size=256, rows=m, cols=n, k=k)
    np.testing.assert_allclose(actual, ref.linear4(*arrays), atol=5e-5, rtol=5e-5)
    np.testing.assert_array_equal(actual, previous)


@pytest.mark.parametrize("m", [17, 23, 24, 25, 31, 40, 128, 129, 257])
@pytest.mark.parametrize("n,k", [(1024, 1024), (2048, 1024), (1024, 3072)])
def test_mixed_partition_matches_f64_and_previous_routes(runtime, m, n, k):
    arrays = list(make(481 + m, m, n, k))
    sentinel = np.full((m, n), np.nan, np.float32)
    actual = project(runtime, arrays, m, n, k, out=sentinel)
    np.testing.assert_allclose(actual, ref.linear4(*arrays), atol=5e-5, rtol=5e-5)
    bufs = [runtime.upload(a) for a in arrays] + [runtime.upload(sentinel)]
    try:
        with runtime.command():
            runtime._dispatch("linear4_tiled", bufs, threads=(m // 8) * (n // 32) * 128,
                              group_size=128, rows=m, cols=n, k=k)
            if m % 8:
                small = m % 8 <= 4
                runtime._dispatch("linear4" if small else "linear4_tail", bufs,
                                  threads=n * 32 if small else (n // 32) * 128,
                                  group_size=32 if small else 128, n=m // 8 * 8, rows=m, cols=n, k=k)
        previous = runtime.read(bufs[-1], (m, n))
    finally:
        for b in bufs:
            b.close()
    np.testing.assert_array_equal(actual, previous)


@pytest.mark.parametrize("m", [2, 3, 4])
def test_small_row_routes_and_output_guard(runtime, m):
    n, k = 1024, 1024
    arrays = list(make(2030 + m, m, n, k))
    sentinel = np.full((m + 2, n), np.nan, np.float32)
    got = project(runtime, arrays, m, n, k, out=sentinel)
    assert np.isnan(got[m:]).all()
    np.testing.assert_allclose(got[:m], ref.linear4(*arrays), atol=5e-5, rtol=5e-5)
    assert runtime.diagnostics()["dispatches"] == {"linear4_small3" if m == 3 else "linear4": 1}


def test_eight_row_offset_preserves_surrounding_rows(runtime):
    m, n, k = 32, 32, 64
    arrays = [np.ones((m, k), np.float32), np.full((n, k // 8), 0x11111111, np.uint32),
              bf16_words(np.ones((n, 1))), bf16_words(np.zeros((n, 1)))]
    bufs = [runtime.upload(a) for a in arrays] + [runtime.upload(np.full((m, n), np.nan, np.float32))]
    try:
        with runtime.command():
            runtime._dispatch("linear4_tiled", bufs, threads=128, group_size=128, n=16, rows=m,
                              cols=n, k=k)
        out = runtime.read(bufs[-1], (m, n))
    finally:
        for b in bufs:
            b.close()
    assert np.isnan(out[:16]).all() and np.isnan(out[24:]).all()
    np.testing.assert_array_equal(out[16:24], 64)


@pytest.mark.parametrize("m,n,k", [(1024, 2048, 1024), (1100, 1024, 2048), (2048, 1024, 1024),
                                   (4096, 3072, 1024), (2050, 1024, 3072),
                                   (2176, 128, 64), (4097, 2048, 1024)])
def test_large_batch_fp16_mfma_path(runtime, m, n, k):
    """From 1024 rows the projection runs on fp16 MFMA over row-scaled hi + lo halves of x. Row
    magnitudes spread over 2^-20 .. 2^20, a zero row, rows near fp32's smallest and largest
    normal values (beyond fp16's range): every output stays within fp32-grade error of the
    float64 product, measured against sum_k |x| |w| of the same element."""
    x, packed, scales, biases = make(907 + m + n, m, n, k)
    rng = np.random.default_rng(m)
    x[5:] *= np.exp2(rng.integers(-20, 21, m - 5)).astype(np.float32)[:, None]
    x[0] = 0.0
    x[1] *= np.float32(1e-36)
    x[2] *= np.float32(1e6)
    x[3] *= np.float32(1e34)
    got = project(runtime, [x, packed, scales, biases], m, n, k)
    w = ref.dequantize(packed, scales, biases, k)
    want = x.astype(np.float64) @ w.T
    bound = np.abs(x).astype(np.float64) @ np.abs(w).T
    assert np.isfinite(got).all()
    err = np.abs(got - want)
    assert np.all(err <= 2e-6 * bound + 1e-37), float((err / (bound + 1e-300)).max())
    assert not np.any(got[0])
