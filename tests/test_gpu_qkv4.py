"""Fused uint4 QKV projection (fp16 activations) against the float64 oracle: every output within
fp16 rounding of the exact projection (|err| <= 2^-11 |y| + 1e-4), for fp16 and bf16 scale words,
rows that are not a multiple of the 128-row tile, and rows left untouched outside [0, M)."""

import numpy as np
import pytest

from oracle import quant4 as ref
from tessery_amd.workloads import bf16_words

pytestmark = pytest.mark.gpu


def weights(rng, n, k, kind):
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    if kind == "f16":
        s = rng.normal(0, 0.02, size=(n, k // 64)).astype(np.float16).view(np.uint16)
        b = rng.normal(0, 0.02, size=(n, k // 64)).astype(np.float16).view(np.uint16)
    else:
        s = bf16_words(rng.normal(0, 0.02, size=(n, k // 64)))
        b = bf16_words(rng.normal(0, 0.02, size=(n, k // 64)))
    return ref.pack(codes), s, b


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("m,k,nq,nkv", [(300, 1024, 2048, 1024), (128, 256, 128, 128), (1, 64, 256, 128),
                                         (65, 320, 128, 128), (257, 448, 256, 128),
                                         (130, 1536, 128, 256), (200, 128, 128, 128)])
def test_qkv4_matches_f64(runtime, kind, m, k, nq, nkv):
    rng = np.random.default_rng(5 + m)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    parts = [weights(rng, n, k, kind) for n in (nq, nkv, nkv)]
    w = np.concatenate([p[0] for p in parts])
    s = np.concatenate([p[1] for p in parts])
    b = np.concatenate([p[2] for p in parts])
    bufs = [runtime.upload(a) for a in (x, w, s, b)]
    outs = [np.full((m + 1, n), np.nan, np.float16) for n in (nq, nkv, nkv)]
    bufs += [runtime.upload(o) for o in outs]
    try:
        with runtime.command():
            runtime._qkv4(bufs, rows=m, k=k, q_cols=nq, kv_cols=nkv, scale_dtype=kind)
        got = [runtime.read(bufs[4 + i], outs[i].shape, np.float16) for i in range(3)]
    finally:
        for buf in bufs:
            buf.close()
    for (packed, sc, bi), y in zip(parts, got):
        expected = ref.linear4(x, packed, sc, bi, kind)
        err = np.abs(y[:m].astype(np.float64) - expected)
        assert np.all(err <= 2.0**-11 * np.abs(expected) + 1e-4), float(err.max())
        assert np.isnan(y[m:]).all()


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("batch,seq,kv,lengths", [(2, 256, 8, (256, 77)), (3, 100, 2, (1, 100, 64)),
                                                  (1, 130, 1, (129,))])
def test_qkv4_then_k_prologue_runs_as_one_kernel_with_the_same_bits(runtime, kind, batch, seq, kv,
                                                                     lengths):
    """qkv4_f16 followed by norm_rope_f16 over its k output (the fused attention's k prologue,
    D = 128) in one command runs as one kernel; q, k, v and both k planes hold the bits of the
    two launches in separate commands, rows past a batch row's length stay untouched, and rows
    that are not a multiple of the 128-row tile are covered."""
    rng = np.random.default_rng(41 + seq)
    m, k, nq, nkv = batch * seq, 256, 2 * kv * 128, kv * 128
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    parts = [weights(rng, n, k, kind) for n in (nq, nkv, nkv)]
    inputs = [x, *(np.concatenate([p[i] for p in parts]) for i in range(3)),
              np.asarray(lengths, np.uint32), bf16_words(1.0 + 0.1 * rng.standard_normal(128))]
    prologue = dict(heads=kv, seq=seq, dim=128, eps=1e-6, theta=1e6, flags=1)

    def run(fused):
        bufs = [runtime.upload(a) for a in inputs]
        outs = [runtime.upload(np.full((m, n), np.nan, np.float16)) for n in (nq, nkv, nkv)]
        planes = runtime.upload(np.full((2, m, nkv), np.nan, np.float16))
        try:
            before = runtime.diagnostics()["fused_pairs"]
            with runtime.command():
                runtime._qkv4([*bufs[:4], *outs], rows=m, k=k, q_cols=nq, kv_cols=nkv,
                              scale_dtype=kind)
                if fused:
                    runtime._dispatch("norm_rope_f16", [outs[1], bufs[5], bufs[4], planes],
                                      threads=m, group_size=256, **prologue)
            if not fused:
                with runtime.command():
                    runtime._dispatch("norm_rope_f16", [outs[1], bufs[5], bufs[4], planes],
                                      threads=m, group_size=256, **prologue)
            assert runtime.diagnostics()["fused_pairs"] == before + int(fused)
            got = [runtime.read(o, (m, n), np.float16) for o, n in zip(outs, (nq, nkv, nkv))]
            return got + [runtime.read(planes, (2, m, nkv), np.float16)]
        finally:
            for buf in bufs + outs + [planes]:
                buf.close()

    fused, separate = run(True), run(False)
    for a, b in zip(fused, separate):
        np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))
    # rows past each batch row's length are never written; every row below it is
    done = ~np.isnan(fused[3][0].reshape(batch, seq, nkv)).any(axis=2)
    assert (done == (np.arange(seq)[None, :] < np.asarray(lengths)[:, None])).all()
