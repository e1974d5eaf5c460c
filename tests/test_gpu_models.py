"""Both model ends and whole-model forwards on the GPU against the float64 oracle.

Routes: embedding4, embedding_position and pool_project (kernels.metal:21-30, 339-360) at model
widths and odd ones. Forwards: Qwen3Backend and BertBackend on synthetic packs written to disk
(SafeTensors + config.json, pinned by sha256), every op a HIP kernel, compared with
oracle.models on the same weights; the second call of a shape replays the recorded plan as a HIP
graph and must give the same bits. Tolerance: 1e-4 absolute on the unit output vectors (the fp32
routes' bar)."""

import numpy as np
import pytest

from oracle import models as ref
from tessery_amd import workloads as wl
from tessery_amd.backends import BertBackend, Qwen3Backend
from tessery_amd.errors import InferenceError
from tests.test_gpu_attention import run

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("vocab,cols,tokens", [(40, 64, 7), (300, 1024, 33), (5, 128, 1)])
def test_embedding4_route(runtime, vocab, cols, tokens):
    rng = np.random.default_rng(cols + tokens)
    packed, s, b = wl.weight4_set(rng, vocab, cols, 0.2)
    ids = rng.integers(0, vocab, tokens).astype(np.uint32)
    ids[0] = vocab - 1
    got = run(runtime, "embedding4", [ids, packed, s, b], (tokens, cols),
              threads=tokens * cols, n=tokens * cols, cols=cols)
    # Each output is code * scale + bias of bf16 values: one fp32 rounding of the float64 value.
    want = ref.embedding4(ids, packed, s, b)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("cols,seq,batch", [(384, 16, 3), (30, 5, 2), (64, 1, 4)])
def test_embedding_position_route(runtime, cols, seq, batch):
    rng = np.random.default_rng(cols)
    words = rng.standard_normal((50, cols)).astype(np.float32)
    positions = rng.standard_normal((seq + 3, cols)).astype(np.float32)
    types = rng.standard_normal((2, cols)).astype(np.float32)
    ids = rng.integers(0, 50, (batch, seq)).astype(np.uint32)
    got = run(runtime, "embedding_position", [ids, words, positions, types],
              (batch * seq, cols), threads=batch * seq * cols, n=batch * seq * cols, cols=cols,
              seq=seq)
    want = ref.embedding_position(ids, words, positions, types)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("first", [False, True])
@pytest.mark.parametrize("cols,dim", [(1024, 1024), (1024, 96), (384, 384), (40, 33)])
def test_pool_project_route(runtime, first, cols, dim):
    rng = np.random.default_rng(dim)
    batch, seq = 5, 9
    x = rng.standard_normal((batch, seq, cols)).astype(np.float32)
    lengths = rng.integers(1, seq + 1, batch).astype(np.uint32)
    got = run(runtime, "pool_project", [x, lengths], (batch, dim), threads=batch * 32,
              group_size=32, seq=seq, cols=cols, dim=dim, first_token=first)
    np.testing.assert_allclose(got, ref.pool_project(x, lengths, dim, first=first), atol=1e-6,
                               rtol=1e-5)


QWEN_SMALL = dict(hidden=128, intermediate=256, layers=2, heads=4, kv_heads=2, head_dim=32,
                  vocab=300)
QWEN_WIDE = dict(hidden=1024, intermediate=3072, layers=2, heads=16, kv_heads=8, head_dim=128,
                 vocab=4096)
BERT_SMALL = dict(hidden=64, intermediate=128, layers=2, heads=4, vocab=50, positions=32, types=2)
BGE_WIDE = dict(hidden=384, intermediate=1536, layers=2, heads=12, vocab=1000, positions=512,
                types=2)


def _ids(vocab, batch, seq, low, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, (batch, seq)).astype(np.uint32)
    lengths = rng.integers(low, seq + 1, batch).astype(np.uint32)
    lengths[-1] = seq
    return ids, lengths


@pytest.mark.parametrize("shape,batch,seq,dims", [
    (QWEN_SMALL, 3, 12, 96), (QWEN_SMALL, 1, 1, 128), (QWEN_WIDE, 4, 64, 1024),
    (QWEN_WIDE, 2, 37, 256),
])
def test_qwen3_backend_forward(tmp_path, shape, batch, seq, dims):
    config, tensors = wl.qwen3_pack_tensors(11, **shape)
    profile = wl.write_pack(str(tmp_path), config, tensors, architecture="qwen3_uint4",
                            max_length=512, min_dimensions=64)
    ids, lengths = _ids(shape["vocab"], batch, seq, 1, seq)
    want = ref.qwen3_forward(wl.weights_of(tensors), ids, lengths, layers=shape["layers"],
                             heads=shape["heads"], kv_heads=shape["kv_heads"],
                             head_dim=shape["head_dim"], eps=config["rms_norm_eps"],
                             theta=config["rope_theta"], dimensions=dims)
    backend = Qwen3Backend(str(tmp_path), profile)
    try:
        first = backend.forward(ids, lengths, dimensions=dims)
        np.testing.assert_allclose(first, want, atol=1e-4, rtol=0)
        again = backend.forward(ids, lengths, dimensions=dims)  # plan replay
        np.testing.assert_array_equal(again, first)
        third = backend.forward(ids, lengths, dimensions=dims)  # same binding: same graph
        np.testing.assert_array_equal(third, first)
        diag = backend.runtime.diagnostics()
        assert (diag["graph_builds"], diag["graph_launches"]) == (1, 2), diag
        with pytest.raises(InferenceError):
            backend.forward(ids + np.uint32(shape["vocab"]), lengths, dimensions=dims)
        with pytest.raises(InferenceError):
            backend.forward(ids, lengths * 0, dimensions=dims)
    finally:
        backend.close()


@pytest.mark.parametrize("shape,batch,seq", [(BERT_SMALL, 3, 10), (BGE_WIDE, 4, 128),
                                             (BGE_WIDE, 2, 2)])
def test_bert_backend_forward(tmp_path, shape, batch, seq):
    config, tensors = wl.bert_pack_tensors(12, **shape)
    profile = wl.write_pack(str(tmp_path), config, tensors, architecture="bert_f32",
                            max_length=min(512, shape["positions"]))
    ids, lengths = _ids(shape["vocab"], batch, seq, 2, seq)
    want = ref.bert_forward(wl.weights_of(tensors), ids, lengths, layers=shape["layers"],
                            heads=shape["heads"], eps=config["layer_norm_eps"])
    backend = BertBackend(str(tmp_path), profile)
    try:
        first = backend.forward(ids, lengths, dimensions=shape["hidden"])
        np.testing.assert_allclose(first, want, atol=1e-4, rtol=0)
        again = backend.forward(ids, lengths, dimensions=shape["hidden"])
        np.testing.assert_array_equal(again, first)
        third = backend.forward(ids, lengths, dimensions=shape["hidden"])
        np.testing.assert_array_equal(third, first)
        diag = backend.runtime.diagnostics()
        assert (diag["graph_builds"], diag["graph_launches"]) == (1, 2), diag
        with pytest.raises(InferenceError):
            backend.forward(ids, lengths, dimensions=shape["hidden"] - 1)
    finally:
        backend.close()
