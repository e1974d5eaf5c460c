"""Weight-pack reading (tessery_amd/weights.py) and the backends' pack checks, on the CPU.

The container cases restate tessery's own (tests/unit/test_standalone_weights.py:12-104): the
same accepted snapshot, malformed tensor records, invalid containers, the no-follow artifact
read and the directory walk. The writer is checked against the safetensors library, and every
config / inventory rejection of the two backends is exercised (they happen before any GPU
allocation, so no device is needed)."""

import hashlib
import json
import os
import struct

import numpy as np
import pytest
import torch

from tessery_amd import workloads as wl
from tessery_amd.backends import BertBackend, ModelProfile, Qwen3Backend
from tessery_amd.errors import ManifestError, UnsupportedProfileError
from tessery_amd.weights import (Artifact, SafeTensors, artifact_of, encode_safetensors,
                                 read_artifact, read_json)


def container(header, payload=b"\x00" * 8):
    encoded = json.dumps(header).encode()
    return struct.pack("<Q", len(encoded)) + encoded + payload


def test_snapshot_views():
    tensors = SafeTensors(container({
        "a": {"dtype": "BF16", "shape": [2], "data_offsets": [0, 4]},
        "b": {"dtype": "U32", "shape": [1], "data_offsets": [4, 8]},
    }))
    assert np.array_equal(tensors.view("a", shape=(2,), dtype="BF16"), np.zeros(4, np.uint8))
    for name, shape, dtype in [("a", (3,), "BF16"), ("none", (2,), "BF16"), ("a", (2,), "U32")]:
        with pytest.raises(ManifestError):
            tensors.view(name, shape=shape, dtype=dtype)


@pytest.mark.parametrize("record", [
    None, [], {},
    {"dtype": "pickle", "shape": [2], "data_offsets": [0, 8]},
    {"dtype": "U32", "shape": [True], "data_offsets": [0, 4]},
    {"dtype": "U32", "shape": [], "data_offsets": [0, 8]},
    {"dtype": "U32", "shape": [2, 2, 2], "data_offsets": [0, 8]},
    {"dtype": "U32", "shape": [2], "data_offsets": [0]},
    {"dtype": "U32", "shape": [2], "data_offsets": [0, True]},
    {"dtype": "U32", "shape": [2], "data_offsets": [-1, 7]},
    {"dtype": "U32", "shape": [2], "data_offsets": [0, 7]},
    {"dtype": "U32", "shape": [2], "data_offsets": [0, 12]},
    {"dtype": "U32", "shape": [200001], "data_offsets": [0, 8]},
    {"dtype": "F16", "shape": [4], "data_offsets": [0, 8]},
    {"dtype": "U32", "shape": [2], "data_offsets": [0, 8], "extra": 1},
])
def test_malformed_tensor(record):
    with pytest.raises(ManifestError):
        SafeTensors(container({"x": record}))


@pytest.mark.parametrize("data", [
    b"", b"1234567", struct.pack("<Q", 0), struct.pack("<Q", 2**32),
    struct.pack("<Q", 20) + b"{}", struct.pack("<Q", 1) + b"!" + b"\0" * 8,
    container([]), container({}),
    container({"a": {"dtype": "U32", "shape": [1], "data_offsets": [4, 8]}}),
    container({"a": {"dtype": "U32", "shape": [1], "data_offsets": [0, 4]},
               "b": {"dtype": "U32", "shape": [1], "data_offsets": [0, 4]}}),
    # duplicate keys and non-finite numbers are not JSON the strict parser accepts
    struct.pack("<Q", 23) + b'{"a":1,"a":2,"b":NaN }' + b"\0" * 8,
])
def test_invalid_container(data):
    with pytest.raises(ManifestError):
        SafeTensors(data)


def test_metadata_is_skipped():
    tensors = SafeTensors(container({
        "__metadata__": {"format": "pt"},
        "w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
    }))
    assert set(tensors.tensors) == {"w"}


def test_safe_read_snapshot(tmp_path):
    root = tmp_path.resolve()
    data = b'{"hello":1}'
    pinned = artifact_of("config.json", "config.json", data)
    file = root / "config.json"
    file.write_bytes(data)
    assert read_json(str(root), pinned) == {"hello": 1}
    (root / "untrusted.py").write_text("raise RuntimeError")
    assert read_artifact(str(root), pinned) == data
    for filename in ["../config.json", "unknown"]:
        with pytest.raises(ManifestError):
            read_artifact(str(root), Artifact("config.json", filename, pinned.size, pinned.sha256))
    file.write_bytes(b"x" * len(data))  # same size, other bytes
    with pytest.raises(ManifestError):
        read_artifact(str(root), pinned)
    file.unlink()
    file.symlink_to(root / "untrusted.py")
    with pytest.raises(ManifestError):
        read_artifact(str(root), pinned)
    file.unlink()
    file.write_bytes(data)
    os.link(file, root / "second_link")  # a hard-linked file is refused
    with pytest.raises(ManifestError):
        read_artifact(str(root), pinned)


def test_directory_failures(tmp_path):
    pinned = Artifact("config.json", "config.json", 1, "0" * 64)
    for path in ["relative", str(tmp_path / ".."), str(tmp_path / "missing")]:
        with pytest.raises(ManifestError):
            read_artifact(path, pinned)


def test_writer_round_trips_through_safetensors_library():
    """encode_safetensors output read by the safetensors library, and the library's own output
    read by SafeTensors: the same bytes either way."""
    from safetensors.torch import load as st_load
    from safetensors.torch import save as st_save

    rng = np.random.default_rng(0)
    arrays = {
        "w.weight": ("U32", rng.integers(0, 2**32, (6, 4), dtype=np.uint32)),
        "w.scales": ("BF16", rng.integers(0, 2**16, (6, 1), dtype=np.uint16)),
        "n.weight": ("F32", rng.standard_normal(5).astype(np.float32)),
        "ids": ("I64", np.arange(7, dtype=np.int64)[None]),
    }
    data = encode_safetensors(arrays)
    loaded = st_load(data)
    for name, (dtype, array) in arrays.items():
        t = loaded[name]
        assert tuple(t.shape) == array.shape
        view = t.view(torch.int16) if dtype == "BF16" else t
        assert view.numpy().tobytes() == array.tobytes()
    snapshot = SafeTensors(data)
    for name, (dtype, array) in arrays.items():
        assert snapshot.view(name, shape=array.shape, dtype=dtype).tobytes() == array.tobytes()
    theirs = st_save({
        "a": torch.from_numpy(arrays["n.weight"][1]),
        "b": torch.from_numpy(arrays["w.scales"][1].view(np.int16)).view(torch.bfloat16),
        "c": torch.from_numpy(arrays["ids"][1]),
    })
    parsed = SafeTensors(theirs)
    assert parsed.view("b", shape=(6, 1), dtype="BF16").tobytes() == arrays["w.scales"][1].tobytes()
    assert parsed.view("c", shape=(1, 7), dtype="I64").tobytes() == arrays["ids"][1].tobytes()


QWEN_TINY = dict(hidden=128, intermediate=256, layers=1, heads=4, kv_heads=2, head_dim=32,
                 vocab=300)
BERT_TINY = dict(hidden=64, intermediate=128, layers=1, heads=4, vocab=50, positions=32, types=2)


def _qwen_pack(tmp_path, config_edit=None, tensor_edit=None):
    config, tensors = wl.qwen3_pack_tensors(1, **QWEN_TINY)
    if config_edit:
        config_edit(config)
    if tensor_edit:
        tensor_edit(tensors)
    return wl.write_pack(str(tmp_path), config, tensors, architecture="qwen3_uint4",
                         max_length=64, min_dimensions=64)


def _bert_pack(tmp_path, config_edit=None, tensor_edit=None, extras=True):
    config, tensors = wl.bert_pack_tensors(1, **BERT_TINY, extras=extras)
    if config_edit:
        config_edit(config)
    if tensor_edit:
        tensor_edit(tensors)
    return wl.write_pack(str(tmp_path), config, tensors, architecture="bert_f32", max_length=32)


@pytest.mark.parametrize("edit", [
    lambda c: c.update(hidden_act="gelu"),
    lambda c: c.update(quantization={"bits": 8, "group_size": 64}),
    lambda c: c.update(num_key_value_heads=3),
    lambda c: c.update(head_dim=33),
    lambda c: c.update(rope_theta=0.5),
    lambda c: c.update(rms_norm_eps=True),
    lambda c: c.update(num_hidden_layers=1.0),
    lambda c: c.update(use_sliding_window=True),
    lambda c: c.update(intermediate_size=200),
])
def test_qwen3_config_rejected(tmp_path, edit):
    profile = _qwen_pack(tmp_path, config_edit=edit)
    with pytest.raises(UnsupportedProfileError):
        Qwen3Backend(str(tmp_path), profile)


@pytest.mark.parametrize("edit", [
    lambda t: t.pop("model.norm.weight"),
    lambda t: t.update({"extra.weight": ("F32", np.zeros(2, np.float32))}),
    lambda t: t.update({"model.norm.weight": ("F32", np.ones(128, np.float32))}),
    lambda t: t.update({"model.layers.0.mlp.up_proj.scales":
                        ("BF16", np.zeros((256, 1), np.uint16))}),
])
def test_qwen3_inventory_rejected(tmp_path, edit):
    profile = _qwen_pack(tmp_path, tensor_edit=edit)
    with pytest.raises(ManifestError):
        Qwen3Backend(str(tmp_path), profile)


def test_pack_pinned_by_hash(tmp_path):
    profile = _qwen_pack(tmp_path)
    data = (tmp_path / "model.safetensors").read_bytes()
    (tmp_path / "model.safetensors").write_bytes(data[:-1] + bytes([data[-1] ^ 1]))
    with pytest.raises(ManifestError):
        Qwen3Backend(str(tmp_path), profile)


@pytest.mark.parametrize("edit", [
    lambda c: c.update(hidden_act="gelu_new"),
    lambda c: c.update(architectures=["BertForMaskedLM"]),
    lambda c: c.update(position_embedding_type="relative_key"),
    lambda c: c.update(num_attention_heads=5),
    lambda c: c.update(max_position_embeddings=16),
])
def test_bert_config_rejected(tmp_path, edit):
    profile = _bert_pack(tmp_path, config_edit=edit)
    with pytest.raises(UnsupportedProfileError):
        BertBackend(str(tmp_path), profile)


def _nan_word_embedding(t):
    bad = t["embeddings.word_embeddings.weight"][1].copy()
    bad[0, 0] = np.nan
    t["embeddings.word_embeddings.weight"] = ("F32", bad)


@pytest.mark.parametrize("edit", [
    _nan_word_embedding,
    lambda t: t.update({"embeddings.position_ids": ("I64", np.zeros((1, 32), np.int64))}),
    lambda t: t.pop("encoder.layer.0.output.LayerNorm.bias"),
    lambda t: t.pop("pooler.dense.bias"),
])
def test_bert_inventory_rejected(tmp_path, edit):
    profile = _bert_pack(tmp_path, tensor_edit=edit)
    with pytest.raises(ManifestError):
        BertBackend(str(tmp_path), profile)


@pytest.mark.parametrize("kwargs", [
    dict(architecture="t5", native_dimensions=64, min_dimensions=64, max_length=32),
])
def test_profile_rejected(kwargs):
    with pytest.raises(UnsupportedProfileError):
        ModelProfile(**kwargs, artifacts=())


@pytest.mark.parametrize("kwargs", [
    dict(architecture="bert_f32", native_dimensions=64, min_dimensions=32, max_length=32),
    dict(architecture="qwen3_uint4", native_dimensions=64, min_dimensions=16, max_length=32),
    dict(architecture="qwen3_uint4", native_dimensions=64, min_dimensions=64, max_length=513),
])
def test_profile_limits(kwargs):
    artifacts = (Artifact("config.json", "config.json", 1, "0" * 64),
                 Artifact("model.safetensors", "model.safetensors", 1, "0" * 64))
    with pytest.raises(ManifestError):
        ModelProfile(**kwargs, artifacts=artifacts)


def test_profile_digest_is_sha256(tmp_path):
    profile = _bert_pack(tmp_path, extras=False)
    data = (tmp_path / "model.safetensors").read_bytes()
    assert profile.artifact("model.safetensors").sha256 == hashlib.sha256(data).hexdigest()
