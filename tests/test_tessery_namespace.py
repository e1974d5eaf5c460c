"""The `tessery` namespace re-exports tessery_amd's implementation under tessery's names
(src/tessery/__init__.py:1-42, src/metal_inference module names), with no device touched."""

import tessery
import tessery.batching
import tessery.bert
import tessery.errors
import tessery.metal
import tessery.qwen3
import tessery.weights
import tessery_amd
from tessery_amd import backends, batching, errors, packs, runtime, weights


def test_public_names_are_the_implementation():
    assert tessery.MetalRuntime is tessery_amd.MetalRuntime is runtime.HipRuntime
    assert tessery.ModelProfile is packs.ModelProfile
    assert tessery.Artifact is weights.Artifact
    assert set(tessery.__all__) <= set(dir(tessery))


def test_module_names_follow_metal_inference():
    assert tessery.metal.MetalRuntime is runtime.HipRuntime
    assert tessery.batching.execution_batches is batching.execution_batches
    assert tessery.qwen3.Qwen3Backend is backends.Qwen3Backend
    assert tessery.bert.BertBackend is backends.BertBackend
    assert tessery.weights.SafeTensors is weights.SafeTensors
    for name in errors.__all__:
        assert getattr(tessery.errors, name) is getattr(errors, name)


def test_out_of_scope_api_is_absent():
    for name in ("EmbeddingModel", "DocumentIndex", "cosine_search"):
        assert not hasattr(tessery, name)
