"""Whole-model embedding forwards on the HIP runtime: Qwen3 (uint4 affine weights) and BERT/BGE
(fp32 weights), loaded from verified SafeTensors packs.

Mirrors tessery's Qwen3Backend (qwen3.py:15-303) and BertBackend (bert.py:13-259): the same
config checks (UnsupportedProfileError), the same tensor inventory (ManifestError on any missing,
extra or mis-shaped tensor, checked before the first GPU allocation), the same input checks on
forward (InferenceError) and the same op sequence, recorded once per (batch, seq, dimensions)
as an execution plan and replayed (as a HIP graph) afterwards. Every op is a HIP kernel of this
package; there is no host compute in the forward.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import numpy as np
from numpy.typing import NDArray

from .errors import ClosedError, InferenceError, ManifestError, UnsupportedProfileError
from .runtime import Buffer, HipRuntime
from .weights import Artifact, SafeTensors, read_artifact, read_json


@dataclass(frozen=True)
class ModelProfile:
    """The pinned description of a pack (the fields of profiles.py:40-95 the backends read).

    architecture: "qwen3_uint4" (last-token pooling) or "bert_f32" (CLS pooling).
    artifacts: config.json and model.safetensors, each pinned by size and sha256.
    """

    architecture: str
    native_dimensions: int
    min_dimensions: int
    max_length: int
    artifacts: tuple[Artifact, ...]

    def __post_init__(self) -> None:
        if self.architecture not in ("qwen3_uint4", "bert_f32"):
            raise UnsupportedProfileError()
        if (any(type(v) is not int for v in (self.native_dimensions, self.min_dimensions,
                                              self.max_length))
                or not 32 <= self.min_dimensions <= self.native_dimensions <= 4096
                or not 1 <= self.max_length <= 512
                or (self.architecture == "bert_f32"
                    and self.min_dimensions != self.native_dimensions)):
            raise ManifestError()
        names = sorted(a.name for a in self.artifacts)
        if names != ["config.json", "model.safetensors"]:
            raise ManifestError()

    def artifact(self, name: str) -> Artifact:
        for a in self.artifacts:
            if a.name == name:
                return a
        raise ManifestError()


def config_int(config: dict[str, Any], key: str, low: int, high: int) -> int:
    """backend.py:35-39: an int (not a bool) in [low, high]."""
    value = config.get(key)
    if type(value) is not int or not low <= value <= high:
        raise UnsupportedProfileError()
    return int(value)


def config_float(config: dict[str, Any], key: str, low: float, high: float) -> float:
    """backend.py:42-51: a finite int or float (not a bool) in [low, high]."""
    value = config.get(key)
    if (not isinstance(value, (int, float)) or isinstance(value, bool)
            or not math.isfinite(value) or not low <= value <= high):
        raise UnsupportedProfileError()
    return float(value)


def _upload(runtime: HipRuntime, snapshot: SafeTensors, specs: dict[str, tuple[tuple[int, ...], str]],
            skip: set[str]) -> dict[str, Buffer]:
    weights: dict[str, Buffer] = {}
    for name, (shape, dtype) in specs.items():
        if name not in skip:
            data = snapshot.view(name, shape=shape, dtype=dtype)
            weights[name] = runtime.buffer(data.nbytes, data)
    return weights


def _check_unit_rows(result: NDArray[np.float32]) -> NDArray[np.float32]:
    if not np.isfinite(result).all() or not np.allclose(
            np.linalg.norm(result, axis=1), 1.0, atol=1e-4, rtol=0.0):
        raise InferenceError()
    return result


class Qwen3Backend:
    """Qwen3 embedding model with uint4 affine group-64 weights (MLX layout: uint32 words of 8
    codes, bf16 scales and biases per 64 inputs), last-token pooling."""

    max_padded_tokens = 4096

    def __init__(self, model_dir: str, profile: ModelProfile, *,
                 workspace_limit_bytes: int = 64 * 1024 * 1024) -> None:
        self._closed = True
        config = read_json(model_dir, profile.artifact("config.json"))
        self.profile = profile
        self.hidden = config_int(config, "hidden_size", 64, 4096)
        self.intermediate = config_int(config, "intermediate_size", 64, 16384)
        self.layers = config_int(config, "num_hidden_layers", 1, 64)
        self.heads = config_int(config, "num_attention_heads", 1, 64)
        self.kv_heads = config_int(config, "num_key_value_heads", 1, self.heads)
        self.head_dim = config_int(config, "head_dim", 2, 256)
        self.vocab_size = config_int(config, "vocab_size", 256, 200000)
        if (profile.architecture != "qwen3_uint4" or self.hidden != profile.native_dimensions
                or self.heads % self.kv_heads or self.head_dim % 2
                or any(v % 64 for v in (self.hidden, self.intermediate, self.heads * self.head_dim))
                or config.get("is_decoder", False) or config.get("add_cross_attention", False)):
            raise UnsupportedProfileError()
        expected: dict[str, Any] = {
            "model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"],
            "hidden_size": self.hidden, "intermediate_size": self.intermediate,
            "num_hidden_layers": self.layers, "num_attention_heads": self.heads,
            "num_key_value_heads": self.kv_heads, "head_dim": self.head_dim,
            "vocab_size": self.vocab_size, "hidden_act": "silu", "attention_bias": False,
            "rope_scaling": None, "use_sliding_window": False,
            "quantization": {"bits": 4, "group_size": 64},
        }
        if any(config.get(key) != value for key, value in expected.items()):
            raise UnsupportedProfileError()
        self.eps = config_float(config, "rms_norm_eps", 1e-12, 1)
        self.theta = config_float(config, "rope_theta", 1, 1e12)
        snapshot = SafeTensors(read_artifact(model_dir, profile.artifact("model.safetensors")))
        specs: dict[str, tuple[tuple[int, ...], str]] = {}

        def norm(prefix: str, dims: int) -> None:
            specs[prefix + ".weight"] = ((dims,), "BF16")

        def quant(prefix: str, outputs: int, inputs: int) -> None:
            specs[prefix + ".weight"] = ((outputs, inputs // 8), "U32")
            specs[prefix + ".scales"] = ((outputs, inputs // 64), "BF16")
            specs[prefix + ".biases"] = ((outputs, inputs // 64), "BF16")

        q_width, kv_width = self.heads * self.head_dim, self.kv_heads * self.head_dim
        quant("model.embed_tokens", self.vocab_size, self.hidden)
        norm("model.norm", self.hidden)
        for layer in range(self.layers):
            p = f"model.layers.{layer}"
            norm(p + ".input_layernorm", self.hidden)
            norm(p + ".post_attention_layernorm", self.hidden)
            quant(p + ".self_attn.q_proj", q_width, self.hidden)
            quant(p + ".self_attn.k_proj", kv_width, self.hidden)
            quant(p + ".self_attn.v_proj", kv_width, self.hidden)
            quant(p + ".self_attn.o_proj", self.hidden, q_width)
            norm(p + ".self_attn.q_norm", self.head_dim)
            norm(p + ".self_attn.k_norm", self.head_dim)
            quant(p + ".mlp.gate_proj", self.intermediate, self.hidden)
            quant(p + ".mlp.up_proj", self.intermediate, self.hidden)
            quant(p + ".mlp.down_proj", self.hidden, self.intermediate)
        if set(specs) != set(snapshot.tensors):
            raise ManifestError()
        for name, (shape, dtype) in specs.items():  # every tensor checked before any allocation
            snapshot.view(name, shape=shape, dtype=dtype)
        self.runtime = HipRuntime(workspace_limit_bytes=workspace_limit_bytes)
        self.weights: dict[str, Buffer] = {}
        self._closed = False
        try:
            self.weights = _upload(self.runtime, snapshot, specs, set())
        except BaseException:
            self.close()
            raise

    def _quant(self, prefix: str) -> list[Buffer]:
        return [self.weights[prefix + s] for s in (".weight", ".scales", ".biases")]

    def forward(self, ids: NDArray[np.uint32], lengths: NDArray[np.uint32], *,
                dimensions: int) -> NDArray[np.float32]:
        """ids [batch, seq] right-padded token ids, lengths [batch] valid tokens per row ->
        [batch, dimensions] unit vectors of the last valid token's final hidden state."""
        if self._closed:
            raise ClosedError()
        if (ids.dtype != np.uint32 or lengths.dtype != np.uint32 or ids.ndim != 2
                or not 1 <= ids.shape[0] <= 32 or not 1 <= ids.shape[1] <= self.profile.max_length
                or ids.size > self.max_padded_tokens or lengths.shape != (ids.shape[0],)
                or not np.all((lengths > 0) & (lengths <= ids.shape[1]))
                or np.any(ids >= self.vocab_size) or type(dimensions) is not int
                or not self.profile.min_dimensions <= dimensions <= self.hidden):
            raise InferenceError()
        rt = self.runtime
        batch, seq = ids.shape
        tokens = batch * seq
        q_width, kv_width = self.heads * self.head_dim, self.kv_heads * self.head_dim

        def norm(x: Buffer, y: Buffer, name: str, rows: int, cols: int) -> None:
            rt._dispatch("rms_norm", [x, self.weights[name + ".weight"], y], threads=rows * 32,
                         group_size=32, cols=cols, eps=self.eps)

        def linear(x: Buffer, y: Buffer, name: str, outputs: int, inputs: int) -> None:
            rt._linear4([x, *self._quant(name), y], rows=tokens, cols=outputs, k=inputs)

        def residual(x: Buffer, y: Buffer) -> None:
            rt._dispatch("add", [x, y, x], threads=tokens * self.hidden, n=tokens * self.hidden)

        with rt._workspace() as new:
            # ids and lengths go into reusable workspace buffers, so a repeated shape binds the
            # same device pointers and its plan replays through the cached graph
            id_buf, len_buf = new(ids.nbytes), new(lengths.nbytes)
            rt.write(id_buf, ids)
            rt.write(len_buf, lengths)
            with rt.command():
                x, normalized, projected = (new(tokens * self.hidden * 4) for _ in range(3))
                q, attended = (new(tokens * q_width * 4) for _ in range(2))
                k, v = (new(tokens * kv_width * 4) for _ in range(2))
                gate, up = (new(tokens * self.intermediate * 4) for _ in range(2))
                output = new(batch * dimensions * 4)
                bindings = [*self.weights.values(), id_buf, len_buf, x, normalized, projected, q,
                            attended, k, v, gate, up, output]
                with rt._execution_plan(("qwen", batch, seq, dimensions), bindings) as replayed:
                    if not replayed:
                        rt._dispatch("embedding4", [id_buf, *self._quant("model.embed_tokens"), x],
                                     threads=tokens * self.hidden, n=tokens * self.hidden,
                                     cols=self.hidden)
                        for layer in range(self.layers):
                            p = f"model.layers.{layer}"
                            attn = p + ".self_attn"
                            norm(x, normalized, p + ".input_layernorm", tokens, self.hidden)
                            linear(normalized, q, attn + ".q_proj", q_width, self.hidden)
                            linear(normalized, k, attn + ".k_proj", kv_width, self.hidden)
                            linear(normalized, v, attn + ".v_proj", kv_width, self.hidden)
                            for value, heads, name in ((q, self.heads, "q"),
                                                       (k, self.kv_heads, "k")):
                                norm(value, value, attn + f".{name}_norm", tokens * heads,
                                     self.head_dim)
                                count = tokens * heads * self.head_dim // 2
                                rt._dispatch("rope", [value], threads=count, n=count,
                                             heads=heads, seq=seq, dim=self.head_dim,
                                             theta=self.theta)
                            rt._attention([q, k, v, len_buf, attended], tokens=tokens, seq=seq,
                                          heads=self.heads, kv_heads=self.kv_heads,
                                          dim=self.head_dim)
                            linear(attended, projected, attn + ".o_proj", self.hidden, q_width)
                            residual(x, projected)
                            norm(x, normalized, p + ".post_attention_layernorm", tokens,
                                 self.hidden)
                            rt._gated4([normalized, *self._quant(p + ".mlp.gate_proj"),
                                        *self._quant(p + ".mlp.up_proj"), gate, up],
                                       rows=tokens, cols=self.intermediate, k=self.hidden)
                            linear(gate, projected, p + ".mlp.down_proj", self.hidden,
                                   self.intermediate)
                            residual(x, projected)
                        norm(x, normalized, "model.norm", tokens, self.hidden)
                        rt._dispatch("pool_project", [normalized, len_buf, output],
                                     threads=batch * 32, group_size=32, seq=seq,
                                     cols=self.hidden, dim=dimensions)
            result = rt.read(output, (batch, dimensions))
        return _check_unit_rows(result)

    def close(self) -> None:
        if not self._closed:
            self._closed = True
            for buffer in self.weights.values():
                buffer.close()
            self.weights.clear()
            self.runtime.close()


class BertBackend:
    """BERT / BGE encoder with fp32 weights, CLS pooling (the encoder state of token 0, not the
    optional tanh pooler)."""

    max_padded_tokens = 4096

    def __init__(self, model_dir: str, profile: ModelProfile, *,
                 workspace_limit_bytes: int = 64 * 1024 * 1024) -> None:
        self._closed = True
        self.profile = profile
        config = read_json(model_dir, profile.artifact("config.json"))
        self.hidden = config_int(config, "hidden_size", 32, 4096)
        self.intermediate = config_int(config, "intermediate_size", 32, 16384)
        self.layers = config_int(config, "num_hidden_layers", 1, 64)
        self.heads = config_int(config, "num_attention_heads", 1, 64)
        self.vocab_size = config_int(config, "vocab_size", 5, 200000)
        positions = config_int(config, "max_position_embeddings", profile.max_length, 8192)
        types = config_int(config, "type_vocab_size", 1, 16)
        if (profile.architecture != "bert_f32" or self.hidden != profile.native_dimensions
                or self.hidden % self.heads or not 1 <= self.hidden // self.heads <= 256
                or config.get("model_type") != "bert"
                or config.get("architectures") != ["BertModel"]
                or config.get("hidden_act") != "gelu"
                or config.get("position_embedding_type", "absolute") != "absolute"
                or config.get("is_decoder", False) or config.get("add_cross_attention", False)
                or config.get("pruned_heads", {})):
            raise UnsupportedProfileError()
        self.head_dim = self.hidden // self.heads
        self.eps = config_float(config, "layer_norm_eps", 1e-12, 1)
        snapshot = SafeTensors(read_artifact(model_dir, profile.artifact("model.safetensors")))
        specs: dict[str, tuple[tuple[int, ...], str]] = {}

        def norm(prefix: str) -> None:
            specs[prefix + ".weight"] = ((self.hidden,), "F32")
            specs[prefix + ".bias"] = ((self.hidden,), "F32")

        def linear(prefix: str, outputs: int, inputs: int) -> None:
            specs[prefix + ".weight"] = ((outputs, inputs), "F32")
            specs[prefix + ".bias"] = ((outputs,), "F32")

        for name, rows in (("word", self.vocab_size), ("position", positions),
                           ("token_type", types)):
            specs[f"embeddings.{name}_embeddings.weight"] = ((rows, self.hidden), "F32")
        norm("embeddings.LayerNorm")
        for layer in range(self.layers):
            p = f"encoder.layer.{layer}"
            for name in ("query", "key", "value"):
                linear(p + ".attention.self." + name, self.hidden, self.hidden)
            linear(p + ".attention.output.dense", self.hidden, self.hidden)
            norm(p + ".attention.output.LayerNorm")
            linear(p + ".intermediate.dense", self.intermediate, self.hidden)
            linear(p + ".output.dense", self.hidden, self.intermediate)
            norm(p + ".output.LayerNorm")
        unused: set[str] = set()
        if "pooler.dense.weight" in snapshot.tensors:
            linear("pooler.dense", self.hidden, self.hidden)
            unused.update(("pooler.dense.weight", "pooler.dense.bias"))
        if "embeddings.position_ids" in snapshot.tensors:
            specs["embeddings.position_ids"] = ((1, positions), "I64")
            unused.add("embeddings.position_ids")
        if set(specs) != set(snapshot.tensors):
            raise ManifestError()
        for name, (shape, dtype) in specs.items():
            data = snapshot.view(name, shape=shape, dtype=dtype)
            if dtype == "F32" and not np.isfinite(data.view(np.float32)).all():
                raise ManifestError()
            if dtype == "I64" and not np.array_equal(data.view(np.int64), np.arange(positions)):
                raise ManifestError()
        self.runtime = HipRuntime(workspace_limit_bytes=workspace_limit_bytes)
        self.weights: dict[str, Buffer] = {}
        self._closed = False
        try:
            self.weights = _upload(self.runtime, snapshot, specs, unused)
        except BaseException:
            self.close()
            raise

    def forward(self, ids: NDArray[np.uint32], lengths: NDArray[np.uint32], *,
                dimensions: int) -> NDArray[np.float32]:
        """ids [batch, seq] right-padded, lengths [batch] (at least 2: CLS and SEP) ->
        [batch, hidden] unit vectors of the CLS token's final encoder state."""
        if self._closed:
            raise ClosedError()
        if (ids.dtype != np.uint32 or lengths.dtype != np.uint32 or ids.ndim != 2
                or not 1 <= ids.shape[0] <= 32 or not 2 <= ids.shape[1] <= self.profile.max_length
                or ids.size > self.max_padded_tokens or lengths.shape != (ids.shape[0],)
                or not np.all((lengths >= 2) & (lengths <= ids.shape[1]))
                or np.any(ids >= self.vocab_size) or type(dimensions) is not int
                or dimensions != self.hidden):
            raise InferenceError()
        rt = self.runtime
        batch, seq = ids.shape
        tokens = batch * seq
        w = self.weights

        def norm(x: Buffer, y: Buffer, name: str) -> None:
            rt._dispatch("layer_norm", [x, w[name + ".weight"], w[name + ".bias"], y],
                         threads=tokens * 32, group_size=32, cols=self.hidden, eps=self.eps)

        def linear(x: Buffer, y: Buffer, name: str, outputs: int, inputs: int) -> None:
            rt._matmul_bias_f32([x, w[name + ".weight"], y, w[name + ".bias"]], rows=tokens,
                                cols=outputs, k=inputs)

        def add(x: Buffer, y: Buffer) -> None:
            rt._dispatch("add", [x, y, x], threads=tokens * self.hidden, n=tokens * self.hidden)

        with rt._workspace() as new:
            id_buf, len_buf = new(ids.nbytes), new(lengths.nbytes)  # reusable: stable bindings
            rt.write(id_buf, ids)
            rt.write(len_buf, lengths)
            with rt.command():
                x, projected, q, k, v, attended = (new(tokens * self.hidden * 4) for _ in range(6))
                activated = new(tokens * self.intermediate * 4)
                output = new(batch * dimensions * 4)
                bindings = [*w.values(), id_buf, len_buf, x, projected, q, k, v, attended,
                            activated, output]
                with rt._execution_plan(("bert", batch, seq, dimensions), bindings) as replayed:
                    if not replayed:
                        rt._dispatch("embedding_position",
                                     [id_buf, w["embeddings.word_embeddings.weight"],
                                      w["embeddings.position_embeddings.weight"],
                                      w["embeddings.token_type_embeddings.weight"], x],
                                     threads=tokens * self.hidden, n=tokens * self.hidden,
                                     cols=self.hidden, seq=seq)
                        norm(x, x, "embeddings.LayerNorm")
                        for layer in range(self.layers):
                            p = f"encoder.layer.{layer}"
                            for target, name in ((q, "query"), (k, "key"), (v, "value")):
                                linear(x, target, p + ".attention.self." + name, self.hidden,
                                       self.hidden)
                            rt._attention([q, k, v, len_buf, attended], tokens=tokens, seq=seq,
                                          heads=self.heads, kv_heads=self.heads,
                                          dim=self.head_dim, bidirectional=True)
                            linear(attended, projected, p + ".attention.output.dense",
                                   self.hidden, self.hidden)
                            add(x, projected)
                            norm(x, x, p + ".attention.output.LayerNorm")
                            linear(x, activated, p + ".intermediate.dense", self.intermediate,
                                   self.hidden)
                            rt._dispatch("gelu_f32", [activated],
                                         threads=tokens * self.intermediate,
                                         n=tokens * self.intermediate)
                            linear(activated, projected, p + ".output.dense", self.hidden,
                                   self.intermediate)
                            add(x, projected)
                            norm(x, x, p + ".output.LayerNorm")
                        rt._dispatch("pool_project", [x, len_buf, output], threads=batch * 32,
                                     group_size=32, seq=seq, cols=self.hidden, dim=dimensions,
                                     first_token=True)
            result = rt.read(output, (batch, dimensions))
        return _check_unit_rows(result)

    def close(self) -> None:
        if not self._closed:
            self._closed = True
            for buffer in self.weights.values():
                buffer.close()
            self.weights.clear()
            self.runtime.close()
