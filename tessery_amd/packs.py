"""Weight packs of the two embedding models: config schemas, tensor inventories and verified upload.

A pack is a directory with config.json and model.safetensors, pinned by a ModelProfile. This
module turns one into a validated set of model dimensions and a DeviceWeights owner holding one
device buffer per tensor:

* the accepted config is declared as data (Schema): integer and real entries with their admitted
  ranges, entries that must hold a fixed value, and named constraints between entries; one parser
  checks any schema and raises UnsupportedProfileError on the first violation;
* the tensor inventory is expanded from a table of per-model and per-layer entries (Family):
  every expected name with its shape and dtype, plus the optional tensors the forward never reads;
* load_weights checks the complete inventory (names, shapes, dtypes, value checks) against the
  SafeTensors index before the first device allocation, then uploads each tensor once.

The config keys and their bounds, the tensor names and the layouts are the pack format of tessery
(qwen3.py:24-87 and bert.py:23-87 read the same packs; profiles.py:40-95 pins them), so a pack
accepted there is accepted here and one rejected there is rejected here.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Callable, Iterator, Mapping

import numpy as np

from .errors import ManifestError, UnsupportedProfileError
from .runtime import Buffer, HipRuntime
from .weights import Artifact, SafeTensors, read_artifact, read_json

# ---- profiles ---------------------------------------------------------------------------------


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
        if self.architecture not in SCHEMAS:
            raise UnsupportedProfileError()
        ints = (self.native_dimensions, self.min_dimensions, self.max_length)
        if (any(type(v) is not int for v in ints)
                or not 32 <= self.min_dimensions <= self.native_dimensions <= 4096
                or not 1 <= self.max_length <= 512
                or (self.architecture == "bert_f32"
                    and self.min_dimensions != self.native_dimensions)):
            raise ManifestError()
        if sorted(a.name for a in self.artifacts) != ["config.json", "model.safetensors"]:
            raise ManifestError()

    def artifact(self, name: str) -> Artifact:
        found = [a for a in self.artifacts if a.name == name]
        if not found:
            raise ManifestError()
        return found[0]


# ---- config schemas ---------------------------------------------------------------------------

# A bound is a number or the name of an entry parsed before it (or of a profile field).
BoundValue = float | int | str


@dataclass(frozen=True)
class Entry:
    """One numeric config entry: integers must be exact ints (not bools); reals may be ints or
    floats (not bools) and must be finite. Bounds are inclusive."""

    key: str
    name: str
    low: BoundValue
    high: BoundValue
    real: bool = False


@dataclass(frozen=True)
class Schema:
    entries: tuple[Entry, ...]
    fixed: Mapping[str, Any]                      # entries that must equal these values
    absent_or: Mapping[str, Any]                  # entries that may be missing, else must equal
    falsy: tuple[str, ...]                        # entries that may be missing, else must be falsy
    constraints: tuple[tuple[str, Callable[[dict[str, Any]], bool]], ...]


def _bound(value: BoundValue, env: Mapping[str, Any]) -> float:
    return float(env[value]) if isinstance(value, str) else float(value)


def parse_config(config: Mapping[str, Any], schema: Schema,
                 context: Mapping[str, Any]) -> dict[str, Any]:
    """The schema's numeric entries of `config` under their short names, or
    UnsupportedProfileError. `context` supplies profile fields that bounds may name."""
    env: dict[str, Any] = dict(context)
    for e in schema.entries:
        value = config.get(e.key)
        if e.real:
            ok = (isinstance(value, (int, float)) and not isinstance(value, bool)
                  and math.isfinite(value))
        else:
            ok = type(value) is int
        if not ok or not _bound(e.low, env) <= value <= _bound(e.high, env):
            raise UnsupportedProfileError()
        env[e.name] = float(value) if e.real else int(value)
    if any(config.get(k) != v for k, v in schema.fixed.items()):
        raise UnsupportedProfileError()
    if any(k in config and config[k] != v for k, v in schema.absent_or.items()):
        raise UnsupportedProfileError()
    if any(config.get(k) for k in schema.falsy):
        raise UnsupportedProfileError()
    for _, holds in schema.constraints:
        if not holds(env):
            raise UnsupportedProfileError()
    return env


QWEN3_SCHEMA = Schema(
    entries=(
        Entry("hidden_size", "hidden", 64, 4096),
        Entry("intermediate_size", "intermediate", 64, 16384),
        Entry("num_hidden_layers", "layers", 1, 64),
        Entry("num_attention_heads", "heads", 1, 64),
        Entry("num_key_value_heads", "kv_heads", 1, "heads"),
        Entry("head_dim", "head_dim", 2, 256),
        Entry("vocab_size", "vocab", 256, 200000),
        Entry("rms_norm_eps", "eps", 1e-12, 1, real=True),
        Entry("rope_theta", "theta", 1, 1e12, real=True),
    ),
    fixed={"model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"], "hidden_act": "silu",
           "attention_bias": False, "rope_scaling": None, "use_sliding_window": False,
           "quantization": {"bits": 4, "group_size": 64}},
    absent_or={},
    falsy=("is_decoder", "add_cross_attention"),
    constraints=(
        ("the model width is the profile's native width", lambda c: c["hidden"] == c["native"]),
        ("query heads share kv heads evenly", lambda c: c["heads"] % c["kv_heads"] == 0),
        ("RoPE rotates pairs of channels", lambda c: c["head_dim"] % 2 == 0),
        ("every projection input is whole uint4 groups of 64",
         lambda c: all(n % 64 == 0 for n in (c["hidden"], c["intermediate"],
                                             c["heads"] * c["head_dim"]))),
    ),
)

BERT_SCHEMA = Schema(
    entries=(
        Entry("hidden_size", "hidden", 32, 4096),
        Entry("intermediate_size", "intermediate", 32, 16384),
        Entry("num_hidden_layers", "layers", 1, 64),
        Entry("num_attention_heads", "heads", 1, 64),
        Entry("vocab_size", "vocab", 5, 200000),
        Entry("max_position_embeddings", "positions", "max_length", 8192),
        Entry("type_vocab_size", "types", 1, 16),
        Entry("layer_norm_eps", "eps", 1e-12, 1, real=True),
    ),
    fixed={"model_type": "bert", "architectures": ["BertModel"], "hidden_act": "gelu"},
    absent_or={"position_embedding_type": "absolute"},
    falsy=("is_decoder", "add_cross_attention", "pruned_heads"),
    constraints=(
        ("the model width is the profile's native width", lambda c: c["hidden"] == c["native"]),
        ("heads split the width into 1..256 channels",
         lambda c: c["hidden"] % c["heads"] == 0 and 1 <= c["hidden"] // c["heads"] <= 256),
    ),
)

SCHEMAS = {"qwen3_uint4": QWEN3_SCHEMA, "bert_f32": BERT_SCHEMA}


@dataclass(frozen=True)
class Qwen3Dims:
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    vocab: int
    eps: float
    theta: float

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim


@dataclass(frozen=True)
class BertDims:
    hidden: int
    intermediate: int
    layers: int
    heads: int
    vocab: int
    positions: int
    types: int
    eps: float

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def read_dims(model_dir: str, profile: ModelProfile) -> Qwen3Dims | BertDims:
    """The pack's config.json, checked against its architecture's schema."""
    config = read_json(model_dir, profile.artifact("config.json"))
    env = parse_config(config, SCHEMAS[profile.architecture],
                       {"native": profile.native_dimensions, "max_length": profile.max_length})
    cls = Qwen3Dims if profile.architecture == "qwen3_uint4" else BertDims
    return cls(**{f: env[f] for f in cls.__dataclass_fields__})


# ---- tensor inventories -----------------------------------------------------------------------


@dataclass(frozen=True)
class TensorSpec:
    shape: tuple[int, ...]
    dtype: str


# A family names how one logical parameter is stored: its tensors as (suffix, shape, dtype)
# given the parameter's (outputs, inputs).
Family = Callable[[int, int], tuple[tuple[str, tuple[int, ...], str], ...]]


def _uint4(outputs: int, inputs: int):
    """MLX affine uint4: words of 8 codes, bf16 scale and bias per group of 64 inputs."""
    return ((".weight", (outputs, inputs // 8), "U32"),
            (".scales", (outputs, inputs // 64), "BF16"),
            (".biases", (outputs, inputs // 64), "BF16"))


def _bf16_vector(outputs: int, _inputs: int):
    return ((".weight", (outputs,), "BF16"),)


def _f32_dense(outputs: int, inputs: int):
    return ((".weight", (outputs, inputs), "F32"), (".bias", (outputs,), "F32"))


def _f32_layernorm(outputs: int, _inputs: int):
    return ((".weight", (outputs,), "F32"), (".bias", (outputs,), "F32"))


def _f32_table(rows: int, cols: int):
    return ((".weight", (rows, cols), "F32"),)


# Qwen3: (parameter, family, outputs, inputs) with sizes named by Qwen3Dims fields / properties.
QWEN3_GLOBAL = (("model.embed_tokens", _uint4, "vocab", "hidden"),
                ("model.norm", _bf16_vector, "hidden", None))
QWEN3_LAYER = (
    ("input_layernorm", _bf16_vector, "hidden", None),
    ("post_attention_layernorm", _bf16_vector, "hidden", None),
    ("self_attn.q_proj", _uint4, "q_width", "hidden"),
    ("self_attn.k_proj", _uint4, "kv_width", "hidden"),
    ("self_attn.v_proj", _uint4, "kv_width", "hidden"),
    ("self_attn.o_proj", _uint4, "hidden", "q_width"),
    ("self_attn.q_norm", _bf16_vector, "head_dim", None),
    ("self_attn.k_norm", _bf16_vector, "head_dim", None),
    ("mlp.gate_proj", _uint4, "intermediate", "hidden"),
    ("mlp.up_proj", _uint4, "intermediate", "hidden"),
    ("mlp.down_proj", _uint4, "hidden", "intermediate"),
)
BERT_GLOBAL = (("embeddings.word_embeddings", _f32_table, "vocab", "hidden"),
               ("embeddings.position_embeddings", _f32_table, "positions", "hidden"),
               ("embeddings.token_type_embeddings", _f32_table, "types", "hidden"),
               ("embeddings.LayerNorm", _f32_layernorm, "hidden", None))
BERT_LAYER = (
    ("attention.self.query", _f32_dense, "hidden", "hidden"),
    ("attention.self.key", _f32_dense, "hidden", "hidden"),
    ("attention.self.value", _f32_dense, "hidden", "hidden"),
    ("attention.output.dense", _f32_dense, "hidden", "hidden"),
    ("attention.output.LayerNorm", _f32_layernorm, "hidden", None),
    ("intermediate.dense", _f32_dense, "intermediate", "hidden"),
    ("output.dense", _f32_dense, "hidden", "intermediate"),
    ("output.LayerNorm", _f32_layernorm, "hidden", None),
)


def _expand(dims: Any, table, prefix: str = "") -> Iterator[tuple[str, TensorSpec]]:
    for name, family, outputs, inputs in table:
        out = getattr(dims, outputs)
        inp = getattr(dims, inputs) if inputs else 0
        for suffix, shape, dtype in family(out, inp):
            yield prefix + name + suffix, TensorSpec(shape, dtype)


@dataclass(frozen=True)
class Inventory:
    """Every tensor a pack must hold (`required`), and groups of tensors it may hold that the
    forward never reads (`optional`): a group is present when its first tensor is, and then every
    tensor of the group must be; present groups are checked, never uploaded."""

    required: dict[str, TensorSpec]
    optional: tuple[dict[str, TensorSpec], ...] = ()

    def expected(self, present: set[str]) -> dict[str, TensorSpec]:
        """The complete set of tensors a pack holding `present` must match exactly."""
        specs = dict(self.required)
        for group in self.optional:
            if next(iter(group)) in present:
                specs.update(group)
        return specs


def qwen3_inventory(d: Qwen3Dims) -> Inventory:
    specs = dict(_expand(d, QWEN3_GLOBAL))
    for layer in range(d.layers):
        specs.update(_expand(d, QWEN3_LAYER, f"model.layers.{layer}."))
    return Inventory(specs)


def bert_inventory(d: BertDims) -> Inventory:
    specs = dict(_expand(d, BERT_GLOBAL))
    for layer in range(d.layers):
        specs.update(_expand(d, BERT_LAYER, f"encoder.layer.{layer}."))
    # CLS pooling reads the encoder state, not the tanh pooler; the position-id buffer some
    # exports carry must be the identity
    pooler = dict(_expand(d, (("pooler.dense", _f32_dense, "hidden", "hidden"),)))
    position_ids = {"embeddings.position_ids": TensorSpec((1, d.positions), "I64")}
    return Inventory(specs, (pooler, position_ids))


# ---- verified upload --------------------------------------------------------------------------


class DeviceWeights:
    """The uploaded tensors of one pack, by tensor name, owned by one runtime."""

    def __init__(self, runtime: HipRuntime) -> None:
        self.runtime = runtime
        self.buffers: dict[str, Buffer] = {}

    def __getitem__(self, name: str) -> Buffer:
        return self.buffers[name]

    def group(self, parameter: str, suffixes: tuple[str, ...]) -> list[Buffer]:
        return [self.buffers[parameter + s] for s in suffixes]

    def close(self) -> None:
        buffers, self.buffers = self.buffers, {}
        for b in buffers.values():
            b.close()


def _value_check(name: str, spec: TensorSpec, data: np.ndarray, d: Any) -> bool:
    if spec.dtype == "F32":
        return bool(np.isfinite(data.view(np.float32)).all())
    if spec.dtype == "I64":  # embeddings.position_ids
        return bool(np.array_equal(data.view(np.int64).reshape(-1), np.arange(d.positions)))
    return True


def load_weights(model_dir: str, profile: ModelProfile, dims: Any, inventory: Inventory,
                 runtime_factory: Callable[[], HipRuntime]) -> DeviceWeights:
    """Verify the pack's tensors against `inventory` (ManifestError on a missing, extra,
    mis-shaped or invalid tensor), and only then create the runtime and upload the required
    tensors, each once."""
    snapshot = SafeTensors(read_artifact(model_dir, profile.artifact("model.safetensors")))
    checks = inventory.expected(set(snapshot.tensors))
    if set(snapshot.tensors) != set(checks):
        raise ManifestError()
    for name, spec in checks.items():
        data = snapshot.view(name, shape=spec.shape, dtype=spec.dtype)
        if profile.architecture == "bert_f32" and not _value_check(name, spec, data, dims):
            raise ManifestError()
    weights = DeviceWeights(runtime_factory())
    try:
        for name, spec in inventory.required.items():
            data = snapshot.view(name, shape=spec.shape, dtype=spec.dtype)
            weights.buffers[name] = weights.runtime.buffer(data.nbytes, data)
    except BaseException:
        weights.close()
        weights.runtime.close()
        raise
    return weights
