"""Whole-model embedding forwards on the HIP runtime: Qwen3 (uint4 affine weights, last-token
pooling) and BERT/BGE (fp32 weights, CLS pooling), from verified packs (packs.py).

A forward is compiled, once per (batch, seq, dimensions), into a Program: a flat tuple of Op
records (kernel family, named slots, static parameters) emitted by per-layer planners, plus the
table of activation slots it needs. One executor runs any Program: it binds the slot names to
weight buffers (tensor names) and to workspace activations, queues the ops through the runtime's
routes inside one command, and lets the runtime record the launches as a prepared plan on the
first call of a shape and replay that plan, as one cached HIP graph, on later calls. The
planners hold each model's layer; the executor, the binding and the plan bookkeeping are shared.

The public surface follows tessery's backends (qwen3.py:15-303, bert.py:13-259): the class names,
the constructor (model_dir, profile, workspace_limit_bytes), forward(ids, lengths, dimensions=)
with its input checks and error classes, the result check (finite unit rows), runtime and close.
The layer op order is the models' own (qwen3.py:194-280, bert.py:186-230).
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache
from typing import Any, Callable, Iterator, Union

import numpy as np
from numpy.typing import NDArray

from .errors import ClosedError, InferenceError, UnsupportedProfileError
from .packs import (BertDims, DeviceWeights, ModelProfile, Qwen3Dims, bert_inventory,
                    load_weights, qwen3_inventory, read_dims)
from .runtime import Buffer, HipRuntime

__all__ = ["BertBackend", "ModelProfile", "Qwen3Backend"]

UINT4 = (".weight", ".scales", ".biases")
DENSE = (".weight", ".bias")

# ---- programs ---------------------------------------------------------------------------------

# A slot is an activation ("%name"), the token ids ("%ids"), the lengths ("%lengths"), or a weight
# parameter: its tensor name, or a parameter prefix whose tensors are taken in a family's order
# ("prefix" + suffixes, written as (prefix, suffixes)).
Slot = Union[str, tuple[str, tuple[str, ...]]]


@dataclass(frozen=True)
class Op:
    kind: str                       # an entry of EMITTERS
    slots: tuple[Slot, ...]
    params: tuple[tuple[str, Any], ...] = ()


@dataclass(frozen=True)
class Program:
    key: tuple[Any, ...]            # the prepared-plan key of this shape
    activations: tuple[tuple[str, int], ...]   # (slot, bytes), in binding order
    output: str                     # the activation holding the [batch, dimensions] result
    output_shape: tuple[int, int]
    ops: tuple[Op, ...]


def op(kind: str, *slots: Slot, **params: Any) -> Op:
    return Op(kind, slots, tuple(sorted(params.items())))


# What each op kind queues on the runtime, given its bound buffers and parameters.
Emitter = Callable[..., None]


def _rms_norm(rt: HipRuntime, b: list[Buffer], *, rows: int, cols: int, eps: float) -> None:
    rt._dispatch("rms_norm", b, threads=rows * 32, group_size=32, cols=cols, eps=eps)


def _rope(rt: HipRuntime, b: list[Buffer], *, pairs: int, heads: int, seq: int, dim: int,
          theta: float) -> None:
    rt._dispatch("rope", b, threads=pairs, n=pairs, heads=heads, seq=seq, dim=dim, theta=theta)


def _layer_norm(rt: HipRuntime, b: list[Buffer], *, rows: int, cols: int, eps: float) -> None:
    rt._dispatch("layer_norm", b, threads=rows * 32, group_size=32, cols=cols, eps=eps)


def _add(rt: HipRuntime, b: list[Buffer], *, n: int) -> None:
    rt._dispatch("add", b, threads=n, n=n)


def _gelu(rt: HipRuntime, b: list[Buffer], *, n: int) -> None:
    rt._dispatch("gelu_f32", b, threads=n, n=n)


def _embed_uint4(rt: HipRuntime, b: list[Buffer], *, n: int, cols: int) -> None:
    rt._dispatch("embedding4", b, threads=n, n=n, cols=cols)


def _embed_bert(rt: HipRuntime, b: list[Buffer], *, n: int, cols: int, seq: int) -> None:
    rt._dispatch("embedding_position", b, threads=n, n=n, cols=cols, seq=seq)


def _pool(rt: HipRuntime, b: list[Buffer], *, batch: int, seq: int, cols: int, dim: int,
          first: bool) -> None:
    rt._dispatch("pool_project", b, threads=batch * 32, group_size=32, seq=seq, cols=cols,
                 dim=dim, first_token=first)


def _linear4(rt: HipRuntime, b: list[Buffer], *, rows: int, cols: int, k: int) -> None:
    rt._linear4(b, rows=rows, cols=cols, k=k)


def _gated4(rt: HipRuntime, b: list[Buffer], *, rows: int, cols: int, k: int) -> None:
    rt._gated4(b, rows=rows, cols=cols, k=k)


def _dense(rt: HipRuntime, b: list[Buffer], *, rows: int, cols: int, k: int) -> None:
    # slots are (x, weight, bias, y); the route takes [x, weight, y, bias]
    rt._matmul_bias_f32([b[0], b[1], b[3], b[2]], rows=rows, cols=cols, k=k)


def _attention(rt: HipRuntime, b: list[Buffer], **shape: int) -> None:
    rt._attention(b, **shape)


EMITTERS: dict[str, Emitter] = {
    "rms_norm": _rms_norm, "rope": _rope, "layer_norm": _layer_norm, "add": _add,
    "gelu": _gelu, "embed_uint4": _embed_uint4, "embed_bert": _embed_bert, "pool": _pool,
    "linear4": _linear4, "gated4": _gated4, "dense": _dense, "attention": _attention,
}


def execute(rt: HipRuntime, program: Program, weights: DeviceWeights, ids: NDArray[np.uint32],
            lengths: NDArray[np.uint32]) -> NDArray[np.float32]:
    """Run `program` on one batch and return its output activation.

    Token ids and lengths are written into workspace buffers and every activation comes from the
    workspace, so a repeated shape binds the same device pointers and its prepared plan replays
    as the same cached graph. The ops are queued only when the plan is recorded."""
    with rt._workspace() as lease:
        bound: dict[str, Buffer] = {"%ids": lease(ids.nbytes), "%lengths": lease(lengths.nbytes)}
        rt.write(bound["%ids"], ids)
        rt.write(bound["%lengths"], lengths)
        with rt.command():
            for slot, nbytes in program.activations:
                bound[slot] = lease(nbytes)

            def resolve(slot: Slot) -> Iterator[Buffer]:
                if isinstance(slot, tuple):
                    yield from weights.group(*slot)
                elif slot.startswith("%"):
                    yield bound[slot]
                else:
                    yield weights[slot]

            bindings = [*weights.buffers.values(), *bound.values()]
            with rt._execution_plan(program.key, bindings) as replayed:
                if not replayed:
                    for o in program.ops:
                        buffers = [b for s in o.slots for b in resolve(s)]
                        EMITTERS[o.kind](rt, buffers, **dict(o.params))
        return rt.read(bound[program.output], program.output_shape)


# ---- Qwen3 ------------------------------------------------------------------------------------


def qwen3_layer_ops(d: Qwen3Dims, layer: int, tokens: int, seq: int) -> Iterator[Op]:
    """One decoder layer (qwen3.py:194-280): pre-norm, q/k/v projections, per-head q/k RMSNorm
    and RoPE, causal GQA attention, o_proj + residual, post-norm, gated MLP, down + residual."""
    p = f"model.layers.{layer}."
    a = p + "self_attn."
    n = tokens * d.hidden
    yield op("rms_norm", "%x", p + "input_layernorm.weight", "%h", rows=tokens, cols=d.hidden,
             eps=d.eps)
    for name, out, width in (("q", "%q", d.q_width), ("k", "%k", d.kv_width),
                             ("v", "%v", d.kv_width)):
        yield op("linear4", "%h", (a + name + "_proj", UINT4), out, rows=tokens, cols=width,
                 k=d.hidden)
    for name, slot, heads in (("q", "%q", d.heads), ("k", "%k", d.kv_heads)):
        yield op("rms_norm", slot, a + name + "_norm.weight", slot, rows=tokens * heads,
                 cols=d.head_dim, eps=d.eps)
        yield op("rope", slot, pairs=tokens * heads * d.head_dim // 2, heads=heads, seq=seq,
                 dim=d.head_dim, theta=d.theta)
    yield op("attention", "%q", "%k", "%v", "%lengths", "%att", tokens=tokens, seq=seq,
             heads=d.heads, kv_heads=d.kv_heads, dim=d.head_dim)
    yield op("linear4", "%att", (a + "o_proj", UINT4), "%proj", rows=tokens, cols=d.hidden,
             k=d.q_width)
    yield op("add", "%x", "%proj", "%x", n=n)
    yield op("rms_norm", "%x", p + "post_attention_layernorm.weight", "%h", rows=tokens,
             cols=d.hidden, eps=d.eps)
    yield op("gated4", "%h", (p + "mlp.gate_proj", UINT4), (p + "mlp.up_proj", UINT4), "%gate",
             "%up", rows=tokens, cols=d.intermediate, k=d.hidden)
    yield op("linear4", "%gate", (p + "mlp.down_proj", UINT4), "%proj", rows=tokens,
             cols=d.hidden, k=d.intermediate)
    yield op("add", "%x", "%proj", "%x", n=n)


@lru_cache(maxsize=16)
def qwen3_program(d: Qwen3Dims, batch: int, seq: int, dimensions: int) -> Program:
    tokens = batch * seq
    f32 = 4
    acts = (("%x", tokens * d.hidden * f32), ("%h", tokens * d.hidden * f32),
            ("%proj", tokens * d.hidden * f32), ("%q", tokens * d.q_width * f32),
            ("%att", tokens * d.q_width * f32), ("%k", tokens * d.kv_width * f32),
            ("%v", tokens * d.kv_width * f32), ("%gate", tokens * d.intermediate * f32),
            ("%up", tokens * d.intermediate * f32), ("%out", batch * dimensions * f32))
    ops = [op("embed_uint4", "%ids", ("model.embed_tokens", UINT4), "%x", n=tokens * d.hidden,
              cols=d.hidden)]
    for layer in range(d.layers):
        ops.extend(qwen3_layer_ops(d, layer, tokens, seq))
    ops.append(op("rms_norm", "%x", "model.norm.weight", "%h", rows=tokens, cols=d.hidden,
                  eps=d.eps))
    # the last valid token of each row, its first `dimensions` channels, L2-normalized
    ops.append(op("pool", "%h", "%lengths", "%out", batch=batch, seq=seq, cols=d.hidden,
                  dim=dimensions, first=False))
    return Program(("qwen", batch, seq, dimensions), acts, "%out", (batch, dimensions),
                   tuple(ops))


# ---- BERT -------------------------------------------------------------------------------------


def bert_layer_ops(d: BertDims, layer: int, tokens: int, seq: int) -> Iterator[Op]:
    """One encoder layer (bert.py:186-230): q/k/v projections with bias, bidirectional attention,
    output projection, residual + LayerNorm, GELU MLP, residual + LayerNorm (x in place)."""
    p = f"encoder.layer.{layer}."
    n = tokens * d.hidden
    for name, out in (("query", "%q"), ("key", "%k"), ("value", "%v")):
        yield op("dense", "%x", (p + "attention.self." + name, DENSE), out, rows=tokens,
                 cols=d.hidden, k=d.hidden)
    yield op("attention", "%q", "%k", "%v", "%lengths", "%att", tokens=tokens, seq=seq,
             heads=d.heads, kv_heads=d.heads, dim=d.head_dim, bidirectional=1)
    yield op("dense", "%att", (p + "attention.output.dense", DENSE), "%proj", rows=tokens,
             cols=d.hidden, k=d.hidden)
    yield op("add", "%x", "%proj", "%x", n=n)
    yield op("layer_norm", "%x", (p + "attention.output.LayerNorm", DENSE), "%x", rows=tokens,
             cols=d.hidden, eps=d.eps)
    yield op("dense", "%x", (p + "intermediate.dense", DENSE), "%act", rows=tokens,
             cols=d.intermediate, k=d.hidden)
    yield op("gelu", "%act", n=tokens * d.intermediate)
    yield op("dense", "%act", (p + "output.dense", DENSE), "%proj", rows=tokens, cols=d.hidden,
             k=d.intermediate)
    yield op("add", "%x", "%proj", "%x", n=n)
    yield op("layer_norm", "%x", (p + "output.LayerNorm", DENSE), "%x", rows=tokens,
             cols=d.hidden, eps=d.eps)


@lru_cache(maxsize=16)
def bert_program(d: BertDims, batch: int, seq: int) -> Program:
    tokens = batch * seq
    f32 = 4
    acts = (("%x", tokens * d.hidden * f32), ("%proj", tokens * d.hidden * f32),
            ("%q", tokens * d.hidden * f32), ("%k", tokens * d.hidden * f32),
            ("%v", tokens * d.hidden * f32), ("%att", tokens * d.hidden * f32),
            ("%act", tokens * d.intermediate * f32), ("%out", batch * d.hidden * f32))
    ops = [op("embed_bert", "%ids", "embeddings.word_embeddings.weight",
              "embeddings.position_embeddings.weight",
              "embeddings.token_type_embeddings.weight", "%x", n=tokens * d.hidden,
              cols=d.hidden, seq=seq),
           op("layer_norm", "%x", ("embeddings.LayerNorm", DENSE), "%x", rows=tokens,
              cols=d.hidden, eps=d.eps)]
    for layer in range(d.layers):
        ops.extend(bert_layer_ops(d, layer, tokens, seq))
    # the CLS token's encoder state (not the tanh pooler), L2-normalized
    ops.append(op("pool", "%x", "%lengths", "%out", batch=batch, seq=seq, cols=d.hidden,
                  dim=d.hidden, first=True))
    return Program(("bert", batch, seq, d.hidden), acts, "%out", (batch, d.hidden), tuple(ops))


# ---- backends ---------------------------------------------------------------------------------


def _unit_rows(result: NDArray[np.float32]) -> NDArray[np.float32]:
    norms = np.linalg.norm(result, axis=1)
    if not np.isfinite(result).all() or not np.allclose(norms, 1.0, atol=1e-4, rtol=0.0):
        raise InferenceError()
    return result


class _Backend:
    """Shared life cycle: dims and weights from a verified pack, one runtime, forward checks."""

    architecture = ""
    max_padded_tokens = 4096
    min_length = 1  # shortest valid row

    def __init__(self, model_dir: str, profile: ModelProfile, *,
                 workspace_limit_bytes: int = 64 * 1024 * 1024) -> None:
        self._weights: DeviceWeights | None = None
        if profile.architecture != self.architecture:
            raise UnsupportedProfileError()
        self.profile = profile
        self.dims = read_dims(model_dir, profile)
        inventory = (qwen3_inventory if isinstance(self.dims, Qwen3Dims) else bert_inventory)
        self._weights = load_weights(
            model_dir, profile, self.dims, inventory(self.dims),
            lambda: HipRuntime(workspace_limit_bytes=workspace_limit_bytes))
        self.runtime = self._weights.runtime

    @property
    def vocab_size(self) -> int:
        return self.dims.vocab

    @property
    def hidden(self) -> int:
        return self.dims.hidden

    def _dimension_ok(self, dimensions: int) -> bool:
        raise NotImplementedError

    def _program(self, batch: int, seq: int, dimensions: int) -> Program:
        raise NotImplementedError

    def forward(self, ids: NDArray[np.uint32], lengths: NDArray[np.uint32], *,
                dimensions: int) -> NDArray[np.float32]:
        """ids [batch, seq] right-padded token ids, lengths [batch] valid tokens per row ->
        [batch, dimensions] unit vectors of the pooled token's final state."""
        if self._weights is None:
            raise ClosedError()
        shape_ok = (ids.dtype == np.uint32 and lengths.dtype == np.uint32 and ids.ndim == 2
                    and 1 <= ids.shape[0] <= 32
                    and max(1, self.min_length) <= ids.shape[1] <= self.profile.max_length
                    and ids.size <= self.max_padded_tokens
                    and lengths.shape == (ids.shape[0],))
        if (not shape_ok or not np.all((lengths >= self.min_length) & (lengths <= ids.shape[1]))
                or np.any(ids >= self.vocab_size) or type(dimensions) is not int
                or not self._dimension_ok(dimensions)):
            raise InferenceError()
        batch, seq = ids.shape
        program = self._program(batch, seq, dimensions)
        result = execute(self.runtime, program, self._weights, np.ascontiguousarray(ids),
                         np.ascontiguousarray(lengths))
        return _unit_rows(result)

    def close(self) -> None:
        weights, self._weights = self._weights, None
        if weights is not None:
            weights.close()
            weights.runtime.close()


class Qwen3Backend(_Backend):
    """Qwen3 embedding model with uint4 affine group-64 weights (MLX layout: uint32 words of 8
    codes, bf16 scales and biases per 64 inputs), last-token pooling."""

    architecture = "qwen3_uint4"
    min_length = 1

    def _dimension_ok(self, dimensions: int) -> bool:
        return self.profile.min_dimensions <= dimensions <= self.dims.hidden

    def _program(self, batch: int, seq: int, dimensions: int) -> Program:
        return qwen3_program(self.dims, batch, seq, dimensions)


class BertBackend(_Backend):
    """BERT / BGE encoder with fp32 weights, CLS pooling (the encoder state of token 0, not the
    optional tanh pooler)."""

    architecture = "bert_f32"
    min_length = 2  # CLS and SEP

    def _dimension_ok(self, dimensions: int) -> bool:
        return dimensions == self.dims.hidden

    def _program(self, batch: int, seq: int, dimensions: int) -> Program:
        return bert_program(self.dims, batch, seq)
