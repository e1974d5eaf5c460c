"""Seeded synthetic workloads of the prefill-attention path and their algorithmic work.

Five workloads, each named by what it is:
  bge_small_c1     BGE-small attention layer, B=2 S=16 H=12 D=32 fp32, lengths [16, 9], bidirectional
  bge_small_32x512 BGE-small encoder attention, B=32 S=512 H=12 D=32 fp32, 12 layers, L ~ U{2..512}
  qwen3_8x512      Qwen3-0.6B causal GQA, B=8 S=512 16q/8kv D=128 fp16, L ~ U{64..512}, q/k norm+RoPE
  qwen3_32x512     Qwen3 causal GQA at maximum batch, B=32, L log-uniform in [1,512], execution width
                   16*ceil(max L/16), 28 layers, q/k norm+RoPE
  qwen3_qkv4       uint4 group-64 QKV projection of x[16,256,1024] fp16 feeding causal GQA, L ~ U{1..256}

Convention: lengths come first from numpy.random.default_rng(seed); layer l's tensors come from
default_rng((seed, l)). Activations are N(0,1); RMSNorm weights U(0.5,1.5) stored as bfloat16
words (truncated, the encoding tessery's own tests use, test_kernels.py:22-23).
"""

from __future__ import annotations

from typing import Any

import math
from dataclasses import dataclass

import numpy as np
from numpy.typing import NDArray

EPS = 1e-6
THETA = 1e6


@dataclass(frozen=True)
class Shape:
    batch: int
    seq: int
    heads: int
    kv_heads: int
    dim: int
    causal: bool

    @property
    def tokens(self) -> int:
        return self.batch * self.seq


def bf16_words(values: NDArray[np.floating]) -> NDArray[np.uint16]:
    """float32 -> bfloat16 storage words by truncation."""
    return (np.asarray(values, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_values(words: NDArray[np.uint16]) -> NDArray[np.float32]:
    return (np.asarray(words, dtype=np.uint32) << 16).view(np.float32)


def normal(rng: np.random.Generator, shape: tuple[int, ...], dtype: type) -> NDArray:
    return rng.standard_normal(shape, dtype=np.float32).astype(dtype, copy=False)


# ---- lengths -------------------------------------------------------------------------------


def lengths_uniform(seed: int, batch: int, low: int, high: int) -> NDArray[np.uint32]:
    return np.random.default_rng(seed).integers(low, high + 1, batch).astype(np.uint32)


def lengths_loguniform(seed: int, batch: int, high: int = 512) -> NDArray[np.uint32]:
    draw = np.random.default_rng(seed).uniform(0.0, math.log(high + 1), batch)
    return np.clip(np.floor(np.exp(draw)), 1, high).astype(np.uint32)


def execution_width(lengths: NDArray[np.uint32], align: int = 16) -> int:
    return align * int(math.ceil(int(lengths.max()) / align))


# ---- workloads -----------------------------------------------------------------------------


def bge_small_c1() -> tuple[Shape, NDArray[np.uint32], dict[str, NDArray]]:
    shape = Shape(2, 16, 12, 12, 32, causal=False)
    lengths = np.array([16, 9], np.uint32)
    rng = np.random.default_rng((1, 0))
    q, k, v = (normal(rng, (2, 16, 12, 32), np.float32) for _ in range(3))
    return shape, lengths, {"q": q, "k": k, "v": v}


def bge_small_32x512() -> tuple[Shape, NDArray[np.uint32]]:
    return Shape(32, 512, 12, 12, 32, causal=False), lengths_uniform(2, 32, 2, 512)


def bge_layer(shape: Shape, layer: int, seed: int = 2) -> dict[str, NDArray]:
    rng = np.random.default_rng((seed, layer))
    q = normal(rng, (shape.batch, shape.seq, shape.heads, shape.dim), np.float32)
    k = normal(rng, (shape.batch, shape.seq, shape.kv_heads, shape.dim), np.float32)
    v = normal(rng, (shape.batch, shape.seq, shape.kv_heads, shape.dim), np.float32)
    return {"q": q, "k": k, "v": v}


def bge_encoder_layer(layer: int, seed: int = 7, batch: int = 32, seq: int = 512) -> dict[str, Any]:
    """BGE-small encoder layer weights and input (bert.py:186-230): hidden 384, 12 heads x 32,
    intermediate 1536; x ~ N(0,1) [batch*seq, 384]; projection weights N(0, 1/K) [N, K] with
    biases N(0, 0.1^2); LayerNorm weights U(0.5,1.5), biases N(0, 0.1^2). fp32."""
    rng = np.random.default_rng((seed, layer))
    hidden, inter = 384, 1536
    w: dict[str, Any] = {"x": normal(rng, (batch * seq, hidden), np.float32)}
    for name, (n, k) in {"q": (hidden, hidden), "k": (hidden, hidden), "v": (hidden, hidden),
                         "o": (hidden, hidden), "i": (inter, hidden), "out": (hidden, inter)}.items():
        w[name] = (normal(rng, (n, k), np.float32) * np.float32(k ** -0.5)).astype(np.float32)
        w[name + "_b"] = (0.1 * normal(rng, (n,), np.float32)).astype(np.float32)
    for ln in ("ln1", "ln2"):
        w[ln + "_w"] = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
        w[ln + "_b"] = (0.1 * normal(rng, (hidden,), np.float32)).astype(np.float32)
    return w


def bge_layer_gemm_flop(tokens: int, hidden: int = 384, inter: int = 1536) -> int:
    """2*T*K*N over the six projections of a BERT layer (q, k, v, o, intermediate, output)."""
    return 2 * tokens * (4 * hidden * hidden + 2 * hidden * inter)


def qwen3_8x512() -> tuple[Shape, NDArray[np.uint32]]:
    return Shape(8, 512, 16, 8, 128, causal=True), lengths_uniform(3, 8, 64, 512)


def qwen3_32x512() -> tuple[Shape, NDArray[np.uint32]]:
    lengths = lengths_loguniform(4, 32)
    return Shape(32, execution_width(lengths), 16, 8, 128, causal=True), lengths


def qwen3_32x512_full() -> tuple[Shape, NDArray[np.uint32]]:
    """The Qwen3 32x512 shape with every length at 512 (the full-length form of the headline)."""
    return Shape(32, 512, 16, 8, 128, causal=True), np.full(32, 512, np.uint32)


def qwen_layer(shape: Shape, layer: int, seed: int) -> dict[str, NDArray]:
    """Pre-norm q/k and v in fp16 plus bf16 q/k norm weights for one layer."""
    rng = np.random.default_rng((seed, layer))
    b, s, h, kv, d = shape.batch, shape.seq, shape.heads, shape.kv_heads, shape.dim
    q = normal(rng, (b, s, h, d), np.float16)
    k = normal(rng, (b, s, kv, d), np.float16)
    v = normal(rng, (b, s, kv, d), np.float16)
    gq = bf16_words(rng.uniform(0.5, 1.5, d))
    gk = bf16_words(rng.uniform(0.5, 1.5, d))
    return {"q": q, "k": k, "v": v, "q_norm": gq, "k_norm": gk}


def qwen_qkv4_16x256(seed: int = 5) -> tuple[Shape, NDArray[np.uint32], dict[str, NDArray]]:
    """uint4 QKV projection feeding causal GQA: x [16*256, 1024] fp16 ~ N(0,1); W_q 1024->2048 and
    W_k, W_v 1024->1024 as weight4 words with codes U{0..15} and group-64 fp16 scale / bias
    ~ N(0, 0.02), concatenated q|k|v along N; lengths U{1..256}; q/k norm weights U(0.5,1.5)."""
    shape = Shape(16, 256, 16, 8, 128, causal=True)
    lengths = lengths_uniform(seed, shape.batch, 1, shape.seq)
    rng = np.random.default_rng((seed, 0))
    k_in = 1024
    x = normal(rng, (shape.tokens, k_in), np.float16)
    n_total = (shape.heads + 2 * shape.kv_heads) * shape.dim
    codes = rng.integers(0, 16, size=(n_total, k_in), dtype=np.uint32)
    packed = np.zeros((n_total, k_in // 8), dtype=np.uint32)
    for j in range(8):
        packed |= codes[:, j::8] << np.uint32(4 * j)
    scales = rng.normal(0.0, 0.02, size=(n_total, k_in // 64)).astype(np.float16).view(np.uint16)
    biases = rng.normal(0.0, 0.02, size=(n_total, k_in // 64)).astype(np.float16).view(np.uint16)
    gq = bf16_words(rng.uniform(0.5, 1.5, shape.dim))
    gk = bf16_words(rng.uniform(0.5, 1.5, shape.dim))
    return shape, lengths, {"x": x, "w": packed, "s": scales, "b": biases,
                            "q_norm": gq, "k_norm": gk}


def weight4_set(rng: np.random.Generator, n: int, k: int, scale: float) -> tuple[NDArray, ...]:
    """weight4 words [n, k/8] with codes U{0..15}, bf16 group-64 scale s = U(0.5,1.5)*scale and
    bias -(7.5 + U(-0.5,0.5))*s, so weights are near zero-mean like an affine-quantized layer (the
    reference's bf16 storage, qwen3.py:70-73)."""
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    packed = np.zeros((n, k // 8), dtype=np.uint32)
    for j in range(8):
        packed |= codes[:, j::8] << np.uint32(4 * j)
    s = rng.uniform(0.5, 1.5, size=(n, k // 64)) * scale
    biases = bf16_words(-(7.5 + rng.uniform(-0.5, 0.5, size=s.shape)) * s)
    return packed, bf16_words(s), biases


def qwen_tail_16x256(layer: int, seed: int = 6) -> dict[str, Any]:
    """Qwen3-0.6B layer tail (qwen3.py:246-280) on 16*256 tokens, fp32 activations: residual x
    [4096, 1024] ~ N(0,1), attention output [4096, 2048] ~ N(0, 0.25), o_proj 2048->1024,
    gate/up 1024->3072, down 3072->1024 as weight4 with bf16 scale/bias, post-attention
    RMSNorm weight U(0.5,1.5) (bf16 words). One independent set per layer."""
    rng = np.random.default_rng((seed, layer))
    tokens, hidden, width, inter = 16 * 256, 1024, 2048, 3072
    return {
        "x": normal(rng, (tokens, hidden), np.float32),
        "attended": (0.5 * normal(rng, (tokens, width), np.float32)).astype(np.float32),
        "o": weight4_set(rng, hidden, width, 0.01),
        "gate": weight4_set(rng, inter, hidden, 0.01),
        "up": weight4_set(rng, inter, hidden, 0.01),
        "down": weight4_set(rng, hidden, inter, 0.01),
        "post_norm": bf16_words(rng.uniform(0.5, 1.5, hidden)),
    }


def tail_flop(tokens: int, hidden: int, width: int, inter: int) -> int:
    """2*T*K*N over the four projections of the layer tail (o, gate, up, down)."""
    return 2 * tokens * (width * hidden + 2 * hidden * inter + inter * hidden)


def qkv4_flop(rows: int, k: int, n_total: int) -> int:
    """2*M*K*N of the three projections."""
    return 2 * rows * k * n_total


def qkv4_bytes(rows: int, k: int, n_total: int) -> int:
    """x fp16 in, packed codes + fp16 scale/bias in, q/k/v fp16 out."""
    return rows * k * 2 + n_total * k // 2 + 2 * n_total * (k // 64) * 2 + rows * n_total * 2


# ---- algorithmic work (per layer) ----------------------------------------------------------


def pairs(shape: Shape, lengths: NDArray[np.uint32]) -> int:
    """Sum over rows and query positions of attended keys: causal n(p) = min(p+1, L),
    bidirectional n(p) = L; padded query rows count (they are outputs)."""
    total = 0
    for length in lengths.astype(np.int64).tolist():
        length = min(length, shape.seq)
        if shape.causal:
            total += length * (length + 1) // 2 + (shape.seq - length) * length
        else:
            total += shape.seq * length
    return total


def attention_flop(shape: Shape, lengths: NDArray[np.uint32]) -> int:
    """QK^T plus PV multiply-adds over attended pairs: 4 * D * H * pairs."""
    return 4 * shape.dim * shape.heads * pairs(shape, lengths)


def dense_flop(shape: Shape) -> int:
    """Dense convention 4*D*H*B*S^2, halved when causal (not mask-exact)."""
    full = 4 * shape.dim * shape.heads * shape.batch * shape.seq * shape.seq
    return full // 2 if shape.causal else full


def attention_bytes(
    shape: Shape, lengths: NDArray[np.uint32], in_bytes: int, out_bytes: int
) -> int:
    """Compulsory HBM traffic of one attention launch: every query row in, valid K/V rows in,
    every output row out, the lengths vector."""
    valid = int(np.minimum(lengths.astype(np.int64), shape.seq).sum())
    q = shape.batch * shape.seq * shape.heads * shape.dim * in_bytes
    kv = 2 * valid * shape.kv_heads * shape.dim * in_bytes
    o = shape.batch * shape.seq * shape.heads * shape.dim * out_bytes
    return q + kv + o + 4 * shape.batch


def k_prologue_bytes(shape: Shape, lengths: NDArray[np.uint32]) -> int:
    """Compulsory HBM traffic of the fused route's k prologue (norm_rope_f16 with hi + lo planes):
    valid k rows in as fp16, two fp16 planes out."""
    valid = int(np.minimum(lengths.astype(np.int64), shape.seq).sum())
    return valid * shape.kv_heads * shape.dim * (2 + 4)


# ---- synthetic weight packs (model.safetensors + config.json of the real model shapes) --------

QWEN3_0P6B = {"hidden": 1024, "intermediate": 3072, "layers": 28, "heads": 16, "kv_heads": 8,
              "head_dim": 128, "vocab": 151669}
BGE_SMALL = {"hidden": 384, "intermediate": 1536, "layers": 12, "heads": 12, "vocab": 30522,
             "positions": 512, "types": 2}


def qwen3_pack_tensors(seed: int, *, hidden: int, intermediate: int, layers: int, heads: int,
                       kv_heads: int, head_dim: int, vocab: int
                       ) -> tuple[dict[str, Any], dict[str, tuple[str, NDArray]]]:
    """A Qwen3 config and its uint4 tensors (names and shapes of qwen3.py:65-92). Projection
    scales 0.2/sqrt(inputs) keep the residual stream O(1) over many layers; embedding scale 0.2;
    RMSNorm weights U(0.5, 1.5)."""
    rng = np.random.default_rng(seed)
    tensors: dict[str, tuple[str, NDArray]] = {}

    def norm(prefix: str, dims: int) -> None:
        tensors[prefix + ".weight"] = ("BF16", bf16_words(rng.uniform(0.5, 1.5, dims)))

    def quant(prefix: str, outputs: int, inputs: int, scale: float) -> None:
        packed, s, b = weight4_set(rng, outputs, inputs, scale)
        tensors[prefix + ".weight"] = ("U32", packed)
        tensors[prefix + ".scales"] = ("BF16", s)
        tensors[prefix + ".biases"] = ("BF16", b)

    qw, kvw = heads * head_dim, kv_heads * head_dim
    quant("model.embed_tokens", vocab, hidden, 0.2)
    norm("model.norm", hidden)
    for layer in range(layers):
        p = f"model.layers.{layer}"
        norm(p + ".input_layernorm", hidden)
        norm(p + ".post_attention_layernorm", hidden)
        for name, outputs in (("q", qw), ("k", kvw), ("v", kvw)):
            quant(p + f".self_attn.{name}_proj", outputs, hidden, 0.2 / math.sqrt(hidden))
        quant(p + ".self_attn.o_proj", hidden, qw, 0.2 / math.sqrt(qw))
        norm(p + ".self_attn.q_norm", head_dim)
        norm(p + ".self_attn.k_norm", head_dim)
        quant(p + ".mlp.gate_proj", intermediate, hidden, 0.2 / math.sqrt(hidden))
        quant(p + ".mlp.up_proj", intermediate, hidden, 0.2 / math.sqrt(hidden))
        quant(p + ".mlp.down_proj", hidden, intermediate, 0.2 / math.sqrt(intermediate))
    config = {
        "model_type": "qwen3", "architectures": ["Qwen3ForCausalLM"], "hidden_size": hidden,
        "intermediate_size": intermediate, "num_hidden_layers": layers,
        "num_attention_heads": heads, "num_key_value_heads": kv_heads, "head_dim": head_dim,
        "vocab_size": vocab, "hidden_act": "silu", "attention_bias": False, "rope_scaling": None,
        "use_sliding_window": False, "quantization": {"bits": 4, "group_size": 64},
        "rms_norm_eps": EPS, "rope_theta": THETA, "max_position_embeddings": 32768,
        "tie_word_embeddings": True,
    }
    return config, tensors


def bert_pack_tensors(seed: int, *, hidden: int, intermediate: int, layers: int, heads: int,
                      vocab: int, positions: int, types: int, extras: bool = True
                      ) -> tuple[dict[str, Any], dict[str, tuple[str, NDArray]]]:
    """A BERT config and its fp32 tensors (names and shapes of bert.py:50-84), with the optional
    pooler and position_ids tensors when extras."""
    rng = np.random.default_rng(seed)
    tensors: dict[str, tuple[str, NDArray]] = {}

    def f32(shape: tuple[int, ...], std: float) -> tuple[str, NDArray]:
        return ("F32", (rng.standard_normal(shape) * std).astype(np.float32))

    def norm(prefix: str) -> None:
        tensors[prefix + ".weight"] = ("F32", rng.uniform(0.5, 1.5, hidden).astype(np.float32))
        tensors[prefix + ".bias"] = f32((hidden,), 0.1)

    def linear(prefix: str, outputs: int, inputs: int) -> None:
        tensors[prefix + ".weight"] = f32((outputs, inputs), 1.0 / math.sqrt(inputs))
        tensors[prefix + ".bias"] = f32((outputs,), 0.1)

    for name, rows in (("word", vocab), ("position", positions), ("token_type", types)):
        tensors[f"embeddings.{name}_embeddings.weight"] = f32((rows, hidden), 0.5)
    norm("embeddings.LayerNorm")
    for layer in range(layers):
        p = f"encoder.layer.{layer}"
        for name in ("query", "key", "value"):
            linear(p + ".attention.self." + name, hidden, hidden)
        linear(p + ".attention.output.dense", hidden, hidden)
        norm(p + ".attention.output.LayerNorm")
        linear(p + ".intermediate.dense", intermediate, hidden)
        linear(p + ".output.dense", hidden, intermediate)
        norm(p + ".output.LayerNorm")
    if extras:
        linear("pooler.dense", hidden, hidden)
        tensors["embeddings.position_ids"] = ("I64", np.arange(positions, dtype=np.int64)[None])
    config = {
        "model_type": "bert", "architectures": ["BertModel"], "hidden_size": hidden,
        "intermediate_size": intermediate, "num_hidden_layers": layers,
        "num_attention_heads": heads, "vocab_size": vocab, "max_position_embeddings": positions,
        "type_vocab_size": types, "hidden_act": "gelu", "layer_norm_eps": 1e-12,
        "position_embedding_type": "absolute",
    }
    return config, tensors


def write_pack(directory: str, config: dict[str, Any], tensors: dict[str, tuple[str, NDArray]],
               *, architecture: str, max_length: int, min_dimensions: int | None = None):
    """Write config.json and model.safetensors into directory; returns the ModelProfile that pins
    both files (sizes and sha256)."""
    import json
    import os

    from .packs import ModelProfile
    from .weights import artifact_of, encode_safetensors

    config_bytes = json.dumps(config).encode()
    model_bytes = encode_safetensors(tensors)
    for name, data in (("config.json", config_bytes), ("model.safetensors", model_bytes)):
        with open(os.path.join(directory, name), "wb") as f:
            f.write(data)
    hidden = int(config["hidden_size"])
    return ModelProfile(
        architecture=architecture, native_dimensions=hidden,
        min_dimensions=hidden if min_dimensions is None else min_dimensions,
        max_length=max_length,
        artifacts=(artifact_of("config.json", "config.json", config_bytes),
                   artifact_of("model.safetensors", "model.safetensors", model_bytes)))


def weights_of(tensors: dict[str, tuple[str, NDArray]]) -> dict[str, NDArray]:
    return {name: array for name, (_, array) in tensors.items()}
