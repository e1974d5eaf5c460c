"""float64 whole-model forwards of tessery's two embedding models, composed from the layer
oracles: the token embeddings, every layer, and the pooled unit vector.

- qwen3_forward follows Qwen3Backend.forward (qwen3.py:112-296): embedding4, per layer
  RMSNorm -> q/k/v uint4 projections -> per-head q/k RMSNorm -> RoPE -> causal GQA attention ->
  layer tail, final RMSNorm, last-token pooling (pool_project, kernels.metal:339-349).
- bert_forward follows BertBackend.forward (bert.py:103-251): embedding_position
  (kernels.metal:351-360) -> LayerNorm, the BERT layers, CLS pooling.

Weights are the numpy arrays of a tessery weight pack, keyed by their SafeTensors names (uint32
words and bf16 words as uint16 for Qwen3, float32 for BERT).
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from . import bert_block as _bert
from . import norm_rope as _norm_rope
from . import quant4 as _quant4
from . import qwen_block as _qwen


def bf16_values(words: NDArray) -> NDArray[np.float64]:
    return (np.asarray(words, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)


def embedding4(ids: NDArray, packed: NDArray, scales: NDArray, biases: NDArray) -> NDArray[np.float64]:
    """Rows ids of the uint4 affine table (kernels.metal:21-30): weight4(table, id, c)."""
    ids = np.asarray(ids).reshape(-1)
    cols = packed.shape[1] * 8
    return _quant4.dequantize(packed[ids], scales[ids], biases[ids], cols)


def embedding_position(ids: NDArray, words: NDArray, positions: NDArray, types: NDArray
                       ) -> NDArray[np.float64]:
    """ids [B, S] -> [B*S, hidden]: (words[id] + types[0]) + positions[s]."""
    batch, seq = ids.shape
    w = np.asarray(words, np.float64)[np.asarray(ids).reshape(-1)]
    p = np.tile(np.asarray(positions, np.float64)[:seq], (batch, 1))
    return (w + np.asarray(types, np.float64)[0]) + p


def pool_project(x: NDArray, lengths: NDArray, dim: int, *, first: bool) -> NDArray[np.float64]:
    """x [B, S, hidden] -> [B, dim]: the first (CLS) or last valid token's first dim columns,
    scaled to unit length."""
    x = np.asarray(x, np.float64)
    rows = np.zeros(x.shape[0], dtype=np.int64) if first else np.asarray(lengths, np.int64) - 1
    picked = x[np.arange(x.shape[0]), rows, :dim]
    return picked / np.linalg.norm(picked, axis=1, keepdims=True)


def _quant(w: dict[str, NDArray], prefix: str) -> tuple[NDArray, NDArray, NDArray]:
    return w[prefix + ".weight"], w[prefix + ".scales"], w[prefix + ".biases"]


def qwen3_forward(w: dict[str, NDArray], ids: NDArray, lengths: NDArray, *, layers: int,
                  heads: int, kv_heads: int, head_dim: int, eps: float, theta: float,
                  dimensions: int, return_hidden: bool = False):
    batch, seq = ids.shape
    x = embedding4(ids, *_quant(w, "model.embed_tokens"))
    for layer in range(layers):
        prefix = f"model.layers.{layer}"
        attn = prefix + ".self_attn"
        normalized = _norm_rope.rms_norm(x, bf16_values(w[prefix + ".input_layernorm.weight"]), eps)
        q = _quant4.linear4(normalized, *_quant(w, attn + ".q_proj"))
        k = _quant4.linear4(normalized, *_quant(w, attn + ".k_proj"))
        v = _quant4.linear4(normalized, *_quant(w, attn + ".v_proj"))
        attended = _qwen.norm_rope_attention(
            q.reshape(batch, seq, heads, head_dim), k.reshape(batch, seq, kv_heads, head_dim),
            v.reshape(batch, seq, kv_heads, head_dim), lengths,
            bf16_values(w[attn + ".q_norm.weight"]), bf16_values(w[attn + ".k_norm.weight"]),
            eps=eps, theta=theta)
        tail = {name: _quant(w, p) for name, p in (
            ("o", attn + ".o_proj"), ("gate", prefix + ".mlp.gate_proj"),
            ("up", prefix + ".mlp.up_proj"), ("down", prefix + ".mlp.down_proj"))}
        x = _qwen.layer_tail(x, attended.reshape(batch * seq, heads * head_dim), tail,
                             bf16_values(w[prefix + ".post_attention_layernorm.weight"]), eps=eps)
    hidden = _norm_rope.rms_norm(x, bf16_values(w["model.norm.weight"]), eps)
    pooled = pool_project(hidden.reshape(batch, seq, -1), lengths, dimensions, first=False)
    return (pooled, hidden) if return_hidden else pooled


def bert_forward(w: dict[str, NDArray], ids: NDArray, lengths: NDArray, *, layers: int,
                 heads: int, eps: float, return_hidden: bool = False):
    batch, seq = ids.shape
    x = embedding_position(ids, w["embeddings.word_embeddings.weight"],
                           w["embeddings.position_embeddings.weight"],
                           w["embeddings.token_type_embeddings.weight"])
    x = _bert.layer_norm(x, w["embeddings.LayerNorm.weight"], w["embeddings.LayerNorm.bias"], eps)
    x = x.reshape(batch, seq, -1)
    for layer in range(layers):
        p = f"encoder.layer.{layer}"
        lw = {
            "q": w[p + ".attention.self.query.weight"], "q_b": w[p + ".attention.self.query.bias"],
            "k": w[p + ".attention.self.key.weight"], "k_b": w[p + ".attention.self.key.bias"],
            "v": w[p + ".attention.self.value.weight"], "v_b": w[p + ".attention.self.value.bias"],
            "o": w[p + ".attention.output.dense.weight"],
            "o_b": w[p + ".attention.output.dense.bias"],
            "ln1_w": w[p + ".attention.output.LayerNorm.weight"],
            "ln1_b": w[p + ".attention.output.LayerNorm.bias"],
            "i": w[p + ".intermediate.dense.weight"], "i_b": w[p + ".intermediate.dense.bias"],
            "out": w[p + ".output.dense.weight"], "out_b": w[p + ".output.dense.bias"],
            "ln2_w": w[p + ".output.LayerNorm.weight"], "ln2_b": w[p + ".output.LayerNorm.bias"],
        }
        x = _bert.layer(x, lengths, lw, heads=heads, eps=eps)
    pooled = pool_project(x, lengths, x.shape[-1], first=True)
    return (pooled, x) if return_hidden else pooled
