"""float64 composition of tessery's Qwen3 layer (qwen3.py:194-280): the attention block
(QKV projection -> per-head q/k RMSNorm -> RoPE -> causal GQA attention) and the layer tail after
it (o_proj -> residual -> post-attention RMSNorm -> gate/up + SiLU -> down_proj -> residual).
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray

from . import attention as _attention
from . import norm_rope as _norm_rope
from . import quant4 as _quant4


def norm_rope_attention(
    q_pre: NDArray,
    k_pre: NDArray,
    v: NDArray,
    lengths: NDArray,
    q_norm: NDArray,
    k_norm: NDArray,
    *,
    eps: float,
    theta: float,
    bidirectional: bool = False,
) -> NDArray[np.float64]:
    """q_pre [B,S,H,D], k_pre/v [B,S,KV,D]; norm weights as float values [D]."""
    q = _norm_rope.norm_rope(q_pre, q_norm, eps, theta)
    k = _norm_rope.norm_rope(k_pre, k_norm, eps, theta)
    return _attention.attention(q, k, v, lengths, bidirectional=bidirectional)


def qkv4(x: NDArray, weights: dict[str, tuple[NDArray, NDArray, NDArray]], kind: str):
    """x [M, K]; weights name -> (packed, scales, biases) for "q", "k", "v"."""
    return {name: _quant4.linear4(x, *weights[name], kind=kind) for name in ("q", "k", "v")}


def layer_tail(x: NDArray, attended: NDArray, weights: dict[str, tuple[NDArray, NDArray, NDArray]],
               post_norm: NDArray, *, eps: float, kind: str = "bf16") -> NDArray[np.float64]:
    """Residual stream after one layer (qwen3.py:246-280). x [T, hidden] is the residual input,
    attended [T, heads * dim] the attention output; weights name -> (packed, scales, biases) for
    "o", "gate", "up", "down"; post_norm the post-attention RMSNorm weight as float values."""
    h = np.asarray(x, dtype=np.float64) + _quant4.linear4(attended, *weights["o"], kind=kind)
    normalized = _norm_rope.rms_norm(h, post_norm, eps)
    mlp = _quant4.gated4(normalized, weights["gate"], weights["up"], kind=kind)
    return h + _quant4.linear4(mlp, *weights["down"], kind=kind)

