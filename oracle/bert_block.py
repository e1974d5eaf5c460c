"""float64 restatement of tessery's BERT (BGE) encoder layer (bert.py:186-230).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

linear:     y = x @ W^T + b, W [N, K] (matmul_bias_f32, kernels.metal:438-487; metal.py:702-731)
gelu:       erf form x * (1 + erf(x / sqrt 2)) / 2 (gelu_f32, kernels.metal:381-394, which
            approximates erf by Abramowitz & Stegun 7.1.26; this oracle uses the exact erf)
layer_norm: (x - mean) / sqrt(var + eps) * w + b over the last axis (kernels.metal:362-374)
layer:      q, k, v = linear(x) -> bidirectional attention with the key-padding mask ->
            x = layer_norm(x + linear(attended)) -> x = layer_norm(x + linear(gelu(linear(x))))
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray
from scipy.special import erf

from . import attention as _attention


def linear(x: NDArray, weight: NDArray, bias: NDArray | None = None) -> NDArray[np.float64]:
    y = np.asarray(x, dtype=np.float64) @ np.asarray(weight, dtype=np.float64).T
    return y if bias is None else y + np.asarray(bias, dtype=np.float64)


def gelu(x: NDArray) -> NDArray[np.float64]:
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))


def layer_norm(x: NDArray, weight: NDArray, bias: NDArray, eps: float) -> NDArray[np.float64]:
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * np.asarray(weight, np.float64) + np.asarray(bias, np.float64)


def layer(x: NDArray, lengths: NDArray, w: dict[str, NDArray], *, heads: int,
          eps: float) -> NDArray[np.float64]:
    """x [B, S, hidden]; w holds "q", "k", "v", "o", "i", "out" weights [N, K] and "<name>_b"
    biases, "ln1_w", "ln1_b", "ln2_w", "ln2_b". Returns the layer output [B, S, hidden]."""
    b, s, hidden = x.shape
    d = hidden // heads
    x2 = np.asarray(x, dtype=np.float64).reshape(b * s, hidden)
    q, k, v = (linear(x2, w[n], w[n + "_b"]).reshape(b, s, heads, d) for n in ("q", "k", "v"))
    attended = _attention.attention(q, k, v, lengths, bidirectional=True).reshape(b * s, hidden)
    h = layer_norm(x2 + linear(attended, w["o"], w["o_b"]), w["ln1_w"], w["ln1_b"], eps)
    inner = gelu(linear(h, w["i"], w["i_b"]))
    out = layer_norm(h + linear(inner, w["out"], w["out_b"]), w["ln2_w"], w["ln2_b"], eps)
    return out.reshape(b, s, hidden)
