"""float64 attention oracle.

Formulation of tessery's own CPU oracle (tests/real_metal/test_kernels.py:198-209): for each
(batch row b, head h): scores = q[b,:,h] @ k[b,:L,kv(h)]^T * scale, causal entries with
key > query position set to -inf, max-subtracted softmax over keys, probabilities @ v[b,:L,kv(h)].
Semantics it encodes (kernels.metal:76-103, 105-170):
  kv(h) = h // (H // KV)
  causal: query p attends keys [0, min(p+1, L)); bidirectional: [0, L)
  padded query rows p >= L are outputs and attend all L valid keys
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray


def attention(
    q: NDArray,
    k: NDArray,
    v: NDArray,
    lengths: NDArray,
    *,
    bidirectional: bool,
    scale: float | None = None,
    dtype: type = np.float64,
) -> NDArray:
    """q [B,S,H,D], k/v [B,S,KV,D], lengths [B] -> out [B,S,H,D] in `dtype` (float64, the
    reference formulation; float32 only as a timing variant of the CPU baseline)."""
    batch, seq, heads, dim = q.shape
    kv_heads = k.shape[2]
    if heads % kv_heads:
        raise ValueError("heads must be a multiple of kv_heads")
    group = heads // kv_heads
    scale = dim**-0.5 if scale is None else scale
    out = np.empty(q.shape, dtype=dtype)
    positions = np.arange(seq)[:, None]
    for b in range(batch):
        length = min(int(lengths[b]), seq)
        keys = np.arange(length)[None, :]
        for h in range(heads):
            kh = h // group
            scores = q[b, :, h].astype(dtype) @ k[b, :length, kh].astype(dtype).T
            scores *= dtype(scale)
            if not bidirectional:
                scores[keys > positions] = -np.inf
            probs = np.exp(scores - scores.max(axis=1, keepdims=True))
            probs /= probs.sum(axis=1, keepdims=True)
            out[b, :, h] = probs @ v[b, :length, kh].astype(dtype)
    return out


def attention_online(
    q: NDArray, k: NDArray, v: NDArray, lengths: NDArray, *, bidirectional: bool
) -> NDArray[np.float64]:
    """Scalar online-softmax loop per (token, head), the order of kernels.metal:76-103.
    Pure Python; for tiny shapes only (cross-checks attention())."""
    batch, seq, heads, dim = q.shape
    group = heads // k.shape[2]
    scale = dim**-0.5
    out = np.zeros(q.shape, dtype=np.float64)
    for b in range(batch):
        length = min(int(lengths[b]), seq)
        for pos in range(seq):
            end = length if bidirectional else min(pos + 1, length)
            for h in range(heads):
                kh = h // group
                maximum, denominator = -np.inf, 0.0
                acc = np.zeros(dim, dtype=np.float64)
                for key in range(end):
                    score = float(np.dot(q[b, pos, h].astype(np.float64), k[b, key, kh])) * scale
                    nxt = max(maximum, score)
                    correction = np.exp(maximum - nxt) if maximum > -np.inf else 0.0
                    prob = np.exp(score - nxt)
                    denominator = denominator * correction + prob
                    acc = acc * correction + prob * v[b, key, kh].astype(np.float64)
                    maximum = nxt
                out[b, pos, h] = acc / denominator
    return out
