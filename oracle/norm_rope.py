"""float64 per-head RMSNorm and rotary position embedding.

rms_norm: y = x / sqrt(mean(x^2) + eps) * w           (kernels.metal:53-63; closed form of
                                                        test_kernels.py:109)
rope:     split-half pairs (c, c + D/2), angle = pos * theta^(-2c/D),
          x_c' = x_c cos - x_{c+D/2} sin, x_{c+D/2}' = x_c sin + x_{c+D/2} cos
                                                       (kernels.metal:65-74; test_kernels.py:273-283)
Positions are the token's index within its padded row, so padded tokens get positions too.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray


def rms_norm(x: NDArray, weight: NDArray, eps: float, dtype: type = np.float64) -> NDArray:
    x = np.asarray(x, dtype=dtype)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + dtype(eps))
    return x * inv * np.asarray(weight, dtype=dtype)


def rope_angles(seq: int, dim: int, theta: float) -> NDArray[np.float64]:
    """[seq, dim/2] angles pos * theta^(-2c/dim)."""
    inv_freq = float(theta) ** (-2.0 * np.arange(dim // 2, dtype=np.float64) / dim)
    return np.arange(seq, dtype=np.float64)[:, None] * inv_freq[None, :]


def rope(x: NDArray, theta: float, dtype: type = np.float64) -> NDArray:
    """x [B, S, heads, D] (position = axis 1) -> rotated, in `dtype` (angles in float64)."""
    x = np.asarray(x, dtype=dtype)
    seq, dim = x.shape[1], x.shape[-1]
    half = dim // 2
    angles = rope_angles(seq, dim, theta)[None, :, None, :]
    cos, sin = np.cos(angles).astype(dtype), np.sin(angles).astype(dtype)
    a, b = x[..., :half], x[..., half:]
    return np.concatenate((a * cos - b * sin, a * sin + b * cos), axis=-1)


def norm_rope(x: NDArray, weight: NDArray, eps: float, theta: float,
              dtype: type = np.float64) -> NDArray:
    """Qwen3 order (qwen3.py:216-237): RMSNorm over D, then RoPE."""
    return rope(rms_norm(x, weight, eps, dtype), theta, dtype)
