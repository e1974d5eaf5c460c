"""uint4 affine group-64 weights: packing, dequantization, projection (float64).

Format (kernels.metal:11-19, weight4): packed u32[N, K/8]; code of column k in row n is nibble
k % 8 of word k // 8, little-nibble first; group = k // 64; w = code * scale[n, g] + bias[n, g].
tessery stores scale/bias as bfloat16 words [N, K/64] (qwen3.py:70-73); the fp16 variant stores
float16 words of the same shape.
"""

from __future__ import annotations

import numpy as np
from numpy.typing import NDArray


def pack(codes: NDArray) -> NDArray[np.uint32]:
    """codes [N, K] in 0..15 -> packed [N, K/8] (layout of test_kernels.py:57-59)."""
    codes = np.asarray(codes, dtype=np.uint32)
    n, k = codes.shape
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    return np.bitwise_or.reduce(codes.reshape(n, k // 8, 8) << shifts, axis=-1).astype(np.uint32)


def unpack(packed: NDArray, k: int) -> NDArray[np.uint32]:
    packed = np.asarray(packed, dtype=np.uint32)
    shifts = np.arange(0, 32, 4, dtype=np.uint32)
    return ((packed[..., None] >> shifts) & 15).reshape(packed.shape[0], k)


def decode_words(words: NDArray, kind: str) -> NDArray[np.float64]:
    """bf16 or fp16 storage words -> float64 values."""
    words = np.asarray(words, dtype=np.uint16)
    if kind == "bf16":
        return (words.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    if kind == "f16":
        return words.view(np.float16).astype(np.float64)
    raise ValueError(kind)


def dequantize(packed: NDArray, scales: NDArray, biases: NDArray, k: int, kind: str = "bf16"):
    codes = unpack(packed, k).astype(np.float64)
    s = decode_words(scales, kind).repeat(64, axis=1)
    b = decode_words(biases, kind).repeat(64, axis=1)
    return codes * s + b


def linear4(x: NDArray, packed: NDArray, scales: NDArray, biases: NDArray, kind: str = "bf16"):
    """y = x @ dequant(W)^T in float64; x [M, K]."""
    k = x.shape[-1]
    return np.asarray(x, dtype=np.float64) @ dequantize(packed, scales, biases, k, kind).T


def weight4_scalar(packed: NDArray, scales: NDArray, biases: NDArray, row: int, col: int,
                   k: int, kind: str = "bf16") -> float:
    """One weight by the kernel's own indexing: word row*(k/8) + col/8, shift 4*(col%8),
    group row*(k/64) + col/64 over the flattened arrays (kernels.metal:11-19)."""
    flat = np.asarray(packed, dtype=np.uint32).reshape(-1)
    code = (int(flat[row * (k // 8) + col // 8]) >> (4 * (col % 8))) & 15
    g = row * (k >> 6) + (col >> 6)
    s = decode_words(np.asarray(scales).reshape(-1)[g : g + 1], kind)[0]
    b = decode_words(np.asarray(biases).reshape(-1)[g : g + 1], kind)[0]
    return code * s + b


def silu_gate(gate: NDArray, up: NDArray) -> NDArray[np.float64]:
    """silu(gate) * up = gate / (1 + exp(-gate)) * up (kernels.metal:334-337), float64."""
    g = np.asarray(gate, dtype=np.float64)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * np.asarray(up, dtype=np.float64)


def gated4(x: NDArray, gate: tuple[NDArray, NDArray, NDArray], up: tuple[NDArray, NDArray, NDArray],
           kind: str = "bf16") -> NDArray[np.float64]:
    """silu(x @ Wg^T) * (x @ Wu^T) with (packed, scales, biases) weight sets (metal.py:501-530,
    kernels.metal:609-656)."""
    return silu_gate(linear4(x, *gate, kind=kind), linear4(x, *up, kind=kind))

