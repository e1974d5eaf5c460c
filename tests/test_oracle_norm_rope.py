"""Pins the RMSNorm / RoPE oracle against torch, transformers' Qwen3 modules, a complex-number
rotation and rotation invariants."""

import numpy as np
import torch
import torch.nn.functional as F
from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm, apply_rotary_pos_emb

from oracle import norm_rope as ref


def test_rms_norm_matches_torch():
    rng = np.random.default_rng(4)
    x = rng.normal(size=(2, 3, 64))
    w = rng.uniform(0.5, 1.5, 64)
    expected = F.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(ref.rms_norm(x, w, 1e-6), expected, atol=1e-13)


def test_rms_norm_matches_qwen3_module():
    rng = np.random.default_rng(6)
    x = rng.normal(size=(5, 128)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    module = Qwen3RMSNorm(128, eps=1e-6)
    with torch.no_grad():
        module.weight.copy_(torch.from_numpy(w))
        expected = module(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(ref.rms_norm(x, w, 1e-6), expected, atol=2e-6, rtol=2e-6)


def test_rope_matches_complex_rotation():
    rng = np.random.default_rng(8)
    x = rng.normal(size=(2, 3, 4, 64))
    got = ref.rope(x, 10000.0)
    angles = np.arange(3)[None, :, None, None] * 10000.0 ** (-2 * np.arange(32) / 64)
    z = (x[..., :32] + 1j * x[..., 32:]) * np.exp(1j * angles)
    np.testing.assert_allclose(got, np.concatenate((z.real, z.imag), axis=-1), atol=1e-13)


def test_rope_matches_qwen3_apply_rotary():
    rng = np.random.default_rng(10)
    b, s, h, d = 2, 37, 3, 128
    x = rng.normal(size=(b, s, h, d))
    inv_freq = 1.0 / (1e6 ** (np.arange(0, d, 2, dtype=np.float64) / d))
    freqs = np.arange(s, dtype=np.float64)[:, None] * inv_freq[None, :]
    emb = np.concatenate((freqs, freqs), axis=-1)
    cos = torch.from_numpy(np.cos(emb))[None]
    sin = torch.from_numpy(np.sin(emb))[None]
    tx = torch.from_numpy(x).transpose(1, 2)  # [b, h, s, d]
    rq, _ = apply_rotary_pos_emb(tx, tx, cos, sin)
    np.testing.assert_allclose(ref.rope(x, 1e6), rq.transpose(1, 2).numpy(), atol=1e-12)


def test_rope_invariants():
    rng = np.random.default_rng(12)
    x = rng.normal(size=(1, 9, 2, 32))
    y = ref.rope(x, 1e6)
    # position 0 is the identity
    np.testing.assert_allclose(y[:, 0], x[:, 0], atol=0)
    # each (c, c + D/2) pair keeps its length
    pair = lambda t: t[..., :16] ** 2 + t[..., 16:] ** 2  # noqa: E731
    np.testing.assert_allclose(pair(y), pair(x), atol=1e-12)
    # q.k after rotation depends only on the position difference
    a = ref.rope(np.repeat(x[:, :1], 9, axis=1), 1e6)
    dots = np.einsum("d,d->", a[0, 2, 0], a[0, 5, 0]), np.einsum("d,d->", a[0, 4, 0], a[0, 7, 0])
    np.testing.assert_allclose(dots[0], dots[1], atol=1e-12)
