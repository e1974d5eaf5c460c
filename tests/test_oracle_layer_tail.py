"""Pins the float64 Qwen3 layer-tail oracle (qwen3.py:246-280): o_proj -> residual ->
post-attention RMSNorm -> gate/up + SiLU -> down_proj -> residual, against torch's rms_norm and
transformers' Qwen3MLP with the dequantized weights, plus a planted-mistake check."""

from types import SimpleNamespace

import numpy as np
import pytest

from oracle import qwen_block
from oracle import quant4 as q4
from tessery_amd.workloads import bf16_words

torch = pytest.importorskip("torch")
qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")


def weight_set(rng, n, k):
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    return (q4.pack(codes), bf16_words(rng.uniform(0.005, 0.05, size=(n, k // 64))),
            bf16_words(rng.uniform(-0.2, 0.0, size=(n, k // 64))))


def test_layer_tail_matches_transformers_modules():
    rng = np.random.default_rng(47)
    tokens, hidden, attn_width, inter, eps = 6, 128, 256, 192, 1e-6
    x = rng.normal(size=(tokens, hidden))
    attended = rng.normal(size=(tokens, attn_width))
    w = {"o": weight_set(rng, hidden, attn_width), "gate": weight_set(rng, inter, hidden),
         "up": weight_set(rng, inter, hidden), "down": weight_set(rng, hidden, inter)}
    gamma = rng.uniform(0.5, 1.5, hidden)
    ours = qwen_block.layer_tail(x, attended, w, gamma, eps=eps)

    cfg = SimpleNamespace(hidden_size=hidden, intermediate_size=inter, hidden_act="silu")
    mlp = qwen3.Qwen3MLP(cfg).double()
    dense = {name: torch.from_numpy(q4.dequantize(*w[name], w[name][0].shape[1] * 8)) for name in w}
    with torch.no_grad():
        mlp.gate_proj.weight.copy_(dense["gate"])
        mlp.up_proj.weight.copy_(dense["up"])
        mlp.down_proj.weight.copy_(dense["down"])
        h = torch.from_numpy(x) + torch.from_numpy(attended) @ dense["o"].T
        normed = torch.nn.functional.rms_norm(h, (hidden,), torch.from_numpy(gamma), eps=eps)
        theirs = (h + mlp(normed)).numpy()
    np.testing.assert_allclose(ours, theirs, rtol=1e-12, atol=1e-12)

    # a planted mistake (the MLP reading the residual stream before the norm) is caught
    bad = x + q4.linear4(attended, *w["o"])
    bad = bad + q4.linear4(q4.gated4(bad, w["gate"], w["up"]), *w["down"])
    assert np.abs(bad - theirs).max() > 1e-3
