"""Pins the uint4 oracle with tessery's known answers and the kernel's own indexing."""

import numpy as np
import pytest

from oracle import quant4 as ref
from tessery_amd.workloads import bf16_words


def test_nibble_order_known_word():
    # column j of a group of eight sits in nibble j, little-nibble first
    codes = ref.unpack(np.array([[0x76543210, 0xFEDCBA98]], np.uint32), 16)
    np.testing.assert_array_equal(codes[0], np.arange(16))
    np.testing.assert_array_equal(ref.pack(codes), [[0x76543210, 0xFEDCBA98]])


def test_known_answer_scale_and_bias():
    """tessery test_kernels.py:55-81: scale 0.125, bias -0.5 -> code * 0.125 - 0.5."""
    rng = np.random.default_rng(1)
    code = rng.integers(0, 16, size=(8, 128), dtype=np.uint32)
    packed = ref.pack(code)
    scales = bf16_words(np.full((8, 2), 0.125))
    biases = bf16_words(np.full((8, 2), -0.5))
    np.testing.assert_array_equal(ref.dequantize(packed, scales, biases, 128), code * 0.125 - 0.5)


def test_all_ones_tile_known_answer():
    """tessery test_kernels.py:759-776: ones x words 0x11111111, scale 1, bias 0 -> 64."""
    x = np.ones((8, 64))
    packed = np.full((32, 8), 0x11111111, np.uint32)
    y = ref.linear4(x, packed, bf16_words(np.ones((32, 1))), bf16_words(np.zeros((32, 1))))
    np.testing.assert_array_equal(y, 64.0)


@pytest.mark.parametrize("kind", ["bf16", "f16"])
def test_dequantize_matches_scalar_kernel_indexing(kind):
    rng = np.random.default_rng(417)
    n, k = 5, 192
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    packed = ref.pack(codes)
    if kind == "bf16":
        scales = bf16_words(rng.uniform(0.01, 0.2, size=(n, k // 64)))
        biases = bf16_words(rng.uniform(-1, 0.1, size=(n, k // 64)))
    else:
        scales = rng.normal(0, 0.02, size=(n, k // 64)).astype(np.float16).view(np.uint16)
        biases = rng.normal(0, 0.02, size=(n, k // 64)).astype(np.float16).view(np.uint16)
    dense = ref.dequantize(packed, scales, biases, k, kind)
    for row in range(n):
        for col in (0, 7, 8, 63, 64, 65, 127, 128, 191):
            assert dense[row, col] == ref.weight4_scalar(packed, scales, biases, row, col, k, kind)
    x = rng.normal(size=(3, k))
    brute = np.array([[sum(x[t, c] * dense[r, c] for c in range(k)) for r in range(n)] for t in range(3)])
    np.testing.assert_allclose(ref.linear4(x, packed, scales, biases, kind), brute, atol=1e-12)


def test_silu_gate_against_torch_and_known_answers():
    """silu_gate (kernels.metal:334-337) against torch.nn.functional.silu in float64, and the
    known answers of tessery's gated tests (test_kernels.py:286-294, 842-857)."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(29)
    g = np.concatenate([rng.normal(scale=4.0, size=500), [0.0, -0.0, 88.0, -88.0, -1000.0, 1000.0]])
    u = rng.normal(size=g.shape)
    expected = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    np.testing.assert_allclose(ref.silu_gate(g, u), expected, rtol=1e-15, atol=1e-300)
    assert ref.silu_gate(np.array([64.0]), np.array([64.0]))[0] == 64.0 / (1 + np.exp(-64.0)) * 64.0
    assert ref.silu_gate(np.array([0.0]), np.array([5.0]))[0] == 0.0


def test_gated4_is_silu_of_gate_times_up_and_matches_qwen3_mlp():
    """gated4 = silu(x Wg^T) * (x Wu^T); with a dense down projection it is transformers'
    Qwen3MLP (the op order of qwen3.py:260-277) in float64."""
    torch = pytest.importorskip("torch")
    qwen3 = pytest.importorskip("transformers.models.qwen3.modeling_qwen3")
    rng = np.random.default_rng(31)
    m, hidden, inter = 5, 128, 192
    x = rng.normal(size=(m, hidden))
    sets = {}
    for name, (n, k) in {"gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}.items():
        codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
        sets[name] = (ref.pack(codes), bf16_words(rng.uniform(0.01, 0.1, size=(n, k // 64))),
                      bf16_words(rng.uniform(-0.5, 0.0, size=(n, k // 64))))
    mlp = ref.gated4(x, sets["gate"], sets["up"])
    np.testing.assert_array_equal(
        mlp, ref.silu_gate(ref.linear4(x, *sets["gate"]), ref.linear4(x, *sets["up"])))
    ours = ref.linear4(mlp, *sets["down"])

    from types import SimpleNamespace
    cfg = SimpleNamespace(hidden_size=hidden, intermediate_size=inter, hidden_act="silu")
    module = qwen3.Qwen3MLP(cfg).double()
    with torch.no_grad():
        for name, proj in (("gate", module.gate_proj), ("up", module.up_proj), ("down", module.down_proj)):
            n, k = proj.weight.shape
            proj.weight.copy_(torch.from_numpy(ref.dequantize(*sets[name], k)))
        theirs = module(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(ours, theirs, rtol=1e-12, atol=1e-12)
