"""Pins the float64 BERT-layer oracle (bert.py:186-230) against torch's gelu / layer_norm and
transformers' BertLayer in float64 with a key-padding mask, plus a planted-mistake check."""

import math

import numpy as np
import pytest

from oracle import bert_block as ref

torch = pytest.importorskip("torch")
modeling_bert = pytest.importorskip("transformers.models.bert.modeling_bert")
BertConfig = pytest.importorskip("transformers").BertConfig


def test_gelu_and_layer_norm_against_torch():
    x = np.linspace(-12, 12, 2001)
    np.testing.assert_allclose(ref.gelu(x), torch.nn.functional.gelu(torch.from_numpy(x)).numpy(),
                               rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(ref.gelu(x), [0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x],
                               rtol=1e-12, atol=1e-15)
    rng = np.random.default_rng(37)
    y = rng.normal(size=(3, 67))
    w, b = rng.normal(size=67), rng.normal(size=67)
    expected = torch.nn.functional.layer_norm(torch.from_numpy(y), (67,), torch.from_numpy(w),
                                              torch.from_numpy(b), eps=1e-12).numpy()
    np.testing.assert_allclose(ref.layer_norm(y, w, b, 1e-12), expected, rtol=1e-12, atol=1e-12)


def test_bert_layer_matches_transformers():
    rng = np.random.default_rng(53)
    batch, seq, hidden, heads, inter, eps = 2, 9, 48, 4, 96, 1e-12
    lengths = np.array([9, 4], np.uint32)
    x = rng.normal(size=(batch, seq, hidden))
    w = {}
    for name, (n, k) in {"q": (hidden, hidden), "k": (hidden, hidden), "v": (hidden, hidden),
                         "o": (hidden, hidden), "i": (inter, hidden), "out": (hidden, inter)}.items():
        w[name] = rng.normal(scale=k ** -0.5, size=(n, k))
        w[name + "_b"] = rng.normal(scale=0.1, size=n)
    for ln in ("ln1", "ln2"):
        w[ln + "_w"], w[ln + "_b"] = rng.uniform(0.5, 1.5, hidden), rng.normal(scale=0.1, size=hidden)
    ours = ref.layer(x, lengths, w, heads=heads, eps=eps)

    cfg = BertConfig(hidden_size=hidden, num_attention_heads=heads, intermediate_size=inter,
                     hidden_act="gelu", layer_norm_eps=eps, attn_implementation="eager",
                     hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)
    layer = modeling_bert.BertLayer(cfg).double().eval()
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    with torch.no_grad():
        sa, so = layer.attention.self, layer.attention.output
        for mod, name in ((sa.query, "q"), (sa.key, "k"), (sa.value, "v"), (so.dense, "o"),
                          (layer.intermediate.dense, "i"), (layer.output.dense, "out")):
            mod.weight.copy_(t(w[name]))
            mod.bias.copy_(t(w[name + "_b"]))
        so.LayerNorm.weight.copy_(t(w["ln1_w"]))
        so.LayerNorm.bias.copy_(t(w["ln1_b"]))
        layer.output.LayerNorm.weight.copy_(t(w["ln2_w"]))
        layer.output.LayerNorm.bias.copy_(t(w["ln2_b"]))
        keep = np.arange(seq)[None, :] < lengths[:, None]
        mask = torch.from_numpy(np.where(keep, 0.0, np.finfo(np.float64).min))[:, None, None, :]
        out = layer(t(x), attention_mask=mask)
        theirs = (out[0] if isinstance(out, tuple) else out).numpy()
    np.testing.assert_allclose(ours, theirs, rtol=1e-10, atol=1e-10)

    # a planted mistake (the residual skipped before the first LayerNorm) is caught
    bad = dict(w)
    bad["o"] = w["o"] + np.eye(hidden)
    assert np.abs(ref.layer(x, lengths, bad, heads=heads, eps=eps) - theirs).max() > 1e-3
