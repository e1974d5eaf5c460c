"""Pins of the whole-model oracle (oracle/models.py): the embedding gathers against the scalar
weight4 indexing of kernels.metal:11-19 and :351-360, pooling against its definition, and both
forwards against transformers' Qwen3Model and BertModel run in float64 on the same weights
(dequantized for Qwen3), with planted mistakes that the pins must catch."""

import numpy as np
import pytest
import torch

from oracle import models as ref
from oracle import quant4
from tessery_amd import workloads as wl

QWEN_TINY = dict(hidden=128, intermediate=256, layers=2, heads=4, kv_heads=2, head_dim=32,
                 vocab=300)
BERT_TINY = dict(hidden=64, intermediate=128, layers=2, heads=4, vocab=50, positions=32, types=2)


def test_embedding4_matches_scalar_indexing():
    rng = np.random.default_rng(0)
    packed, s, b = wl.weight4_set(rng, 20, 128, 0.2)
    ids = np.array([[3, 0], [19, 7]], dtype=np.uint32)
    got = ref.embedding4(ids, packed, s, b)
    for t, token in enumerate(ids.reshape(-1)):
        for c in (0, 1, 7, 8, 63, 64, 100, 127):
            want = quant4.weight4_scalar(packed, s, b, int(token), c, 128)
            assert got[t, c] == want


def test_embedding_position_definition():
    rng = np.random.default_rng(1)
    words, pos, types = (rng.standard_normal(s) for s in ((9, 6), (5, 6), (2, 6)))
    ids = np.array([[1, 8, 2], [0, 0, 4]], dtype=np.uint32)
    got = ref.embedding_position(ids, words, pos, types)
    for bi in range(2):
        for si in range(3):
            np.testing.assert_array_equal(got[bi * 3 + si],
                                          (words[ids[bi, si]] + types[0]) + pos[si])


@pytest.mark.parametrize("first", [True, False])
def test_pool_project(first):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 5, 10))
    lengths = np.array([5, 1, 3])
    got = ref.pool_project(x, lengths, 7, first=first)
    np.testing.assert_allclose(np.linalg.norm(got, axis=1), 1.0, rtol=1e-15)
    for bi in range(3):
        row = x[bi, 0 if first else lengths[bi] - 1, :7]
        np.testing.assert_allclose(got[bi], row / np.sqrt((row * row).sum()), rtol=1e-14)


def _inputs(vocab: int, batch: int, seq: int, low: int, seed: int):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, (batch, seq)).astype(np.uint32)
    lengths = rng.integers(low, seq + 1, batch).astype(np.uint32)
    lengths[0] = seq
    return ids, lengths


def _qwen3_torch(config, w, ids, lengths, monkeypatch):
    from transformers import Qwen3Config, Qwen3Model
    from transformers.models.qwen3 import modeling_qwen3 as mq

    # Its eager attention takes the softmax in float32; the same steps in float64.
    def eager(module, query, key, value, attention_mask, scaling, dropout=0.0, **_):
        key = mq.repeat_kv(key, module.num_key_value_groups)
        value = mq.repeat_kv(value, module.num_key_value_groups)
        scores = torch.matmul(query, key.transpose(2, 3).contiguous()) * scaling
        if attention_mask is not None:
            scores = scores + attention_mask[:, :, :, : key.shape[-2]]
        probs = torch.softmax(scores, dim=-1)
        return torch.matmul(probs, value).transpose(1, 2).contiguous(), probs

    monkeypatch.setattr(mq, "eager_attention_forward", eager)

    hf = Qwen3Config(vocab_size=config["vocab_size"], hidden_size=config["hidden_size"],
                     intermediate_size=config["intermediate_size"],
                     num_hidden_layers=config["num_hidden_layers"],
                     num_attention_heads=config["num_attention_heads"],
                     num_key_value_heads=config["num_key_value_heads"],
                     head_dim=config["head_dim"], rms_norm_eps=config["rms_norm_eps"],
                     rope_theta=config["rope_theta"], max_position_embeddings=4096,
                     attention_bias=False, attn_implementation="eager")
    model = Qwen3Model(hf).to(torch.float64).eval()

    def deq(prefix):
        packed = w[prefix + ".weight"]
        return torch.from_numpy(quant4.dequantize(packed, w[prefix + ".scales"],
                                                  w[prefix + ".biases"], packed.shape[1] * 8))

    def norm(name):
        return torch.from_numpy(ref.bf16_values(w[name]))

    state = {"embed_tokens.weight": deq("model.embed_tokens"), "norm.weight": norm("model.norm.weight")}
    for layer in range(config["num_hidden_layers"]):
        p = f"model.layers.{layer}"
        h = f"layers.{layer}"
        for name in ("q", "k", "v", "o"):
            state[f"{h}.self_attn.{name}_proj.weight"] = deq(f"{p}.self_attn.{name}_proj")
        for name in ("gate", "up", "down"):
            state[f"{h}.mlp.{name}_proj.weight"] = deq(f"{p}.mlp.{name}_proj")
        for name in ("q_norm", "k_norm"):
            state[f"{h}.self_attn.{name}.weight"] = norm(f"{p}.self_attn.{name}.weight")
        for name in ("input_layernorm", "post_attention_layernorm"):
            state[f"{h}.{name}.weight"] = norm(f"{p}.{name}.weight")
    model.load_state_dict(state, strict=True)
    # transformers builds its rotary tables in float32 whatever the model dtype; rebuild them in
    # float64 (same formula: inv_freq = theta^(-2i/d), angles pos * inv_freq, duplicated halves).
    dim, theta = config["head_dim"], config["rope_theta"]
    inv_freq = 1.0 / theta ** (torch.arange(0, dim, 2, dtype=torch.float64) / dim)

    def rotary(x, position_ids):
        angles = position_ids.to(torch.float64)[..., None] * inv_freq
        emb = torch.cat((angles, angles), dim=-1)
        return emb.cos(), emb.sin()

    model.rotary_emb.forward = rotary
    # Qwen3RMSNorm likewise upcasts only to float32; evaluate the same expression in float64.
    for module in model.modules():
        if type(module).__name__ == "Qwen3RMSNorm":
            def rms(x, m=module):
                return m.weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True)
                                                   + m.variance_epsilon))
            module.forward = rms
    mask = torch.from_numpy((np.arange(ids.shape[1])[None] < lengths[:, None]).astype(np.int64))
    with torch.no_grad():
        hidden = model(input_ids=torch.from_numpy(ids.astype(np.int64)),
                       attention_mask=mask).last_hidden_state.numpy()
    return hidden


def test_qwen3_forward_matches_transformers(monkeypatch):
    config, tensors = wl.qwen3_pack_tensors(3, **QWEN_TINY)
    w = wl.weights_of(tensors)
    ids, lengths = _inputs(QWEN_TINY["vocab"], 3, 12, 1, 4)
    kwargs = dict(layers=2, heads=4, kv_heads=2, head_dim=32, eps=config["rms_norm_eps"],
                  theta=config["rope_theta"], dimensions=96)
    pooled, hidden = ref.qwen3_forward(w, ids, lengths, return_hidden=True, **kwargs)
    want = _qwen3_torch(config, w, ids, lengths, monkeypatch)
    valid = np.arange(12)[None] < lengths[:, None]
    np.testing.assert_allclose(hidden.reshape(3, 12, -1)[valid], want[valid], rtol=1e-10,
                               atol=1e-10)
    last = want[np.arange(3), lengths.astype(np.int64) - 1, :96]
    np.testing.assert_allclose(pooled, last / np.linalg.norm(last, axis=1, keepdims=True),
                               rtol=1e-10, atol=1e-12)
    # Planted mistakes: pooling the first token, or skipping a layer, must not pass the pin.
    wrong = ref.pool_project(hidden.reshape(3, 12, -1), lengths, 96, first=True)
    assert np.abs(wrong - pooled).max() > 1e-3
    short = ref.qwen3_forward(w, ids, lengths, **{**kwargs, "layers": 1})
    assert np.abs(short - pooled).max() > 1e-3


def _bert_torch(config, w, ids, lengths):
    from transformers import BertConfig, BertModel

    hf = BertConfig(vocab_size=config["vocab_size"], hidden_size=config["hidden_size"],
                    num_hidden_layers=config["num_hidden_layers"],
                    num_attention_heads=config["num_attention_heads"],
                    intermediate_size=config["intermediate_size"], hidden_act="gelu",
                    max_position_embeddings=config["max_position_embeddings"],
                    type_vocab_size=config["type_vocab_size"],
                    layer_norm_eps=config["layer_norm_eps"], attn_implementation="eager",
                    hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)
    model = BertModel(hf).to(torch.float64).eval()
    # position_ids is arange (the backend checks it) and a non-persistent buffer in transformers.
    state = {name: torch.from_numpy(np.asarray(a, dtype=np.float64)) for name, a in w.items()
             if name != "embeddings.position_ids"}
    model.load_state_dict(state, strict=True)
    mask = torch.from_numpy((np.arange(ids.shape[1])[None] < lengths[:, None]).astype(np.int64))
    with torch.no_grad():
        return model(input_ids=torch.from_numpy(ids.astype(np.int64)), attention_mask=mask,
                     token_type_ids=torch.zeros(ids.shape, dtype=torch.int64)
                     ).last_hidden_state.numpy()


def test_bert_forward_matches_transformers():
    config, tensors = wl.bert_pack_tensors(5, **BERT_TINY)
    w = wl.weights_of(tensors)
    ids, lengths = _inputs(BERT_TINY["vocab"], 3, 10, 2, 6)
    pooled, hidden = ref.bert_forward(w, ids, lengths, layers=2, heads=4,
                                      eps=config["layer_norm_eps"], return_hidden=True)
    want = _bert_torch(config, w, ids, lengths)
    valid = np.arange(10)[None] < lengths[:, None]
    np.testing.assert_allclose(hidden[valid], want[valid], rtol=1e-10, atol=1e-10)
    cls = want[:, 0]
    np.testing.assert_allclose(pooled, cls / np.linalg.norm(cls, axis=1, keepdims=True),
                               rtol=1e-10, atol=1e-12)
    wrong = ref.pool_project(hidden, lengths, hidden.shape[-1], first=False)
    assert np.abs(wrong - pooled).max() > 1e-3
