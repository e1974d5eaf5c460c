"""The compiled forward programs of the two backends, on the CPU (no device is touched).

Each program must read every tensor its pack inventory requires, name only tensors and
activations that exist, and run the model's layer in the order of qwen3.py:194-280 and
bert.py:186-230 (the kernel families per layer are listed below)."""

import pytest

from tessery_amd import backends as bk
from tessery_amd import packs

QWEN = packs.Qwen3Dims(hidden=128, intermediate=256, layers=3, heads=4, kv_heads=2, head_dim=32,
                       vocab=300, eps=1e-6, theta=1e6)
BERT = packs.BertDims(hidden=64, intermediate=128, layers=2, heads=4, vocab=50, positions=32,
                      types=2, eps=1e-12)

QWEN_LAYER = ["rms_norm", "linear4", "linear4", "linear4", "rms_norm", "rope", "rms_norm", "rope",
              "attention", "linear4", "add", "rms_norm", "gated4", "linear4", "add"]
BERT_LAYER = ["dense", "dense", "dense", "attention", "dense", "add", "layer_norm", "dense",
              "gelu", "dense", "add", "layer_norm"]


def tensors_read(program):
    names = set()
    for o in program.ops:
        for s in o.slots:
            if isinstance(s, tuple):
                names.update(s[0] + suffix for suffix in s[1])
            elif not s.startswith("%"):
                names.add(s)
    return names


def activations_read(program):
    return {s for o in program.ops for s in o.slots if isinstance(s, str) and s.startswith("%")}


@pytest.mark.parametrize("dims,program,inventory,layer_kinds,head,tail", [
    (QWEN, bk.qwen3_program(QWEN, 3, 17, 96), packs.qwen3_inventory(QWEN), QWEN_LAYER,
     ["embed_uint4"], ["rms_norm", "pool"]),
    (BERT, bk.bert_program(BERT, 2, 9), packs.bert_inventory(BERT), BERT_LAYER,
     ["embed_bert", "layer_norm"], ["pool"]),
])
def test_program_reads_the_whole_inventory_in_layer_order(dims, program, inventory, layer_kinds,
                                                          head, tail):
    assert tensors_read(program) == set(inventory.required)
    declared = {slot for slot, _ in program.activations} | {"%ids", "%lengths"}
    assert activations_read(program) <= declared
    assert program.output in declared
    kinds = [o.kind for o in program.ops]
    assert kinds == head + layer_kinds * dims.layers + tail
    assert all(o.kind in bk.EMITTERS for o in program.ops)


def test_layer_ops_name_their_own_layer():
    """Layer i's ops read only layer i's tensors (a planted off-by-one in the prefix would read
    the next layer's weights)."""
    for i in range(QWEN.layers):
        ops = list(bk.qwen3_layer_ops(QWEN, i, 51, 17))
        read = tensors_read(bk.Program(("t",), (), "%x", (1, 1), tuple(ops)))
        assert read and all(n.startswith(f"model.layers.{i}.") for n in read)
    for i in range(BERT.layers):
        ops = list(bk.bert_layer_ops(BERT, i, 18, 9))
        read = tensors_read(bk.Program(("t",), (), "%x", (1, 1), tuple(ops)))
        assert read and all(n.startswith(f"encoder.layer.{i}.") for n in read)


def test_programs_are_cached_per_shape():
    assert bk.qwen3_program(QWEN, 3, 17, 96) is bk.qwen3_program(QWEN, 3, 17, 96)
    assert bk.qwen3_program(QWEN, 3, 17, 96) is not bk.qwen3_program(QWEN, 3, 17, 64)
    assert bk.bert_program(BERT, 2, 9).key == ("bert", 2, 9, BERT.hidden)
