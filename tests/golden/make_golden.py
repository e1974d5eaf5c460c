"""Writes the committed golden fixtures of tests/golden/ (run: python tests/golden/make_golden.py).

routes.json    tessery's attention route table: the (seq, dim) cases and expected kernel / group /
               thread counts of test_runtime_loading.py:68-106 (tokens = 2*seq, heads 4, kv 2),
               plus its uint4 projection guard cases (test_runtime_loading.py:9-65).
batching.json  tessery's explicit execution-width expectations (test_batching.py:50-94).
*.npz          seeded inputs of tessery's attention / norm / uint4 test cases and of the small
               BGE configuration, with float64 expected outputs from the oracle.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import attention, norm_rope, quant4  # noqa: E402
from tessery_amd import workloads  # noqa: E402


def attention_routes() -> list[dict]:
    table = [
        (32, 32, False), (63, 128, False), (64, 128, True), (65, 128, False), (127, 32, False),
        (128, 32, True), (129, 32, False), (511, 128, False), (512, 128, True), (128, 64, False),
        (128, 256, False), (65, 32, False), (71, 128, False), (136, 32, False), (513, 32, False),
        (1024, 128, True),
    ]
    cases = []
    for seq, dim, tiled in table:
        tail = 64 <= seq <= 512 and seq % 32 and dim in (32, 128)
        name = f"attention_tail_{dim}" if tail else "attention_tiled" if tiled else "attention"
        threads = (
            2 * ((seq + 7) // 8) * 4 * 128 if tail else (2 * seq // 8 * 4 * 128 if tiled else 2 * seq * 4 * 32)
        )
        cases.append({"seq": seq, "dim": dim, "name": name,
                      "group_size": 128 if (tiled or tail) else 32, "threads": threads})
    return cases


def linear4_guards() -> dict:
    shapes = ((1024, 1024), (2048, 1024), (3072, 1024), (1024, 2048), (1024, 3072))
    bad = ((64, 1024), (1025, 1024), (1024, 64), (1024, 1023), (4096, 1024))
    small3 = [(3, n, k, True) for n, k in shapes] + [(m, 1024, 1024, False) for m in (1, 2, 4, 5, 19)]
    small3 += [(3, n, k, False) for n, k in bad]
    large = [(m, n, k, True) for m in (16, 17, 23, 24, 25, 31, 32, 33, 40, 129, 264, 4095, 4096)
             for n, k in shapes]
    large += [(m, 1024, 1024, False) for m in (1, 4, 7, 8, 15)]
    large += [(16, n, k, False) for n, k in bad]
    return {"small3": small3, "large": large}


def batching() -> dict:
    single = [
        (4, 1, "qwen3_uint4", 4), (7, 1, "qwen3_uint4", 8), (33, 8, "qwen3_uint4", 33),
        (33, 8, "bert_f32", 33), (63, 8, "qwen3_uint4", 64), (129, 1, "qwen3_uint4", 129),
        (129, 1, "bert_f32", 136), (511, 8, "qwen3_uint4", 512), (455, 9, "bert_f32", 455),
        (7, 1, "future_backend", 7),
    ]
    pairs = [
        ([3, 7, 10], 4096, 512, "qwen3_uint4", [([0], 3), ([1, 2], 12)]),
        ([10, 3, 7], 4096, 512, "qwen3_uint4", [([1], 3), ([2, 0], 12)]),
        ([6, 9], 4096, 512, "qwen3_uint4", [([0, 1], 12)]),
        ([7, 11], 4096, 512, "qwen3_uint4", [([0, 1], 12)]),
        ([62, 122], 4096, 512, "qwen3_uint4", [([0, 1], 124)]),
        ([5, 9], 4096, 512, "qwen3_uint4", [([0, 1], 9)]),
        ([7, 10], 4096, 11, "qwen3_uint4", [([0, 1], 10)]),
        ([7, 10], 4096, 12, "qwen3_uint4", [([0, 1], 12)]),
        ([7, 10], 23, 512, "qwen3_uint4", [([0, 1], 10)]),
        ([7, 10], 24, 512, "qwen3_uint4", [([0, 1], 12)]),
        ([7, 10], 4096, 512, "bert_f32", [([0, 1], 10)]),
        ([7, 10], 4096, 512, "future_backend", [([0, 1], 10)]),
        ([7, 7, 7, 7, 7, 10], 4096, 512, "qwen3_uint4", [(list(range(6)), 10)]),
        ([3, 5, 5, 5], 4096, 512, "qwen3_uint4", [(list(range(4)), 5)]),
        ([70, 130], 4096, 512, "qwen3_uint4", [([0, 1], 130)]),
        ([2, 3], 4096, 512, "qwen3_uint4", [([0, 1], 3)]),
    ]
    buckets = {"lengths": [512] + [2] * 31, "budget": 4096,
               "expected": [[list(range(1, 32)), 2], [[0], 512]]}
    uniform = {"lengths": [1] * 5, "budget": 2, "expected_rows": [[0, 1], [2, 3], [4]]}
    return {"single": single, "pairs": pairs, "buckets": buckets, "uniform": uniform}


def attention_cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    # tessery test_kernels.py:127-157 (scalar causal GQA, seed 17)
    rng = np.random.default_rng(17)
    q = rng.normal(size=(2, 5, 4, 64)).astype(np.float32)
    k = rng.normal(size=(2, 5, 2, 64)).astype(np.float32)
    v = rng.normal(size=k.shape).astype(np.float32)
    lengths = np.array([5, 2], np.uint32)
    out.update(s17_q=q, s17_k=k, s17_v=v, s17_lengths=lengths,
               s17_expected=attention.attention(q, k, v, lengths, bidirectional=False))
    # tessery test_kernels.py:359-385 (bidirectional MHA, seed 83)
    rng = np.random.default_rng(83)
    q, k, v = [rng.normal(size=(2, 5, 3, 8)).astype(np.float32) for _ in range(3)]
    lengths = np.array([5, 2], np.uint32)
    out.update(s83_q=q, s83_k=k, s83_v=v, s83_lengths=lengths,
               s83_expected=attention.attention(q, k, v, lengths, bidirectional=True))
    # BGE-small attention layer, B=2 S=16 H=12 D=32, lengths [16, 9], bidirectional
    shape, lengths, t = workloads.bge_small_c1()
    out.update(c1_q=t["q"], c1_k=t["k"], c1_v=t["v"], c1_lengths=lengths,
               c1_expected=attention.attention(t["q"], t["k"], t["v"], lengths, bidirectional=True))
    # tessery test_kernels.py:160-210 ragged cases at seed 393, d=32, widths 64/65/71
    for seq, pair in ((64, (1, 33)), (65, (1, 65)), (71, (33, 71))):
        rng = np.random.default_rng(393)
        q = rng.normal(size=(2, seq, 4, 32)).astype(np.float32)
        k, v = [rng.normal(size=(2, seq, 2, 32)).astype(np.float32) for _ in range(2)]
        lengths = np.array(pair, np.uint32)
        tag = f"r{seq}"
        out.update({f"{tag}_q": q, f"{tag}_k": k, f"{tag}_v": v, f"{tag}_lengths": lengths})
        for bidi in (0, 1):
            out[f"{tag}_expected_b{bidi}"] = attention.attention(q, k, v, lengths, bidirectional=bool(bidi))
    return out


def qwen_small() -> dict[str, np.ndarray]:
    shape = workloads.Shape(2, 40, 4, 2, 128, causal=True)
    lengths = np.array([40, 13], np.uint32)
    t = workloads.qwen_layer(shape, 0, seed=31)
    qn = workloads.bf16_values(t["q_norm"]).astype(np.float64)
    kn = workloads.bf16_values(t["k_norm"]).astype(np.float64)
    q = norm_rope.norm_rope(t["q"], qn, workloads.EPS, workloads.THETA)
    k = norm_rope.norm_rope(t["k"], kn, workloads.EPS, workloads.THETA)
    expected = attention.attention(q, k, t["v"], lengths, bidirectional=False)
    return dict(q=t["q"], k=t["k"], v=t["v"], q_norm=t["q_norm"], k_norm=t["k_norm"],
                lengths=lengths, k_normed=k, expected=expected)


def linear4_small() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(417)
    m, n, k = 7, 64, 128
    codes = rng.integers(0, 16, size=(n, k), dtype=np.uint32)
    packed = quant4.pack(codes)
    scales = workloads.bf16_words(rng.uniform(0.01, 0.2, size=(n, k // 64)))
    biases = workloads.bf16_words(rng.uniform(-1, 0.1, size=(n, k // 64)))
    x = rng.normal(size=(m, k)).astype(np.float32)
    return dict(x=x, packed=packed, scales=scales, biases=biases,
                expected=quant4.linear4(x, packed, scales, biases))


def main() -> None:
    (HERE / "routes.json").write_text(
        json.dumps({"attention": attention_routes(), "linear4": linear4_guards()}, indent=1) + "\n")
    (HERE / "batching.json").write_text(json.dumps(batching(), indent=1) + "\n")
    np.savez_compressed(HERE / "attention_cases.npz", **attention_cases())
    np.savez_compressed(HERE / "qwen_small.npz", **qwen_small())
    np.savez_compressed(HERE / "linear4_small.npz", **linear4_small())


if __name__ == "__main__":
    main()
