"""The committed fixtures still agree with the oracle (guards both against drift)."""

import numpy as np

from oracle import attention, norm_rope, quant4
from tessery_amd import workloads
from tests.conftest import GOLDEN


def test_attention_fixtures():
    f = np.load(GOLDEN / "attention_cases.npz")
    for tag, bidi in (("s17", False), ("s83", True), ("c1", True)):
        got = attention.attention(f[f"{tag}_q"], f[f"{tag}_k"], f[f"{tag}_v"], f[f"{tag}_lengths"],
                                  bidirectional=bidi)
        np.testing.assert_allclose(got, f[f"{tag}_expected"], atol=1e-12)
    for seq in (64, 65, 71):
        tag = f"r{seq}"
        for bidi in (0, 1):
            got = attention.attention(f[f"{tag}_q"], f[f"{tag}_k"], f[f"{tag}_v"],
                                      f[f"{tag}_lengths"], bidirectional=bool(bidi))
            np.testing.assert_allclose(got, f[f"{tag}_expected_b{bidi}"], atol=1e-12)


def test_c1_fixture_is_the_seeded_workload():
    f = np.load(GOLDEN / "attention_cases.npz")
    _, lengths, t = workloads.bge_small_c1()
    np.testing.assert_array_equal(f["c1_q"], t["q"])
    np.testing.assert_array_equal(f["c1_lengths"], lengths)


def test_qwen_fixture():
    f = np.load(GOLDEN / "qwen_small.npz")
    qn = workloads.bf16_values(f["q_norm"])
    kn = workloads.bf16_values(f["k_norm"])
    q = norm_rope.norm_rope(f["q"], qn, workloads.EPS, workloads.THETA)
    k = norm_rope.norm_rope(f["k"], kn, workloads.EPS, workloads.THETA)
    np.testing.assert_allclose(k, f["k_normed"], atol=1e-12)
    got = attention.attention(q, k, f["v"], f["lengths"], bidirectional=False)
    np.testing.assert_allclose(got, f["expected"], atol=1e-12)


def test_linear4_fixture():
    f = np.load(GOLDEN / "linear4_small.npz")
    got = quant4.linear4(f["x"], f["packed"], f["scales"], f["biases"])
    np.testing.assert_allclose(got, f["expected"], atol=1e-12)


def test_workload_lengths_match_published_sums():
    """Seeded lengths behind the algorithmic-work table (sum of valid lengths per workload)."""
    assert int(workloads.bge_small_32x512()[1].sum()) == 8017
    assert int(workloads.qwen3_8x512()[1].sum()) == 2191
    shape, lengths = workloads.qwen3_32x512()
    assert int(lengths.sum()) == 4067 and shape.seq == 464
    assert int(workloads.lengths_uniform(5, 16, 1, 256).sum()) == 1815


def test_algorithmic_work_known_values():
    shape, lengths = workloads.qwen3_32x512()
    # causal pairs by hand for one row: L=3, S=5 -> 1+2+3 + 2*3
    tiny = workloads.Shape(1, 5, 1, 1, 1, causal=True)
    assert workloads.pairs(tiny, np.array([3], np.uint32)) == 12
    assert workloads.pairs(workloads.Shape(1, 5, 1, 1, 1, causal=False), np.array([3], np.uint32)) == 15
    flop = workloads.attention_flop(shape, lengths)
    assert abs(flop / 1e9 - 10.13) < 0.01
    nbytes = workloads.attention_bytes(shape, lengths, 2, 2)
    assert abs(nbytes / 1e6 - 138.3) < 0.1
