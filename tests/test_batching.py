"""Execution-width plan against tessery's explicit expectations (test_batching.py:1-94)."""

import json

import numpy as np
import pytest

from tessery_amd.batching import execution_batches, length_batches
from tests.conftest import GOLDEN

CASES = json.loads((GOLDEN / "batching.json").read_text())


def test_buckets_bound_padding_and_order():
    case = CASES["buckets"]
    groups = list(length_batches(np.array(case["lengths"], np.uint32), case["budget"]))
    assert [[rows.tolist(), width] for rows, width in groups] == case["expected"]
    for length_set in ([3, 8, 2, 8, 2], [512] * 32, [1, 2, 3, 4, 8, 9, 64, 128, 512]):
        values = np.array(length_set, np.uint32)
        groups = list(length_batches(values, 4096))
        assert sorted(np.concatenate([r for r, _ in groups]).tolist()) == list(range(len(values)))
        for rows, width in groups:
            assert width == max(values[rows]) and width <= 2 * min(values[rows])
            assert width * len(rows) <= 4096


def test_empty_and_uniform():
    assert list(length_batches(np.array([], np.uint32), 4096)) == []
    case = CASES["uniform"]
    groups = list(length_batches(np.array(case["lengths"], np.uint32), case["budget"]))
    assert [r.tolist() for r, _ in groups] == case["expected_rows"]


@pytest.mark.parametrize("length,count,architecture,expected", CASES["single"])
def test_execution_padding_selection(length, count, architecture, expected):
    groups = list(execution_batches(np.full(count, length, np.uint32), 4096, 512, architecture))
    assert len(groups) == 1 and groups[0][1] == expected


@pytest.mark.parametrize("lengths,budget,maximum,architecture,expected", CASES["pairs"])
def test_two_input_fallback_alignment(lengths, budget, maximum, architecture, expected):
    groups = execution_batches(np.array(lengths, np.uint32), budget, maximum, architecture)
    assert [[rows.tolist(), width] for rows, width in groups] == [list(e) for e in expected]


@pytest.mark.parametrize("architecture", ["qwen3_uint4", "bert_f32"])
def test_padding_keeps_membership_and_bounds(architecture):
    for maximum in (7, 31, 65, 127, 511, 512):
        for count in (1, 2, 3, 8, 32):
            for longest in range(1, maximum + 1, 3):
                lengths = np.full(count, longest, np.uint32)
                if count > 1:
                    lengths[0] = max(1, longest // 2)
                before = list(length_batches(lengths, 4096))
                after = list(execution_batches(lengths, 4096, maximum, architecture))
                assert len(before) == len(after)
                for (old_rows, old_width), (rows, width) in zip(before, after):
                    np.testing.assert_array_equal(rows, old_rows)
                    assert old_width <= width <= maximum
                    assert width <= 2 * int(lengths[rows].min()) and width * len(rows) <= 4096
    assert list(execution_batches(np.array([], np.uint32), 4096, 512, architecture)) == []
