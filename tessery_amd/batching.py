"""Host-side execution-width plan: which padded width each length bucket runs at.

Restates tessery's bucket and padding policy (src/metal_inference/batching.py:9-69) because the
width it picks decides which attention route runs (tail, tiled or scalar). The outputs must equal
the reference's for every input, so the policy itself is unchanged; the code is this package's.
"""

from __future__ import annotations

from collections.abc import Iterator

import numpy as np
from numpy.typing import NDArray

PADDED_ARCHITECTURES = ("qwen3_uint4", "bert_f32")


def length_batches(
    lengths: NDArray[np.uint32], max_padded_tokens: int
) -> Iterator[tuple[NDArray[np.intp], int]]:
    """Group rows by length (stable ascending order). A bucket grows while the next length is
    at most twice its shortest and the padded token count stays within the budget; its width
    is its longest member. Yields (original row indices, width)."""
    order = np.argsort(lengths, kind="stable")
    count = len(order)
    first = 0
    while first < count:
        shortest = int(lengths[order[first]])
        width = shortest
        last = first + 1
        while last < count:
            candidate = int(lengths[order[last]])
            members = last - first + 1
            if candidate > 2 * shortest or candidate * members > max_padded_tokens:
                break
            width = candidate
            last += 1
        yield order[first:last], width
        first = last


def _round_up(value: int, multiple: int) -> int:
    return -(-value // multiple) * multiple


def execution_batches(
    lengths: NDArray[np.uint32], max_padded_tokens: int, max_length: int, architecture: str
) -> Iterator[tuple[NDArray[np.intp], int]]:
    """Pad each bucket's width to a multiple of 8 when that reaches an attention tile
    (width >= 64, multiple of 32) or removes a partial 8-row projection tile, within the
    bounds max_length, twice the bucket's shortest length and the token budget. Two-row Qwen
    buckets shorter than 128 that cannot take 8-padding may take 4-padding instead."""
    for rows, width in length_batches(lengths, max_padded_tokens):
        members = len(rows)
        shortest = int(lengths[rows].min())

        def admissible(candidate: int) -> bool:
            return (
                candidate <= max_length
                and candidate <= 2 * shortest
                and candidate * members <= max_padded_tokens
            )

        to8 = _round_up(width, 8)
        reaches_tile = to8 >= 64 and to8 % 32 == 0
        partial_rows = (width * members) % 8 != 0 and (
            architecture == "bert_f32" or width < 128
        )
        if (
            architecture in PADDED_ARCHITECTURES
            and width >= 5
            and (reaches_tile or partial_rows)
            and admissible(to8)
        ):
            width = to8
        elif (
            architecture == "qwen3_uint4"
            and members == 2
            and 5 <= width < 128
            and partial_rows
            and admissible(_round_up(width, 4))
        ):
            width = _round_up(width, 4)
        yield rows, width
