"""The attend's split-K rules (host logic, no GPU): the fused step's rule (partials merged in-kernel) and the standalone
attend's (merged by the combine kernel) pick the partition counts that were fastest on MI355X at the measured shapes
(32K with S = 1092 and 128K with S = 4164, B = 1..16, h = 1, 2, 4); the docstring of merged_partitions holds the
timings, where the rule is within 0.4 us of the best P per layer."""
from __future__ import annotations

import pytest

from attention_lab.hip_attend import merged_partitions, sparse_partitions


@pytest.mark.parametrize("BG,S,h,want", [
    (8, 1092, 1, 8), (8, 1092, 2, 8), (8, 1092, 4, 8),
    (16, 1092, 1, 8), (16, 1092, 2, 8), (16, 1092, 4, 8),
    (32, 1092, 1, 8), (32, 1092, 4, 4),
    (64, 1092, 1, 4), (64, 1092, 2, 4), (64, 1092, 4, 2),
    (128, 1092, 1, 2), (128, 1092, 2, 2), (128, 1092, 4, 1),
    (8, 4164, 2, 16), (8, 4164, 4, 8), (16, 4164, 4, 8), (32, 4164, 2, 8), (32, 4164, 4, 4),
])
def test_merged_rule_picks_the_measured_best(BG, S, h, want):
    assert merged_partitions(BG, S, h) == want == sparse_partitions(BG, S, h, merged=True)


def test_short_lists_are_not_split_below_128_rows_and_the_combine_rule_is_unchanged():
    assert merged_partitions(8, 132, 2) == 1 and merged_partitions(8, 300, 2) == 2
    # the standalone attend (combine kernel): B=1 P=8, B=16 h=4 P=1 (two head groups), B=16 h=1 P=1
    assert sparse_partitions(8, 1092, 2) == 8 and sparse_partitions(128, 1092, 4) == 1 and sparse_partitions(128, 1092, 1) == 1
