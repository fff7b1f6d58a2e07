"""
Pins oracle/topk_select.c -- the C restatement of CPU torch.topk's per-row selection
(ATen/native/TopKImpl.h:44-94; libstdc++ nth_element / sort / partial_sort) -- against
torch.topk itself.  The HIP route kernel implements the same algorithm; a dropped step,
a wrong pivot or a wrong comparison would reorder tied indices and fail here, because
the rows below are drawn from a handful of values and are full of exact ties.
"""

import numpy as np
import pytest
import torch

from tests.helpers import oracle_topk, tie_heavy

SHAPES = [(76, 6), (76, 1), (76, 2), (76, 20), (8, 1), (8, 2), (8, 3), (8, 8), (128, 2),
          (200, 3), (300, 40), (5, 5), (3, 2), (1, 1), (64, 1), (65, 1), (17, 17), (33, 18)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("levels", [1, 2, 3, 7, 50, 0])
def test_restatement_matches_torch_topk(n, k, levels):
    rows = 1500
    if levels:
        v = tie_heavy(rows, n, levels, seed=n * 31 + k * 7 + levels)
    else:
        v = (torch.randn(rows, n) * 0.48).bfloat16().float()
    ref = v.topk(k, dim=-1)
    got = oracle_topk(v.numpy(), k)
    assert np.array_equal(got, ref.indices.numpy())


def test_branches_are_all_exercised():
    """k * 64 <= n takes partial_sort, otherwise nth_element + sort (TopKImpl.h:45)."""
    assert any(k * 64 <= n for n, k in SHAPES)
    assert any(k * 64 > n and k - 1 > 16 for n, k in SHAPES)   # introsort inside sort()
    assert any(k * 64 > n and k - 1 <= 16 for n, k in SHAPES)  # insertion sort only


def test_nan_ranks_first():
    v = torch.tensor([[0.5, float("nan"), 1.0, -2.0, float("nan"), 0.5, 0.5, 3.0]])
    for k in range(1, 9):
        assert np.array_equal(oracle_topk(v.numpy(), k), v.topk(k).indices.numpy())
