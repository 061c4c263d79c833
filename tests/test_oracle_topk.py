"""Pins of the top-k selection oracle (CPU)."""

import numpy as np
import pytest
import torch

from oracle.topk import topk_blocks, topk_blocks_bruteforce

INF = float("inf")


def test_known_answers():
    x = np.array([[[0.5, -INF, 2.0, INF, 0.1, -INF],
                   [-INF, -INF, -INF, -INF, 3.0, -INF],
                   [1.0, 2.0, 2.0, 2.0, 0.5, 2.0]]], np.float32)
    assert topk_blocks(x, 4).tolist() == [[[0, 2, 3, 4], [-1, -1, -1, 4], [1, 2, 3, 5]]]
    assert topk_blocks(x, 8).tolist()[0][2] == [-1, -1, 0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("seed", range(6))
def test_against_bruteforce_with_ties(seed):
    rng = np.random.default_rng(seed)
    # few distinct values, +-inf included: ties everywhere
    levels = np.array([-INF, -1.0, 0.0, 0.25, 0.5, INF], np.float32)
    x = levels[rng.integers(0, len(levels), size=(2, 5, 37))]
    for k in (1, 3, 8, 36, 37, 40):
        np.testing.assert_array_equal(topk_blocks(x, k), topk_blocks_bruteforce(x, k))


@pytest.mark.parametrize("seed", range(3))
def test_against_torch_topk_on_distinct_scores(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(2, 7, 300, generator=g)
    for k in (1, 16, 64, 299):
        ref = torch.topk(x, k, dim=-1).indices.sort(-1).values.int().numpy()
        np.testing.assert_array_equal(topk_blocks(x, k), ref)


def _topk_torch_sort(x, k):
    """The same rule through torch's stable descending sort (another library's
    sort than the oracle's numpy argsort)."""
    H, T, NB = x.shape
    kk = min(k, NB)
    vals, idx = torch.sort(x, dim=-1, descending=True, stable=True)
    vals, idx = vals[..., :kk], idx[..., :kk]
    idx = torch.where(vals == -INF, torch.full_like(idx, -1), idx).sort(dim=-1).values
    if kk < k:
        idx = torch.cat([torch.full((H, T, k - kk), -1, dtype=idx.dtype), idx], dim=-1)
    return idx.to(torch.int32)


def test_matches_a_torch_stable_sort():
    g = torch.Generator().manual_seed(9)
    x = torch.randint(-3, 4, (2, 11, 100), generator=g).float()
    x[x == -3] = -INF
    for k in (5, 64, 120):
        np.testing.assert_array_equal(topk_blocks(x, k), _topk_torch_sort(x, k).numpy())
