"""Host logic of the selection pipeline that runs without a GPU: the top-k glue."""

import math

import pytest
import torch

from unum_ops_amd.pipeline import num_blocks, select_blocks, topk_blocks


def test_topk_sorted_and_minus_one_for_empty_windows():
    inf = math.inf
    pooled = torch.tensor([[[0.5, -inf, 2.0, inf, 0.1, -inf],
                            [-inf, -inf, -inf, -inf, 3.0, -inf]]])
    idx = topk_blocks(pooled, 4)
    assert idx.dtype == torch.int32
    assert idx.tolist() == [[[0, 2, 3, 4], [-1, -1, -1, 4]]]


def test_topk_pads_when_fewer_blocks_than_k():
    pooled = torch.tensor([[[1.0, 3.0, 2.0]]])
    assert topk_blocks(pooled, 5).tolist() == [[[-1, -1, 0, 1, 2]]]


def test_num_blocks():
    assert num_blocks(1) == 1 and num_blocks(64) == 1 and num_blocks(65) == 2
    assert num_blocks(135168) == 2112


def test_select_blocks_refuses_cpu_tensors():
    q = torch.zeros(4, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        select_blocks(q, k, cu, cu, torch.zeros(1, 64, dtype=torch.int32),
                      torch.zeros(4, dtype=torch.int32), torch.ones(4, dtype=torch.int32),
                      torch.tensor([64], dtype=torch.int32), 64)


def test_topk_ties_go_to_lower_block_id():
    # Neighbouring windows share a tap, so equal maxima are common.
    pooled = torch.tensor([[[1.0, 2.0, 2.0, 2.0, 0.5, 2.0]]])
    assert topk_blocks(pooled, 2).tolist() == [[[1, 2]]]
    assert topk_blocks(pooled, 4).tolist() == [[[1, 2, 3, 5]]]
