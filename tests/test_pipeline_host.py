"""Host logic of the selection pipeline that runs without a GPU: argument checks and block counts."""

import pytest
import torch

from unum_ops_amd.pipeline import num_blocks, select_blocks, topk_blocks


def test_topk_blocks_refuses_cpu_tensors():
    with pytest.raises(RuntimeError, match="HIP device"):
        topk_blocks(torch.zeros(1, 2, 8), 4)


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


