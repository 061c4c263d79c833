"""Pins of the key-compression oracle (CPU)."""

import numpy as np
import pytest
import torch

from oracle.compress import compress_keys, compress_keys_bruteforce
import workloads


def ulp_diff(a, b):
    """Max distance in bf16 units in the last place (same-sign values)."""
    ia = a.contiguous().view(torch.int16).to(torch.int32)
    ib = b.contiguous().view(torch.int16).to(torch.int32)
    return int((ia - ib).abs().max()) if ia.numel() else 0


@pytest.mark.parametrize("lengths,expected", [
    ([5, 31], [0, 0]), ([32], [1]), ([47], [1]), ([48], [2]), ([1000, 33, 4096], [61, 1, 255])])
def test_window_counts(lengths, expected):
    cu = workloads.prefix(lengths)
    k = torch.randn(sum(lengths), 2, 16).to(torch.bfloat16)
    out, cu_c = compress_keys(k, cu)
    assert (np.diff(cu_c) == np.asarray(expected)).all() and out.shape[0] == sum(expected)


def test_against_torch_mean():
    g = torch.Generator().manual_seed(0)
    lengths = [40, 700, 1333, 96]
    raw = torch.randn(sum(lengths), 2, 128, generator=g).to(torch.bfloat16)
    cu = workloads.prefix(lengths)
    out, _ = compress_keys(raw, cu)
    ref = torch.cat([workloads.compress_keys(raw[int(cu[b]):int(cu[b + 1])])
                     for b in range(len(lengths))]).to(torch.bfloat16)
    assert ref.shape == out.shape
    assert ulp_diff(out, ref) <= 1
    assert (out == ref).float().mean() > 0.999


def test_against_bruteforce():
    g = torch.Generator().manual_seed(1)
    lengths = [33, 64, 81]
    raw = (torch.randn(sum(lengths), 2, 8, generator=g) * 3).to(torch.bfloat16)
    cu = workloads.prefix(lengths)
    out, _ = compress_keys(raw, cu)
    assert ulp_diff(out, compress_keys_bruteforce(raw, cu)) <= 1


def test_constant_and_ramp():
    raw = torch.full((64, 1, 8), 0.375).to(torch.bfloat16)
    out, _ = compress_keys(raw, torch.tensor([0, 64]))
    assert (out.float() == 0.375).all() and out.shape[0] == 3
    ramp = torch.arange(64, dtype=torch.float32)[:, None, None].expand(64, 1, 8).to(torch.bfloat16)
    out, _ = compress_keys(ramp, torch.tensor([0, 64]))
    # window j covers tokens 16j .. 16j+31: mean 16j + 15.5
    assert out[:, 0, 0].float().tolist() == [15.5, 31.5, 47.5]
