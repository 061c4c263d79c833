"""GPU parity: max_pooling_1d_varlen HIP kernel vs the oracle -- bit-exact."""

import numpy as np
import pytest
import torch

from oracle.maxpool import max_pooling_1d_varlen as oracle_pool
import workloads
from unum_ops_amd.infllm_v2 import max_pooling_1d_varlen, max_pooling_1d_varlen_ref_triton

pytestmark = pytest.mark.gpu


def _run(d, dev, fn=max_pooling_1d_varlen, **kw):
    out = fn(d["input"].to(dev), d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev),
             d["cache_lens"].to(dev), **kw)
    torch.cuda.synchronize()
    return out


def _check(d, out, **kw):
    # "absent" equals "raise" wherever the reference stays in bounds
    exp = oracle_pool(d["input"], d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                      oob="absent", **kw)
    got = out.float().cpu().numpy()
    assert out.dtype == d["input"].dtype
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("local_blocks", [1, 2])
def test_cfg2_full_size(local_blocks, dev):
    d = workloads.cfg2_maxpool(local_blocks=local_blocks)
    kw = {k: d[k] for k in ("max_seqlen_q", "max_context_len", "local_blocks", "init_blocks",
                            "block_size", "stride")}
    out = _run(d, dev, **kw)
    assert out.shape == (2, 34816, 256)
    _check(d, out, **kw)


@pytest.mark.parametrize("num_heads", [4, 8, 16])
@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16])
def test_reference_test_shapes(num_heads, batch, dev):
    # test/test_max_pooling_1d.py:8-110: q_b = 8+8i, k_b = 16+8i, bf16 randn input
    # [H, total_q, max_k], max_seqlen_q = max q_b (flat stride max_q//16), init 1, local 32
    q_lens = [8 + 8 * i for i in range(batch)]
    k_lens = [16 + 8 * i for i in range(batch)]
    g = torch.Generator().manual_seed(num_heads * 100 + batch)
    x = torch.randn(num_heads, sum(q_lens), max(k_lens), generator=g).to(torch.bfloat16)
    d = dict(input=x, cu_seqlens_q=workloads.prefix(q_lens), cu_seqlens_k=workloads.prefix(k_lens),
             cache_lens=torch.zeros(batch, dtype=torch.int32))
    kw = dict(max_seqlen_q=max(q_lens), max_context_len=max(q_lens), local_blocks=32,
              init_blocks=1, block_size=64, stride=16)
    out = _run(d, dev, max_pooling_1d_varlen_ref_triton, **kw)
    _check(d, out, **kw)


EDGE = [
    # q_lens, k_lens, cache, F, max_seqlen_q, max_context_len, local, init, dtype
    ([40, 24], [9, 5], [0, 0], 16, 256, 200, 1, 1, torch.float32),
    ([64, 130, 7], [17, 33, 0], [0, 3, 2], 40, 640, 700, 2, 1, torch.float32),
    ([100], [1], [0], 8, 128, 300, 0, 0, torch.float32),
    ([100], [0], [4], 8, 128, 300, 1, 1, torch.float32),
    ([70, 70], [4, 12], [5, 0], 20, 320, 180, 1, 2, torch.bfloat16),
    ([33, 65], [31, 29], [0, 0], 32, 512, 2100, 3, 1, torch.float16),
    ([300, 5], [70, 2], [100, 0], 72, 1152, 9000, 1, 1, torch.float32),   # NB > 256, cache > 0
    ([20], [1023], [0], 1024, 16384, 16384, 1, 1, torch.float32),
    ([20], [1021], [0], 1022, 16352, 16384, 1, 1, torch.float32),         # F not a multiple of 4
    ([9], [30], [0], 30, 480, 1000, 1, 1, torch.bfloat16),                # F*2 not 16-aligned
]


@pytest.mark.parametrize("case", EDGE)
def test_edge_cases(case, dev):
    q_lens, k_lens, cache, Fs, msq, mcl, local, init, dtype = case
    d = workloads.maxpool_inputs(q_lens, F=Fs, H=2, seed=9, k_lens=k_lens, cache=cache)
    d["input"] = torch.randn(d["input"].shape, generator=torch.Generator().manual_seed(3)).to(dtype)
    kw = dict(max_seqlen_q=msq, max_context_len=mcl, local_blocks=local, init_blocks=init)
    out = _run(d, dev, **kw)
    _check(d, out, **kw)


def test_generic_window_path(dev):
    # block_size / stride = 2 (3-tap windows) runs the general kernel
    d = workloads.maxpool_inputs([50, 77], F=24, H=3, seed=2, k_lens=[20, 24], cache=[1, 0])
    kw = dict(max_seqlen_q=24 * 8, max_context_len=500, local_blocks=1, init_blocks=1,
              block_size=16, stride=8)
    out = _run(d, dev, **kw)
    _check(d, out, **kw)


def test_flat_overrun_taps_absent(dev):
    # F = 4 < Lk = 6: the last rows' windows run past the input (reference: out of bounds)
    x = torch.arange(2 * 3 * 4, dtype=torch.float32).reshape(2, 3, 4)
    d = dict(input=x, cu_seqlens_q=torch.tensor([0, 3], dtype=torch.int32),
             cu_seqlens_k=torch.tensor([0, 6], dtype=torch.int32),
             cache_lens=torch.zeros(1, dtype=torch.int32))
    kw = dict(max_seqlen_q=64, max_context_len=128, local_blocks=-1, init_blocks=0)
    out = _run(d, dev, **kw)
    exp = oracle_pool(d["input"], d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                      oob="absent", **kw)
    np.testing.assert_array_equal(out.cpu().numpy(), exp)


def test_row_start_past_end_raises(dev):
    x = torch.zeros(2, 3, 4, device=dev)
    cu = torch.tensor([0, 3], dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        max_pooling_1d_varlen(x, cu, cu, torch.zeros(1, dtype=torch.int32, device=dev),
                              max_seqlen_q=16 * 5, max_context_len=64, local_blocks=1,
                              init_blocks=1)
