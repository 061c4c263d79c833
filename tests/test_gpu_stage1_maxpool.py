"""GPU parity of the fused stage-1 + max-pool entry point (fused in the
K-streaming kernel for rows over 512 keys; shorter rows run the two ops).

The pooled scores must equal, bit for bit, the max-pool the oracle computes
from the scores the same kernel wrote (``return_scores``), and the scores must
match the stage-1 oracle at atol 1e-3 / rtol 1e-2; without ``return_scores``
the pooled output must be the same bits.
"""

import numpy as np
import pytest
import torch

from oracle.maxpool import max_pooling_1d_varlen as oracle_pool
from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1
from unum_ops_amd import workloads
from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1_maxpool

pytestmark = pytest.mark.gpu


def _check(d, dev, max_context_len, local_blocks=1, init_blocks=1, causal=True):
    args = (d["q"].to(dev), d["k"].to(dev), d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev),
            max_context_len)
    kw = dict(max_seqlen_k=d["max_seqlen_k"], causal=causal, local_blocks=local_blocks,
              init_blocks=init_blocks)
    pooled, scores = infllmv2_attn_stage1_maxpool(*args, return_scores=True, **kw)
    pooled_only = infllmv2_attn_stage1_maxpool(*args, **kw)
    torch.cuda.synchronize()
    exp_s = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                          max_seqlen_k=d["max_seqlen_k"], causal=causal)
    torch.testing.assert_close(scores.cpu(), exp_s, atol=1e-3, rtol=1e-2)
    B = d["cu_seqlens_q"].numel() - 1
    exp_p = oracle_pool(scores.cpu(), d["cu_seqlens_q"], d["cu_seqlens_k"],
                        torch.zeros(B, dtype=torch.int32), 16 * scores.shape[-1],
                        max_context_len, local_blocks, init_blocks)
    np.testing.assert_array_equal(pooled.cpu().numpy(), exp_p)
    assert torch.equal(pooled_only, pooled)


@pytest.mark.parametrize("local_blocks,init_blocks", [(1, 1), (2, 3)])
def test_lds_path_prefill(local_blocks, init_blocks, dev):
    d = workloads.stage1_inputs([300, 64, 1000], [8192, 3000, 8192], seed=31)
    _check(d, dev, 8192, local_blocks, init_blocks)


def test_lds_path_cfg3_slice(dev):
    d = workloads.stage1_inputs([8192], [8192], seed=32)
    _check(d, dev, 8192)


@pytest.mark.parametrize("ctx_extra", [0, 8, 70, 2000])
@pytest.mark.parametrize("ctx", [8200, 9000])
def test_pool_width_vs_score_width(ctx, ctx_extra, dev):
    # max_context_len at or above the keys' span: pooled blocks past the
    # computed columns (the tail) hold at most the carried last tap.  8200
    # tokens (511 keys) take the unfused pair, 9000 (561) the fused kernel.
    d = workloads.stage1_inputs([40, 17], [2000, ctx], seed=33)
    _check(d, dev, ctx + ctx_extra)


def test_stream_path_long_context(dev):
    d = workloads.stage1_inputs([96, 7], [40000, 135168], seed=34, raw_keys=False)
    _check(d, dev, 135168)


def test_non_causal_and_orphans(dev):
    d = workloads.stage1_inputs([20, 30], [3000, 600], seed=35)
    q = torch.cat([torch.randn(5, 32, 128).to(torch.bfloat16), d["q"]])
    d["q"] = q
    d["cu_seqlens_q"] = d["cu_seqlens_q"] + 5
    _check(d, dev, 3000, causal=False)


@pytest.mark.parametrize("q_len", [2500, 9000])
def test_prefill_rows_see_fewer_keys_than_the_pool(q_len, dev):
    # A prefill over 561 keys (the fused kernel): early tokens see few keys,
    # so blocks past the columns their piece computes lie over zero scores
    # below the key count and pool to 0, not -inf.
    d = workloads.stage1_inputs([q_len], [9000], seed=34)
    _check(d, dev, 9000)
