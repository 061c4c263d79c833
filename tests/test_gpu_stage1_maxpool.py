"""GPU parity of the fused stage-1 + max-pool entry point (fused in the
LDS-resident kernel for rows of at most 512 keys, in the K-streaming kernels
for longer rows).

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
import workloads
from unum_ops_amd import _lib
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
    # tokens (511 keys) take the LDS-resident kernel, 9000 (561) the
    # streaming one; ctx_extra 2000 puts pooled blocks past the score row.
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


def _fused_c(d, dev, max_context_len, local_blocks, init_blocks, causal, workspace):
    """The fused entry point through the C-ABI, with the key-split workspace
    (key splits, pooling in their second pass) or without it (whole rows)."""
    lib = _lib.load()
    q, k = d["q"].to(dev), d["k"].to(dev)
    cu_q = d["cu_seqlens_q"].to(torch.int32).to(dev)
    cu_k = d["cu_seqlens_k"].to(torch.int32).to(dev)
    B = cu_q.numel() - 1
    Tq, Hq, D = q.shape
    Tk, Hkv, _ = k.shape
    msk = int(d["max_seqlen_k"])
    cols = (msk + 127) // 128 * 128
    nb = (max_context_len + 63) // 64
    scores = torch.empty(Hkv, Tq, cols, device=dev, dtype=torch.float32)
    pooled = torch.empty(Hkv, Tq, nb, device=dev, dtype=torch.float32)
    ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(B, Tq, Hq, Hkv, D, msk) if workspace else 0
    assert (ws_bytes > 0) == workspace
    ws = torch.empty(ws_bytes, device=dev, dtype=torch.uint8) if workspace else None
    with torch.cuda.device(dev):
        st = lib.unum_infllmv2_attn_stage1_maxpool(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(scores), _lib.ptr(pooled),
            B, Tq, Tk, Hq, Hkv, D, msk, cols, D ** -0.5, 1 if causal else 0, nb,
            local_blocks, init_blocks, _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, "infllmv2_attn_stage1_maxpool")
    torch.cuda.synchronize()
    return pooled.cpu(), scores.cpu()


@pytest.mark.parametrize("workspace", [False, True])
@pytest.mark.parametrize("q_lens,ctx_lens,causal,local_blocks,init_blocks", [
    ([2500], [9000], True, 1, 1),             # prefill: early pieces see few keys
    ([64, 300, 17], [20000, 9000, 70000], True, 2, 3),
    ([40, 33], [5000, 30000], False, 1, 1),
])
def test_key_splits_and_whole_rows(q_lens, ctx_lens, causal, local_blocks, init_blocks,
                                   workspace, dev):
    # Pooling in the key-split kernels' second pass (each later split first
    # computes the chunk before its own to carry in the -1 tap; the split
    # whose chunks end a piece's columns writes the blocks past them) and in
    # the whole-row kernel: the pooled blocks are the max-pool of the scores
    # the same launch wrote, bit for bit.
    d = workloads.stage1_inputs(q_lens, ctx_lens, seed=36, raw_keys=False)
    max_context_len = max(ctx_lens)
    pooled, scores = _fused_c(d, dev, max_context_len, local_blocks, init_blocks, causal,
                              workspace)
    exp_s = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                          max_seqlen_k=d["max_seqlen_k"], causal=causal)
    torch.testing.assert_close(scores, exp_s, atol=1e-3, rtol=1e-2)
    B = d["cu_seqlens_q"].numel() - 1
    exp_p = oracle_pool(scores, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        torch.zeros(B, dtype=torch.int32), 16 * scores.shape[-1],
                        max_context_len, local_blocks, init_blocks)
    np.testing.assert_array_equal(pooled.numpy(), exp_p)
