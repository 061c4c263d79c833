"""GPU parity of the whole selection pipeline (stage 1 -> max-pool -> top-k ->
block table) on the chunked-prefill/decode mix and the long-context chunk.

Each stage is checked against the oracle on the same input the GPU stage saw:
stage-1 scores within atol 1e-3 / rtol 1e-2 of the fp32 oracle, the max-pool
of the GPU scores bit-exact, the top-k ids equal to the oracle's top-k of the
GPU pooled scores, and the block table of those ids bit-exact.  The block ids the
oracle end to end selects may differ from the GPU's only where two pooled
scores are within rounding of each other, so their agreement is a recall
figure, not an equality.
"""

import numpy as np
import pytest
import torch

import oracle
import workloads
from unum_ops_amd.pipeline import select_blocks

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2   # stage-1 scores vs the fp32 oracle
TOPK = 64


def _to(d, dev):
    return {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in d.items()}


def _check_pipeline(p, dev, min_recall):
    g = _to(p, dev)
    table, scores, pooled, idx = select_blocks(
        g["q"], g["k"], g["cu_seqlens_q"], g["cu_seqlens_k"], g["block_table"],
        g["token_to_bs"], g["token_pos_in_bs"], g["seqlen_q"], p["max_context_len"],
        max_seqlen_k=p["max_seqlen_k"], topk=TOPK, return_intermediates=True)
    torch.cuda.synchronize()
    scores_c, pooled_c, idx_c = scores.cpu(), pooled.cpu(), idx.cpu()

    exp_s = oracle.infllmv2_attn_stage1(p["q"], p["k"], None, p["cu_seqlens_q"],
                                        p["cu_seqlens_k"], max_seqlen_k=p["max_seqlen_k"],
                                        causal=True)
    torch.testing.assert_close(scores_c, exp_s, atol=ATOL, rtol=RTOL)

    kp = scores.shape[-1]
    B = p["cu_seqlens_q"].numel() - 1
    cache = torch.zeros(B, dtype=torch.int32)
    exp_p = oracle.max_pooling_1d_varlen(scores_c, p["cu_seqlens_q"], p["cu_seqlens_k"], cache,
                                         16 * kp, p["max_context_len"], 1, 1)
    np.testing.assert_array_equal(pooled_c.numpy(), exp_p)

    np.testing.assert_array_equal(idx_c.numpy(), oracle.topk_blocks(pooled_c, TOPK))

    # select_blocks multiplies by H, as the reference's exported Triton
    # functions do (get_table_triton.py:259).
    exp_t = oracle.get_block_table(idx_c, p["block_table"], p["token_to_bs"],
                                   p["token_pos_in_bs"], p["seqlen_q"],
                                   head_group=idx_c.shape[0])
    np.testing.assert_array_equal(table.cpu().numpy(), exp_t)

    # Without intermediates, stage 1 pools in its kernel and the top-k runs
    # over the pooled rows: the same table, bit for bit.
    fast = select_blocks(
        g["q"], g["k"], g["cu_seqlens_q"], g["cu_seqlens_k"], g["block_table"],
        g["token_to_bs"], g["token_pos_in_bs"], g["seqlen_q"], p["max_context_len"],
        max_seqlen_k=p["max_seqlen_k"], topk=TOPK)
    assert torch.equal(fast, table)

    # Selection agreement with the all-oracle pipeline.
    ref_pool = torch.from_numpy(oracle.max_pooling_1d_varlen(
        exp_s, p["cu_seqlens_q"], p["cu_seqlens_k"], cache, 16 * kp, p["max_context_len"], 1, 1))
    ref_idx = oracle.topk_blocks(ref_pool, TOPK)
    got = idx_c.numpy()
    hits = total = 0
    for h in range(got.shape[0]):
        for t in range(got.shape[1]):
            a = set(ref_idx[h, t][ref_idx[h, t] >= 0].tolist())
            if a:
                hits += len(a & set(got[h, t].tolist()))
                total += len(a)
    assert total > 0
    assert hits / total >= min_recall, f"recall {hits / total:.4f}"


def test_cfg4_decode_mix(dev):
    _check_pipeline(workloads.cfg4_pipeline(), dev, min_recall=0.99)


@pytest.mark.parametrize("heads", [(32, 2), (16, 1)])
def test_cfg5_long_context(heads, dev):
    _check_pipeline(workloads.cfg5_pipeline(Hq=heads[0], Hkv=heads[1]), dev, min_recall=0.99)


def test_small_contexts_pad_with_minus_one(dev):
    # Contexts shorter than topk blocks: the ids are padded with -1, which the
    # block table turns into runs of zeros.
    p = workloads.pipeline_inputs([5, 9], [300, 1000], seed=3)
    _check_pipeline(p, dev, min_recall=1.0)
