"""The InfLLM-v2 block-selection pipeline: stage 1 -> max-pool -> top-k -> block table.

The reference has no driver for the whole path (its real caller is an
sglang-style InfLLM-v2 attention backend outside the repository); the order
follows from the layouts of its three ops:

1. ``infllmv2_attn_stage1`` gives per-kv-head scores ``[Hkv, Tq, Kp]`` over
   the compressed keys (``infllmv2_attn_stage1_triton_v2.py:153-228``);
2. ``max_pooling_1d_varlen`` reads that tensor flat with row stride
   ``max_seqlen_q // 16``, so the pipeline passes ``max_seqlen_q = 16 * Kp``
   and each row is read in place (``max_pooling_1d_varlen.py:127-183``);
3. a top-k picks the ``topk`` best 64-token blocks per (head, token), ties
   going to the lower block id;
   the ids are sorted ascending as the reference's tests sort them
   (``test/test_sparse_kernel.py:42-43``) and blocks whose pooled score is
   ``-inf`` (no compressed key in the window) become ``-1``;
4. ``get_block_table`` turns the block ids into physical KV slots
   (``get_table_torch.py:4-44``).

Keys are compressed over the whole context (cached + new tokens), so the
max-pool's ``cache_lens`` are zero: ``cu_seqlens_k`` already counts every
compressed key of each sequence.
"""

import math

import torch

from ._common import require_gpu
from .infllm_v2 import infllmv2_attn_stage1, max_pooling_1d_varlen
from .sparse_kernel_extension import get_block_table


def topk_blocks(pooled, topk):
    """Top-``topk`` block ids per row of ``pooled [H, T, NB]``, sorted ascending,
    int32; among equal scores the lower id wins; ids whose score is ``-inf``
    are ``-1``.  ``topk`` larger than ``NB`` pads with ``-1``."""
    H, T, NB = pooled.shape
    k = min(topk, NB)
    # Neighbouring windows share a tap, so equal pooled scores are common; a
    # stable descending sort breaks ties toward the lower block id, which makes
    # the selection deterministic (torch.topk leaves tie order unspecified).
    vals, idx = torch.sort(pooled, dim=-1, descending=True, stable=True)
    vals, idx = vals[..., :k], idx[..., :k]
    idx = torch.where(vals == float("-inf"), torch.full_like(idx, -1), idx)
    idx = idx.sort(dim=-1).values.to(torch.int32)
    if k < topk:
        pad = torch.full((H, T, topk - k), -1, dtype=torch.int32, device=pooled.device)
        idx = torch.cat([pad, idx], dim=-1)
    return idx


def select_blocks(q, k, cu_seqlens_q, cu_seqlens_k, block_table, token_to_bs, token_pos_in_bs,
                  seqlen_q, max_context_len, *, max_seqlen_k=None, softmax_scale=None,
                  causal=True, topk=64, local_blocks=1, init_blocks=1, block_size=64,
                  stride=16, head_group=2, return_intermediates=False):
    """Physical KV slots ``int32 [Tq, Hkv, topk * 64]`` of the blocks each query
    token attends to.

    ``q [Tq, Hq, D]`` and compressed ``k [Tk, Hkv, D]`` are packed by
    ``cu_seqlens_q`` / ``cu_seqlens_k``; ``block_table [B, L]`` maps token
    positions of sequence b to slots; ``token_to_bs`` / ``token_pos_in_bs`` /
    ``seqlen_q`` are the block-table op's per-token and per-sequence inputs;
    ``max_context_len`` sets the number of 64-token blocks.  With
    ``return_intermediates`` the scores, pooled scores and block ids are
    returned too, as ``(table, scores, pooled, topk_idx)``.
    """
    op = "select_blocks"
    dev = require_gpu(op, q, k, cu_seqlens_q, cu_seqlens_k, block_table)
    scores = infllmv2_attn_stage1(q, k, None, cu_seqlens_q, cu_seqlens_k,
                                  max_seqlen_k=max_seqlen_k, softmax_scale=softmax_scale,
                                  causal=causal)
    kp = scores.shape[-1]
    batch = cu_seqlens_q.numel() - 1
    cache = torch.zeros(max(batch, 1), dtype=torch.int32, device=dev)
    pooled = max_pooling_1d_varlen(scores, cu_seqlens_q, cu_seqlens_k, cache,
                                   max_seqlen_q=stride * kp, max_context_len=max_context_len,
                                   local_blocks=local_blocks, init_blocks=init_blocks,
                                   block_size=block_size, stride=stride)
    idx = topk_blocks(pooled, topk)
    table = get_block_table(idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                            head_group=head_group)
    if return_intermediates:
        return table, scores, pooled, idx
    return table


def num_blocks(max_context_len, block_size=64):
    """Blocks of the pooled output: ``ceil(max_context_len / block_size)``."""
    return math.ceil(max_context_len / block_size)


__all__ = ["select_blocks", "topk_blocks", "num_blocks"]
