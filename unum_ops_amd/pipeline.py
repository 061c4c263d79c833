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
   going to the lower block id (fused with step 2 in one kernel,
   ``maxpool_topk``; or, when the scores are not wanted, steps 1 and 2 run
   as one kernel, ``infllmv2_attn_stage1_maxpool``, and ``topk_blocks``
   selects from its pooled rows);
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

from . import _lib
from ._common import as_i32, as_int, require_gpu
from .infllm_v2 import (infllmv2_attn_stage1, infllmv2_attn_stage1_maxpool,
                        max_pooling_1d_varlen)
from .sparse_kernel_extension import get_block_table

FUSED_MAX_BLOCKS = 4096  # the fused pool + top-k kernel keeps a row's blocks in registers


def topk_blocks(pooled, topk):
    """Top-``topk`` block ids per row of ``pooled [H, T, NB]`` on the GPU, sorted
    ascending, int32; among equal scores the lower id wins; ids whose score is
    ``-inf`` are ``-1``; ``topk`` larger than ``NB`` pads with ``-1`` (first).

    The selection of ``maxpool_topk`` over scores already pooled (the output of
    ``infllmv2_attn_stage1_maxpool``), on gfx950 kernels: a row per wave for up
    to 4096 blocks a row, a row per workgroup for wider rows (the
    same selection, its counts summed through LDS), up to 32768 blocks a row
    (contexts of 2M tokens); wider rows are refused.
    """
    op = "topk_blocks"
    dev = require_gpu(op, pooled)
    if pooled.dim() != 3:
        raise ValueError(f"{op}: pooled must be [H, T, NB]")
    topk = as_int(topk, "topk", op)
    if topk < 1:
        raise ValueError(f"{op}: topk must be >= 1, got {topk}")
    H, T, NB = pooled.shape
    x = pooled if pooled.dtype == torch.float32 else pooled.float()  # exact for bf16 / fp16
    if x.stride(-1) != 1 or (T > 1 and x.stride(1) != NB) or (H > 1 and x.stride(0) != T * NB):
        x = x.contiguous()
    out = torch.empty(H, T, topk, dtype=torch.int32, device=dev)
    if out.numel() == 0 or NB == 0:
        return out.fill_(-1) if NB == 0 else out
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_topk_blocks(_lib.ptr(x), H * T, NB, NB, _lib.ptr(out), topk,
                                  _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


def maxpool_topk(input, cu_seqlens_q, cu_seqlens_k, cache_lens, max_seqlen_q, max_context_len,
                 local_blocks, init_blocks, block_size=64, stride=16, topk=64,
                 return_pooled=False):
    """``topk_blocks(max_pooling_1d_varlen(...), topk)`` in one kernel.

    The arguments are those of ``max_pooling_1d_varlen`` plus ``topk``.
    Returns the int32 block ids ``[H, Tq, topk]`` (or ``(ids, pooled)`` with
    ``return_pooled``).  One gfx950 kernel pools each row into registers and
    selects its blocks, so the pooled scores never go through HBM unless
    asked for.  Inputs the fused kernel does not take (a dtype other than fp32,
    ``block_size / stride != 4``, more than 4096 blocks, unaligned rows) run the
    two ops separately, with the same result.
    """
    op = "maxpool_topk"
    dev = require_gpu(op, input, cu_seqlens_q, cu_seqlens_k, cache_lens)
    if input.dim() != 3:
        raise ValueError(f"{op}: input must be [H, total_q, *]")
    topk = as_int(topk, "topk", op)
    if topk < 1:
        raise ValueError(f"{op}: topk must be >= 1, got {topk}")
    H, n_q, _ = input.shape
    max_seqlen_q = as_int(max_seqlen_q, "max_seqlen_q", op)
    max_context_len = as_int(max_context_len, "max_context_len", op)
    nb = math.ceil(max_context_len / block_size)
    flat_stride = max_seqlen_q // stride
    x = input if input.is_contiguous() else input.contiguous()
    fused = (x.dtype == torch.float32 and block_size // stride == 4 and block_size > 0
             and 1 <= nb <= FUSED_MAX_BLOCKS and flat_stride % 4 == 0
             and x.data_ptr() % 16 == 0 and (not return_pooled or nb % 4 == 0))
    if not fused:
        pooled = max_pooling_1d_varlen(x, cu_seqlens_q, cu_seqlens_k, cache_lens, max_seqlen_q,
                                       max_context_len, local_blocks, init_blocks,
                                       block_size=block_size, stride=stride)
        idx = topk_blocks(pooled, topk)
        return (idx, pooled) if return_pooled else idx
    idx = torch.empty(H, n_q, topk, dtype=torch.int32, device=dev)
    pooled = torch.empty(H, n_q, nb, dtype=x.dtype, device=dev) if return_pooled else None
    if idx.numel() == 0:
        return (idx, pooled) if return_pooled else idx
    batch = cu_seqlens_q.shape[0] - 1
    cu_q = as_i32(cu_seqlens_q, "cu_seqlens_q", op)
    cu_k = as_i32(cu_seqlens_k, "cu_seqlens_k", op)
    cache = as_i32(cache_lens, "cache_lens", op).reshape(-1)
    if cu_k.numel() < batch + 1 or cache.numel() < batch:
        raise ValueError(f"{op}: cu_seqlens_k / cache_lens shorter than the batch ({batch})")
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_max_pooling_1d_varlen_topk(
            _lib.ptr(x), x.numel(), _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(cache),
            _lib.ptr(pooled), _lib.ptr(idx), H, n_q, batch, flat_stride, nb,
            int(block_size), int(stride), int(local_blocks), int(init_blocks), topk,
            _lib.stream_ptr(dev))
    _lib.check(st, op)
    return (idx, pooled) if return_pooled else idx


def select_blocks(q, k, cu_seqlens_q, cu_seqlens_k, block_table, token_to_bs, token_pos_in_bs,
                  seqlen_q, max_context_len, *, max_seqlen_k=None, softmax_scale=None,
                  causal=True, topk=64, local_blocks=1, init_blocks=1, block_size=64,
                  stride=16, head_group=None, return_intermediates=False):
    """Physical KV slots ``int32 [Tq, Hkv, topk * 64]`` of the blocks each query
    token attends to.

    ``q [Tq, Hq, D]`` and compressed ``k [Tk, Hkv, D]`` are packed by
    ``cu_seqlens_q`` / ``cu_seqlens_k``; ``block_table [B, L]`` maps token
    positions of sequence b to slots; ``token_to_bs`` / ``token_pos_in_bs`` /
    ``seqlen_q`` are the block-table op's per-token and per-sequence inputs;
    ``max_context_len`` sets the number of 64-token blocks; ``head_group``
    is the slot multiplier of ``get_block_table`` (default ``Hkv``, as the
    reference's exported Triton functions use).  With
    ``return_intermediates`` the scores, pooled scores and block ids are
    returned too, as ``(table, scores, pooled, topk_idx)``.
    """
    op = "select_blocks"
    dev = require_gpu(op, q, k, cu_seqlens_q, cu_seqlens_k, block_table)
    if not return_intermediates:
        # The scores are not wanted: stage 1 pools its rows in the kernel
        # (the score tensor never goes to HBM), then the top-k runs over the
        # pooled rows -- the same ids as the chain below, bit for bit.
        pooled = infllmv2_attn_stage1_maxpool(q, k, cu_seqlens_q, cu_seqlens_k, max_context_len,
                                              max_seqlen_k=max_seqlen_k,
                                              softmax_scale=softmax_scale, causal=causal,
                                              local_blocks=local_blocks, init_blocks=init_blocks,
                                              block_size=block_size, stride=stride)
        idx = topk_blocks(pooled, topk)
        return get_block_table(idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                               head_group=head_group)
    scores = infllmv2_attn_stage1(q, k, None, cu_seqlens_q, cu_seqlens_k,
                                  max_seqlen_k=max_seqlen_k, softmax_scale=softmax_scale,
                                  causal=causal)
    kp = scores.shape[-1]
    batch = cu_seqlens_q.numel() - 1
    cache = torch.zeros(max(batch, 1), dtype=torch.int32, device=dev)
    res = maxpool_topk(scores, cu_seqlens_q, cu_seqlens_k, cache, max_seqlen_q=stride * kp,
                       max_context_len=max_context_len, local_blocks=local_blocks,
                       init_blocks=init_blocks, block_size=block_size, stride=stride,
                       topk=topk, return_pooled=return_intermediates)
    idx, pooled = res if return_intermediates else (res, None)
    table = get_block_table(idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                            head_group=head_group)
    if return_intermediates:
        return table, scores, pooled, idx
    return table


def num_blocks(max_context_len, block_size=64):
    """Blocks of the pooled output: ``ceil(max_context_len / block_size)``."""
    return math.ceil(max_context_len / block_size)


__all__ = ["select_blocks", "maxpool_topk", "topk_blocks", "num_blocks"]
