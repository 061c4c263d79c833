"""InfLLM-v2 selection ops on gfx950: stage-1 block scores and the varlen max-pool.

Drop-in for ``unum_ops.infllm_v2`` (``src/unum_ops/infllm_v2/__init__.py:1-17``):
the same names, argument lists, ``cu_seqlens`` conventions and output layouts.
Every name here runs the hand-written HIP kernels of ``libunum_ops_amd.so``;
the reference's Triton/torch variant names are kept as aliases so imports keep
working.
"""

import math

import torch

from .. import _lib
from .._common import as_i32, as_int, require_gpu

_OUT_DTYPES = {torch.float32: _lib.UNUM_DTYPE_F32, torch.bfloat16: _lib.UNUM_DTYPE_BF16}
_POOL_DTYPES = {
    torch.float32: _lib.UNUM_DTYPE_F32,
    torch.bfloat16: _lib.UNUM_DTYPE_BF16,
    torch.float16: _lib.UNUM_DTYPE_F16,
}


def round_multiple(x, m):
    """``infllmv2_attn_stage1_triton_v2.py:6-7``."""
    return (x + m - 1) // m * m


def infllmv2_attn_stage1(q, k, v, cu_seqlens_q, cu_seqlens_k, cu_seqlens_v=None,
                         max_seqlen_q=None, max_seqlen_k=None, dropout_p=0.0,
                         softmax_scale=None, causal=False, window_size=(-1, -1),
                         softcap=0.0, alibi_slopes=None, deterministic=False,
                         return_attn_probs=True, block_table=None, *,
                         out_dtype=torch.float32):
    """Stage-1 scores ``[Hkv, total_q, round_up(max_seqlen_k, 128)]``.

    Signature of ``infllmv2_attn_stage1_triton_v2``
    (``infllmv2_attn_stage1_triton_v2.py:153-171``).  As in the reference only
    ``q, k, cu_seqlens_q, cu_seqlens_k, max_seqlen_k, softmax_scale, causal``
    are used; ``v`` and the flash-attention style arguments are accepted and
    ignored.  q/k are read as bf16 (the reference casts loaded values to bf16,
    ``:80-85``, ``:97-103``).

    The scores are fp32 (``out_dtype=torch.bfloat16`` gives the reference's
    storage dtype).  Differences from the reference, all where it is
    undefined or raises later: ``Hq`` not a multiple of ``Hkv`` raises
    ``ValueError``; keys of a sequence beyond the output's columns (a
    ``max_seqlen_k`` smaller than a real length) are dropped instead of
    written past the row.
    """
    op = "infllmv2_attn_stage1"
    dev = require_gpu(op, q, k, cu_seqlens_q, cu_seqlens_k)
    if out_dtype not in _OUT_DTYPES:
        raise ValueError(f"{op}: out_dtype must be float32 or bfloat16, got {out_dtype}")
    if q.dim() != 3 or k.dim() != 3:
        raise ValueError(f"{op}: q must be [total_q, Hq, D] and k [total_k, Hkv, D]")
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    if q.dtype != torch.bfloat16:
        q = q.to(torch.bfloat16)
    if k.dtype != torch.bfloat16:
        k = k.to(torch.bfloat16)
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    total_q, n_heads, head_dim = q.shape
    total_k, n_kv_heads, k_dim = k.shape
    if k_dim != head_dim:
        raise ValueError(f"{op}: head dims differ (q {head_dim}, k {k_dim})")
    if n_kv_heads == 0 or n_heads % n_kv_heads != 0:
        raise ValueError(f"{op}: Hq={n_heads} is not a multiple of Hkv={n_kv_heads}")
    batch = cu_seqlens_q.numel() - 1
    cu_q = as_i32(cu_seqlens_q, "cu_seqlens_q", op)
    cu_k = as_i32(cu_seqlens_k, "cu_seqlens_k", op)
    if cu_k.numel() != batch + 1:
        raise ValueError(f"{op}: cu_seqlens_k has {cu_k.numel()} entries, expected {batch + 1}")
    if max_seqlen_k is None or as_int(max_seqlen_k, "max_seqlen_k", op) == 0:
        # The reference syncs here too (one read per sequence, ``:182-183``).
        max_seqlen_k = int((cu_k[1:] - cu_k[:-1]).max().item()) if batch > 0 else 0
    max_seqlen_k = as_int(max_seqlen_k, "max_seqlen_k", op)
    cols = round_multiple(max_seqlen_k, 128) if max_seqlen_k > 0 else 0
    if cols == 0 or total_q == 0 or batch <= 0:
        return torch.zeros(n_kv_heads, total_q, cols, device=dev, dtype=out_dtype)
    out = torch.empty(n_kv_heads, total_q, cols, device=dev, dtype=out_dtype)
    if total_k == 0:
        return out.zero_()
    lib = _lib.load()
    with _lib.device_guard(dev):
        # Rows over 512 keys split their keys between workgroups through a
        # small workspace (about 1 KiB per 16 rows and split); decode
        # batches run one workgroup per row and need none.
        ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(
            batch, total_q, n_heads, n_kv_heads, head_dim, max_seqlen_k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        st = lib.unum_infllmv2_attn_stage1(
            _lib.ptr(q), q.stride(0), q.stride(1),
            _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(cu_q), _lib.ptr(cu_k),
            _lib.ptr(out), _OUT_DTYPES[out_dtype],
            batch, total_q, total_k, n_heads, n_kv_heads, head_dim,
            max_seqlen_k, cols, float(softmax_scale), 1 if causal else 0,
            _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


def max_pooling_1d_varlen(input, cu_seqlens_q, cu_seqlens_k, cache_lens, max_seqlen_q,
                          max_context_len, local_blocks, init_blocks, block_size=64,
                          stride=16, total_q=-1):
    """Pooled block scores ``[H, total_q, ceil(max_context_len / block_size)]``.

    Signature of ``max_pooling_1d_varlen_ref_triton``
    (``max_pooling_1d_varlen.py:127-139``): ``total_q`` is ignored (taken from
    ``input.shape``, ``:140``) and the padding is fixed at 1 (``:177``).  The
    input is read flat with row stride ``max_seqlen_q // stride`` (``:146``,
    ``:82``), as the reference does.  The output has the input's dtype.

    Differences from the reference, all where it is undefined: a flat row
    stride that puts a row start past the end of the input raises
    ``ValueError``; a tap whose flat address is past the end is treated as
    absent; a non-contiguous input is made contiguous first.
    """
    op = "max_pooling_1d_varlen"
    dev = require_gpu(op, input, cu_seqlens_q, cu_seqlens_k, cache_lens)
    if input.dim() != 3:
        raise ValueError(f"{op}: input must be [H, total_q, *]")
    if input.dtype not in _POOL_DTYPES:
        raise TypeError(f"{op}: unsupported input dtype {input.dtype}")
    num_heads, n_q, _ = input.shape
    batch = cu_seqlens_q.shape[0] - 1
    max_seqlen_q = as_int(max_seqlen_q, "max_seqlen_q", op)
    max_context_len = as_int(max_context_len, "max_context_len", op)
    max_blocks = math.ceil(max_context_len / block_size)
    flat_stride = max_seqlen_q // stride
    out = torch.empty(num_heads, n_q, max_blocks, dtype=input.dtype, device=dev)
    if out.numel() == 0:
        return out
    x = input if input.is_contiguous() else input.contiguous()
    cu_q = as_i32(cu_seqlens_q, "cu_seqlens_q", op)
    cu_k = as_i32(cu_seqlens_k, "cu_seqlens_k", op)
    cache = as_i32(cache_lens, "cache_lens", op).reshape(-1)
    if cu_k.numel() < batch + 1 or cache.numel() < batch:
        raise ValueError(f"{op}: cu_seqlens_k / cache_lens shorter than the batch ({batch})")
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_max_pooling_1d_varlen(
            _lib.ptr(x), x.numel(), _POOL_DTYPES[x.dtype],
            _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(cache), _lib.ptr(out),
            num_heads, n_q, batch, flat_stride, max_blocks,
            int(block_size), int(stride), int(local_blocks), int(init_blocks),
            _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


def infllmv2_attn_stage1_maxpool(q, k, cu_seqlens_q, cu_seqlens_k, max_context_len,
                                 max_seqlen_k=None, softmax_scale=None, causal=True,
                                 local_blocks=1, init_blocks=1, block_size=64, stride=16,
                                 return_scores=False):
    """Pooled block scores ``[Hkv, total_q, ceil(max_context_len / 64)]`` (fp32).

    Equal to ``max_pooling_1d_varlen(infllmv2_attn_stage1(q, k, None,
    cu_seqlens_q, cu_seqlens_k, max_seqlen_k=..., causal=...), cu_seqlens_q,
    cu_seqlens_k, zeros, max_seqlen_q=16 * Kp, max_context_len, local_blocks,
    init_blocks)`` -- each row pooled in place, as the selection pipeline
    chains the two ops -- computed in one kernel, so the fp32 scores only go
    to HBM when ``return_scores`` asks for them (then ``(pooled, scores)``):
    rows of at most 512 keys pool in the LDS-resident stage-1 kernel, longer
    rows in the key-streaming kernels.  Shapes off the MFMA paths (G != 16,
    D != 128, ...) and ``block_size / stride`` other than 64 / 16 run the two
    ops separately.
    """
    op = "infllmv2_attn_stage1_maxpool"
    dev = require_gpu(op, q, k, cu_seqlens_q, cu_seqlens_k)
    if block_size != 64 or stride != 16 or q.dim() != 3 or k.dim() != 3 \
            or q.shape[1] != 16 * k.shape[1] or q.shape[2] != 128:
        sc = infllmv2_attn_stage1(q, k, None, cu_seqlens_q, cu_seqlens_k,
                                  max_seqlen_k=max_seqlen_k, softmax_scale=softmax_scale,
                                  causal=causal)
        batch = cu_seqlens_q.shape[0] - 1
        pooled = max_pooling_1d_varlen(sc, cu_seqlens_q, cu_seqlens_k,
                                       torch.zeros(max(batch, 1), dtype=torch.int32, device=dev),
                                       max_seqlen_q=stride * sc.shape[-1],
                                       max_context_len=max_context_len,
                                       local_blocks=local_blocks, init_blocks=init_blocks,
                                       block_size=block_size, stride=stride)
        return (pooled, sc) if return_scores else pooled
    if q.stride(-1) != 1:
        q = q.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    if q.dtype != torch.bfloat16:
        q = q.to(torch.bfloat16)
    if k.dtype != torch.bfloat16:
        k = k.to(torch.bfloat16)
    if softmax_scale is None:
        softmax_scale = q.shape[-1] ** (-0.5)
    total_q, n_heads, head_dim = q.shape
    total_k, n_kv_heads, _ = k.shape
    batch = cu_seqlens_q.numel() - 1
    cu_q = as_i32(cu_seqlens_q, "cu_seqlens_q", op)
    cu_k = as_i32(cu_seqlens_k, "cu_seqlens_k", op)
    if cu_k.numel() != batch + 1:
        raise ValueError(f"{op}: cu_seqlens_k has {cu_k.numel()} entries, expected {batch + 1}")
    if max_seqlen_k is None or as_int(max_seqlen_k, "max_seqlen_k", op) == 0:
        max_seqlen_k = int((cu_k[1:] - cu_k[:-1]).max().item()) if batch > 0 else 0
    max_seqlen_k = as_int(max_seqlen_k, "max_seqlen_k", op)
    cols = round_multiple(max_seqlen_k, 128) if max_seqlen_k > 0 else 0
    nb = math.ceil(as_int(max_context_len, "max_context_len", op) / block_size)
    pooled = torch.empty(n_kv_heads, total_q, nb, device=dev, dtype=torch.float32)
    scores = torch.empty(n_kv_heads, total_q, cols, device=dev, dtype=torch.float32) \
        if return_scores else None
    if cols == 0 or total_k == 0 or batch <= 0 or softmax_scale <= 0:
        # No keys, or a scale the fused kernels do not take: the two ops.
        return _unfused(q, k, cu_q, cu_k, max_seqlen_k, softmax_scale, causal, max_context_len,
                        local_blocks, init_blocks, return_scores, dev)
    if pooled.numel() == 0:
        return (pooled, scores) if return_scores else pooled
    lib = _lib.load()
    with _lib.device_guard(dev):
        # The key-split workspace of stage 1: rows over 512 keys then pool in
        # the split kernels' second pass.
        ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(
            batch, total_q, n_heads, n_kv_heads, head_dim, max_seqlen_k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        st = lib.unum_infllmv2_attn_stage1_maxpool(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(scores), _lib.ptr(pooled),
            batch, total_q, total_k, n_heads, n_kv_heads, head_dim, max_seqlen_k, cols,
            float(softmax_scale), 1 if causal else 0, nb, int(local_blocks), int(init_blocks),
            _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    if st == _lib.UNUM_ERR_UNSUPPORTED:
        # a layout off the MFMA paths (e.g. unaligned q/k): the two ops take it
        return _unfused(q, k, cu_q, cu_k, max_seqlen_k, softmax_scale, causal, max_context_len,
                        local_blocks, init_blocks, return_scores, dev)
    _lib.check(st, op)
    return (pooled, scores) if return_scores else pooled


def _unfused(q, k, cu_q, cu_k, max_seqlen_k, softmax_scale, causal, max_context_len,
             local_blocks, init_blocks, return_scores, dev):
    sc = infllmv2_attn_stage1(q, k, None, cu_q, cu_k, max_seqlen_k=max_seqlen_k,
                              softmax_scale=softmax_scale, causal=causal)
    batch = cu_q.numel() - 1
    pooled = max_pooling_1d_varlen(sc, cu_q, cu_k,
                                   torch.zeros(max(batch, 1), dtype=torch.int32, device=dev),
                                   max_seqlen_q=16 * max(sc.shape[-1], 1),
                                   max_context_len=max_context_len,
                                   local_blocks=local_blocks, init_blocks=init_blocks)
    return (pooled, sc) if return_scores else pooled


# Names exported by the reference package (``src/unum_ops/infllm_v2/__init__.py``).
infllmv2_attn_stage1_triton = infllmv2_attn_stage1
infllmv2_attn_stage1_triton_v2 = infllmv2_attn_stage1
max_pooling_1d_varlen_ref_triton = max_pooling_1d_varlen

__all__ = [
    "infllmv2_attn_stage1",
    "infllmv2_attn_stage1_maxpool",
    "infllmv2_attn_stage1_triton",
    "infllmv2_attn_stage1_triton_v2",
    "max_pooling_1d_varlen",
    "max_pooling_1d_varlen_ref_triton",
]
