"""Stage-2 sparse attention over the block table's KV slots on gfx950.

The consumer of ``get_block_table``'s output.  The reference ships no portable
implementation of it: its tests hand the table to an NPU paged-attention
operator (``test/test_pa.py:48-71``, ``torch_npu._npu_paged_attention(query,
key_cache, value_cache, num_heads, num_kv_heads, scale_value, block_table,
context_lens, out)``), with the shapes of ``test/test_pa.py:75-80``.  This
module computes the attention those slots define, on one gfx950 kernel.
"""

import torch

from . import _lib
from ._common import as_i32, require_gpu

SPARSE_BLOCK = 64
_OUT_DTYPES = {torch.bfloat16: _lib.UNUM_DTYPE_BF16, torch.float32: _lib.UNUM_DTYPE_F32}


def _cache_rows(cache, name, op):
    """(row stride in elements, rows) of a [num_blocks, block_size, Hkv, D]
    cache viewed as rows of D elements, row ((n * block_size) + s) * Hkv + h;
    raises unless those rows are evenly spaced.  Dimensions of size 1 place
    no constraint, so a one-head slice of a larger cache is accepted."""
    if cache.dim() != 4:
        raise ValueError(f"{op}: {name} must be [num_blocks, block_size, num_kv_heads, head_size]")
    nb, bs, hk, d = cache.shape
    s0, s1, s2, s3 = cache.stride()
    row = s2 if hk > 1 else (s1 if bs > 1 else (s0 if nb > 1 else d))
    if s3 != 1 or (hk > 1 and s2 != row) or (bs > 1 and s1 != hk * row) \
            or (nb > 1 and s0 != bs * hk * row):
        raise ValueError(f"{op}: {name} rows must be evenly spaced (unit stride in the head "
                         f"dimension, strides {cache.stride()})")
    return row, nb * bs * hk


def _kernel_q(query):
    """bf16 query with the kernel's layout: unit stride in D, 16-byte aligned
    base and strides that are multiples of 8 elements (else a packed copy)."""
    q = query if query.dtype == torch.bfloat16 else query.to(torch.bfloat16)
    if (q.stride(-1) != 1 or q.data_ptr() % 16 != 0 or q.stride(0) % 8 != 0
            or q.stride(1) % 8 != 0):
        q = q.contiguous()
    return q


def sparse_paged_attention(query, key_cache, value_cache, num_heads, num_kv_heads, scale_value,
                           topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                           out=None, slots=None, out_dtype=torch.bfloat16):
    """Attention of each query head over the KV slots of its block-table row.

    ``query [T, num_heads, D]`` attends, for kv head h, to the entries of
    ``get_block_table(topk_idx, block_table, token_to_bs, token_pos_in_bs,
    seqlen_q)[t, h]`` that the table marks valid (block id >= 0, position
    below ``seqlen_q[b]`` and ``token_pos_in_bs[t]``).  Slot ``s`` of that
    table (computed with the multiplier ``num_kv_heads``, as the reference's
    Triton functions do, ``get_table_triton.py:259``) is row ``s`` of
    ``key_cache.view(-1, D)``: token slot ``block_table[b, p]``, head h of the
    ``[num_blocks, block_size, num_kv_heads, D]`` caches.  Given ``slots``
    (``get_block_table``'s output with that multiplier) the rows are read
    from it instead of recomputed.  Returns ``out [T, num_heads, D]`` (bf16
    unless ``out`` or ``out_dtype`` says fp32); a (token, head) with no valid
    entry gets zeros.  The selection pipeline's shapes: 16 query heads per kv
    head, D = 128, up to 64 blocks per token.
    """
    op = "sparse_paged_attention"
    dev = require_gpu(op, query, key_cache, value_cache, topk_idx, block_table, token_to_bs,
                      token_pos_in_bs, seqlen_q, slots, out)
    if query.dim() != 3 or topk_idx.dim() != 3 or block_table.dim() != 2:
        raise ValueError(f"{op}: query must be [T, H, D], topk_idx [Hkv, T, K], block_table [B, L]")
    T, Hq, D = query.shape
    Hkv, T2, K = topk_idx.shape
    if Hq != num_heads or Hkv != num_kv_heads or T2 != T:
        raise ValueError(f"{op}: shapes disagree (query {tuple(query.shape)}, topk_idx "
                         f"{tuple(topk_idx.shape)}, num_heads {num_heads}, num_kv_heads "
                         f"{num_kv_heads})")
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        raise ValueError(f"{op}: key_cache and value_cache must have one shape and layout")
    if key_cache.shape[2] != Hkv or key_cache.shape[3] != D:
        raise ValueError(f"{op}: caches must be [num_blocks, block_size, {Hkv}, {D}]")
    row_stride, n_rows = _cache_rows(key_cache, "key_cache", op)
    q = _kernel_q(query)
    if key_cache.dtype != torch.bfloat16 or value_cache.dtype != torch.bfloat16:
        raise TypeError(f"{op}: the caches must be bfloat16")
    if out is None:
        if out_dtype not in _OUT_DTYPES:
            raise ValueError(f"{op}: out_dtype must be bfloat16 or float32")
        out = torch.empty(T, Hq, D, dtype=out_dtype, device=dev)
    elif out.shape != (T, Hq, D) or out.dtype not in _OUT_DTYPES or not out.is_contiguous():
        raise ValueError(f"{op}: out must be a contiguous bf16/fp32 [{T}, {Hq}, {D}] tensor")
    if T == 0:
        return out
    idx = topk_idx if topk_idx.dtype == torch.int32 else as_i32(topk_idx, "topk_idx", op)
    bt = as_i32(block_table, "block_table", op) if (
        block_table.dtype != torch.int32 or block_table.stride(1) != 1) else block_table
    B, L = bt.shape
    bs = as_i32(token_to_bs, "token_to_bs", op).reshape(-1)
    pos = as_i32(token_pos_in_bs, "token_pos_in_bs", op).reshape(-1)
    slen = as_i32(seqlen_q, "seqlen_q", op).reshape(-1)
    if bs.numel() != T:
        raise ValueError(f"{op}: token_to_bs has {bs.numel()} entries, expected T={T}")
    sl = None
    if slots is not None:
        if slots.shape != (T, Hkv, K * SPARSE_BLOCK):
            raise ValueError(f"{op}: slots must be [{T}, {Hkv}, {K * SPARSE_BLOCK}]")
        sl = as_i32(slots, "slots", op)
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_sparse_paged_attention(
            _lib.ptr(q), q.stride(0), q.stride(1),
            _lib.ptr(key_cache), _lib.ptr(value_cache), row_stride, n_rows,
            _lib.ptr(idx), idx.stride(0), idx.stride(1), idx.stride(2),
            _lib.ptr(bt), bt.stride(0), _lib.ptr(sl),
            _lib.ptr(bs), _lib.ptr(pos), pos.numel(), _lib.ptr(slen), slen.numel(),
            _lib.ptr(out), _OUT_DTYPES[out.dtype], T, Hq, Hkv, D, K, B, L,
            float(scale_value), _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


def sparse_gather_calibrate(key_cache, value_cache, num_kv_heads, topk_idx, block_table,
                            token_to_bs, token_pos_in_bs, seqlen_q, slots=None):
    """Measurement tool, not part of the attention: gathers every K and V row
    that ``sparse_paged_attention`` with these arguments attends, in its lane
    pattern and pipeline, with no arithmetic but an XOR checksum.  Returns the
    u32 checksums ``[T, Hkv, 64]`` (as int32).  Its duration is the floor the
    gathers alone set for the selection: the roof the attention kernel's time
    is read against."""
    op = "sparse_gather_calibrate"
    dev = require_gpu(op, key_cache, value_cache, topk_idx, block_table, token_to_bs,
                      token_pos_in_bs, seqlen_q, slots)
    Hkv, T, K = topk_idx.shape
    if Hkv != num_kv_heads or key_cache.shape != value_cache.shape \
            or key_cache.stride() != value_cache.stride() or key_cache.shape[2] != Hkv:
        raise ValueError(f"{op}: caches must be two [num_blocks, block_size, {Hkv}, D] tensors "
                         "of one layout")
    row_stride, n_rows = _cache_rows(key_cache, "key_cache", op)
    out = torch.empty(T, Hkv, 64, dtype=torch.int32, device=dev)
    if T == 0:
        return out
    idx = topk_idx if topk_idx.dtype == torch.int32 else as_i32(topk_idx, "topk_idx", op)
    bt = as_i32(block_table, "block_table", op) if (
        block_table.dtype != torch.int32 or block_table.stride(1) != 1) else block_table
    B, L = bt.shape
    bs = as_i32(token_to_bs, "token_to_bs", op).reshape(-1)
    pos = as_i32(token_pos_in_bs, "token_pos_in_bs", op).reshape(-1)
    slen = as_i32(seqlen_q, "seqlen_q", op).reshape(-1)
    sl = None if slots is None else as_i32(slots, "slots", op)
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_sparse_gather_calibrate(
            _lib.ptr(key_cache), _lib.ptr(value_cache), row_stride, n_rows,
            _lib.ptr(idx), idx.stride(0), idx.stride(1), idx.stride(2),
            _lib.ptr(bt), bt.stride(0), _lib.ptr(sl),
            _lib.ptr(bs), _lib.ptr(pos), pos.numel(), _lib.ptr(slen), slen.numel(),
            _lib.ptr(out), T, Hkv, K, B, L, _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


__all__ = ["sparse_paged_attention", "sparse_gather_calibrate"]
