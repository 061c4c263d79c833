"""Top-k block ids -> paged KV slot table on gfx950.

Drop-in for ``unum_ops.sparse_kernel_extension``
(``src/unum_ops/sparse_kernel_extension/__init__.py:1-21``) and for the CUDA
extension's ``get_block_table_v1/_v2/_v3`` call shape
(``test/test_sparse_kernel.py:148-155``).  Every name runs the same HIP
kernel of ``libunum_ops_amd.so``.
"""

import torch

from .. import _lib
from .._common import as_i32, require_gpu

SPARSE_BLOCK = 64  # kSparseBlockSize, get_table_torch.py:13


def _block_table(op, topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q, topk,
                 head_group):
    dev = require_gpu(op, topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q)
    if topk_idx.dim() != 3 or block_table.dim() != 2:
        raise ValueError(f"{op}: topk_idx must be [H, T, K] and block_table [B, L]")
    H, T, K = topk_idx.shape
    B, L = block_table.shape
    if topk is not None:
        assert topk == K, f"topk={topk} != K={K}"
    head_group = H if head_group is None else int(head_group)
    idx = topk_idx if topk_idx.dtype == torch.int32 else as_i32(topk_idx, "topk_idx", op)
    bt = as_i32(block_table, "block_table", op) if (
        block_table.dtype != torch.int32 or block_table.stride(1) != 1) else block_table
    bs = as_i32(token_to_bs, "token_to_bs", op).reshape(-1)
    pos = as_i32(token_pos_in_bs, "token_pos_in_bs", op).reshape(-1)
    slen = as_i32(seqlen_q, "seqlen_q", op).reshape(-1)
    if bs.numel() != T:
        raise ValueError(f"{op}: token_to_bs has {bs.numel()} entries, expected T={T}")
    out = torch.empty(T, H, K * SPARSE_BLOCK, dtype=torch.int32, device=dev)
    if out.numel() == 0:
        return out
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_get_block_table(
            _lib.ptr(idx), idx.stride(0), idx.stride(1), idx.stride(2),
            _lib.ptr(bt), bt.stride(0), _lib.ptr(bs),
            _lib.ptr(pos), pos.numel(), _lib.ptr(slen), slen.numel(),
            _lib.ptr(out), H, T, K, B, L, head_group, _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out


def get_block_table(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                    topk=None, *, head_group=None):
    """int32 ``[T, H, K*64]`` of KV slots for the selected blocks.

    Entry ``(t, h, 64k+o)`` is ``head_group * block_table[b, min(p, L-1)] + h``
    for ``p = topk_idx[h, t, k]*64 + o`` and ``b = token_to_bs[t]`` when
    ``0 <= p < seqlen_q[b]`` and ``p < token_pos_in_bs[t]`` (a one-element
    ``seqlen_q`` / ``token_pos_in_bs`` broadcasts), else 0 -- so a ``-1`` id
    gives a run of zeros (``get_table_torch.py:4-44``,
    ``get_table_triton.py:6-67``).

    ``head_group`` defaults to ``H`` (``topk_idx.shape[0]``), the multiplier
    of the exported Triton functions (``get_table_triton.py:259``, ``:315``,
    ``:364``); ``get_block_table_ref_torch`` below uses the torch reference's
    constant ``kHeadGroup = 2`` (``get_table_torch.py:12``).  The two agree
    for ``H == 2``.

    ``topk`` must equal K when given (``get_table_triton.py:231-232``).  A
    token whose ``token_to_bs`` is outside ``[0, B)`` gets a zero row (the
    torch reference raises an IndexError there).  A valid position at or past
    ``L`` reads ``block_table[b, L-1]`` as the torch reference's clamp does
    (the Triton kernels read past the row there).
    """
    return _block_table("get_block_table", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, head_group)


def get_block_table_ref_torch(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                              topk=None):
    """``get_table_torch.py:4-44``: the head multiplier is ``kHeadGroup = 2``."""
    return _block_table("get_block_table_ref_torch", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, 2)


def get_block_table_ref_triton(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                               topk=None):
    """``get_table_triton.py:218-264``: the head multiplier is ``H``."""
    return _block_table("get_block_table_ref_triton", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, None)


def get_block_table_ref_triton_v2(topk_idx, block_table, token_to_bs, token_pos_in_bs,
                                  seqlen_q, topk=None):
    """``get_table_triton.py:323-369``: the head multiplier is ``H``."""
    return _block_table("get_block_table_ref_triton_v2", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, None)


def get_block_table_ref_triton_v3(topk_idx, block_table, token_to_bs, token_pos_in_bs,
                                  seqlen_q, topk=None):
    """``get_table_triton.py:267-320``: the head multiplier is ``H``."""
    return _block_table("get_block_table_ref_triton_v3", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, None)


def get_block_table_v1(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                       topk=None):
    """The CUDA extension's ``get_block_table_v1`` call shape
    (``test/test_sparse_kernel.py:148-155``).  That extension ships compiled
    only, and its tests compare it with the other functions at ``H == 2``
    alone, so its multiplier for other ``H`` is not pinned; this build takes
    the torch reference's constant ``kHeadGroup = 2`` (``get_table_torch.py:12``).
    """
    return _block_table("get_block_table_v1", topk_idx, block_table, token_to_bs,
                        token_pos_in_bs, seqlen_q, topk, 2)


# The reference package exports its Triton function under these names too
# (sparse_kernel_extension/__init__.py:7-12): multiplier H.
get_block_table_v2 = get_block_table_ref_triton
get_block_table_v3 = get_block_table_ref_triton

__all__ = [
    "get_block_table",
    "get_block_table_v1",
    "get_block_table_v2",
    "get_block_table_v3",
    "get_block_table_ref_torch",
    "get_block_table_ref_triton",
    "get_block_table_ref_triton_v2",
    "get_block_table_ref_triton_v3",
]
