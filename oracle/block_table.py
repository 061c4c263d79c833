"""Oracle: top-k block ids -> paged KV slot table (test infrastructure only).

Restates ``get_block_table_ref_torch``
(``src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44``) in numpy,
step for step:

* ``pos = topk_idx * 64 + arange(64)`` in the index dtype (int32, wrapping),
  ``get_table_torch.py:18-22``;
* ``valid = (pos >= 0) & (pos < seqlen[bs]) & (pos < token_pos_in_bs)``, with
  a one-element ``seqlen_q`` / ``token_pos_in_bs`` broadcast,
  ``get_table_torch.py:22-33``;
* ``vals = block_table[bs, clamp(pos, 0, L-1)]``, ``get_table_torch.py:35-37``;
* ``out = where(valid, 2 * vals + h, 0)`` (the head multiplier is the constant
  ``kHeadGroup = 2``), ``get_table_torch.py:12,39-42``;
* ``permute(1, 0, 2)`` to ``[T, H, K*64]``, ``get_table_torch.py:44``.
"""

import numpy as np

SPARSE_BLOCK = 64  # kSparseBlockSize, get_table_torch.py:13


def _np(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def get_block_table(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                    topk=None, head_group=2):
    """Return int32 ``[T, H, K*64]`` exactly as the torch reference does."""
    idx = _np(topk_idx).astype(np.int32)
    bt = _np(block_table).astype(np.int32)
    bs = _np(token_to_bs).astype(np.int64).reshape(-1)
    plim = _np(token_pos_in_bs).astype(np.int32).reshape(-1)
    slen = _np(seqlen_q).astype(np.int32).reshape(-1)
    H, T, K = idx.shape
    L = bt.shape[1]
    if topk is not None and topk != K:
        raise AssertionError(f"topk={topk} != K={K}")

    off = np.arange(SPARSE_BLOCK, dtype=np.int32)
    with np.errstate(over="ignore"):
        pos = idx[..., None] * np.int32(SPARSE_BLOCK) + off          # [H,T,K,64] int32 wrap
    pos = pos.reshape(H, T, K * SPARSE_BLOCK)
    seqlen = np.broadcast_to(slen, (T,)) if slen.size == 1 else slen[bs]
    limit = np.broadcast_to(plim, (T,)) if plim.size == 1 else plim
    valid = (pos >= 0) & (pos < seqlen[None, :, None]) & (pos < limit[None, :, None])

    safe = np.clip(pos, 0, L - 1)
    vals = bt[bs[None, :, None], safe]                                 # [H,T,K*64]
    heads = np.arange(H, dtype=np.int32)[:, None, None]
    with np.errstate(over="ignore"):
        out = np.int32(head_group) * vals + heads
    out = np.where(valid, out, np.int32(0)).astype(np.int32)
    return np.ascontiguousarray(out.transpose(1, 0, 2))


def get_block_table_torch(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                          head_group=2):
    """The same steps in torch ops on the CPU (every thread torch is given):
    ``block_table[bs]``, the gather at the clamped positions and the ``where``
    of ``get_table_torch.py:18-44``, as the benchmark's CPU baseline times
    them.  Equal bit for bit to :func:`get_block_table`."""
    import torch

    idx = topk_idx.detach().cpu().to(torch.int32)
    bt = block_table.detach().cpu().to(torch.int32)
    bs = token_to_bs.detach().cpu().to(torch.int64).reshape(-1)
    plim = token_pos_in_bs.detach().cpu().to(torch.int32).reshape(-1)
    slen = seqlen_q.detach().cpu().to(torch.int32).reshape(-1)
    H, T, K = idx.shape
    L = bt.shape[1]
    pos = (idx.unsqueeze(-1) * SPARSE_BLOCK +
           torch.arange(SPARSE_BLOCK, dtype=torch.int32)).reshape(H, T, K * SPARSE_BLOCK)
    seqlen = slen.expand(T) if slen.numel() == 1 else slen[bs]
    limit = plim.expand(T) if plim.numel() == 1 else plim
    valid = (pos >= 0) & (pos < seqlen[None, :, None]) & (pos < limit[None, :, None])
    rows = bt[bs]                                                    # [T, L]
    vals = torch.gather(rows.unsqueeze(0).expand(H, -1, -1), 2, pos.clamp(0, L - 1).long())
    out = head_group * vals + torch.arange(H, dtype=torch.int32).reshape(-1, 1, 1)
    out = torch.where(valid, out, torch.zeros((), dtype=torch.int32))
    return out.permute(1, 0, 2).contiguous()


def get_block_table_bruteforce(topk_idx, block_table, token_to_bs, token_pos_in_bs,
                               seqlen_q, head_group=2):
    """Scalar triple loop over (t, h, k, o) in Python ints; tiny inputs only.

    Used to pin :func:`get_block_table` (independent indexing, no broadcasting).
    """
    idx = _np(topk_idx).astype(np.int64)
    bt = _np(block_table).astype(np.int64)
    bs = [int(v) for v in _np(token_to_bs).reshape(-1)]
    plim = [int(v) for v in _np(token_pos_in_bs).reshape(-1)]
    slen = [int(v) for v in _np(seqlen_q).reshape(-1)]
    H, T, K = idx.shape
    L = bt.shape[1]

    def wrap32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= (1 << 31) else v

    out = np.zeros((T, H, K * SPARSE_BLOCK), dtype=np.int32)
    for t in range(T):
        b = bs[t]
        sl = slen[0] if len(slen) == 1 else slen[b]
        pl = plim[0] if len(plim) == 1 else plim[t]
        for h in range(H):
            for k in range(K):
                blk = int(idx[h, t, k])
                for o in range(SPARSE_BLOCK):
                    p = wrap32(blk * SPARSE_BLOCK + o)
                    if p < 0 or p >= sl or p >= pl:
                        continue
                    slot = int(bt[b, min(p, L - 1)])
                    out[t, h, k * SPARSE_BLOCK + o] = wrap32(head_group * slot + h)
    return out
