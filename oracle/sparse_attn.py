"""Oracle: stage-2 sparse attention over the block table's KV slots (test
infrastructure only).

The reference has no portable implementation of this op: its consumer of the
block table is an NPU paged-attention operator (``test/test_pa.py:48-71``,
``torch_npu._npu_paged_attention(query, key_cache, value_cache, num_heads,
num_kv_heads, scale_value, block_table, context_lens, out)`` with the shapes of
``test/test_pa.py:75-80``: query ``[T, 32, 128]``, caches ``[num_blocks,
block_size, 2, 128]`` bf16, output ``[T, 32, 128]``).  Its result is fixed by
the mathematics -- attention of each query head over the K/V rows the block
table lists -- which this module restates:

* the slot list of (token t, kv head h) is ``get_block_table``'s output
  ``[t, h, :]`` (``get_table_torch.py:4-44``; ``get_table_triton.py:6-67``),
  computed here with the multiplier ``H = num_kv_heads`` of the Triton
  functions (``get_table_triton.py:259``): slot ``H * block_table[b, p] + h``
  is row ``slot`` of the cache viewed as ``[-1, D]`` (``[num_blocks,
  block_size, H, D]`` flattened), i.e. token slot ``block_table[b, p]``, head
  h -- unless a precomputed ``slots`` table is given;
* entry ``(t, h, 64k + o)`` is attended when the block table marks it valid
  (``p = topk_idx[h, t, k] * 64 + o`` in wrapping int32, ``0 <= p <
  seqlen_q[b]``, ``p < token_pos_in_bs[t]``, ``b = token_to_bs[t]`` in
  ``[0, B)``; ``get_table_torch.py:18-33``) and its row lies inside the cache;
  every valid entry counts, repeated rows included (attention over the
  gathered list);
* ``out[t, h*G + i] = softmax_j(scale * q[t, h*G + i] . K[row_j]) @ V[rows]``
  over the valid entries, fp32 math on the bf16 inputs; 0 when no entry of
  (t, h) is valid.

Pinned (tests/test_oracle_sparse_attn.py) by ``F.scaled_dot_product_attention``
on the gathered rows (a library routine), the closed form for ``q = 0`` (the
mean of the listed V rows, with multiplicity), a pure-Python brute force on
tiny inputs, and the slot lists of ``oracle.get_block_table``.
"""

import math

import numpy as np
import torch

SPARSE_BLOCK = 64


def _np(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu().numpy()
    return np.asarray(x)


def valid_entries(topk_idx, token_to_bs, token_pos_in_bs, seqlen_q, num_seqs):
    """bool ``[T, H, K*64]``: the block table's validity of each entry
    (``get_table_torch.py:18-33``), False for tokens outside ``[0, B)``."""
    idx = _np(topk_idx).astype(np.int32)
    H, T, K = idx.shape
    bs = _np(token_to_bs).astype(np.int64).reshape(-1)
    plim = _np(token_pos_in_bs).astype(np.int64).reshape(-1)
    slen = _np(seqlen_q).astype(np.int64).reshape(-1)
    off = np.arange(SPARSE_BLOCK, dtype=np.int32)
    with np.errstate(over="ignore"):
        pos = (idx[..., None] * np.int32(SPARSE_BLOCK) + off).reshape(H, T, K * SPARSE_BLOCK)
    tok_ok = (bs >= 0) & (bs < num_seqs)
    bsafe = np.where(tok_ok, bs, 0)
    seqlen = np.broadcast_to(slen, (T,)) if slen.size == 1 else slen[bsafe]
    limit = np.broadcast_to(plim, (T,)) if plim.size == 1 else plim
    pos = pos.astype(np.int64)
    valid = (pos >= 0) & (pos < seqlen[None, :, None]) & (pos < limit[None, :, None])
    valid &= tok_ok[None, :, None]
    return np.ascontiguousarray(valid.transpose(1, 0, 2))


def slot_table(topk_idx, block_table, token_to_bs, num_kv_heads):
    """int32 ``[T, H, K*64]`` of slots ``H * block_table[b, min(p, L-1)] + h``
    (wrapping int32) -- get_block_table's values with the Triton multiplier --
    for every entry (invalid ones included; callers mask them)."""
    idx = _np(topk_idx).astype(np.int32)
    bt = _np(block_table).astype(np.int32)
    bs = _np(token_to_bs).astype(np.int64).reshape(-1)
    H, T, K = idx.shape
    L = bt.shape[1]
    off = np.arange(SPARSE_BLOCK, dtype=np.int32)
    with np.errstate(over="ignore"):
        pos = (idx[..., None] * np.int32(SPARSE_BLOCK) + off).reshape(H, T, K * SPARSE_BLOCK)
    bsafe = np.clip(bs, 0, bt.shape[0] - 1)
    vals = bt[bsafe[None, :, None], np.clip(pos, 0, L - 1)]
    heads = np.arange(H, dtype=np.int32)[:, None, None]
    with np.errstate(over="ignore"):
        slots = np.int32(num_kv_heads) * vals + heads
    return np.ascontiguousarray(slots.astype(np.int32).transpose(1, 0, 2))


def gathered_rows(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q, num_kv_heads,
                  n_rows, slots=None):
    """Per (t, h), the int64 cache rows attended, in table order."""
    H = _np(topk_idx).shape[0]
    if H != num_kv_heads:
        raise ValueError("topk_idx must have one head per kv head")
    B = _np(block_table).shape[0]
    valid = valid_entries(topk_idx, token_to_bs, token_pos_in_bs, seqlen_q, B)
    table = slot_table(topk_idx, block_table, token_to_bs, num_kv_heads) if slots is None \
        else _np(slots).astype(np.int32)
    rows = table.astype(np.int64)
    valid &= (rows >= 0) & (rows < n_rows)
    T = valid.shape[0]
    return [[rows[t, h][valid[t, h]] for h in range(H)] for t in range(T)]


def sparse_paged_attention(query, key_cache, value_cache, num_heads, num_kv_heads, scale_value,
                           topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                           slots=None, dtype=torch.float32):
    """fp32 ``[T, num_heads, D]`` (CPU tensor); see the module docstring."""
    q = query.detach().cpu().to(torch.bfloat16).to(dtype)
    D = q.shape[-1]
    kf = key_cache.detach().cpu().to(torch.bfloat16).reshape(-1, D)
    vf = value_cache.detach().cpu().to(torch.bfloat16).reshape(-1, D)
    T = q.shape[0]
    G = num_heads // num_kv_heads
    rows = gathered_rows(topk_idx, block_table, token_to_bs, token_pos_in_bs, seqlen_q,
                         num_kv_heads, kf.shape[0], slots)
    out = torch.zeros(T, num_heads, D, dtype=dtype)
    for t in range(T):
        for h in range(num_kv_heads):
            r = rows[t][h]
            if r.size == 0:
                continue
            ri = torch.from_numpy(r)
            kk = kf[ri].to(dtype)                               # [n, D]
            vv = vf[ri].to(dtype)
            qq = q[t, h * G:(h + 1) * G]                        # [G, D]
            s = (qq @ kk.t()) * scale_value                     # [G, n]
            p = torch.softmax(s, dim=-1)
            out[t, h * G:(h + 1) * G] = p @ vv
    return out


def sparse_paged_attention_bruteforce(query, key_cache, value_cache, num_heads, num_kv_heads,
                                      scale_value, topk_idx, block_table, token_to_bs,
                                      token_pos_in_bs, seqlen_q):
    """Python floats, one explicit softmax per (t, head); tiny inputs only.
    Shares no code with the function above: the slot of entry (t, h, 64k+o)
    is worked out from the block-table formula term by term."""
    q = query.detach().cpu().float().tolist()
    D = len(q[0][0])
    kf = key_cache.detach().cpu().float().reshape(-1, D).tolist()
    vf = value_cache.detach().cpu().float().reshape(-1, D).tolist()
    idx = _np(topk_idx).astype(np.int64)
    bt = _np(block_table).astype(np.int64)
    bs = [int(v) for v in _np(token_to_bs).reshape(-1)]
    plim = [int(v) for v in _np(token_pos_in_bs).reshape(-1)]
    slen = [int(v) for v in _np(seqlen_q).reshape(-1)]
    H, T, K = idx.shape
    B, L = bt.shape
    G = num_heads // num_kv_heads

    def wrap32(v):
        v &= 0xFFFFFFFF
        return v - (1 << 32) if v >= (1 << 31) else v

    out = [[[0.0] * D for _ in range(num_heads)] for _ in range(T)]
    for t in range(T):
        b = bs[t]
        for h in range(H):
            rows = []
            if 0 <= b < B:
                sl = slen[0] if len(slen) == 1 else slen[b]
                pl = plim[0] if len(plim) == 1 else plim[t]
                for k in range(K):
                    for o in range(SPARSE_BLOCK):
                        p = wrap32(int(idx[h, t, k]) * SPARSE_BLOCK + o)
                        if 0 <= p < sl and p < pl:
                            row = wrap32(num_kv_heads * int(bt[b, min(p, L - 1)]) + h)
                            if 0 <= row < len(kf):
                                rows.append(row)
            for i in range(G):
                hq = h * G + i
                if not rows:
                    continue
                s = [scale_value * sum(q[t][hq][d] * kf[r][d] for d in range(D)) for r in rows]
                m = max(s)
                e = [math.exp(x - m) for x in s]
                z = sum(e)
                for d in range(D):
                    out[t][hq][d] = sum(e[j] * vf[rows[j]][d] for j in range(len(rows))) / z
    return torch.tensor(out, dtype=torch.float32)
