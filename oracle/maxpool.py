"""Oracle: varlen 1-D max-pool of compressed-block scores (test infrastructure only).

Restates the Triton kernel ``_max_pooling_1d_varlen_kernel`` and its wrapper
(``src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:33-183``); the reference
has no torch implementation of this op.

For head ``h``, token ``t`` and output block ``n``:

* ``b`` is the sequence with ``cu_q[b] <= t < cu_q[b+1]`` (none -> ``Lk = 0``,
  ``ob = 0``), ``max_pooling_1d_varlen.py:69-80``;
* ``Lk = (cu_k[b+1] - cu_k[b]) + cache_lens[b]`` and
  ``ob = (t - cu_q[b]) // block_size``, ``:79-80``;
* taps ``p = n*P - 1 + i`` for ``i < P+1`` (``P = block_size // stride``,
  padding 1), kept when ``0 <= p < Lk``, ``:84-106``;
* values are read from the FLAT input at ``(h*Tq + t) * F + p`` with
  ``F = max_seqlen_q // stride`` -- not from row ``t`` of the last dimension,
  ``:82``, ``:146``;
* ``+inf`` when ``n < init_blocks`` or ``n <= ob <= n + local_blocks``; else the
  max of the kept taps, or ``-inf`` when no tap is kept, ``:108-116``;
* the result has the input dtype, ``:122``, ``:148-153``.

The max is ``fmax`` (a NaN tap loses to a number), as Triton's ``tl.maximum``
without NaN propagation.
"""

import math

import numpy as np


def _np(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu()
        if str(x.dtype) == "torch.bfloat16":
            x = x.float()
        x = x.numpy()
    return np.asarray(x)


def row_params(cu_seqlens_q, cu_seqlens_k, cache_lens, total_q, block_size):
    """Per-token ``(Lk, ob)`` following ``max_pooling_1d_varlen.py:69-80``."""
    cq = _np(cu_seqlens_q).astype(np.int64)
    ck = _np(cu_seqlens_k).astype(np.int64)
    cache = _np(cache_lens).astype(np.int64).reshape(-1)
    B = cq.size - 1
    t = np.arange(total_q, dtype=np.int64)
    lk = np.zeros(total_q, dtype=np.int64)
    ob = np.zeros(total_q, dtype=np.int64)
    # The reference scans every b and keeps the LAST hit; with non-decreasing
    # cu_seqlens the hit is unique, so a scan in order is equivalent.
    for b in range(B):
        hit = (t >= cq[b]) & (t < cq[b + 1])
        lk = np.where(hit, (ck[b + 1] - ck[b]) + cache[b], lk)
        ob = np.where(hit, (t - cq[b]) // block_size, ob)
    return lk, ob


def max_pooling_1d_varlen(input, cu_seqlens_q, cu_seqlens_k, cache_lens, max_seqlen_q,
                          max_context_len, local_blocks, init_blocks, block_size=64,
                          stride=16, total_q=-1, oob="raise"):
    """Return ``[H, Tq, NB]`` as float32 (bf16 input values are exact in float32);
    see the module docstring.

    A kept tap whose flat address is past the end of the input is an
    out-of-bounds read in the reference (undefined).  ``oob="raise"`` raises
    ``IndexError`` for it; ``oob="absent"`` drops such taps, which is the
    behaviour the HIP kernel defines for that case.
    """
    x = _np(input).astype(np.float32)
    H, Tq = x.shape[0], x.shape[1]
    NB = math.ceil(max_context_len / block_size)
    P = block_size // stride
    KS = P + 1
    pad = 1
    F = max_seqlen_q // stride
    flat = x.reshape(-1)
    numel = flat.size

    lk, ob = row_params(cu_seqlens_q, cu_seqlens_k, cache_lens, Tq, block_size)
    n = np.arange(NB, dtype=np.int64)
    ws = n * P - pad                                        # window start, may be -1
    out = np.full((H, Tq, NB), -np.inf, dtype=np.float32)
    for h in range(H):
        base = (h * Tq + np.arange(Tq, dtype=np.int64)) * F  # [Tq]
        m = np.full((Tq, NB), -np.inf, dtype=np.float32)
        for i in range(KS):
            p = ws + i                                        # [NB]
            keep = (p[None, :] >= 0) & (p[None, :] < lk[:, None])
            addr = base[:, None] + np.maximum(p, 0)[None, :]
            bad = keep & (addr >= numel)
            if bad.any():
                if oob == "raise":
                    raise IndexError("flat read past the end of the input "
                                     "(the reference reads out of bounds here)")
                keep = keep & ~bad
            vals = np.where(keep, flat[np.minimum(addr, numel - 1)], -np.inf)
            m = np.fmax(m, vals.astype(np.float32))
        force = (n[None, :] < init_blocks) | ((ob[:, None] >= n[None, :]) &
                                              (ob[:, None] <= n[None, :] + local_blocks))
        has_win = np.minimum(ws[None, :] + KS, lk[:, None]) > np.maximum(ws, 0)[None, :]
        out[h] = np.where(force, np.inf, np.where(has_win, m, -np.inf))
    return out


def max_pooling_1d_varlen_torch(input, cu_seqlens_q, cu_seqlens_k, cache_lens, max_seqlen_q,
                                max_context_len, local_blocks, init_blocks, block_size=64,
                                stride=16):
    """The same restatement as :func:`max_pooling_1d_varlen` in torch ops (CPU,
    every thread torch is given): the form the benchmark times as the CPU
    baseline (the reference ships no torch max-pool).  Taps past the end of
    the flat input are dropped (``oob="absent"``).  Returns float32
    ``[H, Tq, NB]``, equal bit for bit to the numpy form."""
    import torch

    x = input.detach().cpu().float()
    H, Tq = x.shape[0], x.shape[1]
    NB = math.ceil(max_context_len / block_size)
    P = block_size // stride
    F = max_seqlen_q // stride
    flat = x.reshape(-1)
    numel = flat.numel()
    lk_np, ob_np = row_params(cu_seqlens_q, cu_seqlens_k, cache_lens, Tq, block_size)
    lk, ob = torch.from_numpy(lk_np), torch.from_numpy(ob_np)
    n = torch.arange(NB, dtype=torch.int64)
    ws = n * P - 1
    force = (n[None, :] < init_blocks) | ((ob[:, None] >= n[None, :]) &
                                          (ob[:, None] <= n[None, :] + local_blocks))
    has_win = torch.minimum(ws[None, :] + P + 1, lk[:, None]) > ws.clamp(min=0)[None, :]
    out = torch.empty(H, Tq, NB, dtype=torch.float32)
    ninf = torch.tensor(-math.inf)
    for h in range(H):
        base = (h * Tq + torch.arange(Tq, dtype=torch.int64)) * F
        m = torch.full((Tq, NB), -math.inf)
        for i in range(P + 1):
            p = ws + i
            addr = base[:, None] + p.clamp(min=0)[None, :]
            keep = (p[None, :] >= 0) & (p[None, :] < lk[:, None]) & (addr < numel)
            vals = torch.where(keep, flat[addr.clamp(max=numel - 1)], ninf)
            m = torch.fmax(m, vals)
        out[h] = torch.where(force, torch.tensor(math.inf), torch.where(has_win, m, ninf))
    return out


def max_pooling_1d_varlen_bruteforce(input, cu_seqlens_q, cu_seqlens_k, cache_lens,
                                     max_seqlen_q, max_context_len, local_blocks,
                                     init_blocks, block_size=64, stride=16):
    """Scalar loops in Python floats; tiny inputs only (pins the vectorised form)."""
    x = _np(input).astype(np.float32)
    H, Tq = x.shape[0], x.shape[1]
    flat = [float(v) for v in x.reshape(-1)]
    cq = [int(v) for v in _np(cu_seqlens_q).reshape(-1)]
    ck = [int(v) for v in _np(cu_seqlens_k).reshape(-1)]
    cache = [int(v) for v in _np(cache_lens).reshape(-1)]
    NB = -(-max_context_len // block_size)
    P = block_size // stride
    F = max_seqlen_q // stride
    out = np.empty((H, Tq, NB), dtype=np.float32)
    for h in range(H):
        for t in range(Tq):
            lk, ob = 0, 0
            for b in range(len(cq) - 1):
                if cq[b] <= t < cq[b + 1]:
                    lk = ck[b + 1] - ck[b] + cache[b]
                    ob = (t - cq[b]) // block_size
            for nn in range(NB):
                if nn < init_blocks or (nn <= ob <= nn + local_blocks):
                    out[h, t, nn] = math.inf
                    continue
                best = -math.inf
                for p in range(nn * P - 1, nn * P + P):
                    if 0 <= p < lk:
                        v = flat[(h * Tq + t) * F + p]
                        if v == v and v > best:      # fmax: a NaN tap loses
                            best = v
                out[h, t, nn] = best
    return out
