"""Oracle: key compression (test infrastructure only).

The reference has no code for this step; its benchmark configurations define
the compressed keys as the mean of windows of 32 raw keys, 16 apart, per
sequence (``(L - 32) // 16 + 1`` windows).  Restated in numpy float32 in the
summation order the build fixes -- per 16-token half-block, tokens added in
order; a window is ``(h_j + h_{j+1}) * (1/32)`` -- then rounded to bf16
(nearest-even).  Pinned against ``torch``'s ``mean`` over ``unfold`` windows
(within one bf16 ulp: only the fp32 summation order differs) and a
Python-float brute force.
"""

import numpy as np
import torch


def compress_keys(k, cu_seqlens, kernel_size=32, stride=16):
    """bf16 ``[T_c, H, D]`` and int64 ``cu_seqlens_compressed`` (CPU)."""
    assert kernel_size == 2 * stride
    x = k.detach().cpu().to(torch.float32).numpy()
    cu = [int(v) for v in np.asarray(cu_seqlens.detach().cpu()).reshape(-1)]
    outs, cu_c = [], [0]
    for b in range(len(cu) - 1):
        seq = x[cu[b]:cu[b + 1]]
        L = seq.shape[0]
        lk = (L - kernel_size) // stride + 1 if L >= kernel_size else 0
        cu_c.append(cu_c[-1] + lk)
        if lk == 0:
            continue
        m = lk + 1                                   # half-blocks used
        h = seq[0:stride * m:stride].copy()          # token 0 of each half-block
        for i in range(1, stride):
            h = h + seq[i:stride * m:stride]         # float32, in token order
        win = (h[:-1] + h[1:]) * np.float32(1.0 / kernel_size)
        outs.append(win.astype(np.float32))
    H, D = x.shape[1], x.shape[2]
    out = np.concatenate(outs, 0) if outs else np.zeros((0, H, D), np.float32)
    return torch.from_numpy(out).to(torch.bfloat16), np.asarray(cu_c, np.int64)


def compress_keys_bruteforce(k, cu_seqlens, kernel_size=32, stride=16):
    """Exact window means (Python floats, math.fsum), rounded once to bf16."""
    import math
    x = k.detach().cpu().to(torch.float64).numpy()
    cu = [int(v) for v in np.asarray(cu_seqlens).reshape(-1)]
    rows = []
    for b in range(len(cu) - 1):
        L = cu[b + 1] - cu[b]
        lk = (L - kernel_size) // stride + 1 if L >= kernel_size else 0
        for j in range(lk):
            w = x[cu[b] + stride * j: cu[b] + stride * j + kernel_size]
            mean = np.empty(w.shape[1:])
            for h in range(w.shape[1]):
                for d in range(w.shape[2]):
                    mean[h, d] = math.fsum(w[:, h, d]) / kernel_size
            rows.append(mean)
    H, D = k.shape[1], k.shape[2]
    arr = np.stack(rows) if rows else np.zeros((0, H, D))
    return torch.from_numpy(arr).to(torch.bfloat16)
