"""Oracle: top-k block selection over pooled scores (test infrastructure only).

The reference selects blocks from the pooled scores with a top-k and sorts the
ids ascending (its tests: ``test/test_sparse_kernel.py:42-43``; the exported
ops stop at the pooled scores, ``max_pooling_1d_varlen.py:127-183``).  A
top-k leaves the order of equal scores open; the build fixes it -- equal
scores are taken in ascending block id -- and writes ``-1`` for a taken block
whose score is ``-inf`` (a window with no key) and for slots past the block
count, the ``-1`` entries first.  Restated here in numpy: a stable sort on
the negated scores, then the first ``k`` ids, sorted.
"""

import numpy as np


def topk_blocks(pooled, k):
    """int32 ``[H, T, k]`` block ids of ``pooled [H, T, NB]`` (any float dtype)."""
    x = pooled.detach().cpu().float().numpy() if hasattr(pooled, "detach") else np.asarray(pooled)
    x = x.astype(np.float32)
    H, T, NB = x.shape
    kk = min(k, NB)
    order = np.argsort(-x, axis=-1, kind="stable")[..., :kk]          # score desc, id asc
    vals = np.take_along_axis(x, order, axis=-1)
    ids = np.where(vals == -np.inf, -1, order).astype(np.int32)
    ids = np.sort(ids, axis=-1)
    if kk < k:
        ids = np.concatenate([np.full((H, T, k - kk), -1, np.int32), ids], axis=-1)
    return ids


def topk_blocks_bruteforce(pooled, k):
    """Python ``sorted`` over (score, id) pairs per row; tiny inputs only."""
    x = np.asarray(pooled, dtype=np.float32)
    H, T, NB = x.shape
    out = np.zeros((H, T, k), np.int32)
    for h in range(H):
        for t in range(T):
            pairs = sorted(((-float(x[h, t, n]), n) for n in range(NB)))[:k]
            ids = [(-1 if s == float("inf") else n) for s, n in pairs]
            ids += [-1] * (k - len(ids))
            out[h, t] = sorted(ids)
    return out
