"""Oracle: InfLLM-v2 stage-1 block scores (test infrastructure only).

Restates the exported ``infllmv2_attn_stage1`` -- the Triton v2 kernel and its
wrapper, ``src/unum_ops/infllm_v2/infllmv2_attn_stage1_triton_v2.py:20-228``
(aliased at ``src/unum_ops/infllm_v2/__init__.py:3-5``) -- in fp32 torch on the
CPU.  The torch "ref" in ``infllmv2_attn_stage1.py`` is NOT followed for its
causal offset or batching (it floors, uses the padded key length and only
works for batch 1); only its math form (fp32 ``q @ k^T * scale``, softmax,
sum over the heads of a group; ``infllmv2_attn_stage1.py:67-111``) is shared.

For token ``t`` of sequence ``b`` and kv group ``g`` (``G = Hq // Hkv``):

* ``lq = t - cu_q[b]``, ``Lq = cu_q[b+1] - cu_q[b]``, ``Lk = cu_k[b+1] - cu_k[b]``
  (``_triton_v2.py:55-64``); rows with no sequence or ``Lk <= 0`` stay 0
  (``:66-67``);
* causal visible count ``vis = clamp(tdiv(lq - 15, 16) + Lk - tdiv(Lq - 15, 16),
  0, Lk)`` where ``tdiv`` truncates toward zero (Triton's signed integer
  ``//``), ``:69-74``; non-causal ``vis = Lk``;
* ``s_i[j] = scale * sum_d bf16(q[t, gG+i, d]) * bf16(k[cu_k[b]+j, g, d])``
  accumulated in fp32 (``:105``), ``-inf`` for ``j >= vis`` (``:106-111``);
* ``out[g, t, j] = sum_i softmax_j(s_i)[j]`` for ``j < Lk`` (``:121-150``);
  a fully masked row is NaN in the kernel and scrubbed to 0 (``:227``);
* output ``[Hkv, Tq, round_up(max_seqlen_k, 128)]``, zero elsewhere
  (``:185-197``).  The reference stores bf16; this oracle returns fp32.
"""

import math

import numpy as np
import torch


def tdiv(a, b):
    """Signed integer division truncating toward zero (Triton ``//`` on int32)."""
    a = np.asarray(a, dtype=np.int64)
    q = np.abs(a) // b
    return np.where(a < 0, -q, q)


def round_multiple(x, m):
    return (x + m - 1) // m * m


def visible_counts(lq, Lq, Lk, causal=True):
    """Visible compressed-key count per query (``_triton_v2.py:69-74``)."""
    lq = np.asarray(lq, dtype=np.int64)
    if not causal:
        return np.full(lq.shape, Lk, dtype=np.int64)
    v = tdiv(lq - 15, 16) + Lk - tdiv(Lq - 16 + 1, 16)
    return np.clip(v, 0, Lk)


def _cpu_list(x):
    if hasattr(x, "detach"):
        x = x.detach().cpu()
    return [int(v) for v in np.asarray(x).reshape(-1)]


def infllmv2_attn_stage1(q, k, v, cu_seqlens_q, cu_seqlens_k, cu_seqlens_v=None,
                         max_seqlen_q=None, max_seqlen_k=None, dropout_p=0.0,
                         softmax_scale=None, causal=False, window_size=(-1, -1),
                         softcap=0.0, alibi_slopes=None, deterministic=False,
                         return_attn_probs=True, block_table=None, drop_past_cols=False):
    """fp32 scores ``[Hkv, Tq, round_up(max_seqlen_k, 128)]`` (CPU tensor).

    A sequence with more keys than the output has columns (a ``max_seqlen_k``
    below a real length) makes the reference store past the row
    (``_triton_v2.py:146-150``): undefined there, so this oracle raises --
    unless ``drop_past_cols``, the build's documented contract for that input:
    the visible count is computed from the real key count and then capped at
    the column count, so each row is the softmax over its first
    ``min(vis, Kp)`` keys (the dropped keys are in no denominator).
    """
    q = q.detach().cpu()
    k = k.detach().cpu()
    Tq, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    scale = D ** (-0.5) if softmax_scale is None else float(softmax_scale)
    cq = _cpu_list(cu_seqlens_q)
    ck = _cpu_list(cu_seqlens_k)
    B = len(cq) - 1
    if max_seqlen_k is None or max_seqlen_k == 0:
        max_seqlen_k = max([ck[i + 1] - ck[i] for i in range(B)] + [0])
    Kp = round_multiple(max_seqlen_k, 128) if max_seqlen_k > 0 else 0
    out = torch.zeros(Hkv, Tq, Kp, dtype=torch.float32)
    if Kp == 0 or Tq == 0:
        return out
    # bf16 -> fp32 is exact, so fp32 products equal the bf16 products of the
    # kernel; only the fp32 accumulation order differs.
    qf = q.to(torch.bfloat16).float()
    kf = k.to(torch.bfloat16).float()
    for b in range(B):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        Lq, Lk = qe - qs, ke - ks
        if Lq <= 0 or Lk <= 0:
            continue
        if Lk > Kp and not drop_past_cols:
            raise ValueError("sequence key length exceeds round_up(max_seqlen_k, 128)")
        vis = visible_counts(np.arange(Lq), Lq, Lk, causal)            # [Lq]
        vis = np.minimum(vis, Kp)
        nk = min(Lk, Kp)                                                # keys scored
        cols = np.arange(nk)
        masked = torch.from_numpy(cols[None, :] >= vis[:, None])       # [Lq, nk]
        for g in range(Hkv):
            qg = qf[qs:qe, g * G:(g + 1) * G, :]                          # [Lq, G, D]
            kg = kf[ks:ks + nk, g, :]                                     # [nk, D]
            s = torch.matmul(qg, kg.t()) * scale                          # [Lq, G, nk]
            s = s.masked_fill(masked[:, None, :], -math.inf)
            p = torch.softmax(s, dim=-1)
            p = torch.nan_to_num(p, nan=0.0)
            out[g, qs:qe, :nk] = p.sum(dim=1)
    return out
