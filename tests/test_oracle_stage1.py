"""Pins of the stage-1 oracle (CPU).

* library reduction: ``F.scaled_dot_product_attention`` with an identity value
  matrix returns the probability matrix; summed over a group's heads it must
  equal the oracle (non-causal, and causal with the visible-count mask);
* uniform closed form: ``q = 0`` makes every visible score equal, so each row
  is ``G / vis`` on ``j < vis`` and 0 elsewhere -- this pins where the causal
  mask falls independently of the softmax code;
* visible counts: a hand-derived table for the reference's rule with Triton's
  truncating division (the floor-division torch ref differs on several rows);
* invariants: row sums are ``G`` (or 0 when nothing is visible).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.stage1 import infllmv2_attn_stage1, tdiv, visible_counts
import workloads


def _sdpa_reference(q, k, cu_q, cu_k, Hkv, causal, scale=None):
    """Per sequence: SDPA(q, k, I) = softmax(q k^T * scale) (masked), summed per group."""
    Tq, Hq, D = q.shape
    G = Hq // Hkv
    scale = D ** -0.5 if scale is None else scale
    cq, ck = [int(v) for v in cu_q], [int(v) for v in cu_k]
    kp = ((max(ck[i + 1] - ck[i] for i in range(len(ck) - 1)) + 127) // 128) * 128
    out = torch.zeros(Hkv, Tq, kp)
    for b in range(len(cq) - 1):
        Lq, Lk = cq[b + 1] - cq[b], ck[b + 1] - ck[b]
        if Lq == 0 or Lk == 0:
            continue
        qb = q[cq[b]:cq[b + 1]].float().transpose(0, 1)            # [Hq, Lq, D]
        kb = k[ck[b]:ck[b + 1]].float().transpose(0, 1)            # [Hkv, Lk, D]
        kb = kb.repeat_interleave(G, dim=0).contiguous()            # [Hq, Lk, D]
        eye = torch.eye(Lk).expand(Hq, Lk, Lk).contiguous()
        mask = None
        if causal:
            vis = torch.from_numpy(visible_counts(np.arange(Lq), Lq, Lk))
            mask = torch.arange(Lk)[None, :] < vis[:, None]          # [Lq, Lk] True = keep
        p = F.scaled_dot_product_attention(qb, kb, eye, attn_mask=mask, scale=scale)
        p = torch.nan_to_num(p, nan=0.0)
        out[:, cq[b]:cq[b + 1], :Lk] = p.reshape(Hkv, G, Lq, Lk).sum(1)
    return out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("q_lens,ctx,Hq,Hkv,D", [
    ([64], [272], 32, 2, 128),
    ([40, 17, 100], [512, 300, 1000], 32, 2, 64),
    ([33], [2000], 16, 1, 128),
    ([20, 9], [200, 90], 32, 4, 32),
])
def test_matches_sdpa(causal, q_lens, ctx, Hq, Hkv, D):
    d = workloads.stage1_inputs(q_lens, ctx, Hq=Hq, Hkv=Hkv, D=D, seed=1)
    ours = infllmv2_attn_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                                max_seqlen_k=d["max_seqlen_k"], causal=causal)
    ref = _sdpa_reference(d["q"], d["k"], d["cu_seqlens_q"], d["cu_seqlens_k"], Hkv, causal)
    torch.testing.assert_close(ours, ref, atol=2e-5, rtol=1e-4)


def test_matches_sdpa_peaky():
    d = workloads.stage1_inputs([50], [900], seed=2)
    k = d["k"].float() * 8
    ours = infllmv2_attn_stage1(d["q"], k.to(torch.bfloat16), None, d["cu_seqlens_q"],
                                d["cu_seqlens_k"], causal=True)
    ref = _sdpa_reference(d["q"], k.to(torch.bfloat16), d["cu_seqlens_q"], d["cu_seqlens_k"], 2,
                          True)
    torch.testing.assert_close(ours, ref, atol=2e-5, rtol=1e-4)


# (Lq, Lk) -> {lq: vis}, derived by hand from
#   vis = clamp(tdiv(lq-15, 16) + Lk - tdiv(Lq-15, 16), 0, Lk), tdiv truncating.
VIS_TABLE = {
    (40, 10): {0: 9, 14: 9, 15: 9, 30: 9, 31: 10, 39: 10},
    (20, 3): {0: 3, 14: 3, 19: 3},                     # floor division would give 2 at lq<15
    (8192, 511): {0: 0, 30: 0, 31: 1, 46: 1, 47: 2, 8191: 511},
    (4096, 8447): {0: 8192, 31: 8193, 4095: 8447},
    (1, 100): {0: 100},
    (16, 1): {0: 1, 15: 1},
    (100, 2): {0: 0, 62: 0, 63: 0, 79: 1, 95: 2, 99: 2},
}


@pytest.mark.parametrize("key", list(VIS_TABLE))
def test_visible_count_table(key):
    Lq, Lk = key
    for lq, v in VIS_TABLE[key].items():
        assert int(visible_counts(np.array([lq]), Lq, Lk)[0]) == v, (Lq, Lk, lq)


def test_tdiv_truncates():
    assert list(tdiv(np.array([-17, -16, -15, -1, 0, 1, 15, 16, 17]), 16)) == \
        [-1, -1, 0, 0, 0, 0, 0, 1, 1]


@pytest.mark.parametrize("Lq,ctx", [(40, 176), (20, 64), (100, 48), (16, 32), (300, 3000)])
def test_uniform_closed_form(Lq, ctx):
    Lk = workloads.compressed_len(ctx)
    d = workloads.stage1_inputs([Lq], [ctx], seed=3)
    q = torch.zeros_like(d["q"])
    out = infllmv2_attn_stage1(q, d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                               causal=True)
    checked = set()
    for lq in range(Lq):
        row = out[0, lq]
        nz = int((row != 0).sum())
        if nz:
            assert torch.allclose(row[:nz], torch.full((nz,), 16.0 / nz), rtol=1e-6)
        assert torch.all(row[nz:] == 0)
        if (Lq, Lk) in VIS_TABLE and lq in VIS_TABLE[(Lq, Lk)]:
            assert nz == VIS_TABLE[(Lq, Lk)][lq]
            checked.add(lq)
    assert Lq == 300 or checked == set(VIS_TABLE[(Lq, Lk)])


def test_row_sums_and_empty_rows():
    # sequences: normal, no keys (Lk = 0), and tokens past cu_seqlens_q[-1]
    d = workloads.stage1_inputs([30, 12], [600, 20], seed=4)
    q = torch.cat([d["q"], torch.randn(5, 32, 128).to(torch.bfloat16)])
    out = infllmv2_attn_stage1(q, d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                               causal=True)
    assert out.shape == (2, 47, 128)
    sums = out.sum(-1)
    vis = visible_counts(np.arange(30), 30, workloads.compressed_len(600))
    exp = torch.where(torch.from_numpy(vis) > 0, 16.0, 0.0).float()
    torch.testing.assert_close(sums[:, :30], exp.expand(2, 30), atol=1e-4, rtol=0)
    assert torch.all(out[:, 30:] == 0)        # Lk = 0 and out-of-batch tokens


def test_output_columns_round_to_128():
    d = workloads.stage1_inputs([4], [2100], seed=5)
    lk = workloads.compressed_len(2100)
    out = infllmv2_attn_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"])
    assert out.shape[-1] == 128 * math.ceil(lk / 128)
    out2 = infllmv2_attn_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                                max_seqlen_k=lk + 200)
    assert out2.shape[-1] == 128 * math.ceil((lk + 200) / 128)
    torch.testing.assert_close(out2[..., :out.shape[-1]], out)


def test_drop_past_cols_closed_form_and_sums():
    # A max_seqlen_k below the real key count: the oracle raises by default;
    # with drop_past_cols each row is the softmax over its first
    # min(vis, Kp) keys.  q = 0 makes every kept score equal: G / min(vis, Kp)
    # (a denominator that counted the dropped keys would give less), and a
    # random q still gives rows summing to G.
    Lq, Lk, max_k = 40, 700, 300
    g = torch.Generator().manual_seed(5)
    k = torch.randn(Lk, 2, 128, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0, Lq], dtype=torch.int32)
    cu_k = torch.tensor([0, Lk], dtype=torch.int32)
    q0 = torch.zeros(Lq, 32, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        infllmv2_attn_stage1(q0, k, None, cu_q, cu_k, max_seqlen_k=max_k, causal=True)
    out = infllmv2_attn_stage1(q0, k, None, cu_q, cu_k, max_seqlen_k=max_k, causal=True,
                               drop_past_cols=True)
    kp = out.shape[-1]
    assert kp == 384
    vis = np.minimum(visible_counts(np.arange(Lq), Lq, Lk), kp)
    assert vis.max() == kp and vis.min() > 0
    j = np.arange(kp)[None, :]
    exp = np.where(j < vis[:, None], 16.0 / vis[:, None], 0.0)
    np.testing.assert_allclose(out[0].numpy(), exp, rtol=1e-6, atol=1e-7)
    q = torch.randn(Lq, 32, 128, generator=g).to(torch.bfloat16)
    out = infllmv2_attn_stage1(q, k, None, cu_q, cu_k, max_seqlen_k=max_k, causal=True,
                               drop_past_cols=True)
    np.testing.assert_allclose(out.sum(-1).numpy(), 16.0, rtol=1e-5)
