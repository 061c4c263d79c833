"""GPU parity: infllmv2_attn_stage1 HIP kernels vs the fp32 oracle.

Tolerance (stated by the task): |hip - oracle| <= 1e-3 + 1e-2 * |oracle|.
"""

import numpy as np
import pytest
import torch

from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1, visible_counts
import workloads
from unum_ops_amd.infllm_v2 import (infllmv2_attn_stage1, infllmv2_attn_stage1_triton,
                                    infllmv2_attn_stage1_triton_v2)

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2


def _run(d, dev, fn=infllmv2_attn_stage1, causal=True, **kw):
    q, k = d["q"].to(dev), d["k"].to(dev)
    out = fn(q, k, k, d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev),
             max_seqlen_q=d.get("max_seqlen_q"), max_seqlen_k=d.get("max_seqlen_k"),
             causal=causal, **kw)
    torch.cuda.synchronize()
    return out


def _check(d, out, causal=True):
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=d.get("max_seqlen_k"), causal=causal)
    assert out.shape == exp.shape
    torch.testing.assert_close(out.float().cpu(), exp, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("seqlen_q", [64, 256])
@pytest.mark.parametrize("seqlen_k", [15, 16, 128])
def test_reference_test_shapes(seqlen_q, seqlen_k, dev):
    # test/test_infllmv2_attn_stage1.py:35-110: B=1, Hq=32, Hkv=2, D=128, randn q/k, non-causal
    g = torch.Generator().manual_seed(seqlen_q * 1000 + seqlen_k)
    d = dict(q=torch.randn(seqlen_q, 32, 128, generator=g).to(torch.bfloat16),
             k=torch.randn(seqlen_k, 2, 128, generator=g).to(torch.bfloat16),
             cu_seqlens_q=torch.tensor([0, seqlen_q], dtype=torch.int32),
             cu_seqlens_k=torch.tensor([0, seqlen_k], dtype=torch.int32),
             max_seqlen_q=seqlen_q, max_seqlen_k=seqlen_k)
    for fn in (infllmv2_attn_stage1, infllmv2_attn_stage1_triton, infllmv2_attn_stage1_triton_v2):
        out = _run(d, dev, fn, causal=False)
        assert not torch.isnan(out).any()
        _check(d, out, causal=False)


@pytest.mark.parametrize("q_lens,ctx", [
    ([1], [64]), ([14], [300]), ([15], [300]), ([16], [300]), ([17], [300]), ([31], [512]),
    ([32], [1000]), ([100], [96]), ([200], [8192]),
    ([40, 17, 100, 5], [512, 300, 1000, 2048]),           # varlen batch
    ([64, 64], [40, 9000]),                                # Lk > 512: two-pass path
    ([3, 8], [20, 8448]),                                  # an empty sequence (Lk = 0)
])
def test_causal_corners(q_lens, ctx, dev):
    d = workloads.stage1_inputs(q_lens, ctx, seed=len(q_lens) * 31 + sum(q_lens))
    _check(d, _run(d, dev))


@pytest.mark.parametrize("causal", [False, True])
def test_last_quad_half_boundaries(causal, dev):
    # Rows whose last 64-key quad ends just before, at and just after its
    # second half (32 keys in) and its second half's second tile, for every
    # quad count of a 512-column row: the resident kernel computes a last
    # quad's second half only when one of its keys is visible.
    lens = sorted({64 * qd + o for qd in range(8) for o in (1, 16, 17, 31, 32, 33, 48, 49, 63, 64)
                   if 64 * qd + o <= 512})
    q_lens = [3] * len(lens)
    ctx = [16 * (L - 1) + 32 for L in lens]  # compressed to exactly L keys
    d = workloads.stage1_inputs(q_lens, ctx, seed=97 + causal)
    assert [int(v) for v in d["cu_seqlens_k"][1:] - d["cu_seqlens_k"][:-1]] == lens
    _check(d, _run(d, dev, causal=causal), causal=causal)


@pytest.mark.parametrize("peaky", [False, True])
def test_peaky_keys(peaky, dev):
    d = workloads.stage1_inputs([128, 64], [4096, 12000], seed=11, peaky=peaky)
    _check(d, _run(d, dev))


def test_generic_kernel_shapes(dev):
    # G = 8 and D = 64 run the general kernel
    for Hq, Hkv, D in [(32, 4, 128), (16, 1, 64), (32, 2, 64)]:
        d = workloads.stage1_inputs([20, 33], [400, 700], Hq=Hq, Hkv=Hkv, D=D, seed=Hq + D)
        _check(d, _run(d, dev))


def test_gqa_16_1(dev):
    d = workloads.stage1_inputs([64], [4096], Hq=16, Hkv=1, seed=21)
    _check(d, _run(d, dev))


def test_bf16_output(dev):
    d = workloads.stage1_inputs([50], [2000], seed=22)
    out = _run(d, dev, out_dtype=torch.bfloat16)
    assert out.dtype == torch.bfloat16
    _check(d, out)


def test_max_seqlen_k_none_and_padding(dev):
    d = workloads.stage1_inputs([30, 9], [1000, 3000], seed=23)
    d["max_seqlen_k"] = None
    out = _run(d, dev)
    assert out.shape[-1] == 256
    _check(d, out)
    d["max_seqlen_k"] = 300                     # wider than needed: more zero columns
    out = _run(d, dev)
    assert out.shape[-1] == 384
    _check(d, out)


def test_noncontiguous_q(dev):
    d = workloads.stage1_inputs([40], [800], seed=24)
    q = d["q"].to(dev)
    qt = torch.empty(q.shape[1], q.shape[0], q.shape[2], dtype=q.dtype, device=dev)
    qt.copy_(q.transpose(0, 1))
    out = infllmv2_attn_stage1(qt.transpose(0, 1), d["k"].to(dev), None,
                               d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev),
                               max_seqlen_k=d["max_seqlen_k"], causal=True)
    _check(d, out)


def test_cfg3_full_size_properties(dev):
    """cfg3 at full size: row sums are G (or 0), zeros past the visible count, and
    a band of rows of every sequence matches the oracle."""
    d = workloads.cfg3_stage1()
    out = _run(d, dev)
    assert out.shape == (2, 32768, 512)
    sums = out.sum(-1).cpu()
    vis = np.concatenate([visible_counts(np.arange(8192), 8192, 511)] * 4)
    exp = torch.where(torch.from_numpy(vis) > 0, 16.0, 0.0).float()
    # The head sum runs on the matrix core with the exponentials and 1/l in
    # f16 (relative rounding 2^-11 each), so a row sum of 16 carries up to
    # ~16 * 5e-4 of rounding; 1e-2 bounds it with margin.
    torch.testing.assert_close(sums, exp.expand(2, -1), atol=1e-2, rtol=0)
    cols = torch.arange(512, device=dev)
    mask = cols[None, :] >= torch.from_numpy(vis).to(dev)[:, None]
    assert torch.all(out[:, mask] == 0)
    # exact rows: the last 96 tokens of each sequence (a sub-problem with the same
    # causal offsets: the oracle is run on the whole sequence, then sliced)
    for b in range(4):
        qs = 8192 * b
        part = dict(q=d["q"][qs:qs + 8192], k=d["k"][511 * b:511 * (b + 1)],
                    cu_seqlens_q=torch.tensor([0, 8192], dtype=torch.int32),
                    cu_seqlens_k=torch.tensor([0, 511], dtype=torch.int32), max_seqlen_k=511)
        exp_b = oracle_stage1(part["q"], part["k"], None, part["cu_seqlens_q"],
                              part["cu_seqlens_k"], max_seqlen_k=511, causal=True)
        rows = list(range(0, 96)) + list(range(4000, 4096)) + list(range(8096, 8192))
        torch.testing.assert_close(out[:, qs + torch.tensor(rows)].cpu(), exp_b[:, rows],
                                   atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("boost", [4.0, 60.0])
def test_later_keys_far_above_first_quad(boost, dev):
    """Keys after the first 64 scaled up: the first quad's max is then far below
    the row max (boost 60 pushes the per-head sums past 2^14, so those rows are
    redone against their exact max; boost 4 stays on the first pass)."""
    d = workloads.stage1_inputs([300, 77], [5000, 3000], seed=25)
    k = d["k"].float()
    cu_k = d["cu_seqlens_k"].tolist()
    for b in range(2):
        k[cu_k[b] + 64:cu_k[b + 1]] *= boost
    d["k"] = k.to(torch.bfloat16)
    _check(d, _run(d, dev))


@pytest.mark.parametrize("q_lens", [[1], [3], [5], [7, 2], [129, 130, 131], [1023, 1]])
def test_odd_lengths_and_pair_split(q_lens, dev):
    """Odd sequence lengths (one token pair is split) and lengths that put a
    workgroup boundary inside a pair."""
    ctx = [16 * q + 900 for q in q_lens]
    d = workloads.stage1_inputs(q_lens, ctx, seed=sum(q_lens))
    _check(d, _run(d, dev))


def _c_entry_nan(d, dev):
    """Stage 1 through the C entry point into an output that starts as NaN."""
    import ctypes

    from unum_ops_amd import _lib

    q, k = d["q"].to(dev), d["k"].to(dev)
    cu_q, cu_k = d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev)
    cols = (d["max_seqlen_k"] + 127) // 128 * 128
    out = torch.full((2, q.shape[0], cols), float("nan"), device=dev)
    lib = _lib.load()
    st = lib.unum_infllmv2_attn_stage1(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
        _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
        cu_q.numel() - 1, q.shape[0], k.shape[0], 32, 2, 128, d["max_seqlen_k"], cols,
        ctypes.c_float(128 ** -0.5), 1, None, 0, _lib.stream_ptr(dev))
    _lib.check(st, "stage1")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("n_seq", [70, 150])
def test_many_sequences_with_gaps(n_seq, dev):
    """Rows of at most 512 keys: workgroups walk pieces of eight tokens across
    more than 64 sequences, sequences without tokens, a sequence without keys,
    and tokens outside every sequence (zero rows).  The output starts as NaN,
    so an element left unwritten fails the comparison."""
    g = torch.Generator().manual_seed(50 + n_seq)
    q_lens = torch.randint(0, 40, (n_seq,), generator=g).tolist()
    q_lens[0], q_lens[-1], q_lens[3] = 5, 17, 0
    ctx = torch.randint(40, 8000, (n_seq,), generator=g).tolist()
    ctx[1] = 8          # no compressed key: an all-zero row for each token
    d = workloads.stage1_inputs(q_lens, ctx, seed=50)
    assert d["max_seqlen_k"] <= 512
    pre, post = 3, 6
    d["q"] = torch.cat([torch.randn(pre, 32, 128).to(torch.bfloat16), d["q"],
                        torch.randn(post, 32, 128).to(torch.bfloat16)])
    d["cu_seqlens_q"] = d["cu_seqlens_q"] + pre
    out = _c_entry_nan(d, dev)
    assert not torch.isnan(out).any()
    assert float(out[:, :pre].abs().max()) == 0.0 and float(out[:, -post:].abs().max()) == 0.0
    _check(d, out)


@pytest.mark.parametrize("split", [64, 256])
def test_key_halves_far_apart(split, dev):
    """Keys from `split` on scaled far up: the waves that share a row's keys then
    hold references far apart, and the one below gets tiny head-sum weights."""
    d = workloads.stage1_inputs([700, 301], [8192, 6000], seed=26)
    k = d["k"].float()
    cu_k = d["cu_seqlens_k"].tolist()
    for b in range(2):
        k[cu_k[b] + split:cu_k[b + 1]] *= 12.0
    d["k"] = k.to(torch.bfloat16)
    _check(d, _run(d, dev))
