"""GPU regression tests: stage 1 on inputs outside the reference's contract.

* ``max_seqlen_k`` below a sequence's real key count (SURVEY-style quirk: the
  reference stores past the row there, ``infllmv2_attn_stage1_triton_v2.py:
  146-150``).  The build's contract: keys at or past the output's columns are
  dropped, the visible count is taken from the real key count and capped at
  the column count, and each row is the softmax over the keys it keeps -- so
  every row with a visible key sums to G.  Pinned by the closed form G/vis'
  on zero keys (uniform softmax) and by the oracle's ``drop_past_cols``.
* A negative first ``cu_seqlens_k`` entry: the sequence's keys are outside k,
  so no key is read (they read as zero, a uniform softmax: G/vis per column)
  and nothing outside k is touched.

Each case runs every kernel family: the LDS-resident kernel (at most 512
columns), the key-streaming kernels (whole rows and key splits), the decode
kernel (at most two new tokens per sequence), the row-MFMA kernel (a
non-positive scale) and the generic kernel (four heads per group, or a q
whose base is not 16-byte aligned).
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1, visible_counts
import workloads
from unum_ops_amd import _lib

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2
SCALE = 128 ** -0.5

# (q_lens, real key counts, max_seqlen_k given, key-split workspace, query
# heads (two kv heads), scale, q offset in elements): the column count
# round_up(max_seqlen_k, 128), the workspace, the head count, the sign of the
# scale and the alignment of q pick the kernel.
CASES = {
    "lds": ([40, 300], [700, 200], 300, False, 32, SCALE, 0),            # 384 columns, 700 keys
    "stream_split": ([64, 64], [3000, 900], 1000, True, 32, SCALE, 0),   # 1024 columns
    "stream_whole": ([64, 64], [3000, 900], 1000, False, 32, SCALE, 0),  # no workspace
    "decode": ([1, 2, 1], [3000, 2500, 800], 1000, False, 32, SCALE, 0),  # Tq <= 2B
    "row_mfma": ([40, 300], [700, 200], 300, False, 32, -SCALE, 0),      # non-positive scale
    "generic_g4": ([40, 70], [700, 200], 300, False, 8, SCALE, 0),       # 4 heads per group
    "generic_unaligned": ([40, 70], [700, 200], 300, False, 32, SCALE, 1),  # q base + 2 bytes
}


def _inputs(q_lens, k_lens, seed, zero_keys=False, hq=32):
    g = torch.Generator().manual_seed(seed)
    Tq, Tk = sum(q_lens), sum(k_lens)
    q = torch.randn(Tq, hq, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(Tk, 2, 128, generator=g).mul(0.25).to(torch.bfloat16)
    if zero_keys:
        k.zero_()
    return q, k, workloads.prefix(q_lens), workloads.prefix(k_lens)


def _run(q, k, cu_q, cu_k, max_k, with_ws, dev, scale=SCALE, q_offset=0):
    """Stage 1 through the C entry point (NaN-filled output, so an unwritten
    element shows), with or without the key-split workspace; q_offset > 0
    places q that many elements past a 16-byte boundary."""
    hq = q.shape[1]
    if q_offset:
        buf = torch.empty(q.numel() + q_offset, dtype=q.dtype, device=dev)
        qd = buf[q_offset:].view(q.shape)
        qd.copy_(q.to(dev))
    else:
        qd = q.to(dev)
    k, cu_q, cu_k = k.to(dev), cu_q.to(dev), cu_k.to(dev)
    B = cu_q.numel() - 1
    cols = (max_k + 127) // 128 * 128
    lib = _lib.load()
    ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(B, qd.shape[0], hq, 2, 128, max_k)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if with_ws else None
    out = torch.full((2, qd.shape[0], cols), float("nan"), device=dev)
    st = lib.unum_infllmv2_attn_stage1(
        _lib.ptr(qd), qd.stride(0), qd.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
        _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
        B, qd.shape[0], k.shape[0], hq, 2, 128, max_k, cols,
        ctypes.c_float(scale), 1, _lib.ptr(ws), ws_bytes if with_ws else 0,
        _lib.stream_ptr(dev))
    _lib.check(st, "stage1")
    torch.cuda.synchronize()
    if with_ws:
        assert ws_bytes > 0, "the case was meant to split its keys"
    return out.cpu()


def _capped_vis(q_lens, k_lens, cols):
    vis = [np.minimum(visible_counts(np.arange(lq), lq, lk), cols)
           for lq, lk in zip(q_lens, k_lens)]
    return np.concatenate(vis)


@pytest.mark.parametrize("case", sorted(CASES))
def test_keys_past_columns_dropped_closed_form(case, dev):
    q_lens, k_lens, max_k, ws, hq, scale, qo = CASES[case]
    G = hq // 2
    q, k, cu_q, cu_k = _inputs(q_lens, k_lens, seed=1, zero_keys=True, hq=hq)
    out = _run(q, k, cu_q, cu_k, max_k, ws, dev, scale, qo)
    cols = out.shape[-1]
    vis = _capped_vis(q_lens, k_lens, cols)
    j = np.arange(cols)[None, :]
    exp = np.where(j < vis[:, None], G / np.maximum(vis[:, None], 1), 0.0)
    for g in range(2):
        np.testing.assert_allclose(out[g].numpy(), exp, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("case", sorted(CASES))
def test_keys_past_columns_dropped_oracle(case, dev):
    q_lens, k_lens, max_k, ws, hq, scale, qo = CASES[case]
    G = hq // 2
    q, k, cu_q, cu_k = _inputs(q_lens, k_lens, seed=2, hq=hq)
    out = _run(q, k, cu_q, cu_k, max_k, ws, dev, scale, qo)
    exp = oracle_stage1(q, k, None, cu_q, cu_k, max_seqlen_k=max_k, causal=True,
                        drop_past_cols=True, softmax_scale=scale)
    torch.testing.assert_close(out, exp, atol=ATOL, rtol=RTOL)
    vis = _capped_vis(q_lens, k_lens, out.shape[-1])
    sums = out.double().sum(-1).numpy()
    np.testing.assert_allclose(sums, np.where(vis > 0, float(G), 0.0)[None, :].repeat(2, 0),
                               rtol=1e-3)


@pytest.mark.parametrize("case", sorted(CASES))
def test_negative_first_key_offset_reads_nothing(case, dev):
    q_lens, k_lens, max_k, ws, hq, scale, qo = CASES[case]
    G = hq // 2
    q, k, cu_q, cu_k = _inputs(q_lens, k_lens, seed=3, hq=hq)
    # Sequence 0 claims keys [-5, cu_k[1]): its start lies before k.
    cu_k = cu_k.clone()
    cu_k[0] = -5
    lens = [int(cu_k[1] - cu_k[0])] + list(k_lens[1:])
    out = _run(q, k, cu_q, cu_k, max_k, ws, dev, scale, qo)
    cols = out.shape[-1]
    # Sequence 0: every key reads as zero -> G / vis over its visible columns.
    vis0 = np.minimum(visible_counts(np.arange(q_lens[0]), q_lens[0], lens[0]), cols)
    j = np.arange(cols)[None, :]
    exp0 = np.where(j < vis0[:, None], G / np.maximum(vis0[:, None], 1), 0.0)
    for g in range(2):
        np.testing.assert_allclose(out[g, :q_lens[0]].numpy(), exp0, atol=ATOL, rtol=RTOL)
    # The other sequences are unaffected.
    exp = oracle_stage1(q, k, None, cu_q, cu_k.clamp(min=0), max_seqlen_k=max_k, causal=True,
                        drop_past_cols=True, softmax_scale=scale)
    torch.testing.assert_close(out[:, q_lens[0]:], exp[:, q_lens[0]:], atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("case", ["lds", "stream_split", "decode", "row_mfma", "generic_g4"])
def test_keys_past_the_end_of_k_read_as_zero(case, dev):
    # The last sequence claims more keys than k holds: its keys at rows past
    # the end of k score as zero keys, on every path alike.  The oracle gets
    # the same keys with zero rows appended.
    q_lens, k_lens, max_k, ws, hq, scale, qo = CASES[case]
    q, k, cu_q, cu_k = _inputs(q_lens, k_lens, seed=4, hq=hq)
    short = k_lens[-1] // 3
    k_cut = k[:k.shape[0] - short]
    out = _run(q, k_cut, cu_q, cu_k, max_k, ws, dev, scale, qo)
    k_zero = torch.cat([k_cut, torch.zeros(short, 2, 128, dtype=k.dtype)])
    exp = oracle_stage1(q, k_zero, None, cu_q, cu_k, max_seqlen_k=max_k, causal=True,
                        drop_past_cols=True, softmax_scale=scale)
    torch.testing.assert_close(out, exp, atol=ATOL, rtol=RTOL)
