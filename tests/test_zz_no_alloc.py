"""GPU: unum_infllmv2_attn_stage1_noalloc (the entry point that allocates
nothing: its key-split workspace is a device array inside the library)
against unum_infllmv2_attn_stage1 with a caller workspace, through the C ABI.

The two run the same kernels on the same split plan, so their outputs must
be equal bit for bit; both are also checked against the fp32 oracle at the
stage-1 tolerance (atol 1e-3, rtol 1e-2).  Two calls in a row, the second
smaller, show that the array's leftover contents do not leak into a later
call.
"""

import ctypes

import pytest
import torch

from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1
import workloads
from unum_ops_amd import _lib

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2
SCRATCH_BYTES = 4 << 20


def _args(d, dev):
    q, k = d["q"].to(dev), d["k"].to(dev)
    cu_q, cu_k = d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev)
    B = cu_q.numel() - 1
    cols = (d["max_seqlen_k"] + 127) // 128 * 128
    return q, k, cu_q, cu_k, B, cols


def _with_workspace(d, dev):
    lib = _lib.load()
    q, k, cu_q, cu_k, B, cols = _args(d, dev)
    ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(B, q.shape[0], 32, 2, 128,
                                                            d["max_seqlen_k"])
    assert 0 < ws_bytes <= SCRATCH_BYTES, ws_bytes  # the case splits its keys
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.full((2, q.shape[0], cols), float("nan"), device=dev)
    st = lib.unum_infllmv2_attn_stage1(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
        _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
        B, q.shape[0], k.shape[0], 32, 2, 128, d["max_seqlen_k"], cols,
        ctypes.c_float(128 ** -0.5), 1, _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(st, "stage1")
    torch.cuda.synchronize()
    return out.cpu()


def _noalloc(d, dev):
    lib = _lib.load()
    q, k, cu_q, cu_k, B, cols = _args(d, dev)
    out = torch.full((2, q.shape[0], cols), float("nan"), device=dev)
    st = lib.unum_infllmv2_attn_stage1_noalloc(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
        _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
        B, q.shape[0], k.shape[0], 32, 2, 128, d["max_seqlen_k"], cols,
        ctypes.c_float(128 ** -0.5), 1, _lib.stream_ptr(dev))
    _lib.check(st, "stage1_noalloc")
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(d):
    return oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                         max_seqlen_k=d["max_seqlen_k"], causal=True)


def test_noalloc_matches_the_workspace_entry_twice(dev):
    # A long prefill chunk (key splits over about 2.5K keys), then a smaller
    # mixed batch: the second call must not see the first one's split sums.
    big = workloads.stage1_inputs([600], [40000], seed=71, raw_keys=False)
    small = workloads.stage1_inputs([9, 40], [30000, 9000], seed=72, raw_keys=False)
    for d in (big, small):
        print(f"noalloc case: q_lens={d['q_lens']} ctx={d['ctx_lens']}", flush=True)
        got = _noalloc(d, dev)
        ref = _with_workspace(d, dev)
        assert not torch.isnan(got).any()
        assert torch.equal(got, ref)
        torch.testing.assert_close(got, _oracle(d), atol=ATOL, rtol=RTOL)


def test_noalloc_paths_without_split(dev):
    # Rows of at most 512 keys and a decode batch: no scratch is used.
    for d in (workloads.stage1_inputs([70, 33], [4000, 8192], seed=73),
              workloads.stage1_inputs([1, 2, 1], [20000, 9000, 3000], seed=74, raw_keys=False)):
        print(f"noalloc case: q_lens={d['q_lens']} ctx={d['ctx_lens']}", flush=True)
        got = _noalloc(d, dev)
        assert not torch.isnan(got).any()
        torch.testing.assert_close(got, _oracle(d), atol=ATOL, rtol=RTOL)


def test_split_plan_fits_the_array(dev):
    # The split plan targets six workgroups per CU: its workspace stays below
    # 12 KiB + 288 bytes per CU (3.07 MiB at 256 CUs; the worst problem found,
    # one kv head, 8 sequences, ~23K tokens over 2047 keys, reaches 2.97 MiB),
    # so every problem fits the 4 MiB array on this GPU and the refusal past
    # it never fires here.
    lib = _lib.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    worst = 0
    for Hkv in (1, 2):
        for B in (1, 2, 8, 64, 256):
            tqs = [B, 2 * B + 1, 16 * B, 64 * B, 300 * B]
            if B == 1:
                tqs += [20000, 24021, 30000, 40000]
            if B == 8:
                tqs += [22939]
            for Tq in tqs:
                for max_k in (513, 700, 1000, 2047, 4095, 8447, 30000, 131071, 131072):
                    worst = max(worst, lib.unum_infllmv2_attn_stage1_workspace_size(
                        B, Tq, 16 * Hkv, Hkv, 128, max_k))
    assert 0 < worst < (12 * 1024 + 288) * cus, worst
    assert worst <= SCRATCH_BYTES, worst
