"""Pins of the max-pool oracle (CPU): library reduction, brute force, known answers."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.maxpool import max_pooling_1d_varlen, max_pooling_1d_varlen_bruteforce
import workloads


def _library_pool(x, cu_q, cu_k, cache, max_seqlen_q, max_context_len, local, init,
                  block_size=64, stride=16):
    """Reduction to F.max_pool1d: gather each row through the flat-stride view
    (torch.as_strided), mask taps >= Lk to -inf, pad, pool with k=P+1, s=P, p=1,
    then force the init/local blocks to +inf."""
    x = torch.as_tensor(x, dtype=torch.float32)
    H, Tq = x.shape[0], x.shape[1]
    NB = math.ceil(max_context_len / block_size)
    P = block_size // stride
    Fs = max_seqlen_q // stride
    span = P * NB + P + 1                       # taps any window can touch
    flat = torch.cat([x.reshape(-1), torch.full((span,), float("nan"))])  # pad, never kept
    rows = torch.as_strided(flat, (H, Tq, span), (Tq * Fs, Fs, 1))
    out = torch.empty(H, Tq, NB)
    cq, ck, ca = list(map(int, cu_q)), list(map(int, cu_k)), list(map(int, cache))
    for t in range(Tq):
        lk, ob = 0, 0
        for b in range(len(cq) - 1):
            if cq[b] <= t < cq[b + 1]:
                lk, ob = ck[b + 1] - ck[b] + ca[b], (t - cq[b]) // block_size
        r = rows[:, t, :].clone()
        r[:, lk:] = -math.inf
        pooled = F.max_pool1d(r[:, None, :], kernel_size=P + 1, stride=P, padding=1)[:, 0, :NB]
        n = torch.arange(NB)
        force = (n < init) | ((ob >= n) & (ob <= n + local))
        out[:, t, :] = torch.where(force, torch.full_like(pooled, math.inf), pooled)
    return out.numpy()


CASES = [
    # q_lens, k_lens, cache, F, max_seqlen_q, max_context_len, local, init
    ([40, 24], [9, 5], [0, 0], 16, 256, 200, 1, 1),
    ([64, 130, 7], [17, 33, 0], [0, 3, 2], 40, 640, 700, 2, 1),
    ([100], [1], [0], 8, 128, 300, 0, 0),
    ([70, 70], [4, 12], [5, 0], 20, 320, 180, 1, 2),
    ([33, 65], [31, 29], [0, 0], 32, 512, 2100, 3, 1),
]


@pytest.mark.parametrize("case", CASES)
def test_matches_library_pool(case):
    q_lens, k_lens, cache, Fs, msq, mcl, local, init = case
    d = workloads.maxpool_inputs(q_lens, F=Fs, H=2, seed=3, k_lens=k_lens, cache=cache)
    # random values, not just softmax rows, so every tap matters
    x = torch.randn(d["input"].shape, generator=torch.Generator().manual_seed(7))
    ours = max_pooling_1d_varlen(x, d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                                 msq, mcl, local, init, oob="absent")
    lib = _library_pool(x, d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"], msq, mcl,
                        local, init)
    # taps past the end of the input are "absent" in ours and NaN-padded in the
    # library form; F.max_pool1d propagates NaN, so compare where lib is not NaN
    ok = ~np.isnan(lib)
    np.testing.assert_array_equal(ours[ok], lib[ok])


@pytest.mark.parametrize("case", CASES[:3])
def test_matches_bruteforce(case):
    q_lens, k_lens, cache, Fs, msq, mcl, local, init = case
    d = workloads.maxpool_inputs(q_lens, F=Fs, H=2, seed=5, k_lens=k_lens, cache=cache)
    x = d["input"]
    args = (x, d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"], msq, mcl, local, init)
    try:
        ours = max_pooling_1d_varlen(*args)
    except IndexError:
        pytest.skip("case reads past the end of the input")
    np.testing.assert_array_equal(ours, max_pooling_1d_varlen_bruteforce(*args))


def test_known_answer():
    # H=1, one 70-token sequence with Lk = 10 keys, F = 10: row t holds t*100 + p.
    Tq, Fs = 70, 10
    x = (np.arange(Tq)[:, None] * 100 + np.arange(Fs)[None, :]).astype(np.float32)[None]
    cu_q = np.array([0, 70], np.int32)
    cu_k = np.array([0, 10], np.int32)
    out = max_pooling_1d_varlen(x, cu_q, cu_k, np.array([0], np.int32), max_seqlen_q=160,
                                max_context_len=256, local_blocks=0, init_blocks=1)
    assert out.shape == (1, 70, 4)
    # t = 3 (ob = 0): n=0 forced by init; n=1 -> taps 3..7 -> 307; n=2 -> taps 7..9 -> 309;
    # n=3 -> taps 11.. (>= Lk) -> -inf
    np.testing.assert_array_equal(out[0, 3], [math.inf, 307, 309, -math.inf])
    # t = 65 (ob = 1, local 0): n=1 forced
    np.testing.assert_array_equal(out[0, 65], [math.inf, math.inf, 6509, -math.inf])


def test_flat_stride_reads_across_rows():
    # F = 4 < Lk = 6: taps 4, 5 of row t are elements 0, 1 of row t+1 (max_pooling_1d_varlen.py:82)
    x = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4)
    out = max_pooling_1d_varlen(x, np.array([0, 3], np.int32), np.array([0, 6], np.int32),
                                np.array([0], np.int32), max_seqlen_q=64, max_context_len=64,
                                local_blocks=0, init_blocks=0, block_size=64, stride=16)
    # row (h=0, t=0) base 0: window n=0 taps 0..3 -> max 3 (forced? ob=0, local 0 -> n=0 forced)
    assert out[0, 0, 0] == math.inf
    args = (x, np.array([0, 3], np.int32), np.array([0, 6], np.int32), np.array([0], np.int32))
    kw = dict(max_seqlen_q=64, max_context_len=128, local_blocks=-1, init_blocks=0)
    # row (h=1, t=2): base (1*3+2)*4 = 20 -> window n=1 keeps taps 23, 24, 25, and
    # 24, 25 are past the 24-element input: the reference reads out of bounds
    with pytest.raises(IndexError):
        max_pooling_1d_varlen(*args, **kw)
    out2 = max_pooling_1d_varlen(*args, **kw, oob="absent")
    # local -1 never forces; n=1 -> taps 3..5 -> flat[base+3..base+5]; row t=0: 3,4,5 -> 5
    assert out2[0, 0, 1] == 5.0
    # row (h=0, t=1): base 4 -> taps 7, 8, 9 = elements of rows t=1 and t=2 -> 9
    assert out2[0, 1, 1] == 9.0
    # the overrunning row keeps only tap 23
    assert out2[1, 2, 1] == 23.0


def test_cfg2_shapes_and_forcing():
    d = workloads.maxpool_inputs([256, 384], F=64, H=2, seed=1)
    out = max_pooling_1d_varlen(d["input"], d["cu_seqlens_q"], d["cu_seqlens_k"],
                                d["cache_lens"], 1024, 1024, 1, 1)
    assert out.shape == (2, 640, 16)
    # init block and local blocks n in [ob-1, ob] are +inf on every row
    assert np.all(out[:, :, 0] == np.inf)
    for t in [0, 63, 64, 200, 255, 256, 300, 639]:
        b0 = 0 if t < 256 else 256
        ob = (t - b0) // 64
        for n in range(16):
            if n <= ob <= n + 1 or n == 0:
                assert np.all(out[:, t, n] == np.inf)


@pytest.mark.parametrize("case", CASES)
def test_torch_form_matches(case):
    # the torch form the benchmark times as its CPU baseline is bit-exact
    from oracle.maxpool import max_pooling_1d_varlen_torch
    q_lens, k_lens, cache, Fs, msq, mcl, local, init = case
    d = workloads.maxpool_inputs(q_lens, F=Fs, H=2, seed=5, k_lens=k_lens, cache=cache)
    x = torch.randn(d["input"].shape, generator=torch.Generator().manual_seed(9))
    exp = max_pooling_1d_varlen(x, d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                                msq, mcl, local, init, oob="absent")
    got = max_pooling_1d_varlen_torch(x, d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                                      msq, mcl, local, init)
    np.testing.assert_array_equal(got.numpy(), exp)
