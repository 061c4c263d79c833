"""GPU parity of the fused max-pool + block top-k kernel (bit-exact).

The block ids must equal the oracle's selection (equal scores by ascending
id, ``-1`` for ``-inf`` blocks and missing slots, ``-1`` first) on the oracle's
pooled scores of the same input, and the optional pooled output must equal
the oracle's max-pool bit for bit.  Inputs the fused kernel does not take run
the unfused pair and must give the same result.
"""

import numpy as np
import pytest
import torch

from oracle.maxpool import max_pooling_1d_varlen as oracle_pool
from oracle.topk import topk_blocks as oracle_topk
import workloads
from unum_ops_amd.pipeline import maxpool_topk, topk_blocks

pytestmark = pytest.mark.gpu


def _check(d, dev, topk, return_pooled=True, **kw):
    res = maxpool_topk(d["input"].to(dev), d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev),
                       d["cache_lens"].to(dev), topk=topk, return_pooled=return_pooled, **kw)
    torch.cuda.synchronize()
    idx, pooled = res if return_pooled else (res, None)
    exp_pool = oracle_pool(d["input"], d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                           oob="absent", **kw)
    if pooled is not None:
        np.testing.assert_array_equal(pooled.float().cpu().numpy(), exp_pool)
    exp_idx = oracle_topk(exp_pool, topk)
    assert idx.dtype == torch.int32 and tuple(idx.shape) == exp_idx.shape
    np.testing.assert_array_equal(idx.cpu().numpy(), exp_idx)
    return idx


def _kw(max_seqlen_q, max_context_len, local_blocks=1, init_blocks=1):
    return dict(max_seqlen_q=max_seqlen_q, max_context_len=max_context_len,
                local_blocks=local_blocks, init_blocks=init_blocks)


@pytest.mark.parametrize("local_blocks", [1, 2])
def test_cfg2(local_blocks, dev):
    d = workloads.cfg2_maxpool(local_blocks=local_blocks)
    _check(d, dev, 64, **_kw(16384, 16384, local_blocks))


def test_long_rows_2112_blocks(dev):
    # cfg5's pooled width: 8447 compressed keys per row, flat stride 8448
    d = workloads.maxpool_inputs([300, 211], F=8448, H=2, seed=5, k_lens=[8447, 5000])
    _check(d, dev, 64, **_kw(16 * 8448, 135168))


@pytest.mark.parametrize("topk", [1, 7, 64, 100])
def test_ties_everywhere(topk, dev):
    # few distinct scores: the tie-break decides most of the selection
    d = workloads.maxpool_inputs([70, 33, 129], F=1024, H=2, seed=6)
    x = d["input"]
    d["input"] = torch.where(x > 0, torch.floor(x * 4096.0) / 8.0, x)
    _check(d, dev, topk, **_kw(16384, 64 * 200, 2, 3))


@pytest.mark.parametrize("topk", [1, 7, 64, 100])
def test_ties_on_long_rows(topk, dev):
    # 600 blocks (three chunks a lane): the search runs on the per-wave list
    # of keys between its bounds; few distinct scores put ties at the cut.
    d = workloads.maxpool_inputs([40, 25], F=2400, H=2, seed=11, k_lens=[2399, 1500])
    x = d["input"]
    d["input"] = torch.where(x > 0, torch.floor(x * 8192.0) / 16.0, x)
    _check(d, dev, topk, **_kw(16 * 2400, 64 * 600, 1, 1))


def test_most_keys_between_the_bounds(dev):
    # Rows of one repeated score with a few larger ones: more than 512 keys
    # lie between the bounds, so the search falls back to every key.
    d = workloads.maxpool_inputs([30, 20], F=8448, H=2, seed=12, k_lens=[8447, 8000])
    x = torch.full_like(d["input"], 0.25)
    x[:, :, 1000:1003] = 0.75
    x[:, 7:9, 5000] = 0.9
    x[:, 30:, 8000:] = 0.0
    d["input"] = x
    _check(d, dev, 64, **_kw(16 * 8448, 64 * 2112))


def _list_rows(T, ties, seed):
    """2112-block rows (nine chunks a lane) for the selection over the list:
    lane 0's largest score, 0.1, is the lower bound; every other lane holds an
    anchor in [0.12, 0.18] (lane 63 also a +inf block); everything else is
    below 0.05 but for m_r large scores outside lane 0, so row r's list holds
    65 + m_r entries."""
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(1, T, 2112, generator=g) * 0.05
    anchor = 4 * torch.arange(64)                   # block 4l: lane l, chunk 0
    x[0, :, anchor] = 0.12 + torch.rand(T, 64, generator=g) * 0.06
    x[0, :, 0] = 0.1
    free = torch.arange(2112) % 256 >= 4            # lane 0 keeps 0.1 as its largest
    free[anchor] = False
    free_cols = torch.nonzero(free).flatten()
    ms = []
    for r in range(T):
        m = min(r * 26, 1500) if r < T - 2 else 1500
        cols = free_cols[torch.randperm(free_cols.numel(), generator=g)[:m]]
        v = 0.2 + torch.rand(m, generator=g) * 0.8
        if ties:
            v = torch.floor(v * 64.0) / 64.0
        x[0, r, cols] = v
        ms.append(m)
    x[0, :, 4 * 63 + 1] = float("inf")
    return x, ms


@pytest.mark.parametrize("ties", [False, True])
def test_short_list_of_every_length(ties, dev):
    # Lists of 65 to 1565 entries: one to ten a lane, and past 640 (the row
    # then runs topk_select, whose own short list takes up to 1024 keys).
    x, _ = _list_rows(40, ties, 31 + ties)
    for topk in (1, 64):
        got = topk_blocks(x.to(dev), topk)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))


def test_minus_inf_blocks_on_long_rows(dev):
    # Short key counts leave most of a 2112-block row at -inf.  With 38 or 10
    # finite blocks some lanes hold only -inf, the bounds take every key and
    # -inf blocks are selected (as -1); with 275 finite blocks every lane has
    # one, and the -inf blocks stay below the short list's lower bound.
    d = workloads.maxpool_inputs([20, 20, 20, 20], F=8448, H=2, seed=13,
                                 k_lens=[8447, 150, 40, 1100])
    _check(d, dev, 64, **_kw(16 * 8448, 64 * 2112))


def test_fewer_blocks_than_topk(dev):
    d = workloads.maxpool_inputs([40, 9], F=128, H=2, seed=7, k_lens=[50, 20])
    _check(d, dev, 64, **_kw(2048, 1000))           # 16 blocks < 64


def test_block_count_not_multiple_of_four(dev):
    d = workloads.maxpool_inputs([40, 90], F=256, H=2, seed=8)
    _check(d, dev, 8, return_pooled=False, **_kw(4096, 64 * 13))   # 13 blocks, fused
    _check(d, dev, 8, return_pooled=True, **_kw(4096, 64 * 13))    # pooled asked: unfused


@pytest.mark.parametrize("n_seq", [63, 64, 70])
def test_many_sequences(n_seq, dev):
    # A row's sequence is found by ballots over cu_seqlens_q, 64 entries a
    # step: B + 1 = 64, 65 and 71 entries, with cached keys and 40 tokens past
    # the last sequence.
    g = np.random.default_rng(n_seq)
    q_lens = [int(x) for x in g.integers(120, 200, n_seq)]
    k_lens = [int(x) for x in g.integers(200, 990, n_seq)]
    cache = [int(x) for x in g.integers(0, 30, n_seq)]
    d = workloads.maxpool_inputs(q_lens, F=1024, H=2, seed=20 + n_seq, k_lens=k_lens, cache=cache)
    d["cu_seqlens_q"][-1] -= 40
    _check(d, dev, 64, **_kw(16 * 1024, 64 * 256, 2, 1))
    _check(d, dev, 64, return_pooled=False, **_kw(16 * 1024, 64 * 256, 2, 1))


def test_tokens_outside_sequences(dev):
    d = workloads.maxpool_inputs([50, 30], F=512, H=2, seed=9)
    d["cu_seqlens_q"] = torch.tensor([0, 20, 60], dtype=torch.int32)  # tokens 60..79 orphan
    _check(d, dev, 16, **_kw(8192, 8192))


def test_unfused_shapes(dev):
    d = workloads.maxpool_inputs([64, 20], F=1100, H=2, seed=10, k_lens=[1050, 400])
    _check(d, dev, 32, **_kw(16 * 1100, 64 * 4100))     # 4100 blocks > 4096
    db = dict(d, input=d["input"].to(torch.bfloat16))
    _check(db, dev, 32, **_kw(16 * 1100, 64 * 300))     # bf16 input


# ----------------------------------------------------------------------------
# topk_blocks: the same selection over rows already pooled (one kernel, the
# selection of the fused kernel above) -- bit-exact against the oracle.

def _pooled_rows(H, T, NB, seed, ties=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(H, T, NB, generator=g)
    if ties:
        x = torch.floor(x * 3.0) / 3.0
    r = torch.rand(H, T, NB, generator=g)
    x = torch.where(r < 0.05, torch.full_like(x, float("-inf")), x)
    x = torch.where(r > 0.98, torch.full_like(x, float("inf")), x)
    return x


@pytest.mark.parametrize("NB", [1, 3, 63, 64, 128, 255, 256, 257, 1000, 2112, 4096])
@pytest.mark.parametrize("topk", [1, 64, 100])
def test_topk_blocks_matches_oracle(NB, topk, dev):
    x = _pooled_rows(2, 37, NB, seed=NB * 7 + topk, ties=NB % 2 == 1)
    got = topk_blocks(x.to(dev), topk)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))


def test_topk_blocks_small_cases(dev):
    inf = float("inf")
    pooled = torch.tensor([[[0.5, -inf, 2.0, inf, 0.1, -inf],
                            [-inf, -inf, -inf, -inf, 3.0, -inf]]])
    assert topk_blocks(pooled.to(dev), 4).cpu().tolist() == [[[0, 2, 3, 4], [-1, -1, -1, 4]]]
    assert topk_blocks(torch.tensor([[[1.0, 3.0, 2.0]]]).to(dev), 5).cpu().tolist() == \
        [[[-1, -1, 0, 1, 2]]]
    ties = torch.tensor([[[1.0, 2.0, 2.0, 2.0, 0.5, 2.0]]]).to(dev)
    assert topk_blocks(ties, 2).cpu().tolist() == [[[1, 2]]]
    assert topk_blocks(ties, 4).cpu().tolist() == [[[1, 2, 3, 5]]]


def _list_case_rows(kind, T, NB, g):
    """Rows of two chunks or more for the list selection (topk <= 64) and the
    cases it hands to topk_select."""
    inf = float("inf")
    u = torch.rand(T, NB, generator=g)
    if kind == "uniform":
        return u
    if kind == "negative":            # no score >= 0: each lane's largest is its least negative
        return -u - 1.0
    if kind == "signed_zeros":        # -0.0 and +0.0 are one score: ties by ascending id
        x = torch.where(torch.rand(T, NB, generator=g) < 0.5, torch.tensor(-0.0), torch.tensor(0.0))
        x[:, torch.randperm(NB, generator=g)[:20]] = 1.0
        x[:, torch.randperm(NB, generator=g)[:NB // 2]] = -1.0
        return x
    if kind == "many_inf":            # more +inf blocks than slots
        x = u.clone()
        x[:, torch.randperm(NB, generator=g)[:100]] = inf
        return x
    if kind == "mostly_minus_inf":    # fewer finite blocks than slots: -inf selected (-1)
        x = torch.full((T, NB), -inf)
        x[:, torch.randperm(NB, generator=g)[:30]] = u[:, :30]
        return x
    if kind == "wide_tie":            # 64 + tied blocks at the cut, every lane holding one
        x = u * 0.1
        x[:, 0:256:4] = 0.5
        x[:, torch.randperm(NB, generator=g)[:40]] = 0.5
        x[:, torch.randperm(NB, generator=g)[:10]] = 0.9
        return x
    if kind == "coarse":              # few distinct scores: ties and long lists
        return torch.floor(u * 6.0)
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["uniform", "negative", "signed_zeros", "many_inf",
                                  "mostly_minus_inf", "wide_tie", "coarse"])
@pytest.mark.parametrize("NB", [257, 600, 2112, 4096])
def test_topk_blocks_list_selection(kind, NB, dev):
    g = torch.Generator().manual_seed(NB * 13 + len(kind))
    x = _list_case_rows(kind, 12, NB, g).reshape(1, 12, NB)
    for topk in (1, 7, 64, 65):       # 65: past the list selection
        got = topk_blocks(x.to(dev), topk)
        np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))


@pytest.mark.parametrize("seed", range(12))
def test_topk_blocks_random_rows(seed, dev):
    # Random widths (one chunk to sixteen), slot counts and score mixes: normal
    # scores, a coarse grid (ties), sprinkled +-inf and -0.0, negative rows.
    g = torch.Generator().manual_seed(1000 + seed)
    NB = int(torch.randint(2, 4097, (1,), generator=g))
    topk = int(torch.randint(1, 66, (1,), generator=g))
    x = torch.randn(2, 9, NB, generator=g)
    if seed % 3 == 1:
        x = torch.floor(x * 3.0) / 3.0
    if seed % 4 == 2:
        x = -x.abs() - 0.5
    r = torch.rand(2, 9, NB, generator=g)
    x = torch.where(r < 0.03, torch.full_like(x, float("-inf")), x)
    x = torch.where(r > 0.995, torch.full_like(x, float("inf")), x)
    x = torch.where((r > 0.4) & (r < 0.41), torch.full_like(x, -0.0), x)
    got = topk_blocks(x.to(dev), topk)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))


@pytest.mark.parametrize("NB", [200, 2112, 5000])
def test_topk_blocks_signed_zeros(NB, dev):
    # One chunk, the list selection, and one workgroup a row: -0.0 ranks as
    # +0.0 everywhere (the oracle's argsort compares them equal).
    x = torch.zeros(2, 5, NB)
    x[:, :, 1::3] = -0.0
    x[:, :, 7] = 2.0
    x[1, :, ::5] = -1.0
    got = topk_blocks(x.to(dev), 64)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, 64))


def test_topk_blocks_bf16_strided_and_wide(dev):
    x = _pooled_rows(3, 20, 300, seed=11, ties=True)
    wide = torch.zeros(3, 20, 320)
    wide[..., 7:307] = x
    got = topk_blocks(wide.to(dev)[..., 7:307], 64)            # non-contiguous rows
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, 64))
    xb = x.to(torch.bfloat16)
    got = topk_blocks(xb.to(dev), 64)                           # converted to fp32 exactly
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(xb.float(), 64))
    # past 4096 blocks a row: the workgroup-per-row kernel, same order
    x = _pooled_rows(1, 5, 5000, seed=12, ties=True)
    got = topk_blocks(x.to(dev), 64)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, 64))


# Rows past 4096 blocks (contexts past 262 144 tokens): one workgroup per row
# (256 threads of 32 blocks up to 8192 blocks, then 1024 threads of 16 or
# 32), every count summed through LDS.  Block counts at and around each
# size's edge, odd counts (the scalar loads), ties, +-inf blocks.
@pytest.mark.parametrize("NB", [4097, 5000, 8192, 8193, 16384, 16385, 30001, 32768])
@pytest.mark.parametrize("topk", [1, 64, 100])
def test_topk_blocks_wide_rows(NB, topk, dev):
    x = _pooled_rows(2, 3, NB, seed=NB + topk, ties=NB % 2 == 1)
    got = topk_blocks(x.to(dev), topk)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))


def test_topk_blocks_wide_rows_edge_cases(dev):
    inf = float("inf")
    NB = 6000
    g = torch.Generator().manual_seed(5)
    rows = torch.randn(8, NB, generator=g)
    rows[0] = 1.0                                   # every score equal: the lowest ids
    rows[1, 10:] = -inf                             # ten finite blocks, the rest -inf
    rows[2] = -inf                                  # nothing but -inf
    rows[3, ::7] = inf                              # more +inf blocks than topk
    rows[4] = torch.floor(rows[4] * 2.0) / 2.0      # heavy ties at the threshold
    rows[5, :5000] = -inf                           # a finite tail only
    rows[6, -3:] = inf                              # +inf at the last thread's blocks
    x = rows.reshape(1, 8, NB)
    for topk in (1, 7, 64, 200, 5999, 6000, 6100):  # up to more slots than blocks
        got = topk_blocks(x.to(dev), topk)
        np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, topk))
    # rows that are views: bf16, and fp32 at an unaligned offset of a wider buffer
    wide = torch.zeros(1, 8, NB + 5)
    wide[..., 1:NB + 1] = x
    got = topk_blocks(wide.to(dev)[..., 1:NB + 1], 64)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x, 64))
    got = topk_blocks(x.to(torch.bfloat16).to(dev), 64)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(x.to(torch.bfloat16).float(), 64))


def test_topk_blocks_refuses_rows_past_32768_blocks(dev):
    with pytest.raises(ValueError, match="exceed"):
        topk_blocks(torch.zeros(1, 1, 32769, device=dev), 4)


def test_topk_blocks_of_fused_stage1_maxpool(dev):
    # The fused stage-1 + max-pool output of cfg5's chunk, then the top-k: the
    # same ids as the fused pool + top-k over stage 1's scores.
    from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1_maxpool
    p = workloads.cfg5_pipeline()
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    pooled, scores = infllmv2_attn_stage1_maxpool(
        g["q"], g["k"], g["cu_seqlens_q"], g["cu_seqlens_k"], p["max_context_len"],
        max_seqlen_k=p["max_seqlen_k"], return_scores=True)
    got = topk_blocks(pooled, 64)
    kp = scores.shape[-1]
    exp = maxpool_topk(scores, g["cu_seqlens_q"], g["cu_seqlens_k"],
                       torch.zeros(1, dtype=torch.int32, device=dev), max_seqlen_q=16 * kp,
                       max_context_len=p["max_context_len"], local_blocks=1, init_blocks=1, topk=64)
    assert torch.equal(got, exp)
    np.testing.assert_array_equal(got.cpu().numpy(), oracle_topk(pooled.cpu(), 64))
