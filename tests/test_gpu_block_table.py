"""GPU parity: get_block_table HIP kernel vs the oracle -- bit-exact."""

import numpy as np
import pytest
import torch

from oracle.block_table import get_block_table as oracle_bt
import workloads
from unum_ops_amd import sparse_kernel_extension as ske
from unum_ops_amd.sparse_kernel_extension import (get_block_table, get_block_table_v1,
                                                  get_block_table_v2, get_block_table_v3)

pytestmark = pytest.mark.gpu


def _run(d, dev, fn=get_block_table, **kw):
    args = [d[k].to(dev) for k in ("topk_idx", "block_table", "token_to_bs",
                                   "token_pos_in_bs", "seqlen_q")]
    out = fn(*args, topk=d.get("topk"), **kw)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _oracle(d, **kw):
    return oracle_bt(d["topk_idx"], d["block_table"], d["token_to_bs"], d["token_pos_in_bs"],
                     d["seqlen_q"], **kw)


@pytest.mark.parametrize("variant", ["a", "b", "c"])
def test_cfg1(variant, dev):
    d = workloads.cfg1_block_table(variant)
    np.testing.assert_array_equal(_run(d, dev), _oracle(d))


@pytest.mark.parametrize("batch,seq_len,topk", [
    (1, 256, 4), (2, 512, 8), (4, 1024, 16), (8, 2048, 32), (4, 4096, 64), (2, 8192, 96)])
@pytest.mark.parametrize("fn", [get_block_table_v1, get_block_table_v2, get_block_table_v3])
def test_reference_test_shapes(batch, seq_len, topk, fn, dev):
    d = workloads.reference_test_block_table(batch, seq_len, topk)
    np.testing.assert_array_equal(_run(d, dev, fn), _oracle(d))


@pytest.mark.parametrize("seed", range(4))
def test_random_with_negatives_clamp_and_scalars(seed, dev):
    g = torch.Generator().manual_seed(100 + seed)
    H, T, K, B, L = 3, 37, 9, 5, 300
    d = dict(topk_idx=torch.randint(-3, 8, (H, T, K), generator=g, dtype=torch.int32),
             block_table=torch.randint(-100, 1 << 20, (B, L), generator=g, dtype=torch.int32),
             token_to_bs=torch.randint(0, B, (T,), generator=g, dtype=torch.int32),
             token_pos_in_bs=torch.randint(0, 600, (1 if seed % 2 else T,), generator=g,
                                           dtype=torch.int32),
             seqlen_q=torch.randint(0, 600, (1 if seed >= 2 else B,), generator=g,
                                    dtype=torch.int32))
    for hg in (2, H):
        np.testing.assert_array_equal(_run(d, dev, head_group=hg), _oracle(d, head_group=hg))


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes(seed, dev):
    # heads, tokens, K, sequences and table widths drawn per seed; block ids
    # past the table, -1 and other negatives, negative physical ids
    rng = np.random.default_rng(300 + seed)
    H, T = int(rng.integers(1, 5)), int(rng.integers(1, 300))
    K, B, L = int(rng.integers(1, 80)), int(rng.integers(1, 70)), int(rng.integers(1, 1200))
    g = torch.Generator().manual_seed(300 + seed)
    d = dict(topk_idx=torch.randint(-2, L // 64 + 3, (H, T, K), generator=g, dtype=torch.int32),
             block_table=torch.randint(-5, 1 << 22, (B, L), generator=g, dtype=torch.int32),
             token_to_bs=torch.randint(0, B, (T,), generator=g, dtype=torch.int32),
             token_pos_in_bs=torch.randint(0, 64 * (L // 64 + 2), (T,), generator=g,
                                           dtype=torch.int32),
             seqlen_q=torch.randint(0, 64 * (L // 64 + 2), (B,), generator=g, dtype=torch.int32))
    for hg in (2, H):
        np.testing.assert_array_equal(_run(d, dev, head_group=hg), _oracle(d, head_group=hg))


def test_strided_topk_and_unaligned_table(dev):
    g = torch.Generator().manual_seed(7)
    H, T, K, B, L = 2, 16, 12, 3, 777
    big = torch.randint(-1, 12, (T, K, H), generator=g, dtype=torch.int32)
    topk = big.permute(2, 0, 1)                         # non-contiguous [H, T, K]
    bt_full = torch.randint(0, 1 << 16, (B, L + 3), generator=g, dtype=torch.int32)
    d = dict(topk_idx=topk, block_table=bt_full[:, 1:L + 1],   # row stride L+3, offset 1
             token_to_bs=torch.randint(0, B, (T,), generator=g, dtype=torch.int32),
             token_pos_in_bs=torch.full((T,), 10 ** 6, dtype=torch.int32),
             seqlen_q=torch.full((B,), 10 ** 6, dtype=torch.int32))
    dev_args = dict(topk_idx=big.to(dev).permute(2, 0, 1), block_table=bt_full.to(dev)[:, 1:L + 1],
                    token_to_bs=d["token_to_bs"].to(dev), token_pos_in_bs=d["token_pos_in_bs"].to(dev),
                    seqlen_q=d["seqlen_q"].to(dev))
    out = get_block_table(**dev_args).cpu().numpy()
    np.testing.assert_array_equal(out, _oracle(d))


def test_out_of_range_token_to_bs_gives_zero_rows(dev):
    d = workloads.cfg1_block_table("c")
    d["token_to_bs"] = torch.tensor([0, 7, -1, 3], dtype=torch.int32)
    out = _run(d, dev)
    assert np.all(out[1] == 0) and np.all(out[2] == 0)
    ok = dict(d)
    ok["token_to_bs"] = torch.tensor([0, 0, 0, 3], dtype=torch.int32)
    exp = _oracle(ok)
    np.testing.assert_array_equal(out[[0, 3]], exp[[0, 3]])


def test_pipeline_scale_properties(dev):
    # cfg5-sized output (134 MB): bit-exact vs the oracle on identical ids
    g = torch.Generator().manual_seed(5)
    T, H, K = 4096, 2, 64
    ctx = 135168
    page = torch.randperm(2112, generator=g).to(torch.int32).view(1, 2112)
    bt = workloads.expand_pages(page)
    ids = torch.rand(H, T, 2112, generator=g).topk(K, dim=-1).indices.sort(-1).values.int()
    pos = torch.arange(131072 + 1, 131072 + T + 1, dtype=torch.int32)
    d = dict(topk_idx=ids, block_table=bt, token_to_bs=torch.zeros(T, dtype=torch.int32),
             token_pos_in_bs=pos, seqlen_q=torch.tensor([ctx], dtype=torch.int32))
    out = _run(d, dev)
    np.testing.assert_array_equal(out, _oracle(d))


# Head multiplier of each exported name, as its reference function uses it:
# the torch reference's constant kHeadGroup = 2 (get_table_torch.py:12), the
# Triton functions' H (get_table_triton.py:259, :315, :364; the package
# exports the first as get_block_table_v2/_v3, sparse_kernel_extension/
# __init__.py:7-12).  get_block_table_v1 (compiled-only CUDA extension,
# pinned by the reference tests at H = 2 only) takes 2 here.
_MULTIPLIER = {
    "get_block_table": "H",
    "get_block_table_ref_torch": 2,
    "get_block_table_ref_triton": "H",
    "get_block_table_ref_triton_v2": "H",
    "get_block_table_ref_triton_v3": "H",
    "get_block_table_v1": 2,
    "get_block_table_v2": "H",
    "get_block_table_v3": "H",
}


def test_every_exported_name_has_a_multiplier():
    assert sorted(_MULTIPLIER) == sorted(ske.__all__)


@pytest.mark.parametrize("H", [1, 2, 3])
@pytest.mark.parametrize("name", sorted(_MULTIPLIER))
def test_alias_head_multiplier(name, H, dev):
    g = torch.Generator().manual_seed(40 + H)
    T, K, B, L = 29, 7, 4, 640
    d = dict(topk_idx=torch.randint(-1, 10, (H, T, K), generator=g, dtype=torch.int32),
             block_table=torch.randint(0, 1 << 20, (B, L), generator=g, dtype=torch.int32),
             token_to_bs=torch.randint(0, B, (T,), generator=g, dtype=torch.int32),
             token_pos_in_bs=torch.randint(1, L + 1, (T,), generator=g, dtype=torch.int32),
             seqlen_q=torch.randint(1, L + 1, (B,), generator=g, dtype=torch.int32))
    mult = H if _MULTIPLIER[name] == "H" else _MULTIPLIER[name]
    got = _run(d, dev, getattr(ske, name))
    np.testing.assert_array_equal(got, _oracle(d, head_group=mult))
    if H != 2:  # the multiplier matters: the other one gives a different table
        other = 2 if mult == H else H
        assert not np.array_equal(got, _oracle(d, head_group=other))


def test_cfg5_variant_16_1_slots(dev):
    # The block-table stage of the Hq16/Hkv1 variant: H = 1, so the Triton
    # names give slot + 0 (multiplier 1) and the torch name 2 * slot.
    g = torch.Generator().manual_seed(11)
    T, K = 512, 64
    page = torch.randperm(2112, generator=g).to(torch.int32).view(1, 2112)
    bt = workloads.expand_pages(page)
    ids = torch.rand(1, T, 2112, generator=g).topk(K, dim=-1).indices.sort(-1).values.int()
    pos = torch.arange(131072 + 1, 131072 + T + 1, dtype=torch.int32)
    d = dict(topk_idx=ids, block_table=bt, token_to_bs=torch.zeros(T, dtype=torch.int32),
             token_pos_in_bs=pos, seqlen_q=torch.tensor([135168], dtype=torch.int32))
    np.testing.assert_array_equal(_run(d, dev, get_block_table_v2), _oracle(d, head_group=1))
    np.testing.assert_array_equal(_run(d, dev, ske.get_block_table_ref_torch),
                                  _oracle(d, head_group=2))
