"""Pins of the stage-2 sparse-attention oracle (CPU).

* library reduction: per (token, kv head), ``F.scaled_dot_product_attention``
  over the K/V rows gathered at the block table's valid slots;
* closed form: ``q = 0`` makes every listed key equally likely, so each output
  row is the mean of the listed V rows, repeats counted;
* brute force: Python floats with an explicit softmax on tiny inputs, the
  slot of each entry worked out from the block-table formula;
* slot lists: exactly the entries ``oracle.get_block_table`` (Triton
  multiplier ``H``) marks valid, in table order.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.block_table import get_block_table as oracle_block_table
from oracle.sparse_attn import (gathered_rows, slot_table, sparse_paged_attention,
                                sparse_paged_attention_bruteforce, valid_entries)


def _problem(seed, T=6, Hkv=2, G=4, D=16, K=3, B=2, n_blocks=10, block_size=64, L=None,
             neg=0.2):
    g = torch.Generator().manual_seed(seed)
    L = L or 4 * 64
    q = torch.randn(T, Hkv * G, D, generator=g).to(torch.bfloat16)
    kc = torch.randn(n_blocks, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, L // 64, (Hkv, T, K), generator=g, dtype=torch.int32)
    idx = torch.where(torch.rand(Hkv, T, K, generator=g) < neg, torch.full_like(idx, -1), idx)
    slots = n_blocks * block_size
    bt = torch.randint(0, slots, (B, L), generator=g, dtype=torch.int32)
    tok = torch.randint(0, B, (T,), generator=g, dtype=torch.int32)
    pos = torch.randint(1, L + 40, (T,), generator=g, dtype=torch.int32)
    slen = torch.randint(1, L + 40, (B,), generator=g, dtype=torch.int32)
    return dict(query=q, key_cache=kc, value_cache=vc, num_heads=Hkv * G, num_kv_heads=Hkv,
                scale_value=D ** -0.5, topk_idx=idx, block_table=bt, token_to_bs=tok,
                token_pos_in_bs=pos, seqlen_q=slen)


@pytest.mark.parametrize("seed", range(3))
def test_matches_sdpa_on_gathered_rows(seed):
    p = _problem(seed)
    out = sparse_paged_attention(**p)
    D = p["query"].shape[-1]
    kf = p["key_cache"].float().reshape(-1, D)
    vf = p["value_cache"].float().reshape(-1, D)
    rows = gathered_rows(p["topk_idx"], p["block_table"], p["token_to_bs"], p["token_pos_in_bs"],
                         p["seqlen_q"], p["num_kv_heads"], kf.shape[0])
    G = p["num_heads"] // p["num_kv_heads"]
    n_checked = 0
    for t in range(p["query"].shape[0]):
        for h in range(p["num_kv_heads"]):
            r = torch.from_numpy(rows[t][h])
            qq = p["query"][t, h * G:(h + 1) * G].float()[None]           # [1, G, D]
            if r.numel() == 0:
                assert float(out[t, h * G:(h + 1) * G].abs().max()) == 0.0
                continue
            ref = F.scaled_dot_product_attention(qq, kf[r][None], vf[r][None],
                                                 scale=p["scale_value"])[0]
            torch.testing.assert_close(out[t, h * G:(h + 1) * G], ref, atol=1e-5, rtol=1e-5)
            n_checked += 1
    assert n_checked > 0


def test_zero_query_is_the_mean_of_listed_rows():
    p = _problem(7, neg=0.0)
    p["query"] = torch.zeros_like(p["query"])
    # force repeats: two ids equal per token, so a row is listed twice
    p["topk_idx"][:, :, 1] = p["topk_idx"][:, :, 0]
    out = sparse_paged_attention(**p)
    D = p["query"].shape[-1]
    vf = p["value_cache"].float().reshape(-1, D)
    valid = valid_entries(p["topk_idx"], p["token_to_bs"], p["token_pos_in_bs"], p["seqlen_q"],
                          p["block_table"].shape[0])
    table = oracle_block_table(p["topk_idx"], p["block_table"], p["token_to_bs"],
                               p["token_pos_in_bs"], p["seqlen_q"],
                               head_group=p["num_kv_heads"]).astype(np.int64)
    G = p["num_heads"] // p["num_kv_heads"]
    for t in range(out.shape[0]):
        for h in range(p["num_kv_heads"]):
            r = table[t, h][valid[t, h]]
            exp = vf[torch.from_numpy(r)].mean(0) if r.size else torch.zeros(D)
            for i in range(G):
                torch.testing.assert_close(out[t, h * G + i], exp, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("seed", range(2))
def test_bruteforce(seed):
    p = _problem(10 + seed, T=3, Hkv=2, G=2, D=8, K=2, B=2, n_blocks=4, block_size=64, L=192)
    torch.testing.assert_close(sparse_paged_attention(**p),
                               sparse_paged_attention_bruteforce(**p), atol=1e-5, rtol=1e-5)


def test_slot_lists_are_the_block_tables_valid_entries():
    p = _problem(3, T=9, K=4)
    kf_rows = p["key_cache"].reshape(-1, p["key_cache"].shape[-1]).shape[0]
    rows = gathered_rows(p["topk_idx"], p["block_table"], p["token_to_bs"], p["token_pos_in_bs"],
                         p["seqlen_q"], p["num_kv_heads"], kf_rows)
    table = oracle_block_table(p["topk_idx"], p["block_table"], p["token_to_bs"],
                               p["token_pos_in_bs"], p["seqlen_q"], head_group=p["num_kv_heads"])
    valid = valid_entries(p["topk_idx"], p["token_to_bs"], p["token_pos_in_bs"], p["seqlen_q"],
                          p["block_table"].shape[0])
    # invalid entries of the block table are exactly its zeros outside valid slots
    assert np.all(table[~valid] == 0)
    for t in range(table.shape[0]):
        for h in range(table.shape[1]):
            np.testing.assert_array_equal(rows[t][h], table[t, h][valid[t, h]].astype(np.int64))
    np.testing.assert_array_equal(slot_table(p["topk_idx"], p["block_table"], p["token_to_bs"],
                                             p["num_kv_heads"])[valid], table[valid])


def test_tokens_without_valid_slots_are_zero():
    p = _problem(4)
    p["token_to_bs"] = torch.tensor([0, -1, 5, 1, 0, 1], dtype=torch.int32)   # 5 >= B
    p["topk_idx"][:, 4] = -1                                                     # no block
    out = sparse_paged_attention(**p)
    for t in (1, 2, 4):
        assert float(out[t].abs().max()) == 0.0
    assert float(out[0].abs().max()) > 0.0 or float(out[3].abs().max()) > 0.0
