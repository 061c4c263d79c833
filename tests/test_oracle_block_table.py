"""Pins of the block-table oracle (CPU): brute force, known answers, closed forms."""

import numpy as np
import pytest

from oracle.block_table import get_block_table, get_block_table_bruteforce
import workloads


def _rand_case(seed, H=2, T=5, K=3, B=3, L=200, scalar_pos=False, scalar_len=False):
    rng = np.random.default_rng(seed)
    idx = rng.integers(-2, 6, size=(H, T, K)).astype(np.int32)
    bt = rng.integers(-5, 10000, size=(B, L)).astype(np.int32)
    bs = rng.integers(0, B, size=T).astype(np.int32)
    pos = rng.integers(0, 400, size=1 if scalar_pos else T).astype(np.int32)
    sl = rng.integers(0, 400, size=1 if scalar_len else B).astype(np.int32)
    return idx, bt, bs, pos, sl


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("scalar_pos,scalar_len", [(False, False), (True, False), (False, True), (True, True)])
def test_vectorised_matches_bruteforce(seed, scalar_pos, scalar_len):
    args = _rand_case(seed, scalar_pos=scalar_pos, scalar_len=scalar_len)
    np.testing.assert_array_equal(get_block_table(*args), get_block_table_bruteforce(*args))


@pytest.mark.parametrize("head_group", [1, 2, 3])
def test_head_group_bruteforce(head_group):
    args = _rand_case(11, H=3)
    np.testing.assert_array_equal(get_block_table(*args, head_group=head_group),
                                  get_block_table_bruteforce(*args, head_group=head_group))


def test_known_answer():
    # One token, two heads, two slots; a table row 0..299 so slot value = position.
    bt = np.arange(300, dtype=np.int32)[None, :]
    idx = np.array([[[1, -1]], [[4, 0]]], dtype=np.int32)         # [H=2, T=1, K=2]
    out = get_block_table(idx, bt, np.array([0], np.int32), np.array([270], np.int32),
                          np.array([1000], np.int32))
    assert out.shape == (1, 2, 128)
    # head 0, slot 0: block 1 -> positions 64..127, all < 270 -> 2*p + 0
    np.testing.assert_array_equal(out[0, 0, :64], 2 * np.arange(64, 128))
    # head 0, slot 1: id -1 -> zeros (not -1)
    np.testing.assert_array_equal(out[0, 0, 64:], np.zeros(64))
    # head 1, slot 0: block 4 -> positions 256..319; valid while p < 270 (pos limit);
    # 256..269 -> 2*p + 1, the rest 0
    exp = np.where(np.arange(256, 320) < 270, 2 * np.arange(256, 320) + 1, 0)
    np.testing.assert_array_equal(out[0, 1, :64], exp)
    # head 1, slot 1: block 0 -> 2*p + 1
    np.testing.assert_array_equal(out[0, 1, 64:], 2 * np.arange(64) + 1)


def test_clamp_to_last_column():
    # L = 100 < seqlen: valid positions >= 100 read block_table[b, 99] (get_table_torch.py:35).
    bt = (np.arange(100, dtype=np.int32) * 7)[None, :]
    idx = np.array([[[1]]], dtype=np.int32)
    out = get_block_table(idx, bt, np.array([0], np.int32), np.array([1 << 20], np.int32),
                          np.array([1 << 20], np.int32))
    p = np.arange(64, 128)
    np.testing.assert_array_equal(out[0, 0], 2 * bt[0, np.minimum(p, 99)])


def test_closed_forms_on_reference_test_inputs():
    for batch, seq_len, topk in [(1, 256, 4), (4, 1024, 16), (2, 8192, 96)]:
        d = workloads.reference_test_block_table(batch, seq_len, topk)
        out = get_block_table(d["topk_idx"], d["block_table"], d["token_to_bs"],
                              d["token_pos_in_bs"], d["seqlen_q"], topk=d["topk"])
        H, T, K = d["topk_idx"].shape
        assert out.shape == (T, H, K * 64) and out.dtype == np.int32
        idx = d["topk_idx"].numpy()
        sl = d["seqlen_q"].numpy()
        bt = d["block_table"].numpy()
        for t in range(T):
            for h in range(H):
                row = out[t, h].reshape(K, 64)
                for k in range(K):
                    p = idx[h, t, k] * 64 + np.arange(64)
                    valid = p < sl[t]
                    # parity with the head index where valid, zero elsewhere
                    assert np.all(row[k][valid] % 2 == h)
                    assert np.all(row[k][~valid] == 0)
                    np.testing.assert_array_equal(row[k][valid], 2 * bt[t, p[valid]] + h)


def test_int32_wraparound():
    # ids * 64 overflow int32 exactly like the torch reference's int32 arithmetic
    idx = np.array([[[2 ** 25 + 3]]], dtype=np.int32)
    bt = np.arange(10, dtype=np.int32)[None, :]
    big = np.array([2 ** 31 - 1], np.int32)
    args = (idx, bt, np.array([0], np.int32), big, big)
    np.testing.assert_array_equal(get_block_table(*args), get_block_table_bruteforce(*args))


def test_torch_inputs_accepted():
    d = workloads.cfg1_block_table("c")
    out = get_block_table(**d)
    assert out.shape == (4, 2, 16 * 64)
    heads = np.broadcast_to(np.arange(2)[None, :, None], out.shape)
    assert np.all(out[out != 0] % 2 == heads[out != 0])


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("scalar_pos,scalar_len", [(False, False), (True, True)])
def test_torch_form_matches(seed, scalar_pos, scalar_len):
    # the torch form the benchmark times as its CPU baseline gives the same ints
    import torch
    from oracle.block_table import get_block_table_torch
    args = _rand_case(40 + seed, scalar_pos=scalar_pos, scalar_len=scalar_len)
    got = get_block_table_torch(*(torch.from_numpy(a) for a in args))
    np.testing.assert_array_equal(got.numpy(), get_block_table(*args))
    wrap = (np.array([[[2 ** 25 + 3, -1]]], np.int32), np.arange(10, dtype=np.int32)[None, :],
            np.array([0], np.int32), np.array([2 ** 31 - 1], np.int32),
            np.array([2 ** 31 - 1], np.int32))
    np.testing.assert_array_equal(get_block_table_torch(*(torch.from_numpy(a) for a in wrap)).numpy(),
                                  get_block_table(*wrap))
