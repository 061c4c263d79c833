"""GPU parity: stage-2 sparse attention (sparse_paged_attention) vs the oracle.

The oracle attends, in fp32, over the K/V rows of the block table's valid
slots (oracle/sparse_attn.py).  The kernel's P.V products take each softmax
weight as two bf16 terms (to about 2^-15) with fp32 accumulation, so the bar
is |gpu - oracle| <= 1e-4 + 1e-3 |oracle| with an fp32 output (measured:
at most 7e-5 on the random shapes below), and the same plus one bf16
rounding of the result (2^-8 relative) with a bf16 output.  The two ways of naming
the slots -- recomputed from the block table, or read from get_block_table's
output -- run the same arithmetic and must agree bit for bit.
"""

import numpy as np
import pytest
import torch

import workloads
from oracle.sparse_attn import sparse_paged_attention as oracle_attn
from unum_ops_amd.pipeline import select_blocks
from unum_ops_amd.sparse_attention import sparse_paged_attention
from unum_ops_amd.sparse_kernel_extension import get_block_table

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3
RTOL_BF16_OUT = RTOL + 2.0 ** -8


def _problem(seed, T=7, Hkv=2, K=5, B=3, n_blocks=40, block_size=64, L=640, neg=0.15,
             scale=128 ** -0.5, kscale=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, 16 * Hkv, 128, generator=g).to(torch.bfloat16)
    kc = (torch.randn(n_blocks, block_size, Hkv, 128, generator=g) * kscale).to(torch.bfloat16)
    vc = torch.randn(n_blocks, block_size, Hkv, 128, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, L // 64, (Hkv, T, K), generator=g, dtype=torch.int32)
    idx = torch.where(torch.rand(Hkv, T, K, generator=g) < neg, torch.full_like(idx, -1), idx)
    bt = torch.randint(0, n_blocks * block_size, (B, L), generator=g, dtype=torch.int32)
    tok = torch.randint(0, B, (T,), generator=g, dtype=torch.int32)
    pos = torch.randint(1, L + 50, (T,), generator=g, dtype=torch.int32)
    slen = torch.randint(1, L + 50, (B,), generator=g, dtype=torch.int32)
    return dict(query=q, key_cache=kc, value_cache=vc, num_heads=16 * Hkv, num_kv_heads=Hkv,
                scale_value=scale, topk_idx=idx, block_table=bt, token_to_bs=tok,
                token_pos_in_bs=pos, seqlen_q=slen)


def _gpu(p, dev, **kw):
    args = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    out = sparse_paged_attention(**args, **kw)
    torch.cuda.synchronize()
    return out.cpu()


def _check(p, dev, out_dtype=torch.float32):
    exp = oracle_attn(**p)
    got = _gpu(p, dev, out_dtype=out_dtype)
    assert not torch.isnan(got).any()
    rtol = RTOL if out_dtype == torch.float32 else RTOL_BF16_OUT
    torch.testing.assert_close(got.float(), exp, atol=ATOL, rtol=rtol)
    return got, exp


@pytest.mark.parametrize("seed", range(4))
def test_random_small(seed, dev):
    _check(_problem(seed), dev)


@pytest.mark.parametrize("seed", range(16))
def test_random_shapes(seed, dev):
    # token counts, kv heads, K, sequences, cache sizes, context lengths, the
    # share of -1 ids and the key scale drawn per seed
    rng = np.random.default_rng(900 + seed)
    L = 64 * int(rng.integers(1, 40))
    p = _problem(900 + seed, T=int(rng.integers(1, 40)), Hkv=int(rng.integers(1, 5)),
                 K=int(rng.integers(1, 65)), B=int(rng.integers(1, 9)),
                 n_blocks=int(rng.integers(1, 80)), L=L, neg=float(rng.uniform(0, 0.5)),
                 kscale=float(rng.choice([0.5, 1.0, 4.0])))
    print(f"seed {seed}: T {p['query'].shape[0]} Hkv {p['num_kv_heads']} K "
          f"{p['topk_idx'].shape[2]} L {L}", flush=True)
    _check(p, dev)


@pytest.mark.parametrize("seed", range(2))
def test_bf16_output(seed, dev):
    got, exp = _check(_problem(20 + seed), dev, out_dtype=torch.bfloat16)
    assert got.dtype == torch.bfloat16


@pytest.mark.parametrize("seed", range(3))
def test_slot_table_path_is_bit_identical(seed, dev):
    p = _problem(30 + seed, T=11, K=7)
    fused = _gpu(p, dev)
    pd = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    slots = get_block_table(pd["topk_idx"], pd["block_table"], pd["token_to_bs"],
                            pd["token_pos_in_bs"], pd["seqlen_q"], head_group=p["num_kv_heads"])
    table = _gpu(p, dev, slots=slots)
    assert torch.equal(fused, table)


@pytest.mark.parametrize("Hkv", [3, 4])
def test_three_and_four_kv_heads(Hkv, dev):
    # The cache row of slot s for head h is Hkv*s + h; q and out carry 16*Hkv heads.
    _check(_problem(70 + Hkv, T=6, Hkv=Hkv, K=6), dev)


def test_peaky_scores_and_one_kv_head(dev):
    # Large scores move the running max many times (the lazy rescale); Hkv = 1.
    _check(_problem(41, Hkv=1, kscale=6.0), dev)


def test_edge_cases(dev):
    p = _problem(50, T=9, K=4, neg=0.0)
    p["token_to_bs"][1] = -1                     # outside every sequence: zeros
    p["token_to_bs"][2] = 7                      # b >= B: zeros
    p["topk_idx"][:, 3] = -1                     # no block: zeros
    p["topk_idx"][:, 4, 1] = p["topk_idx"][:, 4, 0]   # a repeated block counts twice
    p["token_pos_in_bs"][5] = 1                  # only position 0 is visible
    p["token_pos_in_bs"][6] = 64 * 3 + 17        # a partial block
    got, _ = _check(p, dev)
    for t in (1, 2, 3):
        assert float(got[t].abs().max()) == 0.0


def test_slots_outside_the_cache_are_skipped(dev):
    p = _problem(60, T=5, K=3, neg=0.0)
    pd = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    slots = get_block_table(pd["topk_idx"], pd["block_table"], pd["token_to_bs"],
                            pd["token_pos_in_bs"], pd["seqlen_q"], head_group=2)
    bad = slots.clone()
    n_rows = p["key_cache"].numel() // 128
    bad[:, :, 5] = n_rows + 3          # past the cache
    bad[:, :, 9] = -7                  # negative
    got = _gpu(p, dev, slots=bad)  # bf16 output
    exp = oracle_attn(**p, slots=bad.cpu())
    torch.testing.assert_close(got.float(), exp, atol=ATOL, rtol=RTOL_BF16_OUT)


def test_q_strides_and_cache_row_padding(dev):
    p = _problem(70, T=6)
    g = torch.Generator().manual_seed(71)
    big_q = torch.randn(6, 40, 136, generator=g).to(torch.bfloat16)
    p["query"] = big_q[:, 3:35, 8:136]            # strided query (16-byte aligned)
    kc_pad = torch.randn(40, 64, 2, 136, generator=g).to(torch.bfloat16)
    vc_pad = torch.randn(40, 64, 2, 136, generator=g).to(torch.bfloat16)
    pd = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    pd["query"] = big_q.to(dev)[:, 3:35, 8:136]
    pd["key_cache"] = kc_pad.to(dev)[..., :128]   # rows 136 elements apart
    pd["value_cache"] = vc_pad.to(dev)[..., :128]
    got = sparse_paged_attention(**pd, out_dtype=torch.float32).cpu()
    p["key_cache"], p["value_cache"] = kc_pad[..., :128], vc_pad[..., :128]
    torch.testing.assert_close(got, oracle_attn(**p), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("scale", [0.0, -0.05, -128 ** -0.5, 0.7])
def test_any_scale(scale, dev):
    # The scores are scaled before the running max and the key mask: a zero
    # scale gives the mean of the attended V rows, a negative one the softmax
    # of the negated products -- in partly masked stages too (-1 ids, partial
    # blocks, the position limit).
    p = _problem(80, T=9, K=6, neg=0.3, scale=scale)
    p["token_pos_in_bs"][2] = 64 * 2 + 5
    _check(p, dev)
    _check(p, dev, out_dtype=torch.bfloat16)


def test_misaligned_query_and_one_head_cache_slice(dev):
    # q at an odd element offset with odd strides (copied to the kernel's
    # layout by the wrapper), and the caches as one-head slices of two-head
    # caches: slots s1 apart, s2 belonging to the parent.
    p = _problem(90, T=6, Hkv=1, K=4)
    g = torch.Generator().manual_seed(91)
    big_q = torch.randn(6 * 17 + 1, 19, 131, generator=g).to(torch.bfloat16)
    kc2 = torch.randn(40, 64, 2, 128, generator=g).to(torch.bfloat16)
    vc2 = torch.randn(40, 64, 2, 128, generator=g).to(torch.bfloat16)
    pd = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    qd = big_q.to(dev).view(-1)[1:1 + 6 * 17 * 19 * 131].view(6, 17 * 19, 131)
    pd["query"] = qd[:, 3:19, 2:130]
    assert pd["query"].data_ptr() % 16 != 0
    pd["key_cache"] = kc2.to(dev)[:, :, 1:2]
    pd["value_cache"] = vc2.to(dev)[:, :, 1:2]
    got = sparse_paged_attention(**pd, out_dtype=torch.float32).cpu()
    p["query"] = pd["query"].cpu()
    p["key_cache"], p["value_cache"] = kc2[:, :, 1:2].contiguous(), vc2[:, :, 1:2].contiguous()
    torch.testing.assert_close(got, oracle_attn(**p), atol=ATOL, rtol=RTOL)


def _gather_checksum(p, slots):
    """The calibration kernel's checksum on the CPU: per (t, h, lane l =
    16r + s), the XOR of the 32-bit words of chunk s (16 bytes) of K xor V
    over the attended rows of keys 4r + i (i < 4) of every live stage."""
    from oracle.sparse_attn import valid_entries
    kc = p["key_cache"].contiguous().view(torch.int32).reshape(-1, 64).numpy()
    vc = p["value_cache"].contiguous().view(torch.int32).reshape(-1, 64).numpy()
    idx = p["topk_idx"].numpy().astype(np.int64)
    Hkv, T, K = idx.shape
    valid = valid_entries(p["topk_idx"], p["token_to_bs"], p["token_pos_in_bs"], p["seqlen_q"],
                          p["block_table"].shape[0])
    n_rows = kc.shape[0]
    out = np.zeros((T, Hkv, 64), dtype=np.uint32)
    for t in range(T):
        for h in range(Hkv):
            for k in range(K):
                for q4 in range(4):
                    e0 = 64 * k + 16 * q4
                    p0 = ((int(idx[h, t, k]) * 64 + 16 * q4 + 2 ** 31) % 2 ** 32) - 2 ** 31
                    if not (p0 >= 0 and _live(p, t, p0)):
                        continue
                    for lane in range(64):
                        r, s = divmod(lane, 16)
                        x = 0
                        for i in range(4):
                            e = e0 + 4 * r + i
                            row = int(slots[t, h, e])
                            if valid[t, h, e] and 0 <= row < n_rows:
                                w = kc[row, 4 * s:4 * s + 4] ^ vc[row, 4 * s:4 * s + 4]
                                x ^= int(np.bitwise_xor.reduce(w.astype(np.uint32)))
                        out[t, h, lane] ^= np.uint32(x)
    return out


def _live(p, t, p0):
    """Quarter starting at position p0 >= 0 of token t can hold an attended
    entry: p0 below min(seqlen_q[b], token_pos_in_bs[t])."""
    b = int(p["token_to_bs"][t])
    if not 0 <= b < p["block_table"].shape[0]:
        return False
    sl = p["seqlen_q"].reshape(-1)
    ps = p["token_pos_in_bs"].reshape(-1)
    lim = min(int(sl[0] if sl.numel() == 1 else sl[b]), int(ps[0] if ps.numel() == 1 else ps[t]))
    return p0 < lim


@pytest.mark.parametrize("seed", range(3))
def test_gather_calibration_checksum(seed, dev):
    # The calibration kernel gathers exactly the rows stage 2 attends (same
    # stages, row checks and lane pattern): its checksum equals the CPU's.
    from unum_ops_amd.sparse_attention import sparse_gather_calibrate
    p = _problem(110 + seed, T=5, K=5, neg=0.2)
    p["token_pos_in_bs"][1] = 64 + 7
    pd = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    slots = get_block_table(pd["topk_idx"], pd["block_table"], pd["token_to_bs"],
                            pd["token_pos_in_bs"], pd["seqlen_q"], head_group=2)
    exp = _gather_checksum(p, slots.cpu().numpy())
    for sl in (None, slots):
        got = sparse_gather_calibrate(pd["key_cache"], pd["value_cache"], 2, pd["topk_idx"],
                                      pd["block_table"], pd["token_to_bs"],
                                      pd["token_pos_in_bs"], pd["seqlen_q"], slots=sl)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), exp)


def _pipeline_case(p, dev, n_pages_pool, seed, check_tokens):
    """Stage 1 -> max-pool -> top-64 on the GPU for the block ids, then stage 2
    over random paged K/V caches; the oracle checks `check_tokens`."""
    g = {k: (v.to(dev) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    _, _, _, idx = select_blocks(g["q"], g["k"], g["cu_seqlens_q"], g["cu_seqlens_k"],
                                 g["block_table"], g["token_to_bs"], g["token_pos_in_bs"],
                                 g["seqlen_q"], p["max_context_len"],
                                 max_seqlen_k=p["max_seqlen_k"], topk=64,
                                 return_intermediates=True)
    Hkv = p["k"].shape[1]
    gen = torch.Generator(device=dev).manual_seed(seed)
    kc = torch.randn(n_pages_pool, 64, Hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(n_pages_pool, 64, Hkv, 128, generator=gen, device=dev).to(torch.bfloat16)
    # the page table of the case, folded into the pool (pages may repeat)
    bt = (g["block_table"] // 64 % n_pages_pool) * 64 + g["block_table"] % 64
    Hq = p["q"].shape[1]
    out = sparse_paged_attention(g["q"], kc, vc, Hq, Hkv, 128 ** -0.5, idx, bt,
                                 g["token_to_bs"], g["token_pos_in_bs"], g["seqlen_q"],
                                 out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    sel = torch.as_tensor(check_tokens)
    exp = oracle_attn(p["q"][sel], kc.cpu(), vc.cpu(), Hq, Hkv, 128 ** -0.5, idx.cpu()[:, sel],
                      bt.cpu(), p["token_to_bs"][sel], p["token_pos_in_bs"][sel], p["seqlen_q"])
    torch.testing.assert_close(out.cpu()[sel], exp, atol=ATOL, rtol=RTOL)
    # the slot-table path gives the same bits
    slots = get_block_table(idx, bt, g["token_to_bs"], g["token_pos_in_bs"], g["seqlen_q"],
                            head_group=Hkv)
    out2 = sparse_paged_attention(g["q"], kc, vc, Hq, Hkv, 128 ** -0.5, idx, bt,
                                  g["token_to_bs"], g["token_pos_in_bs"], g["seqlen_q"],
                                  slots=slots, out_dtype=torch.float32)
    assert torch.equal(out, out2)


def test_cfg4_selection(dev):
    p = workloads.cfg4_pipeline()
    T = int(p["cu_seqlens_q"][-1])
    _pipeline_case(p, dev, n_pages_pool=4096, seed=4, check_tokens=range(T))


@pytest.mark.parametrize("heads", [(32, 2), (16, 1)])
def test_cfg5_selection(heads, dev):
    p = workloads.cfg5_pipeline(Hq=heads[0], Hkv=heads[1])
    rng = np.random.default_rng(5)
    toks = np.sort(np.concatenate([np.arange(8), np.arange(4088, 4096),
                                   rng.choice(4096, 112, replace=False)]))
    _pipeline_case(p, dev, n_pages_pool=2112, seed=5, check_tokens=np.unique(toks))
