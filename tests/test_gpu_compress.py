"""GPU parity of key compression against the oracle -- bit-exact (the kernel
and the oracle fix the same fp32 summation order), plus the composition with
stage 1."""

import numpy as np
import pytest
import torch

from oracle.compress import compress_keys as oracle_compress
from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1
import workloads
from unum_ops_amd.compression import compress_keys
from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1

pytestmark = pytest.mark.gpu


def _check(raw, lengths, dev):
    cu = workloads.prefix(lengths)
    out, cu_c, max_c = compress_keys(raw.to(dev), cu.to(dev))
    torch.cuda.synchronize()
    exp, exp_cu = oracle_compress(raw, cu)
    np.testing.assert_array_equal(cu_c.cpu().numpy(), exp_cu)
    assert max_c == int(np.diff(exp_cu).max(initial=0))
    assert out.dtype == torch.bfloat16 and out.shape == exp.shape
    assert torch.equal(out.cpu().view(torch.int16), exp.view(torch.int16))
    return out, cu_c, max_c


def test_cfg5_context(dev):
    g = torch.Generator().manual_seed(5)
    raw = torch.randn(135168, 2, 128, generator=g).to(torch.bfloat16)
    out, _, max_c = _check(raw, [135168], dev)
    assert max_c == 8447


def test_ragged_batch_with_short_sequences(dev):
    lengths = [5, 31, 32, 33, 47, 48, 1000, 4096, 0, 77]
    g = torch.Generator().manual_seed(6)
    _check(torch.randn(sum(lengths), 2, 128, generator=g).to(torch.bfloat16), lengths, dev)


@pytest.mark.parametrize("H,D", [(1, 128), (4, 128), (2, 64), (8, 64), (4, 32)])
def test_head_shapes(H, D, dev):
    lengths = [300, 1111]
    g = torch.Generator().manual_seed(H * 100 + D)
    _check((torch.randn(sum(lengths), H, D, generator=g) * 4).to(torch.bfloat16), lengths, dev)


@pytest.mark.parametrize("seed", range(16))
def test_random_batches(seed, dev):
    # ragged batches (more than 64 sequences for some seeds), empty and short
    # sequences, head counts and widths drawn per seed
    rng = np.random.default_rng(700 + seed)
    B = int(rng.integers(1, 90))
    lengths = [int(v) for v in rng.integers(0, 3000, B)]
    lengths = [L if rng.random() > 0.2 else int(rng.integers(0, 48)) for L in lengths]
    H, D = [(1, 128), (2, 128), (4, 64), (2, 64)][seed % 4]
    g = torch.Generator().manual_seed(700 + seed)
    _check(torch.randn(sum(lengths), H, D, generator=g).to(torch.bfloat16), lengths, dev)


def test_strided_keys(dev):
    lengths = [500, 129]
    g = torch.Generator().manual_seed(8)
    wide = torch.randn(sum(lengths), 2, 256, generator=g).to(torch.bfloat16)
    cu = workloads.prefix(lengths)
    out, _, _ = compress_keys(wide.to(dev)[:, :, 64:192], cu.to(dev))
    exp, _ = oracle_compress(wide[:, :, 64:192].contiguous(), cu)
    assert torch.equal(out.cpu().view(torch.int16), exp.view(torch.int16))


def test_unsupported_shapes_raise(dev):
    with pytest.raises(NotImplementedError):
        compress_keys(torch.zeros(64, 8, 128, dtype=torch.bfloat16, device=dev),
                      torch.tensor([0, 64], dtype=torch.int32, device=dev))


def test_feeds_stage1(dev):
    # raw keys -> compressed keys -> stage-1 scores, against the oracle chain
    q_lens, ctx = [40, 17], [3000, 9000]
    g = torch.Generator().manual_seed(9)
    raw = torch.randn(sum(ctx), 2, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(q_lens), 32, 128, generator=g).to(torch.bfloat16)
    cu_q, cu_raw = workloads.prefix(q_lens), workloads.prefix(ctx)
    kc, cu_c, max_c = compress_keys(raw.to(dev), cu_raw.to(dev))
    out = infllmv2_attn_stage1(q.to(dev), kc, None, cu_q.to(dev), cu_c, max_seqlen_k=max_c,
                               causal=True)
    torch.cuda.synchronize()
    kc_ref, cu_c_ref = oracle_compress(raw, cu_raw)
    exp = oracle_stage1(q, kc_ref, None, cu_q, torch.from_numpy(cu_c_ref), max_seqlen_k=max_c,
                        causal=True)
    torch.testing.assert_close(out.cpu(), exp, atol=1e-3, rtol=1e-2)


def test_plan_reuse_matches(dev):
    from unum_ops_amd.compression import CompressionPlan
    lengths = [700, 64, 3000]
    g = torch.Generator().manual_seed(10)
    raw = torch.randn(sum(lengths), 2, 128, generator=g).to(torch.bfloat16).to(dev)
    cu = workloads.prefix(lengths)
    plan = CompressionPlan(cu, 2, 128, dev)
    a, cu_a, m_a = compress_keys(raw, cu.to(dev), plan=plan)
    b, cu_b, m_b = compress_keys(raw, cu.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(cu_a, cu_b) and m_a == m_b
