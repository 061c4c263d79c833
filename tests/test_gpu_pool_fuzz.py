"""GPU parity on seeded random max-pool problems: the max-pool and the fused
max-pool + top-k against the oracle, bit for bit.

Each seed draws ragged sequences (empty ones included), a flat row stride F
(not always a multiple of 4), key counts up to F, cache lengths, the pooled
width (max_context_len), the forced init / local blocks, the head count, the
input dtype and K.  The input is N(0,1) noise, so negative and tied-after-
rounding scores occur; the top-k takes the oracle's order (score descending,
block id ascending), -1 past the row's blocks.
"""

import numpy as np
import pytest
import torch

from oracle.maxpool import max_pooling_1d_varlen as oracle_pool
from oracle.topk import topk_blocks as oracle_topk
import workloads
from unum_ops_amd.infllm_v2 import max_pooling_1d_varlen
from unum_ops_amd.pipeline import maxpool_topk

pytestmark = pytest.mark.gpu


def _problem(seed):
    rng = np.random.default_rng(5000 + seed)
    B = int(rng.integers(1, 9))
    H = int(rng.integers(1, 4))
    # the fused top-k kernel takes fp32 rows of a stride that is a multiple of 4
    # (pooled widths a multiple of 4 when the pooled scores are returned too)
    F = int(rng.integers(8, 2200)) if seed % 4 == 3 else 4 * int(rng.integers(2, 550))
    q_lens = [int(v) for v in rng.integers(0, 200, B)]
    k_lens = [int(v) for v in rng.integers(0, F + 1, B)]
    cache = [int(v) for v in rng.integers(0, 300, B)]
    mcl = int(rng.integers(64, 20000))
    if seed % 2 == 0:
        mcl = 256 * (mcl // 256 + 1)
    local, init = int(rng.integers(0, 4)), int(rng.integers(0, 4))
    dtype = [torch.float32, torch.float32, torch.bfloat16, torch.float16][seed % 4]
    topk = [1, 7, 16, 64, 100][seed % 5]
    d = workloads.maxpool_inputs(q_lens, F=F, H=H, seed=seed, k_lens=k_lens, cache=cache)
    d["input"] = torch.randn(d["input"].shape,
                             generator=torch.Generator().manual_seed(seed)).to(dtype)
    kw = dict(max_seqlen_q=16 * F, max_context_len=mcl, local_blocks=local, init_blocks=init)
    return d, kw, topk


@pytest.mark.parametrize("seed", range(40))
def test_random_pools(seed, dev):
    d, kw, topk = _problem(seed)
    print(f"seed {seed}: shape {tuple(d['input'].shape)} {d['input'].dtype} {kw} topk {topk}",
          flush=True)
    args = [d[n].to(dev) for n in ("input", "cu_seqlens_q", "cu_seqlens_k", "cache_lens")]
    exp = oracle_pool(d["input"], d["cu_seqlens_q"], d["cu_seqlens_k"], d["cache_lens"],
                      oob="absent", **kw)
    out = max_pooling_1d_varlen(*args, **kw)
    torch.cuda.synchronize()
    assert out.dtype == d["input"].dtype
    np.testing.assert_array_equal(out.float().cpu().numpy(), exp)

    exp_idx = oracle_topk(exp, topk)
    idx, pooled = maxpool_topk(*args, topk=topk, return_pooled=True, **kw)
    idx_only = maxpool_topk(*args, topk=topk, **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(pooled.float().cpu().numpy(), exp)
    np.testing.assert_array_equal(idx.cpu().numpy(), exp_idx)
    np.testing.assert_array_equal(idx_only.cpu().numpy(), exp_idx)
