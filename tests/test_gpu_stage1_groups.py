"""GPU parity of stage 1 with three and four kv groups of 16 query heads.

The MFMA kernels take a (token, group) row's 16 heads as one 4 KiB run of q,
group g's keys at column g of each key row, and write group g's scores at
``out[g]``; the other tests run them with one or two groups.  Here every MFMA
path -- the LDS-resident kernel (rows of at most 512 keys), the streaming
kernel's whole rows and key splits, and the decode kernel -- runs Hq/Hkv = 48/3
and 64/4 against the fp32 oracle (atol 1e-3 / rtol 1e-2), and the fused
stage-1 + max-pool entry is checked bit for bit against the oracle's pool of
the scores it returns.
"""

import numpy as np
import pytest
import torch

from oracle.maxpool import max_pooling_1d_varlen as oracle_pool
from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1
import workloads
from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1, infllmv2_attn_stage1_maxpool

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2

# (Hq, Hkv, new tokens per sequence, context per sequence); the comment names
# the kernel the shape takes.
CASES = {
    "lds_3": (48, 3, [200, 64], [6000, 8192]),           # <= 512 keys: LDS-resident
    "lds_4": (64, 4, [96, 33], [3000, 8000]),
    "split_3": (48, 3, [40, 9, 1], [9000, 30000, 12000]),  # few tokens, long rows: key splits
    "rows_4": (64, 4, [300], [12000]),                    # one long prefill piece set
    "decode_3": (48, 3, [1] * 6, [20000] * 6),            # Tq <= 2B, <= 4096 keys: decode
    "decode_4": (64, 4, [1, 2, 1, 1], [9000, 16000, 7000, 12000]),
}


def _inputs(name):
    Hq, Hkv, q_lens, ctx = CASES[name]
    return workloads.stage1_inputs(q_lens, ctx, Hq=Hq, Hkv=Hkv, seed=Hq + 7 * Hkv + len(q_lens))


@pytest.mark.parametrize("name", sorted(CASES))
def test_stage1_groups(name, dev):
    d = _inputs(name)
    out = infllmv2_attn_stage1(d["q"].to(dev), d["k"].to(dev), None, d["cu_seqlens_q"].to(dev),
                               d["cu_seqlens_k"].to(dev), max_seqlen_k=d["max_seqlen_k"],
                               causal=True)
    torch.cuda.synchronize()
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=d["max_seqlen_k"], causal=True)
    assert out.shape == exp.shape and out.shape[0] == CASES[name][1]
    torch.testing.assert_close(out.cpu(), exp, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("name", ["lds_3", "split_3", "rows_4"])
def test_stage1_maxpool_groups(name, dev):
    d = _inputs(name)
    ctx = max(CASES[name][3])
    args = (d["q"].to(dev), d["k"].to(dev), d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev), ctx)
    kw = dict(max_seqlen_k=d["max_seqlen_k"], causal=True, local_blocks=1, init_blocks=1)
    pooled, scores = infllmv2_attn_stage1_maxpool(*args, return_scores=True, **kw)
    pooled_only = infllmv2_attn_stage1_maxpool(*args, **kw)
    torch.cuda.synchronize()
    exp_s = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                          max_seqlen_k=d["max_seqlen_k"], causal=True)
    torch.testing.assert_close(scores.cpu(), exp_s, atol=ATOL, rtol=RTOL)
    B = d["cu_seqlens_q"].numel() - 1
    exp_p = oracle_pool(scores.cpu(), d["cu_seqlens_q"], d["cu_seqlens_k"],
                        torch.zeros(B, dtype=torch.int32), 16 * scores.shape[-1], ctx, 1, 1)
    np.testing.assert_array_equal(pooled.cpu().numpy(), exp_p)
    assert torch.equal(pooled_only, pooled)
