"""GPU parity on seeded random batches that cross every stage-1 path.

Each seed draws a batch of ragged sequences (empty ones included) in one of
four regimes: rows of at most 512 keys (the LDS-resident kernel), longer rows
(the streaming kernel, whole rows or key splits), decode batches (one or two
new tokens per sequence: the one-workgroup-a-row kernel) and a mix, with
peaky keys, bf16 score outputs, other softmax scales and strided q / k for
some seeds.  Stage 1 must match the oracle at atol 1e-3 / rtol 1e-2 (the bar of test_gpu_stage1),
and the fused stage-1 + max-pool entry must return, bit for bit, the oracle's
max-pool of the scores it wrote.
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


def _batch(seed):
    rng = np.random.default_rng(1000 + seed)
    regime = seed % 4
    B = int(rng.integers(1, 9))
    if regime == 0:    # rows of at most 512 keys
        q = rng.integers(0, 49, B)
        ctx = q + rng.integers(0, 8192 - 48, B)
    elif regime == 1:  # rows over 512 keys
        q = rng.integers(0, 49, B)
        ctx = q + rng.integers(8200, 20000, B)
    elif regime == 2:  # decode batches
        q = rng.integers(1, 3, B)
        ctx = q + rng.integers(2000, 40000, B)
    else:              # a mix, short contexts included (no keys below 32 tokens)
        q = rng.integers(0, 33, B)
        ctx = q + rng.integers(0, 12000, B)
        short = rng.random(B) < 0.2
        ctx[short] = q[short]  # contexts of just the new tokens
    hq, hkv = [(32, 2), (16, 1), (48, 3)][seed % 3]
    return [int(v) for v in q], [int(v) for v in ctx], hq, hkv, bool(seed % 5)


@pytest.mark.parametrize("seed", range(48))
def test_random_batches(seed, dev):
    q_lens, ctx, hq, hkv, causal = _batch(seed)
    # every seventh seed peaky keys (x8), every fourth a bf16 score output; the
    # softmax scale varies too (a non-positive one runs the per-row MFMA kernel)
    peaky, out_dtype = seed % 7 == 3, torch.bfloat16 if seed % 4 == 1 else torch.float32
    scale = [None, None, 0.05, 0.3, None, -0.08, 1.0 / 64, 0.0][seed % 8]
    d = workloads.stage1_inputs(q_lens, ctx, Hq=hq, Hkv=hkv, seed=seed, raw_keys=False,
                                peaky=peaky)
    print(f"seed {seed}: q {q_lens} ctx {ctx} Hq {hq} Hkv {hkv} causal {causal} peaky {peaky} "
          f"{out_dtype} scale {scale}", flush=True)
    q, k = d["q"].to(dev), d["k"].to(dev)
    if seed % 6 == 5:  # rows of a wider tensor: head strides 136, token strides 136*H
        wq = torch.zeros(q.shape[0], q.shape[1], 136, dtype=q.dtype, device=dev)
        wk = torch.zeros(k.shape[0], k.shape[1], 136, dtype=k.dtype, device=dev)
        wq[:, :, 8:] = q
        wk[:, :, :128] = k
        q, k = wq[:, :, 8:], wk[:, :, :128]
    cq, ck = d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev)
    msk = max(d["max_seqlen_k"], 1)
    out = infllmv2_attn_stage1(q, k, None, cq, ck, max_seqlen_k=msk, softmax_scale=scale,
                               causal=causal, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.dtype == out_dtype
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=msk, softmax_scale=scale, causal=causal)
    torch.testing.assert_close(out.float().cpu(), exp, atol=ATOL, rtol=RTOL)

    max_ctx = max(max(ctx), 1)
    pooled, scores = infllmv2_attn_stage1_maxpool(q, k, cq, ck, max_ctx, max_seqlen_k=msk,
                                                  softmax_scale=scale, causal=causal,
                                                  return_scores=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(scores.cpu(), exp, atol=ATOL, rtol=RTOL)
    exp_p = oracle_pool(scores.cpu(), d["cu_seqlens_q"], d["cu_seqlens_k"],
                        torch.zeros(len(q_lens), dtype=torch.int32), 16 * scores.shape[-1],
                        max_ctx, 1, 1)
    np.testing.assert_array_equal(pooled.cpu().numpy(), exp_p)


@pytest.mark.parametrize("seed", range(8))
def test_random_generic_shapes(seed, dev):
    # head groups other than 16 and head dims other than 128: the generic kernel
    q_lens, ctx, _, _, causal = _batch(4 * seed)  # rows of at most 512 keys
    hq, hkv, D = [(32, 4, 128), (16, 1, 64), (8, 8, 128), (24, 2, 64)][seed % 4]
    d = workloads.stage1_inputs(q_lens, ctx, Hq=hq, Hkv=hkv, D=D, seed=seed, raw_keys=False)
    print(f"seed {seed}: q {q_lens} ctx {ctx} Hq {hq} Hkv {hkv} D {D} causal {causal}", flush=True)
    msk = max(d["max_seqlen_k"], 1)
    out = infllmv2_attn_stage1(d["q"].to(dev), d["k"].to(dev), None, d["cu_seqlens_q"].to(dev),
                               d["cu_seqlens_k"].to(dev), max_seqlen_k=msk, causal=causal)
    torch.cuda.synchronize()
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=msk, causal=causal)
    torch.testing.assert_close(out.cpu(), exp, atol=ATOL, rtol=RTOL)
