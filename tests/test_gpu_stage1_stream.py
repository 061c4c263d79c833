"""GPU parity of the K-streaming stage-1 kernel (rows longer than 512 compressed
keys) against the fp32 oracle, at atol 1e-3 / rtol 1e-2.

Cases aimed at the kernel's own structure: pieces of tokens (16 on whole
rows, 8 on key splits) that straddle sequence boundaries, tokens that see no key, chunks cut by the sequence end,
tokens outside every sequence, bf16 output, strided queries, and scores that
grow along the keys far enough to force the running reference maximum to
move (the rare re-do path).
"""

import pytest
import torch

from oracle.stage1 import infllmv2_attn_stage1 as oracle_stage1
import workloads
from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2


def _run_check(d, dev, causal=True, out_dtype=torch.float32, q=None):
    qd = (d["q"] if q is None else q).to(dev)
    out = infllmv2_attn_stage1(qd, d["k"].to(dev), None, d["cu_seqlens_q"].to(dev),
                               d["cu_seqlens_k"].to(dev), max_seqlen_k=d["max_seqlen_k"],
                               causal=causal, out_dtype=out_dtype)
    torch.cuda.synchronize()
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=d["max_seqlen_k"], causal=causal)
    assert out.shape == exp.shape and out.shape[-1] > 512
    if out_dtype == torch.bfloat16:
        torch.testing.assert_close(out.float().cpu(), exp.to(torch.bfloat16).float(),
                                   atol=2e-3, rtol=2e-2)
    else:
        torch.testing.assert_close(out.cpu(), exp, atol=ATOL, rtol=RTOL)
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_pieces_straddle_sequences(causal, dev):
    d = workloads.stage1_inputs([5, 30, 1, 17, 9], [9000, 600, 3000, 700, 5000], seed=41)
    _run_check(d, dev, causal)


def test_tokens_without_visible_keys(dev):
    # 1000 queries on 100 context tokens (5 compressed keys): the early tokens
    # see nothing; the second sequence makes the rows long.
    d = workloads.stage1_inputs([1000, 4], [100, 9000], seed=42)
    out = _run_check(d, dev)
    assert float(out[:, :40].abs().max()) == 0.0


@pytest.mark.parametrize("ctx", [32 + 16 * 512, 32 + 16 * 513, 32 + 16 * 766])
def test_chunk_boundaries(ctx, dev):
    # compressed lengths 513 / 514 / 767: the last 128-key chunk is cut
    d = workloads.stage1_inputs([20], [ctx], seed=ctx)
    _run_check(d, dev)


def test_tokens_outside_sequences(dev):
    d = workloads.stage1_inputs([10, 20], [3000, 9000], seed=43)
    q = torch.cat([torch.randn(3, 32, 128).to(torch.bfloat16), d["q"],
                   torch.randn(6, 32, 128).to(torch.bfloat16)])
    d["q"] = q
    d["cu_seqlens_q"] = d["cu_seqlens_q"] + 3
    out = _run_check(d, dev)
    assert float(out[:, :3].abs().max()) == 0.0 and float(out[:, -6:].abs().max()) == 0.0


def test_bf16_output(dev):
    d = workloads.stage1_inputs([33, 7], [9000, 2000], seed=44)
    _run_check(d, dev, out_dtype=torch.bfloat16)


def test_strided_queries(dev):
    d = workloads.stage1_inputs([24, 9], [6000, 9000], seed=45)
    wide = torch.zeros(d["q"].shape[0], 48, 128, dtype=torch.bfloat16)
    wide[:, 8:40] = d["q"]
    _run_check(d, dev, q=wide[:, 8:40])


@pytest.mark.parametrize("causal", [True, False])
def test_growing_scores_move_the_reference(causal, dev):
    # Scores rise linearly along the keys up to ~2000 (log2-domain ~260), far
    # above the first quad's maximum: pass 1 must re-base its reference.
    Lq, ctx = 40, 48032
    Lk = workloads.compressed_len(ctx)
    q = torch.ones(Lq, 32, 128).to(torch.bfloat16)
    ramp = (torch.arange(Lk, dtype=torch.float32) / Lk * 16.0)
    k = ramp[:, None, None].expand(Lk, 2, 128).contiguous().to(torch.bfloat16)
    d = dict(q=q, k=k, cu_seqlens_q=torch.tensor([0, Lq], dtype=torch.int32),
             cu_seqlens_k=torch.tensor([0, Lk], dtype=torch.int32), max_seqlen_k=Lk)
    out = _run_check(d, dev, causal)
    assert torch.isfinite(out).all()


def test_large_magnitude_keys(dev):
    d = workloads.stage1_inputs([50, 16], [20000, 7000], seed=46)
    d["k"] = (d["k"].float() * 40.0).to(torch.bfloat16)
    _run_check(d, dev)


def test_decode_mix_many_short_sequences(dev):
    # cfg4's shape in small: many sequences of a few query tokens over long
    # contexts -- the rows are split over keys between workgroups.
    g = torch.Generator().manual_seed(47)
    q_lens = torch.randint(1, 17, (12,), generator=g).tolist()
    ctx = torch.randint(8000, 20000, (12,), generator=g).tolist()
    d = workloads.stage1_inputs(q_lens, ctx, seed=47, raw_keys=False)
    _run_check(d, dev)


# Decode batches (at most two new tokens per sequence on average, rows of at
# most 4096 keys) run one workgroup per row, its waves splitting the keys.

def test_decode_one_token_per_sequence(dev):
    g = torch.Generator().manual_seed(61)
    ctx = torch.randint(9000, 65000, (40,), generator=g).tolist()
    d = workloads.stage1_inputs([1] * 40, ctx, seed=61, raw_keys=False)
    _run_check(d, dev)


def test_decode_ragged_with_gaps(dev):
    # 0-3 new tokens per sequence, short and long rows (some under 64 keys),
    # and tokens outside every sequence.
    g = torch.Generator().manual_seed(62)
    q_lens = torch.randint(0, 4, (90,), generator=g).tolist()
    q_lens[0] = 3
    ctx = torch.randint(200, 60000, (90,), generator=g).tolist()
    ctx[1] = 40
    d = workloads.stage1_inputs(q_lens, ctx, seed=62, raw_keys=False)
    pre, post = 3, 5
    d["q"] = torch.cat([torch.randn(pre, 32, 128).to(torch.bfloat16), d["q"],
                        torch.randn(post, 32, 128).to(torch.bfloat16)])
    d["cu_seqlens_q"] = d["cu_seqlens_q"] + pre
    assert d["q"].shape[0] <= 2 * 90
    out = _run_check(d, dev)
    assert float(out[:, :pre].abs().max()) == 0.0 and float(out[:, -post:].abs().max()) == 0.0


def test_decode_scores_far_above_the_first_quad(dev):
    # Scores rise along the keys far above each wave's first quad: the
    # reference moves (the quad is summed again).
    Lk = 3900
    q = torch.ones(2, 32, 128).to(torch.bfloat16)
    ramp = (torch.arange(Lk, dtype=torch.float32) / Lk * 16.0)
    k = ramp[:, None, None].expand(Lk, 2, 128).contiguous().to(torch.bfloat16)
    d = dict(q=q, k=k, cu_seqlens_q=torch.tensor([0, 1, 2], dtype=torch.int32),
             cu_seqlens_k=torch.tensor([0, Lk - 700, Lk], dtype=torch.int32), max_seqlen_k=Lk - 700)
    out = _run_check(d, dev)
    assert torch.isfinite(out).all()


def test_decode_bf16_output_and_large_keys(dev):
    d = workloads.stage1_inputs([1, 2, 1, 1], [30000, 20000, 9000, 50000], seed=63, raw_keys=False)
    d["k"] = (d["k"].float() * 40.0).to(torch.bfloat16)
    _run_check(d, dev)
    _run_check(d, dev, out_dtype=torch.bfloat16)


@pytest.mark.parametrize("n_seq", [70, 150])
def test_more_than_64_sequences_with_gaps(n_seq, dev):
    # Workgroups find their piece from a prefix over cu_seqlens_q, 64
    # sequences per step: batches past 64 sequences, empty sequences, and
    # tokens outside every sequence (zeroed by the workgroups past the last
    # piece), on the key-split kernels (short rows) and the whole-row kernel.
    g = torch.Generator().manual_seed(49 + n_seq)
    q_lens = torch.randint(0, 12, (n_seq,), generator=g).tolist()
    q_lens[0], q_lens[-1] = 5, 17
    ctx = torch.randint(8300, 9000, (n_seq,), generator=g).tolist()
    d = workloads.stage1_inputs(q_lens, ctx, seed=49, raw_keys=False)
    pre, post = 4, 7
    d["q"] = torch.cat([torch.randn(pre, 32, 128).to(torch.bfloat16), d["q"],
                        torch.randn(post, 32, 128).to(torch.bfloat16)])
    d["cu_seqlens_q"] = d["cu_seqlens_q"] + pre
    out = _run_check(d, dev)                       # with a workspace: key splits
    assert float(out[:, :pre].abs().max()) == 0.0 and float(out[:, -post:].abs().max()) == 0.0
    whole = _c_entry(d, dev, with_ws=False)        # without: the whole-row kernel
    torch.testing.assert_close(whole.cpu(), out.cpu(), atol=1e-4, rtol=1e-3)
    assert float(whole[:, :pre].abs().max()) == 0.0 and float(whole[:, -post:].abs().max()) == 0.0


def _c_entry(d, dev, with_ws):
    """Stage 1 through the C entry point, with or without the split workspace."""
    import ctypes

    from unum_ops_amd import _lib

    q, k = d["q"].to(dev), d["k"].to(dev)
    cu_q, cu_k = d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev)
    B = cu_q.numel() - 1
    cols = (d["max_seqlen_k"] + 127) // 128 * 128
    lib = _lib.load()
    ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(B, q.shape[0], 32, 2, 128,
                                                            d["max_seqlen_k"])
    out = torch.full((2, q.shape[0], cols), float("nan"), device=dev)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if with_ws else None
    st = lib.unum_infllmv2_attn_stage1(
        _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
        _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
        B, q.shape[0], k.shape[0], 32, 2, 128, d["max_seqlen_k"], cols,
        ctypes.c_float(128 ** -0.5), 1, _lib.ptr(ws), ws_bytes if with_ws else 0,
        _lib.stream_ptr(dev))
    _lib.check(st, "stage1")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("q_lens,ctx", [([40, 9], [9000, 30000]), ([300], [12000])])
def test_workspace_absent_runs_the_unsplit_kernel(q_lens, ctx, dev):
    """The C entry point without a workspace runs the whole-row kernel; with one
    it splits the keys.  Both match the oracle."""
    import ctypes

    from unum_ops_amd import _lib

    d = workloads.stage1_inputs(q_lens, ctx, seed=48, raw_keys=False)
    exp = oracle_stage1(d["q"], d["k"], None, d["cu_seqlens_q"], d["cu_seqlens_k"],
                        max_seqlen_k=d["max_seqlen_k"], causal=True)
    q, k = d["q"].to(dev), d["k"].to(dev)
    cu_q, cu_k = d["cu_seqlens_q"].to(dev), d["cu_seqlens_k"].to(dev)
    B = cu_q.numel() - 1
    cols = exp.shape[-1]
    lib = _lib.load()
    ws_bytes = lib.unum_infllmv2_attn_stage1_workspace_size(B, q.shape[0], 32, 2, 128,
                                                            d["max_seqlen_k"])
    assert ws_bytes > 0
    outs = []
    for with_ws in (False, True):
        out = torch.full((2, q.shape[0], cols), float("nan"), device=dev)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if with_ws else None
        st = lib.unum_infllmv2_attn_stage1(
            _lib.ptr(q), q.stride(0), q.stride(1), _lib.ptr(k), k.stride(0), k.stride(1),
            _lib.ptr(cu_q), _lib.ptr(cu_k), _lib.ptr(out), _lib.UNUM_DTYPE_F32,
            B, q.shape[0], k.shape[0], 32, 2, 128, d["max_seqlen_k"], cols,
            ctypes.c_float(128 ** -0.5), 1, _lib.ptr(ws), ws_bytes if with_ws else 0,
            _lib.stream_ptr(dev))
        _lib.check(st, "stage1")
        torch.cuda.synchronize()
        torch.testing.assert_close(out.cpu(), exp, atol=ATOL, rtol=RTOL)
        outs.append(out)
    torch.testing.assert_close(outs[0], outs[1], atol=1e-4, rtol=1e-3)
