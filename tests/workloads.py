"""Seeded synthetic inputs for the benchmark configurations of the selection path
(test and benchmark infrastructure: the GPU tests, `bench.py` and `smoke()` use it;
the product package does not).

All inputs come from ``torch.Generator('cpu').manual_seed(seed)`` and are CPU
tensors; callers move them to the GPU.  The five configurations:

* ``cfg1``: ``get_block_table`` on 4 decode tokens (contexts 1K-8K), top-16,
  ~10 % of ids ``-1``, a 4x256 page table from a permutation of 1024 pages.
* ``cfg2``: ``max_pooling_1d_varlen`` on 4 sequences (q lengths 4K/6K/8K/16K,
  compressed lengths ``(len-32)//16+1``), fp32 rows of softmax-normalised
  N(0,1) logits, flat row stride 1024, 256 output blocks.
* ``cfg3``: ``infllmv2_attn_stage1`` prefill, 4 x 8192 tokens, Hq=32, Hkv=2,
  D=128, keys mean-pooled (kernel 32, stride 16) from N(0,1) raw keys, causal.
* ``cfg4``: the whole selection pipeline on 64 sequences with 1-16 new tokens
  and 16K-64K cached tokens (chunked prefill / decode mix).
* ``cfg5``: the pipeline on one 131072-token context with a 4096-token chunk
  (Hq/Hkv = 32/2 or 16/1).

Page tables are expanded to the reference's token-granular layout:
``block_table[b, p] = page[b, p // 64] * 64 + p % 64``.
"""

import math

import torch

PAGE = 64          # tokens per KV page / sparse block
KC_KERNEL = 32     # key compression kernel
KC_STRIDE = 16     # key compression stride


def _gen(seed):
    return torch.Generator(device="cpu").manual_seed(seed)


def compressed_len(n):
    """Compressed keys of an n-token context: ``(n - 32) // 16 + 1`` (0 if n < 32)."""
    return 0 if n < KC_KERNEL else (n - KC_KERNEL) // KC_STRIDE + 1


def compress_keys(raw):
    """Mean-pool raw keys ``[L, H, D]`` with kernel 32 / stride 16 -> ``[Lk, H, D]`` fp32."""
    L = raw.shape[0]
    lk = compressed_len(L)
    if lk == 0:
        return raw.new_zeros((0,) + tuple(raw.shape[1:]))
    win = raw.float().unfold(0, KC_KERNEL, KC_STRIDE)  # [Lk, H, D, 32]
    return win.mean(dim=-1)[:lk]


def expand_pages(page_table):
    """Token-granular block table ``[B, pages*64]`` from a page table ``[B, pages]``."""
    B, n = page_table.shape
    off = torch.arange(PAGE, dtype=torch.int32)
    return (page_table.to(torch.int32)[:, :, None] * PAGE + off).reshape(B, n * PAGE)


def prefix(lengths):
    out = torch.zeros(len(lengths) + 1, dtype=torch.int32)
    out[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int64), 0).to(torch.int32)
    return out


# --------------------------------------------------------------------- cfg1
def cfg1_block_table(variant="a", seed=0):
    """``get_block_table`` decode case; variants: a) literal ``seqlen_q=[1]``,
    b) ``seqlen_q = ctx`` on the literal 4x256 page table (clamp path),
    c) ``seqlen_q = ctx`` on the token-granular expansion of the page table."""
    g = _gen(seed)
    ctx = torch.tensor([1024, 2048, 4096, 8192], dtype=torch.int32)
    H, T, K = 2, 4, 16
    nblk = torch.tensor([math.ceil(c / PAGE) for c in ctx.tolist()], dtype=torch.float64)
    u = torch.rand(H, T, K, generator=g, dtype=torch.float64)
    topk = torch.floor(u * nblk[None, :, None]).to(torch.int32)
    drop = torch.rand(H, T, K, generator=g) < 0.1
    topk = torch.where(drop, torch.full_like(topk, -1), topk)
    page = torch.randperm(1024, generator=g).to(torch.int32).view(4, 256)
    d = dict(topk_idx=topk, token_to_bs=torch.arange(4, dtype=torch.int32),
             token_pos_in_bs=ctx.clone())
    if variant == "a":
        d.update(block_table=page, seqlen_q=torch.tensor([1], dtype=torch.int32))
    elif variant == "b":
        d.update(block_table=page, seqlen_q=ctx.clone())
    elif variant == "c":
        d.update(block_table=expand_pages(page), seqlen_q=ctx.clone())
    else:
        raise ValueError(variant)
    return d


def reference_test_block_table(batch, seq_len, topk, seed_offset=0):
    """Inputs of the reference's block-table test (``test/test_sparse_kernel.py:66-125``),
    regenerated from its seeds: sorted distinct ids padded with 0 to 96 slots,
    a ``randint(1, 10000)`` token table, ``seqlen_q`` a random multiple of 64
    passed as both ``token_pos_in_bs`` and ``seqlen_q`` (``:177-192``)."""
    head_group, slots = 2, 96
    tmax = seq_len // PAGE
    actual = min(topk, tmax)
    seed = (42 + seed_offset + batch + seq_len + topk) % 1000000
    g = _gen(seed)
    scores = torch.rand((head_group, batch, tmax), generator=g)
    idx = scores.topk(actual, dim=-1, largest=False).indices.sort(dim=-1).values
    topk_idx = torch.zeros((head_group, batch, slots), dtype=torch.int32)
    topk_idx[:, :, :actual] = idx.to(torch.int32)
    g2 = _gen(seed + 10000)
    bt = torch.randint(1, 10000, (batch, seq_len), dtype=torch.int32, generator=g2)
    g3 = _gen(seed + 20000)
    sl = torch.randint(tmax // 4, tmax + 1, (batch,), dtype=torch.int32, generator=g3) * PAGE
    return dict(topk_idx=topk_idx, block_table=bt, token_to_bs=torch.arange(batch, dtype=torch.int32),
                token_pos_in_bs=sl.clone(), seqlen_q=sl, topk=slots)


# --------------------------------------------------------------------- cfg2
def maxpool_inputs(q_lens, F, H=2, seed=0, dtype=torch.float32, k_lens=None, cache=None):
    """Rows of seq b are softmax(N(0,1)) over its ``Lk_b`` compressed columns, 0 elsewhere."""
    g = _gen(seed)
    k_lens = [compressed_len(q) for q in q_lens] if k_lens is None else list(k_lens)
    Tq = sum(q_lens)
    x = torch.zeros(H, Tq, F, dtype=torch.float32)
    r = 0
    for q, lk in zip(q_lens, k_lens):
        if lk > 0:
            logits = torch.randn(H, q, lk, generator=g)
            x[:, r:r + q, :lk] = torch.softmax(logits, dim=-1)
        r += q
    cache = torch.zeros(len(q_lens), dtype=torch.int32) if cache is None else \
        torch.tensor(cache, dtype=torch.int32)
    return dict(input=x.to(dtype), cu_seqlens_q=prefix(q_lens), cu_seqlens_k=prefix(k_lens),
                cache_lens=cache)


def cfg2_maxpool(local_blocks=1, seed=0):
    q_lens = [4096, 6144, 8192, 16384]
    d = maxpool_inputs(q_lens, F=1024, H=2, seed=seed)
    d.update(max_seqlen_q=16384, max_context_len=16384, local_blocks=local_blocks,
             init_blocks=1, block_size=64, stride=16)
    return d


# --------------------------------------------------------------------- cfg3
def stage1_inputs(q_lens, ctx_lens, Hq=32, Hkv=2, D=128, seed=0, peaky=False,
                  raw_keys=True):
    """Queries N(0,1) bf16 ``[sum q, Hq, D]``; keys mean-pooled from N(0,1) raw keys.

    ``raw_keys=False`` draws the 16-token half-block means directly (each
    ~N(0, 1/16)) and averages neighbours -- the same distribution without
    materialising the raw keys (used for the 16K-64K-token contexts)."""
    g = _gen(seed)
    Tq = sum(q_lens)
    q = torch.randn(Tq, Hq, D, generator=g).to(torch.bfloat16)
    ks = []
    for n in ctx_lens:
        lk = compressed_len(n)
        if raw_keys:
            kc = compress_keys(torch.randn(n, Hkv, D, generator=g))
        else:
            half = torch.randn(lk + 1, Hkv, D, generator=g) / 4.0
            kc = 0.5 * (half[:-1] + half[1:])
        if peaky:
            kc = kc * 8.0
        ks.append(kc)
    k = torch.cat(ks, 0).to(torch.bfloat16) if ks else torch.zeros(0, Hkv, D, dtype=torch.bfloat16)
    k_lens = [compressed_len(n) for n in ctx_lens]
    return dict(q=q, k=k, cu_seqlens_q=prefix(q_lens), cu_seqlens_k=prefix(k_lens),
                max_seqlen_q=max(q_lens), max_seqlen_k=max(k_lens), causal=True,
                q_lens=list(q_lens), ctx_lens=list(ctx_lens))


def cfg3_stage1(peaky=False, seed=0, n_seq=4, seqlen=8192):
    return stage1_inputs([seqlen] * n_seq, [seqlen] * n_seq, seed=seed, peaky=peaky)


# --------------------------------------------------------------- cfg4 / cfg5
def pipeline_inputs(q_lens, cache_lens, Hq=32, Hkv=2, D=128, seed=0, pages_per_seq=None,
                    raw_keys=True, page_pool=None):
    """Stage-1 inputs for chunks of ``q_lens`` new tokens after ``cache_lens``
    cached ones, plus the block-table inputs of each token: ``token_to_bs``,
    ``token_pos_in_bs = cache + i + 1`` and ``seqlen_q = ctx``."""
    ctx = [c + q for c, q in zip(cache_lens, q_lens)]
    d = stage1_inputs(q_lens, ctx, Hq=Hq, Hkv=Hkv, D=D, seed=seed, raw_keys=raw_keys)
    g = _gen(seed + 1)
    B = len(q_lens)
    pages = pages_per_seq or max(math.ceil(c / PAGE) for c in ctx)
    pool = page_pool or B * pages
    page = torch.randperm(pool, generator=g)[: B * pages].to(torch.int32).view(B, pages)
    tok_bs, tok_pos = [], []
    for b, (c, q) in enumerate(zip(cache_lens, q_lens)):
        tok_bs += [b] * q
        tok_pos += [c + i + 1 for i in range(q)]
    d.update(page_table=page, block_table=expand_pages(page),
             token_to_bs=torch.tensor(tok_bs, dtype=torch.int32),
             token_pos_in_bs=torch.tensor(tok_pos, dtype=torch.int32),
             seqlen_q=torch.tensor(ctx, dtype=torch.int32), cache_lens_tokens=list(cache_lens),
             max_context_len=max(ctx))
    return d


def cfg4_pipeline(seed=0, n_seq=64):
    g = _gen(seed + 4)
    q_lens = torch.randint(1, 17, (n_seq,), generator=g).tolist()
    cache = torch.randint(16384, 65537, (n_seq,), generator=g).tolist()
    return pipeline_inputs(q_lens, cache, seed=seed, pages_per_seq=1024, page_pool=65536,
                           raw_keys=False)


def cfg5_pipeline(seed=0, Hq=32, Hkv=2):
    return pipeline_inputs([4096], [131072], Hq=Hq, Hkv=Hkv, seed=seed, pages_per_seq=2112)


# ------------------------------------------------------------ roofline math
def stage1_work(cu_q, cu_k, Hq, Hkv, D, out_cols, causal=True, out_bytes=4):
    """Useful FLOP (QK^T over visible keys, once) and compulsory HBM bytes."""
    cq = [int(v) for v in cu_q]
    ck = [int(v) for v in cu_k]
    sum_vis = 0
    for b in range(len(cq) - 1):
        Lq, Lk = cq[b + 1] - cq[b], ck[b + 1] - ck[b]
        if Lk <= 0:
            continue
        for lq in range(Lq):
            if causal:
                a = lq - 15
                a = -((-a) // 16) if a < 0 else a // 16
                c = Lq - 15
                c = -((-c) // 16) if c < 0 else c // 16
                v = min(max(a + Lk - c, 0), Lk)
            else:
                v = Lk
            sum_vis += v
    Tq = cq[-1]
    flop = 2.0 * Hq * D * sum_vis
    nbytes = 2.0 * Tq * Hq * D + 2.0 * ck[-1] * Hkv * D + out_bytes * Hkv * Tq * out_cols
    return flop, nbytes, sum_vis


def maxpool_bytes(cu_q, cu_k, cache, H, NB, elem=4):
    cq = [int(v) for v in cu_q]
    ck = [int(v) for v in cu_k]
    ca = [int(v) for v in cache]
    rd = 0
    for b in range(len(cq) - 1):
        lk = ck[b + 1] - ck[b] + ca[b]
        rd += (cq[b + 1] - cq[b]) * min(lk, 4 * NB + 3)
    return elem * H * rd + elem * H * cq[-1] * NB


def block_table_bytes(topk_idx, token_to_bs, H, T, K, B):
    """Output + ids + one 256-byte table run per distinct valid (b, id) + per-token scalars."""
    idx = topk_idx.reshape(H, T, K)
    bs = token_to_bs.reshape(1, T, 1).expand(H, T, K)
    valid = idx >= 0
    pairs = torch.unique(torch.stack([bs[valid].long(), idx[valid].long()], 0), dim=1)
    U = pairs.shape[1]
    return 4 * T * H * K * 64 + 4 * H * T * K + 256 * U + 4 * (2 * T + B)


def sparse_attn_work(topk_idx, token_to_bs, token_pos_in_bs, seqlen_q, num_seqs, G=16, D=128,
                     out_bytes=2):
    """Stage-2 sparse attention: (algorithmic HBM bytes, useful FLOP, attended entries).

    Bytes: every attended entry's K row and V row gathered once per (token, kv
    head) (``2 * 2 * D`` bytes), the queries read once and the output written
    once.  FLOP: ``2 * G * D`` for the scores plus ``2 * G * D`` for P.V per
    attended entry.  An entry is attended as the block table marks it valid
    (``get_table_torch.py:18-33``)."""
    idx = topk_idx.detach().cpu().to(torch.int64)              # [H, T, K]
    H, T, K = idx.shape
    bs = token_to_bs.detach().cpu().to(torch.int64).reshape(-1)
    pos = token_pos_in_bs.detach().cpu().to(torch.int64).reshape(-1)
    sl = seqlen_q.detach().cpu().to(torch.int64).reshape(-1)
    ok = (bs >= 0) & (bs < num_seqs)
    lim_s = sl.expand(T) if sl.numel() == 1 else sl[bs.clamp(0, num_seqs - 1)]
    lim_p = pos.expand(T) if pos.numel() == 1 else pos
    lim = torch.where(ok, torch.minimum(lim_s, lim_p), torch.zeros_like(lim_s))   # [T]
    p0 = idx * PAGE                                             # [H, T, K]
    # entries p0 + o (o < 64) with 0 <= p < lim
    lo = p0.clamp(min=0)
    hi = torch.minimum(p0 + PAGE, lim[None, :, None])
    n = (hi - lo).clamp(min=0).sum().item()
    nbytes = n * 2 * 2 * D + T * H * G * D * 2 + T * H * G * D * out_bytes
    return float(nbytes), float(n * 4 * G * D), int(n)
