/*
 * unum_ops_amd -- C ABI of the MI355X (gfx950) InfLLM-v2 selection path.
 *
 * Plain C: raw device pointers, element strides and sizes, a HIP stream passed
 * as `void*` (a `hipStream_t`), and an int status.  No torch types cross this
 * boundary.  The library never allocates, frees or synchronises: every
 * launch is asynchronous on `stream`; outputs and workspaces are owned by the
 * caller.  Kernels are compiled for gfx950 only.
 *
 * Status: UNUM_OK (0) on success, a negative UNUM_ERR_* code otherwise; the
 * thread-local message of the last failure is returned by unum_last_error().
 *
 * Devices: the stage-1 entry points plan for the current device (its CU
 * count; the no-allocation entry its scratch array), so their `stream` must
 * belong to the current device -- the null stream is the current device's;
 * a stream of another device returns UNUM_ERR_INVALID_ARGUMENT.
 *
 * Reference interfaces replaced (paths relative to Yanguan619/unum_ops):
 *   unum_infllmv2_attn_stage1  <- infllmv2_attn_stage1 =
 *       src/unum_ops/infllm_v2/infllmv2_attn_stage1_triton_v2.py:153-228
 *       (exported at src/unum_ops/infllm_v2/__init__.py:3-5)
 *   unum_max_pooling_1d_varlen <- max_pooling_1d_varlen =
 *       src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:127-183
 *       (exported at src/unum_ops/infllm_v2/__init__.py:7-9)
 *   unum_get_block_table       <- get_block_table_ref_torch
 *       src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44 and the
 *       exported get_block_table_v2/_v3 (sparse_kernel_extension/__init__.py:7-12
 *       -> get_table_triton.py:218-264)
 */
#ifndef UNUM_OPS_AMD_H_
#define UNUM_OPS_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UNUM_ABI_VERSION 2

enum unum_status {
  UNUM_OK = 0,
  UNUM_ERR_INVALID_ARGUMENT = -1, /* shape / stride / value outside the contract */
  UNUM_ERR_UNSUPPORTED = -2,      /* a combination no kernel implements         */
  UNUM_ERR_WORKSPACE = -3,        /* workspace missing or too small             */
  UNUM_ERR_LAUNCH = -4,           /* the HIP runtime rejected a launch          */
};

enum unum_dtype {
  UNUM_DTYPE_F32 = 0,
  UNUM_DTYPE_BF16 = 1,
  UNUM_DTYPE_F16 = 2,
};

/* Message of the last failing call on this thread ("" if none). */
const char* unum_last_error(void);

/* UNUM_ABI_VERSION of the built library. */
int unum_abi_version(void);

/*
 * Stage-1 block scores (InfLLM-v2), replacing infllmv2_attn_stage1
 * (infllmv2_attn_stage1_triton_v2.py:153-228, kernel :20-150).
 *
 *   q   bf16 [Tq, Hq, D]   element strides (q_stride_t, q_stride_h, 1)
 *   k   bf16 [Tk, Hkv, D]  element strides (k_stride_t, k_stride_h, 1)
 *   cu_seqlens_q / cu_seqlens_k  int32 [B+1] prefix sums
 *   out [Hkv, Tq, out_cols] contiguous, dtype out_dtype (F32 or BF16);
 *       out_cols = round_up(max_seqlen_k, 128) in the reference.
 *
 * For token t of sequence b and kv group g (G = Hq / Hkv heads):
 *   out[g, t, j] = sum_{i<G} softmax_j(scale * q[t, gG+i] . k[cu_k[b]+j, g])
 * over the visible keys j < vis(t) (causal rule of the reference, truncating
 * division), 0 for vis <= j < out_cols, and 0 for the whole row when
 * vis == 0 or the sequence has no keys.  Every element of `out` is written
 * when cu_seqlens_q is non-decreasing within [0, Tq].  The rows of a
 * sequence reaching outside [0, Tq) (malformed cu_seqlens_q) are left
 * unwritten, never indexed.
 *
 * Inputs outside the reference's contract (where it stores past the row or
 * reads outside k):
 *   - a sequence with more keys than out_cols (max_seqlen_k below its real
 *     length): vis is computed from the real key count, then capped at
 *     out_cols; the row is the softmax over the keys it keeps (the dropped
 *     keys are in no denominator), so it still sums to G;
 *   - key ranges of cu_seqlens_k outside [0, Tk): a sequence whose first
 *     key row cu_seqlens_k[b] lies outside [0, Tk) reads none of its keys,
 *     and keys at rows past the end of k are not read; a key not read
 *     scores as a zero key (q . k = 0), on every kernel path.  No load
 *     leaves k.
 * q and k must be finite: the reference maps a NaN score row to 0
 * (infllmv2_attn_stage1_triton_v2.py:227); this library is built without NaN
 * semantics, and the result for an inf or NaN input is not defined.
 *
 * `workspace` (device memory, caller-owned, no initial contents needed) of
 * unum_infllmv2_attn_stage1_workspace_size(...) bytes lets rows over 512 keys
 * split their keys between workgroups (two launches on `stream`: per-split
 * log-sum-exps, then the scores); NULL or a smaller workspace runs the
 * whole-row kernel, with the same results to within fp32 rounding.  Batches
 * of at most two new tokens per sequence over rows of at most 4096 keys run
 * one workgroup per row and leave the workspace unused.  Calls that share
 * one workspace must not overlap.
 */
int unum_infllmv2_attn_stage1(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                              const void* k, int64_t k_stride_t, int64_t k_stride_h,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              void* out, int32_t out_dtype, int64_t B, int64_t Tq,
                              int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
                              int64_t max_seqlen_k, int64_t out_cols, float scale,
                              int32_t causal, void* workspace, int64_t workspace_bytes,
                              void* stream);

/* Workspace bytes unum_infllmv2_attn_stage1 and
 * unum_infllmv2_attn_stage1_maxpool use for this problem on the current
 * device (>= 0; 0: rows of at most 512 keys, never split), with out_cols =
 * round_up(max_seqlen_k, 128).  B is the number of sequences. */
int64_t unum_infllmv2_attn_stage1_workspace_size(int64_t B, int64_t Tq, int64_t Hq,
                                                 int64_t Hkv, int64_t D,
                                                 int64_t max_seqlen_k);

/*
 * unum_infllmv2_attn_stage1 without a caller workspace and without any
 * allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Arguments and results are those
 * of unum_infllmv2_attn_stage1 minus the workspace.
 *
 * The key-split workspace lives in a 4 MiB device array inside the library
 * (one per device, held until the process ends).  Its address on a device is
 * resolved on the first call there (with that device current); make that
 * first call outside graph capture.  A problem whose key split needs more
 * than 4 MiB returns UNUM_ERR_WORKSPACE without launching.  The split plan
 * targets six workgroups per CU: pieces * splits < 6 * CUs + pieces, with
 * fewer than 6 * CUs pieces whenever keys split, and 1 KiB per (piece,
 * split) plus 48 bytes per piece, so the workspace stays below 12.3 KiB per
 * CU -- 3.07 MiB on a 256-CU MI355X (2.97 MiB is the largest problem found
 * there), and the 4 MiB array holds every problem on GPUs of up to 333
 * CUs.  Every
 * call on one device shares that device's array: calls that overlap on one
 * device (other streams, other threads) race and must be serialised by the
 * caller.  Nothing in the array needs clearing: each call writes every
 * element it reads before reading it.
 */
int unum_infllmv2_attn_stage1_noalloc(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                      const void* k, int64_t k_stride_t, int64_t k_stride_h,
                                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      void* out, int32_t out_dtype, int64_t B, int64_t Tq,
                                      int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t max_seqlen_k, int64_t out_cols, float scale,
                                      int32_t causal, void* stream);

/*
 * Stage 1 with the max-pool fused into it.  No single reference function: it
 * equals max_pooling_1d_varlen (max_pooling_1d_varlen.py:127-183; block 64,
 * stride 16, cache_lens 0) applied to infllmv2_attn_stage1's fp32 scores with
 * max_seqlen_q = 16 * out_cols, i.e. each row pooled in place -- the way the
 * selection pipeline chains the two -- without the scores going through HBM.
 *
 *   scores  optional fp32 [Hkv, Tq, out_cols] (NULL: not written)
 *   pooled  fp32 [Hkv, Tq, num_blocks]
 *   workspace / workspace_bytes  as unum_infllmv2_attn_stage1 (size from
 *          unum_infllmv2_attn_stage1_workspace_size): with it, rows over 512
 *          keys run the key-split kernels, pooling in their second pass;
 *          NULL runs whole rows.  Rows of at most 512 keys need none.
 * Other arguments as unum_infllmv2_attn_stage1 and unum_max_pooling_1d_varlen.
 * Fused on the MFMA paths (G = 16, D = 128, 16-byte aligned q/k, scale > 0):
 * rows of at most 512 keys pool in the LDS-resident kernel, longer rows in
 * the key-streaming kernels.  Other shapes return UNUM_ERR_UNSUPPORTED; run
 * unum_infllmv2_attn_stage1 and unum_max_pooling_1d_varlen there.
 */
int unum_infllmv2_attn_stage1_maxpool(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                      const void* k, int64_t k_stride_t, int64_t k_stride_h,
                                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      void* scores, float* pooled, int64_t B, int64_t Tq,
                                      int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
                                      int64_t max_seqlen_k, int64_t out_cols, float scale,
                                      int32_t causal, int64_t num_blocks, int32_t local_blocks,
                                      int32_t init_blocks, void* workspace,
                                      int64_t workspace_bytes, void* stream);

/*
 * Varlen 1-D max-pool of compressed-block scores, replacing
 * max_pooling_1d_varlen (max_pooling_1d_varlen.py:127-183, kernel :33-124).
 *
 *   input  [H, Tq, *] of dtype `dtype` (F32, BF16 or F16), read FLAT:
 *          tap p of row (h, t) is input_flat[(h*Tq + t) * flat_stride + p]
 *          with flat_stride = max_seqlen_q / stride (the reference's
 *          convention); input_numel bounds every read.
 *   cu_seqlens_q / cu_seqlens_k int32 [B+1], cache_lens int32 [B]
 *   out    [H, Tq, num_blocks] contiguous, same dtype as input.
 *
 * Window n covers taps n*P-1 .. n*P+P-1 (P = block_size / stride, padding 1)
 * that fall in [0, Lk), Lk = cu_k[b+1]-cu_k[b]+cache_lens[b]; +inf for
 * n < init_blocks or n <= (t-cu_q[b])/block_size <= n+local_blocks; -inf for an
 * empty window.  A tap whose flat address is >= input_numel is treated as
 * absent (the reference reads out of bounds there).  H <= 65535 and
 * Tq * ceil(num_blocks / 256) < 2^31 (UNUM_ERR_INVALID_ARGUMENT otherwise).
 */
int unum_max_pooling_1d_varlen(const void* input, int64_t input_numel, int32_t dtype,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                               const int32_t* cache_lens, void* out, int64_t H,
                               int64_t Tq, int64_t B, int64_t flat_stride,
                               int64_t num_blocks, int32_t block_size, int32_t stride,
                               int32_t local_blocks, int32_t init_blocks, void* stream);

/*
 * Max-pool fused with the block selection that follows it.  No single
 * reference function: it is max_pooling_1d_varlen (max_pooling_1d_varlen.py:
 * 127-183, fp32 input, block_size / stride == 4) followed by the top-k the
 * reference's tests apply to pooled scores (test/test_sparse_kernel.py:42-43:
 * top-k ids, sorted ascending), with a deterministic tie-break.
 *
 *   topk_idx int32 [H, Tq, topk]: per (h, t), the topk blocks with the largest
 *            pooled scores, equal scores (-0.0 and +0.0 are one score) taken
 *            in ascending block id, listed in ascending id; a selected block
 *            scoring -inf and every slot past num_blocks is -1, and the -1
 *            entries come first.  NaN inputs are outside the contract.
 *   pooled   optional [H, Tq, num_blocks] fp32 (NULL: not written); when given
 *            it must be 16-byte aligned with num_blocks % 4 == 0.
 * Other arguments as unum_max_pooling_1d_varlen.  num_blocks <= 4096,
 * H <= 65535, Tq < 2^31; the input rows must be 16-byte aligned (input
 * aligned, flat_stride % 4 == 0).
 */
int unum_max_pooling_1d_varlen_topk(const void* input, int64_t input_numel,
                                    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                    const int32_t* cache_lens, void* pooled, int32_t* topk_idx,
                                    int64_t H, int64_t Tq, int64_t B, int64_t flat_stride,
                                    int64_t num_blocks, int32_t block_size, int32_t stride,
                                    int32_t local_blocks, int32_t init_blocks, int32_t topk,
                                    void* stream);

/*
 * The block selection of unum_max_pooling_1d_varlen_topk over rows already
 * pooled (e.g. the output of unum_infllmv2_attn_stage1_maxpool).  No single
 * reference function: the top-k the reference's tests apply to pooled scores
 * (test/test_sparse_kernel.py:42-43), with the same deterministic tie-break.
 *
 *   pooled   fp32, `rows` rows of num_blocks scores, row r at r * row_stride
 *   topk_idx int32 [rows, topk] contiguous, as unum_max_pooling_1d_varlen_topk
 *            writes it: the topk largest scores, equal scores (-0.0 and +0.0
 *            are one score) in ascending block id, listed in ascending id; -1
 *            for a selected block scoring -inf and for every slot past
 *            num_blocks, -1 entries first.
 * 1 <= num_blocks <= 32768 (when rows > 0), row_stride >= num_blocks,
 * rows < 2^31 past 4096 blocks (one workgroup per row there) and < 2^33
 * below; NaN scores are outside the contract.
 */
int unum_topk_blocks(const float* pooled, int64_t rows, int64_t row_stride, int64_t num_blocks,
                     int32_t* topk_idx, int32_t topk, void* stream);

/*
 * Top-k block ids -> per-token paged KV slots, replacing
 * get_block_table_ref_torch (get_table_torch.py:4-44) and the exported
 * get_block_table_v2/_v3 (get_table_triton.py:218-264, kernel :6-67).
 *
 *   topk_idx    int32 [H, T, K], element strides (s_h, s_t, s_k)
 *   block_table int32 [B, L], row stride bt_stride_b, unit column stride
 *   token_to_bs int32 [T]
 *   token_pos_in_bs int32 [T] or one element (pos_numel == 1 broadcasts)
 *   seqlen_q    int32 [>= B] indexed by b, or one element (seqlen_numel == 1
 *               broadcasts)
 *   out         int32 [T, H, K*64] contiguous
 *
 *   p = topk_idx[h,t,k]*64 + o (int32, wrapping), b = token_to_bs[t]
 *   out[t,h,64k+o] = (p >= 0 && p < seqlen[b] && p < pos[t])
 *                    ? head_group * block_table[b, min(p, L-1)] + h : 0
 * head_group is 2 in the torch reference (kHeadGroup) and H in the Triton
 * kernels; they agree for H == 2.  A token whose token_to_bs is outside
 * [0, B) gets an all-zero row (the reference raises or reads out of bounds).
 * Every element of `out` is written.
 */
int unum_get_block_table(const int32_t* topk_idx, int64_t topk_stride_h,
                         int64_t topk_stride_t, int64_t topk_stride_k,
                         const int32_t* block_table, int64_t bt_stride_b,
                         const int32_t* token_to_bs, const int32_t* token_pos_in_bs,
                         int64_t pos_numel, const int32_t* seqlen_q, int64_t seqlen_numel,
                         int32_t* out, int64_t H, int64_t T, int64_t K, int64_t B,
                         int64_t L, int32_t head_group, void* stream);

/*
 * Stage-2 sparse attention over the KV slots of the block table.  No
 * portable reference function: the reference's consumer of get_block_table's
 * output is an NPU paged-attention operator (test/test_pa.py:48-71,
 * torch_npu._npu_paged_attention(query, key_cache, value_cache, num_heads,
 * num_kv_heads, scale_value, block_table, context_lens, out); shapes
 * test/test_pa.py:75-80).  This is the attention those slots define.
 *
 *   q            bf16 [T, Hq, D], element strides (q_stride_t, q_stride_h, 1)
 *   key_cache, value_cache  bf16, viewed as n_rows rows of D elements, row r at
 *                element r * kv_row_stride -- a [num_blocks, block_size,
 *                Hkv, D] cache has n_rows = num_blocks*block_size*Hkv, and row
 *                s*Hkv + h holds token slot s, kv head h
 *   topk_idx     int32 [Hkv, T, K] block ids, element strides (h, t, k)
 *   block_table  int32 [B, L] token-granular table, row stride bt_stride_b
 *                (unused when `slots` is given)
 *   slots        optional int32 [T, Hkv, K*64] contiguous: get_block_table's
 *                output for these inputs with head_group = Hkv (NULL: the
 *                slots are computed from block_table)
 *   token_to_bs, token_pos_in_bs (T or 1 entries), seqlen_q (>= B or 1)
 *                as for unum_get_block_table
 *   out          [T, Hq, D] contiguous, out_dtype BF16 or F32
 *
 * For token t and kv head h, entry (t, h, 64k + o) is attended when the block
 * table marks it valid (p = topk_idx[h,t,k]*64 + o, wrapping int32; b =
 * token_to_bs[t] in [0, B); 0 <= p < seqlen_q[b]; p < token_pos_in_bs[t])
 * and its row -- slots[t,h,64k+o], or Hkv*block_table[b, min(p, L-1)] + h
 * (wrapping int32) -- lies in [0, n_rows).  Then
 *   out[t, h*G+i] = sum_j softmax_j(scale * q[t,h*G+i] . K[row_j]) V[row_j]
 * over the attended entries (repeats counted), fp32 math, and 0 when (t, h)
 * has none.  Any finite scale is accepted (zero gives the mean of the
 * attended V rows, a negative one the softmax of the negated products).  G = Hq / Hkv must be 16 and D 128; K <= 64; q, the caches and
 * out 16-byte aligned.
 */
int unum_sparse_paged_attention(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                const void* key_cache, const void* value_cache,
                                int64_t kv_row_stride, int64_t n_rows, const int32_t* topk_idx,
                                int64_t topk_stride_h, int64_t topk_stride_t,
                                int64_t topk_stride_k, const int32_t* block_table,
                                int64_t bt_stride_b, const int32_t* slots,
                                const int32_t* token_to_bs, const int32_t* token_pos_in_bs,
                                int64_t pos_numel, const int32_t* seqlen_q, int64_t seqlen_numel,
                                void* out, int32_t out_dtype, int64_t T, int64_t Hq, int64_t Hkv,
                                int64_t D, int64_t K, int64_t B, int64_t L, float scale,
                                void* stream);

/*
 * Gather-rate calibration for unum_sparse_paged_attention (a measurement
 * tool; no reference counterpart).  Walks the same stages with the same
 * table loads, row checks and K / V gathers, in the same lane pattern and
 * pipeline depth, and does no arithmetic but an XOR of the gathered words:
 * out, u32 [T, Hkv, 64] contiguous, receives each (t, h, lane)'s checksum.
 * Its duration is the floor the gathers alone set for that selection, the
 * roof against which the attention kernel's time is read.  Arguments and
 * validation as unum_sparse_paged_attention.
 */
int unum_sparse_gather_calibrate(const void* key_cache, const void* value_cache,
                                 int64_t kv_row_stride, int64_t n_rows, const int32_t* topk_idx,
                                 int64_t topk_stride_h, int64_t topk_stride_t,
                                 int64_t topk_stride_k, const int32_t* block_table,
                                 int64_t bt_stride_b, const int32_t* slots,
                                 const int32_t* token_to_bs, const int32_t* token_pos_in_bs,
                                 int64_t pos_numel, const int32_t* seqlen_q,
                                 int64_t seqlen_numel, uint32_t* out, int64_t T, int64_t Hkv,
                                 int64_t K, int64_t B, int64_t L, void* stream);

/*
 * Key compression: mean-pool raw keys into the compressed keys stage 1 takes.
 * No reference function: the reference's stage 1 receives compressed keys;
 * the pooling (kernel 32, stride 16) is the one its benchmark configurations
 * describe ("compressed k ... built as mean-pooled blocks of raw keys").
 *
 *   k      bf16 [T_raw, H, D], element strides (k_stride_t, k_stride_h, 1)
 *   cu_seqlens_raw  int32 [B+1]; cu_seqlens_comp int32 [B+1] with
 *          Lk_b = (L_b - kernel_size) / stride + 1 (0 if L_b < kernel_size)
 *   unit_prefix int32 [B+1]: first work unit of each sequence,
 *          units_b = ceil(Lk_b / windows_per_unit); n_units = unit_prefix[B]
 *   out    bf16 [T_comp, H, D] contiguous:
 *          out[cu_comp[b]+j] = bf16_rne(((h_j + h_{j+1}) / kernel_size)),
 *          h_m = sum over the stride tokens stride*m .. stride*m+stride-1 of
 *          the sequence, in fp32 in token order.
 * kernel_size == 2 * stride == 32; D % 8 == 0 and H*D/8 <= 64;
 * windows_per_unit a multiple of the lane groups per wave, 64 / (H*D/w) with
 * w = 4 when H*D/4 <= 64 and w = 8 otherwise (a multiple of 64 / (H*D/8)
 * always is one).
 */
int unum_compress_keys(const void* k, int64_t k_stride_t, int64_t k_stride_h,
                       const int32_t* cu_seqlens_raw, const int32_t* cu_seqlens_comp,
                       const int32_t* unit_prefix, int64_t n_units, void* out, int64_t B,
                       int64_t T_raw, int64_t T_comp, int64_t H, int64_t D, int32_t kernel_size,
                       int32_t stride, int32_t windows_per_unit, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UNUM_OPS_AMD_H_ */
