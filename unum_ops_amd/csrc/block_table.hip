// get_block_table: top-k block ids -> per-token paged KV slots (gfx950).
//
// Reference semantics: get_block_table_ref_torch
// (src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44); the exported
// Triton kernel (get_table_triton.py:6-67) computes the same gather.
//
// Work decomposition: the output [T, H, K*64] int32 is a flat array of
// "items" (t, h, k), each a 64-entry run.  One thread owns four consecutive
// entries of one item, so a 64-lane wave writes four whole items (1 KiB) with
// one dwordx4 store per lane; the block-table gather for those entries is one
// dwordx4 load when the four positions are valid, in range and 16-byte
// aligned.  The kernel is bound by the output write (see the roofline note in
// the launcher).
#include "common.h"

namespace unum {
namespace {

constexpr int kSparseBlock = 64;  // kSparseBlockSize, get_table_torch.py:13

struct BlockTableArgs {
  const int32_t* topk;
  int64_t s_h, s_t, s_k;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t* token_to_bs;
  const int32_t* pos;
  const int32_t* seqlen;
  int32_t* out;
  int32_t H, T, K, B, L;
  int32_t pos_scalar, seqlen_scalar;
  int32_t head_group;
  int64_t n_quads;  // T*H*K*16
};

__device__ __forceinline__ int32_t wrap_add_i32(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}
__device__ __forceinline__ int32_t wrap_mul_i32(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) * static_cast<uint32_t>(b));
}

template <bool kVecTable>
__global__ __launch_bounds__(256) void block_table_kernel(BlockTableArgs a) {
  const int64_t quad = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (quad >= a.n_quads) return;
  const int32_t item = static_cast<int32_t>(quad >> 4);  // (t*H + h)*K + k
  const int32_t o0 = static_cast<int32_t>(quad & 15) * 4;
  const int32_t k = item % a.K;
  const int32_t th = item / a.K;
  const int32_t h = th % a.H;
  const int32_t t = th / a.H;

  i32x4 res = {0, 0, 0, 0};
  const int32_t b = a.token_to_bs[t];
  if (b >= 0 && b < a.B) {
    const int32_t idx = a.topk[h * a.s_h + t * a.s_t + k * a.s_k];
    const int32_t limit_pos = a.pos[a.pos_scalar ? 0 : t];
    const int32_t limit_len = a.seqlen[a.seqlen_scalar ? 0 : b];
    const int32_t p0 = wrap_add_i32(wrap_mul_i32(idx, kSparseBlock), o0);
    const int32_t* row = a.bt + static_cast<int64_t>(b) * a.bt_stride;
    int32_t p[4];
    bool valid[4];
    bool all_fast = true;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[e] = wrap_add_i32(p0, e);
      valid[e] = p[e] >= 0 && p[e] < limit_len && p[e] < limit_pos;
      all_fast = all_fast && valid[e] && p[e] < a.L;
    }
    int32_t v[4];
    if (kVecTable && all_fast) {  // all four valid and < L: p0..p0+3 consecutive
      const i32x4 w = *reinterpret_cast<const i32x4*>(row + p0);
      v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t c = p[e] < 0 ? 0 : (p[e] > a.L - 1 ? a.L - 1 : p[e]);
        v[e] = valid[e] ? row[c] : 0;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = valid[e] ? wrap_add_i32(wrap_mul_i32(a.head_group, v[e]), h) : 0;
    res = i32x4{v[0], v[1], v[2], v[3]};
  }
  *reinterpret_cast<i32x4*>(a.out + static_cast<int64_t>(item) * kSparseBlock + o0) = res;
}

}  // namespace
}  // namespace unum

extern "C" int unum_get_block_table(const int32_t* topk_idx, int64_t topk_stride_h,
                                    int64_t topk_stride_t, int64_t topk_stride_k,
                                    const int32_t* block_table, int64_t bt_stride_b,
                                    const int32_t* token_to_bs,
                                    const int32_t* token_pos_in_bs, int64_t pos_numel,
                                    const int32_t* seqlen_q, int64_t seqlen_numel,
                                    int32_t* out, int64_t H, int64_t T, int64_t K,
                                    int64_t B, int64_t L, int32_t head_group,
                                    void* stream) {
  using namespace unum;
  clear_error();
  UNUM_REQUIRE(H >= 0 && T >= 0 && K >= 0 && B >= 0 && L >= 0,
               "get_block_table: negative size (H=%lld T=%lld K=%lld B=%lld L=%lld)",
               (long long)H, (long long)T, (long long)K, (long long)B, (long long)L);
  const int64_t n_items = H * T * K;
  if (n_items == 0) return UNUM_OK;
  UNUM_REQUIRE(n_items <= (int64_t(1) << 31) / 64,
               "get_block_table: H*T*K=%lld too large", (long long)n_items);
  UNUM_REQUIRE(B > 0 && L > 0, "get_block_table: empty block_table [%lld, %lld]",
               (long long)B, (long long)L);
  UNUM_REQUIRE(pos_numel == 1 || pos_numel == T,
               "get_block_table: token_pos_in_bs has %lld elements, expected 1 or T=%lld",
               (long long)pos_numel, (long long)T);
  UNUM_REQUIRE(seqlen_numel == 1 || seqlen_numel >= B,
               "get_block_table: seqlen_q has %lld elements, expected 1 or >= B=%lld",
               (long long)seqlen_numel, (long long)B);
  UNUM_REQUIRE(topk_idx && block_table && token_to_bs && token_pos_in_bs && seqlen_q && out,
               "get_block_table: null pointer");
  UNUM_REQUIRE(L <= INT32_MAX && T <= INT32_MAX && B <= INT32_MAX,
               "get_block_table: size exceeds int32");

  BlockTableArgs a;
  a.topk = topk_idx;
  a.s_h = topk_stride_h;
  a.s_t = topk_stride_t;
  a.s_k = topk_stride_k;
  a.bt = block_table;
  a.bt_stride = bt_stride_b;
  a.token_to_bs = token_to_bs;
  a.pos = token_pos_in_bs;
  a.seqlen = seqlen_q;
  a.out = out;
  a.H = (int32_t)H;
  a.T = (int32_t)T;
  a.K = (int32_t)K;
  a.B = (int32_t)B;
  a.L = (int32_t)L;
  a.pos_scalar = pos_numel == 1;
  a.seqlen_scalar = seqlen_numel == 1;
  a.head_group = head_group;
  a.n_quads = n_items * 16;

  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "get_block_table: output must be 16-byte aligned");
  const bool vec = (reinterpret_cast<uintptr_t>(block_table) & 15) == 0 && (bt_stride_b % 4) == 0;
  const int threads = 256;
  const int64_t blocks = (a.n_quads + threads - 1) / threads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(block_table_kernel<true>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  else
    hipLaunchKernelGGL(block_table_kernel<false>, dim3((unsigned)blocks), dim3(threads), 0, s, a);
  return check_launch("get_block_table");
}
