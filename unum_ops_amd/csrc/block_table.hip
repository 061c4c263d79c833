// get_block_table: top-k block ids -> per-token paged KV slots (gfx950).
//
// Reference semantics: get_block_table_ref_torch
// (src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44); the exported
// Triton kernel (get_table_triton.py:6-67) computes the same gather.
//
// Work decomposition: one wave owns 16 ids of one (token, head) row of the
// output -- 16 runs of 64 entries.  The per-token scalars (sequence, position
// limit, sequence length) are read once per wave; the ids are read one per
// lane and broadcast with a lane shuffle; each store step writes four whole
// runs (1 KiB, one dwordx4 per lane).  The block-table gather for those
// entries is one dwordx4 load when the four positions are in range and
// 16-byte aligned, all four steps' loads issued before the first store.  The
// kernel is bound by the output write; its stores are non-temporal (nothing
// here re-reads the output).
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
};

__device__ __forceinline__ int32_t wrap_add_i32(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}
__device__ __forceinline__ int32_t wrap_mul_i32(int32_t a, int32_t b) {
  return static_cast<int32_t>(static_cast<uint32_t>(a) * static_cast<uint32_t>(b));
}

// Finish four entries of a run from the dwordx4 `raw` loaded at the clamped
// address `safe`: entries whose position the vector covered take it, the
// others (positions outside [0, L-4], the clamp to L-1) read the table one by
// one.  Invalid entries are 0.
__device__ __forceinline__ i32x4 finish4(const BlockTableArgs& a, const int32_t* row, i32x4 raw,
                                         bool raw_ok, int32_t p0, int32_t limit_len,
                                         int32_t limit_pos, int32_t h) {
  int32_t p[4];
  bool valid[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    p[e] = wrap_add_i32(p0, e);
    valid[e] = p[e] >= 0 && p[e] < limit_len && p[e] < limit_pos;
  }
  int32_t v[4] = {raw.x, raw.y, raw.z, raw.w};
  if (!raw_ok) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int32_t c = p[e] < 0 ? 0 : (p[e] > a.L - 1 ? a.L - 1 : p[e]);
      v[e] = valid[e] ? row[c] : 0;
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
    v[e] = valid[e] ? wrap_add_i32(wrap_mul_i32(a.head_group, v[e]), h) : 0;
  return i32x4{v[0], v[1], v[2], v[3]};
}

// One wave per unit of 16 ids of a (token, head) row: four store steps of
// four runs.  Units this small give the grid enough waves that the last
// round of waves is short (whole-row waves left a long tail).
constexpr int kIdsPerUnit = 16;

template <bool kVecTable>
__global__ __launch_bounds__(256) void block_table_kernel(BlockTableArgs a, int64_t n_units,
                                                          int32_t units_per_row) {
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (unit >= n_units) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t th = unit / units_per_row;  // t*H + h
  const int32_t kb = kIdsPerUnit * static_cast<int32_t>(unit - th * units_per_row);
  const int32_t t = static_cast<int32_t>(th / a.H);
  const int32_t h = static_cast<int32_t>(th - static_cast<int64_t>(t) * a.H);
  i32x4* out = reinterpret_cast<i32x4*>(a.out + th * a.K * kSparseBlock);
  const int32_t sub = lane >> 4;       // run within a store step
  const int32_t o0 = (lane & 15) * 4;  // first entry of the lane in its run
  const int32_t b = a.token_to_bs[t];
  if (b < 0 || b >= a.B) {
#pragma unroll
    for (int st = 0; st < kIdsPerUnit / 4; ++st) {
      const int32_t k = kb + 4 * st + sub;
      if (k < a.K) __builtin_nontemporal_store(i32x4{0, 0, 0, 0}, out + static_cast<int64_t>(k) * 16 + (lane & 15));
    }
    return;
  }
  const int32_t limit_pos = a.pos[a.pos_scalar ? 0 : t];
  const int32_t limit_len = a.seqlen[a.seqlen_scalar ? 0 : b];
  const int32_t* row = a.bt + static_cast<int64_t>(b) * a.bt_stride;
  const int32_t* ids = a.topk + static_cast<int64_t>(h) * a.s_h + static_cast<int64_t>(t) * a.s_t;
  const int32_t vec_hi = a.L - 4;  // a dwordx4 at p0 (a multiple of 4) covers p0..p0+3 <= L-1
  const int32_t my = (lane < kIdsPerUnit && kb + lane < a.K) ? ids[static_cast<int64_t>(kb + lane) * a.s_k] : -1;
  // All table loads of the unit go out before the first is used.
  int32_t p0[kIdsPerUnit / 4];
  i32x4 raw[kIdsPerUnit / 4];
#pragma unroll
  for (int st = 0; st < kIdsPerUnit / 4; ++st) {
    const int32_t idx = __shfl(my, 4 * st + sub);
    p0[st] = wrap_add_i32(wrap_mul_i32(idx, kSparseBlock), o0);
    if (kVecTable) {
      const int32_t safe = (p0[st] >= 0 && p0[st] <= vec_hi) ? p0[st] : 0;
      raw[st] = *reinterpret_cast<const i32x4*>(row + safe);
    } else {
      raw[st] = i32x4{0, 0, 0, 0};
    }
  }
#pragma unroll
  for (int st = 0; st < kIdsPerUnit / 4; ++st) {
    const int32_t k = kb + 4 * st + sub;
    const bool raw_ok = kVecTable && p0[st] >= 0 && p0[st] <= vec_hi;
    if (k < a.K)
      __builtin_nontemporal_store(finish4(a, row, raw[st], raw_ok, p0[st], limit_len, limit_pos, h),
                                  out + static_cast<int64_t>(k) * 16 + (lane & 15));
  }
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

  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "get_block_table: output must be 16-byte aligned");
  const bool vec = (reinterpret_cast<uintptr_t>(block_table) & 15) == 0 && (bt_stride_b % 4) == 0 &&
                   L >= 4;
  const int threads = 256;  // four units per block
  const int32_t units_per_row = (int32_t)((K + kIdsPerUnit - 1) / kIdsPerUnit);
  const int64_t n_units = T * H * units_per_row;
  const int64_t blocks = (n_units + 3) / 4;
  UNUM_REQUIRE(blocks <= INT32_MAX, "get_block_table: T*H=%lld too large", (long long)(T * H));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(block_table_kernel<true>, dim3((unsigned)blocks), dim3(threads), 0, s, a,
                       n_units, units_per_row);
  else
    hipLaunchKernelGGL(block_table_kernel<false>, dim3((unsigned)blocks), dim3(threads), 0, s, a,
                       n_units, units_per_row);
  return check_launch("get_block_table");
}
