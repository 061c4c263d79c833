// compress_keys: mean-pool raw keys into the compressed keys stage 1 scores
// against (kernel 32, stride 16 in the benchmark configurations).
//
// The reference has no kernel for this step (its stage 1 takes compressed
// keys as input); the definition is the mean of each window of `kernel`
// consecutive tokens of a sequence, windows `stride` apart:
//   Lk_b = (L_b - kernel) / stride + 1   (0 if L_b < kernel)
//   kc[j] = (1/kernel) * sum_{i < kernel} k[16j + i]     (per head, per dim)
// With kernel == 2*stride each window is two half-blocks:
//   h_j   = sum_{i < stride} k[stride*j + i]   (fp32, in token order)
//   kc[j] = bf16_rne((h_j + h_{j+1}) * (1/kernel))
// The summation order is fixed, so the result is reproducible bit for bit
// (kernel a power of two: the scale is exact).
//
// Work decomposition: a wave owns a unit of consecutive windows of one
// sequence; each lane owns one 4- or 8-element slice (8 or 16 bytes) of one
// head, a row of the group's lanes covering all heads and dims of a token,
// and the wave's lane groups split the unit's windows between them.  A lane group
// walks its consecutive windows loading and summing every half-block once
// (16 token loads at once, the next two or three half-blocks' while the
// current one is summed): each raw key is read once.  A workgroup is one
// wave, so the few hundred units of a long sequence spread over every CU
// (four-wave workgroups left half the CUs without one: cfg5's keys 17.3 ->
// 16.4 us with both changes, bit-identical).
#include "common.h"

namespace unum {
namespace {

struct CompressArgs {
  const __bf16* k;
  int64_t k_st, k_sh;
  const int32_t* cu_raw;
  const int32_t* cu_comp;
  const int32_t* unit_prefix;  // [B+1]: first unit of each sequence
  uint16_t* out;               // [T_comp, H, D] bf16 bits
  int64_t B, n_units, T_raw, T_comp;
  int32_t H, D, stride, per_group;  // windows per lane group
  float inv_kernel;
};

__device__ __forceinline__ int find_seq(const int32_t* prefix, int64_t B, int64_t u) {
  const int lane = threadIdx.x & (kWave - 1);
  int count = 0;
  for (int64_t base = 0; base <= B; base += kWave) {
    const int64_t i = base + lane;
    const bool le = (i <= B) && (prefix[i] <= u);
    count += __popcll(__ballot(le));
  }
  return count - 1;
}

typedef int i32x2 __attribute__((ext_vector_type(2)));

// A lane's slice of kSW bf16 elements of one token row (16 or 8 bytes).
template <int kSW>
struct SliceT;
template <>
struct SliceT<8> {
  typedef i32x4 type;
};
template <>
struct SliceT<4> {
  typedef i32x2 type;
};

template <int kSW>
__device__ __forceinline__ void add_slice(float* acc, typename SliceT<kSW>::type w) {
#pragma unroll
  for (int e = 0; e < kSW / 2; ++e) {
    const uint32_t u = static_cast<uint32_t>(w[e]);
    acc[2 * e] += __uint_as_float(u << 16);
    acc[2 * e + 1] += __uint_as_float(u & 0xffff0000u);
  }
}

// Half-block hb of a lane's slice: its kStride token rows, loaded at once.
template <int kStride, int kSW>
__device__ __forceinline__ void half_load(const __bf16* kb, int64_t k_st, int64_t hb,
                                          typename SliceT<kSW>::type (&w)[kStride]) {
#pragma unroll
  for (int i = 0; i < kStride; ++i)
    w[i] = *reinterpret_cast<const typename SliceT<kSW>::type*>(kb + (hb * kStride + i) * k_st);
}

// Their sum, in token order.
template <int kStride, int kSW>
__device__ __forceinline__ void half_sum(const typename SliceT<kSW>::type (&w)[kStride], float* h) {
#pragma unroll
  for (int e = 0; e < kSW; ++e) h[e] = 0.f;
#pragma unroll
  for (int i = 0; i < kStride; ++i) add_slice<kSW>(h, w[i]);
}

// Window j = (half-block j + half-block j+1) / kernel, rounded to bf16.
template <int kSW>
__device__ __forceinline__ void store_window(uint16_t* o, const float* h0, const float* h1, float inv) {
  typename SliceT<kSW>::type v;
#pragma unroll
  for (int e = 0; e < kSW / 2; ++e) {
    const uint32_t lo = f32_to_bf16_bits((h0[2 * e] + h1[2 * e]) * inv);
    const uint32_t hi = f32_to_bf16_bits((h0[2 * e + 1] + h1[2 * e + 1]) * inv);
    v[e] = static_cast<int>(lo | (hi << 16));
  }
  *reinterpret_cast<typename SliceT<kSW>::type*>(o) = v;
}

// Lanes per token row take kSW-element slices: 8 bytes when a row fits in
// the wave that way (twice the waves for the same windows per lane, so twice
// the loads in flight: cfg5's keys measured faster), 16 bytes otherwise.
__host__ __device__ inline int slice_elems(int64_t H, int64_t D) {
  return H * (D / 4) <= kWave ? 4 : 8;
}

// Half-block buffers of a lane group's ring: four for 8-byte slices (three
// half-blocks of 16 loads in flight, within the 63 a wave may have
// outstanding), three for 16-byte slices (register space).
template <int kSW>
constexpr int cmp_ring() { return kSW == 4 ? 4 : 3; }

template <int kStride, int kSW>
__global__ __launch_bounds__(kWave) void compress_keys_kernel(CompressArgs a) {
  const int64_t unit = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (unit >= a.n_units) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int b = find_seq(a.unit_prefix, a.B, unit);
  if (b < 0 || b >= a.B) return;
  const int32_t slices = a.D / kSW;             // slices per head
  const int32_t row_lanes = a.H * slices;       // lanes per token row
  const int32_t groups = kWave / row_lanes;
  const int32_t grp = lane / row_lanes;
  if (grp >= groups) return;                    // lanes past the last full group
  const int32_t h = (lane % row_lanes) / slices;
  const int32_t d0 = kSW * ((lane % row_lanes) % slices);
  const int64_t run = unit - a.unit_prefix[b];
  // Windows of the sequence, clamped to what its raw keys (inside the key
  // tensor) and its output rows (inside the output) allow.
  const int64_t r0 = a.cu_raw[b], c0 = a.cu_comp[b];
  int64_t raw_len = (a.cu_raw[b + 1] < a.T_raw ? a.cu_raw[b + 1] : a.T_raw) - r0;
  int64_t lk = a.cu_comp[b + 1] - c0;
  const int64_t lk_raw = raw_len >= 2 * kStride ? (raw_len - 2 * kStride) / kStride + 1 : 0;
  lk = lk < lk_raw ? lk : lk_raw;
  lk = lk < a.T_comp - c0 ? lk : a.T_comp - c0;
  if (r0 < 0 || c0 < 0) return;
  const int64_t j_lo = (run * groups + grp) * a.per_group;
  int64_t j_hi = j_lo + a.per_group;
  j_hi = j_hi < lk ? j_hi : lk;
  if (j_lo >= j_hi) return;
  const __bf16* kb = a.k + r0 * a.k_st + h * a.k_sh + d0;
  uint16_t* ob = a.out + (c0 * a.H + h) * a.D + d0;
  const int64_t o_st = static_cast<int64_t>(a.H) * a.D;
  // Windows j_lo .. j_hi-1 use half-blocks j_lo .. j_hi, each loaded and
  // summed once, through a ring of kCmpRing register buffers: kCmpRing-1
  // half-blocks load while one is summed.  Past j_hi the ring reloads j_hi,
  // so every step issues the same loads and the compiler's wait before a
  // sum stays a partial one.
  constexpr int kCmpRing = cmp_ring<kSW>();
  typename SliceT<kSW>::type w[kCmpRing][kStride];
  float hp[kSW], hn[kSW];
#pragma unroll
  for (int r = 0; r < kCmpRing - 1; ++r) {
    const int64_t hb = j_lo + r < j_hi ? j_lo + r : j_hi;
    half_load<kStride, kSW>(kb, a.k_st, hb, w[r]);
  }
  for (int64_t base = j_lo;; base += kCmpRing) {
#pragma unroll
    for (int r = 0; r < kCmpRing; ++r) {
      const int64_t hb = base + r;  // the half-block summed at this step
      if (hb > j_hi) return;
      const int64_t nxt = hb + kCmpRing - 1 < j_hi ? hb + kCmpRing - 1 : j_hi;
      half_load<kStride, kSW>(kb, a.k_st, nxt, w[(r + kCmpRing - 1) % kCmpRing]);
      half_sum<kStride, kSW>(w[r], hn);
      if (hb > j_lo) store_window<kSW>(ob + (hb - 1) * o_st, hp, hn, a.inv_kernel);
#pragma unroll
      for (int e = 0; e < kSW; ++e) hp[e] = hn[e];
    }
  }
}

}  // namespace
}  // namespace unum

extern "C" int unum_compress_keys(const void* k, int64_t k_stride_t, int64_t k_stride_h,
                                  const int32_t* cu_seqlens_raw, const int32_t* cu_seqlens_comp,
                                  const int32_t* unit_prefix, int64_t n_units, void* out,
                                  int64_t B, int64_t T_raw, int64_t T_comp, int64_t H, int64_t D,
                                  int32_t kernel_size, int32_t stride, int32_t windows_per_unit,
                                  void* stream) {
  using namespace unum;
  clear_error();
  UNUM_REQUIRE(B >= 0 && T_raw >= 0 && T_comp >= 0 && n_units >= 0 && H > 0 && D > 0,
               "compress_keys: bad sizes (B=%lld T_comp=%lld units=%lld H=%lld D=%lld)",
               (long long)B, (long long)T_comp, (long long)n_units, (long long)H, (long long)D);
  UNUM_REQUIRE(kernel_size == 2 * stride && stride == 16,
               "compress_keys: kernel_size=%d stride=%d (supported: 32 / 16)", kernel_size, stride);
  UNUM_REQUIRE(D % 8 == 0 && H * (D / 8) <= kWave,
               "compress_keys: H*D/8 = %lld must be at most 64 with D %% 8 == 0",
               (long long)(H * (D / 8)));
  UNUM_REQUIRE(windows_per_unit > 0, "compress_keys: windows_per_unit=%d", windows_per_unit);
  if (T_comp == 0 || B == 0 || n_units == 0) return UNUM_OK;
  UNUM_REQUIRE(k && out && cu_seqlens_raw && cu_seqlens_comp && unit_prefix,
               "compress_keys: null pointer");
  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(k) & 15) == 0 && (k_stride_t % 8) == 0 &&
                   (k_stride_h % 8) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "compress_keys: keys and output must be 16-byte aligned (strides %% 8 == 0)");
  const int32_t groups = static_cast<int32_t>(kWave / (H * (D / slice_elems(H, D))));
  UNUM_REQUIRE(windows_per_unit % groups == 0,
               "compress_keys: windows_per_unit=%d not a multiple of the %d lane groups",
               windows_per_unit, groups);
  const int64_t blocks = n_units;
  UNUM_REQUIRE(blocks <= INT32_MAX, "compress_keys: too many units (%lld)", (long long)n_units);
  CompressArgs a;
  a.k = static_cast<const __bf16*>(k);
  a.k_st = k_stride_t;
  a.k_sh = k_stride_h;
  a.cu_raw = cu_seqlens_raw;
  a.cu_comp = cu_seqlens_comp;
  a.unit_prefix = unit_prefix;
  a.out = static_cast<uint16_t*>(out);
  a.B = B;
  a.n_units = n_units;
  a.T_raw = T_raw;
  a.T_comp = T_comp;
  a.H = static_cast<int32_t>(H);
  a.D = static_cast<int32_t>(D);
  a.stride = stride;
  a.per_group = windows_per_unit / groups;
  a.inv_kernel = 1.0f / static_cast<float>(kernel_size);
  if (slice_elems(H, D) == 4)
    hipLaunchKernelGGL((compress_keys_kernel<16, 4>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                       static_cast<hipStream_t>(stream), a);
  else
    hipLaunchKernelGGL((compress_keys_kernel<16, 8>), dim3(static_cast<unsigned>(blocks)), dim3(kWave), 0,
                       static_cast<hipStream_t>(stream), a);
  return check_launch("compress_keys");
}
