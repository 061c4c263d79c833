// max_pooling_1d_varlen: pool compressed-block scores into 64-token blocks.
//
// Reference semantics: the Triton kernel _max_pooling_1d_varlen_kernel and its
// wrapper (src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:33-183).
//
// Work decomposition: one wave owns a 256-output chunk of one row (h, t);
// lane i owns outputs n0..n0+3 with n0 = 256*chunk + 4i.  With the reference's
// block_size 64 / stride 16 (P = 4 taps per step, 5-tap windows, padding 1)
// those four windows cover taps 4*n0-1 .. 4*n0+15: sixteen consecutive input
// elements that the lane reads as 16-byte vectors, plus the one tap before
// them.  A wave therefore streams one contiguous 1024-element stretch of the
// row in and one 256-element stretch of the output out, with every input
// element read from HBM once -- the kernel is bound by HBM bandwidth.  The
// row -> sequence lookup is one 64-lane vector load of cu_seqlens_q and a
// ballot, done once per wave.
#include "common.h"

namespace unum {
namespace {

struct PoolArgs {
  const void* in;
  int64_t numel;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* cache;
  void* out;
  int64_t H, Tq, B, F, NB;
  int32_t block_size, P, local_blocks, init_blocks;
  int64_t n_chunks;  // chunks of 256 outputs per row
  int64_t n_waves;   // H * Tq * n_chunks
};

template <typename T>
struct Elem;
template <>
struct Elem<float> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    static_cast<float*>(p)[i] = v;
  }
};
template <>
struct Elem<__bf16> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);  // exact: v is an input value or +-inf
  }
};
template <>
struct Elem<_Float16> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v);
  }
};

// Find the sequence of token t: b with cu_q[b] <= t < cu_q[b+1], or -1.
// cu_q is non-decreasing, so b+1 = #{i <= B : cu_q[i] <= t}; each lane tests
// up to ceil((B+1)/64) entries and a ballot counts them.
__device__ __forceinline__ int find_sequence(const int32_t* cu_q, int64_t B, int64_t t) {
  const int lane = threadIdx.x & (kWave - 1);
  int count = 0;
  for (int64_t base = 0; base <= B; base += kWave) {
    const int64_t i = base + lane;
    const bool le = (i <= B) && (cu_q[i] <= t);
    count += __popcll(__ballot(le));
  }
  const int b = count - 1;
  if (b < 0 || b >= B) return -1;
  return (t < cu_q[b + 1]) ? b : -1;
}

// Fast path: P == 4 (block_size / stride), vector loads and stores allowed.
template <typename T, bool kVec>
__global__ __launch_bounds__(256) void maxpool_p4_kernel(PoolArgs a) {
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (wave >= a.n_waves) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = wave / a.n_chunks;  // h*Tq + t
  const int64_t chunk = wave - row * a.n_chunks;
  const int64_t t = row % a.Tq;

  const int b = find_sequence(a.cu_q, a.B, t);
  int64_t lk = 0, ob = 0;
  if (b >= 0) {
    lk = static_cast<int64_t>(a.cu_k[b + 1] - a.cu_k[b]) + a.cache[b];
    ob = (t - a.cu_q[b]) / a.block_size;
  }
  const int64_t base = row * a.F;
  // Taps beyond either the key length or the end of the input are absent.
  const int64_t lim = lk < (a.numel - base) ? lk : (a.numel - base);

  const int64_t n0 = chunk * 256 + 4 * lane;
  if (n0 >= a.NB) return;
  const int64_t p0 = 4 * n0;  // first of the 16 taps owned by this lane

  float v[17];  // v[0] = tap p0-1, v[1+j] = tap p0+j
  if (kVec && p0 + 15 < lim) {
    const T* src = static_cast<const T*>(a.in) + base + p0;
    if constexpr (sizeof(T) == 4) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 w = reinterpret_cast<const f32x4*>(src)[q];
        v[1 + 4 * q] = w.x; v[2 + 4 * q] = w.y; v[3 + 4 * q] = w.z; v[4 + 4 * q] = w.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const i32x4 w = reinterpret_cast<const i32x4*>(src)[q];
        const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t lo = static_cast<uint16_t>(u[e] & 0xffffu);
          const uint16_t hi = static_cast<uint16_t>(u[e] >> 16);
          if constexpr (sizeof(T) == 2 && __is_same(T, __bf16)) {
            v[1 + 8 * q + 2 * e] = bf16_bits_to_f32(lo);
            v[2 + 8 * q + 2 * e] = bf16_bits_to_f32(hi);
          } else {
            v[1 + 8 * q + 2 * e] = f16_bits_to_f32(lo);
            v[2 + 8 * q + 2 * e] = f16_bits_to_f32(hi);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int64_t p = p0 + j;
      v[1 + j] = (p < lim) ? Elem<T>::load(a.in, base + p) : -INFINITY;
    }
  }
  {
    const int64_t p = p0 - 1;
    v[0] = (p >= 0 && p < lim) ? Elem<T>::load(a.in, base + p) : -INFINITY;
  }

  float r[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t n = n0 + e;
    float m = v[4 * e];
#pragma unroll
    for (int j = 1; j < 5; ++j) m = fmaxf(m, v[4 * e + j]);
    const int64_t ws = 4 * n - 1;
    const int64_t w_lo = ws < 0 ? 0 : ws;
    const int64_t w_hi = (ws + 5) < lk ? (ws + 5) : lk;
    const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
    r[e] = force ? INFINITY : ((w_hi > w_lo) ? m : -INFINITY);
  }

  const int64_t o = row * a.NB + n0;
  if (kVec && n0 + 3 < a.NB) {
    if constexpr (sizeof(T) == 4) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + o) = f32x4{r[0], r[1], r[2], r[3]};
    } else {
      uint16_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float tmp = r[e];
        uint16_t bits;
        if constexpr (__is_same(T, __bf16)) bits = f32_to_bf16_bits(tmp);
        else bits = f32_to_f16_bits(tmp);
        h[e] = bits;
      }
      uint2 pk;
      pk.x = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
      pk.y = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + o) = pk;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n0 + e < a.NB) Elem<T>::store(a.out, o + e, r[e]);
  }
}

// General path: any P >= 1 (window of P+1 taps, padding 1); one output per lane.
template <typename T>
__global__ __launch_bounds__(256) void maxpool_generic_kernel(PoolArgs a) {
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (wave >= a.n_waves) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = wave / a.n_chunks;
  const int64_t chunk = wave - row * a.n_chunks;
  const int64_t t = row % a.Tq;
  const int b = find_sequence(a.cu_q, a.B, t);
  int64_t lk = 0, ob = 0;
  if (b >= 0) {
    lk = static_cast<int64_t>(a.cu_k[b + 1] - a.cu_k[b]) + a.cache[b];
    ob = (t - a.cu_q[b]) / a.block_size;
  }
  const int64_t base = row * a.F;
  const int64_t lim = lk < (a.numel - base) ? lk : (a.numel - base);
  const int P = a.P;
  for (int e = 0; e < 4; ++e) {
    const int64_t n = chunk * 256 + 4 * lane + e;
    if (n >= a.NB) break;
    const int64_t ws = n * P - 1;
    float m = -INFINITY;
    for (int j = 0; j <= P; ++j) {
      const int64_t p = ws + j;
      if (p >= 0 && p < lim) m = fmaxf(m, Elem<T>::load(a.in, base + p));
    }
    const int64_t w_lo = ws < 0 ? 0 : ws;
    const int64_t w_hi = (ws + P + 1) < lk ? (ws + P + 1) : lk;
    const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
    Elem<T>::store(a.out, row * a.NB + n, force ? INFINITY : ((w_hi > w_lo) ? m : -INFINITY));
  }
}

template <typename T>
int launch_pool(const PoolArgs& a, hipStream_t s) {
  const int threads = 256;
  const int64_t blocks = (a.n_waves * kWave + threads - 1) / threads;
  if (blocks > INT32_MAX) UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, "max_pooling_1d_varlen: too many rows");
  if (a.P == 4) {
    const bool vec = (reinterpret_cast<uintptr_t>(a.in) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                     ((a.F * (int64_t)sizeof(T)) % 16) == 0 && (a.NB % 4) == 0;
    if (vec)
      hipLaunchKernelGGL((maxpool_p4_kernel<T, true>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
    else
      hipLaunchKernelGGL((maxpool_p4_kernel<T, false>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
  } else {
    hipLaunchKernelGGL((maxpool_generic_kernel<T>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
  }
  return check_launch("max_pooling_1d_varlen");
}

}  // namespace
}  // namespace unum

extern "C" int unum_max_pooling_1d_varlen(const void* input, int64_t input_numel,
                                          int32_t dtype, const int32_t* cu_seqlens_q,
                                          const int32_t* cu_seqlens_k,
                                          const int32_t* cache_lens, void* out, int64_t H,
                                          int64_t Tq, int64_t B, int64_t flat_stride,
                                          int64_t num_blocks, int32_t block_size,
                                          int32_t stride, int32_t local_blocks,
                                          int32_t init_blocks, void* stream) {
  using namespace unum;
  clear_error();
  UNUM_REQUIRE(H >= 0 && Tq >= 0 && B >= 0 && num_blocks >= 0 && flat_stride >= 0,
               "max_pooling_1d_varlen: negative size");
  UNUM_REQUIRE(block_size > 0 && stride > 0, "max_pooling_1d_varlen: block_size=%d stride=%d",
               block_size, stride);
  const int P = block_size / stride;
  UNUM_REQUIRE(P >= 1, "max_pooling_1d_varlen: block_size (%d) < stride (%d)", block_size,
               stride);
  if (H == 0 || Tq == 0 || num_blocks == 0) return UNUM_OK;
  UNUM_REQUIRE(input && out && cu_seqlens_q && cu_seqlens_k && cache_lens,
               "max_pooling_1d_varlen: null pointer");
  UNUM_REQUIRE(B >= 1, "max_pooling_1d_varlen: cu_seqlens must hold at least 2 entries");
  UNUM_REQUIRE(H * Tq * flat_stride <= input_numel,
               "max_pooling_1d_varlen: flat row stride %lld (max_seqlen_q // stride) times "
               "H*Tq=%lld rows exceeds the input's %lld elements",
               (long long)flat_stride, (long long)(H * Tq), (long long)input_numel);
  PoolArgs a;
  a.in = input;
  a.numel = input_numel;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.cache = cache_lens;
  a.out = out;
  a.H = H;
  a.Tq = Tq;
  a.B = B;
  a.F = flat_stride;
  a.NB = num_blocks;
  a.block_size = block_size;
  a.P = P;
  a.local_blocks = local_blocks;
  a.init_blocks = init_blocks;
  a.n_chunks = (num_blocks + 255) / 256;
  a.n_waves = H * Tq * a.n_chunks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case UNUM_DTYPE_F32: return launch_pool<float>(a, s);
    case UNUM_DTYPE_BF16: return launch_pool<__bf16>(a, s);
    case UNUM_DTYPE_F16: return launch_pool<_Float16>(a, s);
    default: UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "max_pooling_1d_varlen: unsupported dtype %d", dtype);
  }
}
