// max_pooling_1d_varlen: pool compressed-block scores into 64-token blocks.
//
// Reference semantics: the Triton kernel _max_pooling_1d_varlen_kernel and its
// wrapper (src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:33-183).
//
// Work decomposition: one wave owns a 256-output chunk of one row (h, t) and
// walks it in four steps of 64 outputs, one output n per lane.  With the
// reference's block_size 64 / stride 16 (P = 4 taps per step, 5-tap windows,
// padding 1) window n covers taps 4n-1 .. 4n+3: the lane reads taps 4n..4n+3
// as one vector -- a wave's load is one contiguous 1 KiB (fp32) -- and takes
// tap 4n-1 from the lane below (lane 0 from the previous step).  Every input
// element is read from HBM once and every output written once, so the kernel
// is bound by HBM bandwidth.  The row -> sequence lookup is one 64-lane
// vector load of cu_seqlens_q and a ballot, done once per wave.
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
  int64_t n_units;   // (row, chunk) units: H * Tq * n_chunks
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

template <typename T>
struct Vec4;
template <>
struct Vec4<float> {
  static __device__ __forceinline__ f32x4 load(const void* p, int64_t i) {
    return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  }
};
template <>
struct Vec4<__bf16> {
  static __device__ __forceinline__ f32x4 load(const void* p, int64_t i) {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u),
                 __uint_as_float(w.y << 16), __uint_as_float(w.y & 0xffff0000u)};
  }
};
template <>
struct Vec4<_Float16> {
  static __device__ __forceinline__ f32x4 load(const void* p, int64_t i) {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    return f32x4{f16_bits_to_f32(static_cast<uint16_t>(w.x & 0xffffu)),
                 f16_bits_to_f32(static_cast<uint16_t>(w.x >> 16)),
                 f16_bits_to_f32(static_cast<uint16_t>(w.y & 0xffffu)),
                 f16_bits_to_f32(static_cast<uint16_t>(w.y >> 16))};
  }
};

// Fast path: P == 4 (block_size / stride == 4).  A wave processes kUnits
// consecutive (row, 256-output chunk) units; every input load of all units is
// issued before the first one is used, so a wave keeps 16 KiB of reads in
// flight.
constexpr int kUnits = 4;

template <typename T, bool kVec>
__global__ __launch_bounds__(256) void maxpool_p4_kernel(PoolArgs a) {
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  const int64_t u0 = wave * kUnits;
  if (u0 >= a.n_units) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);

  f32x4 v[kUnits][4];
  float carry[kUnits];
  int64_t lk[kUnits], ob[kUnits], out_base[kUnits], nfirst[kUnits];
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    const int64_t u = u0 + i < a.n_units ? u0 + i : a.n_units - 1;  // tail: redo the last unit
    const int64_t row = u / a.n_chunks;  // h*Tq + t
    const int64_t chunk = u - row * a.n_chunks;
    const int64_t t = row % a.Tq;
    const int b = find_sequence(a.cu_q, a.B, t);
    lk[i] = 0;
    ob[i] = 0;
    if (b >= 0) {
      lk[i] = static_cast<int64_t>(a.cu_k[b + 1] - a.cu_k[b]) + a.cache[b];
      ob[i] = (t - a.cu_q[b]) / a.block_size;
    }
    const int64_t base = row * a.F;
    // Taps are present below the key length, inside the input, and below the
    // last tap any output window uses (4*NB - 1).
    int64_t lim = lk[i] < (a.numel - base) ? lk[i] : (a.numel - base);
    lim = lim < 4 * a.NB ? lim : 4 * a.NB;
    nfirst[i] = chunk * 256;
    out_base[i] = row * a.NB;
    const int64_t p_first = 4 * nfirst[i];
    {
      const int64_t p = p_first - 1;
      carry[i] = (p >= 0 && p < lim) ? Elem<T>::load(a.in, base + p) : -INFINITY;
    }
    if (kVec && p_first + 1023 < lim) {  // the whole chunk is present: plain vector loads
#pragma unroll
      for (int st = 0; st < 4; ++st) v[i][st] = Vec4<T>::load(a.in, base + p_first + 256 * st + 4 * lane);
    } else {
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int64_t p0 = p_first + 256 * st + 4 * lane;
        if (kVec && p0 + 3 < lim) {
          v[i][st] = Vec4<T>::load(a.in, base + p0);
        } else {
          v[i][st].x = (p0 + 0 < lim) ? Elem<T>::load(a.in, base + p0 + 0) : -INFINITY;
          v[i][st].y = (p0 + 1 < lim) ? Elem<T>::load(a.in, base + p0 + 1) : -INFINITY;
          v[i][st].z = (p0 + 2 < lim) ? Elem<T>::load(a.in, base + p0 + 2) : -INFINITY;
          v[i][st].w = (p0 + 3 < lim) ? Elem<T>::load(a.in, base + p0 + 3) : -INFINITY;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kUnits; ++i) {
    if (u0 + i >= a.n_units) break;
    float cy = carry[i];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const f32x4 w = v[i][st];
      float prev = __shfl_up(w.w, 1);
      prev = lane == 0 ? cy : prev;
      cy = __shfl(w.w, kWave - 1);
      const float m = fmaxf(fmaxf(fmaxf(prev, w.x), fmaxf(w.y, w.z)), w.w);
      const int64_t n = nfirst[i] + 64 * st + lane;
      const int64_t ws = 4 * n - 1;
      const int64_t w_lo = ws < 0 ? 0 : ws;
      const int64_t w_hi = (ws + 5) < lk[i] ? (ws + 5) : lk[i];
      const bool force = n < a.init_blocks || (ob[i] >= n && ob[i] <= n + a.local_blocks);
      const float r = force ? INFINITY : ((w_hi > w_lo) ? m : -INFINITY);
      if (n < a.NB) Elem<T>::store(a.out, out_base[i] + n, r);
    }
  }
}

// General path: any P >= 1 (window of P+1 taps, padding 1); one output per lane.
template <typename T>
__global__ __launch_bounds__(256) void maxpool_generic_kernel(PoolArgs a) {
  const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
  if (wave >= a.n_units) return;
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
  const int64_t blocks = (a.n_units * kWave + threads - 1) / threads;  // generic: one wave per unit
  if (blocks > INT32_MAX) UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, "max_pooling_1d_varlen: too many rows");
  if (a.P == 4) {
    const int64_t waves = (a.n_units + kUnits - 1) / kUnits;
    const int64_t blocks4 = (waves * kWave + threads - 1) / threads;
    const bool vec = (reinterpret_cast<uintptr_t>(a.in) & 15) == 0 && (a.F % 4) == 0;
    if (vec)
      hipLaunchKernelGGL((maxpool_p4_kernel<T, true>), dim3((unsigned)blocks4), dim3(threads), 0, s, a);
    else
      hipLaunchKernelGGL((maxpool_p4_kernel<T, false>), dim3((unsigned)blocks4), dim3(threads), 0, s, a);
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
  a.n_units = H * Tq * a.n_chunks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case UNUM_DTYPE_F32: return launch_pool<float>(a, s);
    case UNUM_DTYPE_BF16: return launch_pool<__bf16>(a, s);
    case UNUM_DTYPE_F16: return launch_pool<_Float16>(a, s);
    default: UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "max_pooling_1d_varlen: unsupported dtype %d", dtype);
  }
}
