// max_pooling_1d_varlen: pool compressed-block scores into 64-token blocks.
//
// Reference semantics: the Triton kernel _max_pooling_1d_varlen_kernel and its
// wrapper (src/unum_ops/infllm_v2/max_pooling_1d_varlen.py:33-183).
//
// Work decomposition: one wave owns one (row, 256-output chunk) unit; lane i
// owns four consecutive outputs n0..n0+3 (n0 = 256*chunk + 4i).  With the
// reference's block_size 64 / stride 16 (P = 4 taps per step, 5-tap windows,
// padding 1) their windows cover taps 4*n0-1 .. 4*n0+15: the lane reads the
// sixteen taps 4*n0 .. 4*n0+15 as 16-byte vectors, takes tap 4*n0-1 from the
// lane below (lane 0 reads it), and writes its four outputs with one 16-byte
// store.  Every input element is read from HBM once and every output written
// once, so the kernel is bound by HBM bandwidth; waves are kept light (about
// 32 VGPRs) so many are resident, which measured faster than fewer waves
// with deeper per-wave batches.  The row -> sequence lookup is one 64-lane
// vector load of cu_seqlens_q and a ballot.
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

// Fast path: P == 4 (block_size / stride == 4).
template <typename T>
struct Vec16;  // sixteen consecutive taps as fp32
template <>
struct Vec16<float> {
  static __device__ __forceinline__ void load(const void* p, int64_t i, float* v) {
    const f32x4* q = reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 w = q[k];
      v[4 * k] = w.x; v[4 * k + 1] = w.y; v[4 * k + 2] = w.z; v[4 * k + 3] = w.w;
    }
  }
};
template <typename H, bool kBf16>
struct Vec16Half {
  static __device__ __forceinline__ void load(const void* p, int64_t i, float* v) {
    const i32x4* q = reinterpret_cast<const i32x4*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const i32x4 w = q[k];
      const uint32_t u[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (kBf16) {
          v[8 * k + 2 * e] = __uint_as_float(u[e] << 16);
          v[8 * k + 2 * e + 1] = __uint_as_float(u[e] & 0xffff0000u);
        } else {
          v[8 * k + 2 * e] = f16_bits_to_f32(static_cast<uint16_t>(u[e] & 0xffffu));
          v[8 * k + 2 * e + 1] = f16_bits_to_f32(static_cast<uint16_t>(u[e] >> 16));
        }
      }
    }
  }
};
template <>
struct Vec16<__bf16> : Vec16Half<__bf16, true> {};
template <>
struct Vec16<_Float16> : Vec16Half<_Float16, false> {};

// Output stores are non-temporal: the pooled rows are not re-read by this
// kernel, and keeping them out of the cache measured 8-16% faster (plain
// stores evict input lines that neighbouring waves still read).
template <typename T>
__device__ __forceinline__ void store4(void* out, int64_t o, const float* r) {
  if constexpr (sizeof(T) == 4) {
    __builtin_nontemporal_store(f32x4{r[0], r[1], r[2], r[3]},
                                reinterpret_cast<f32x4*>(static_cast<float*>(out) + o));
  } else {
    uint16_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (__is_same(T, __bf16)) h[e] = f32_to_bf16_bits(r[e]);
      else h[e] = f32_to_f16_bits(r[e]);
    }
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 pk = {(uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16)};
    __builtin_nontemporal_store(pk, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(out) + o));
  }
}

// Row context of the P == 4 path: key length, block of the token, flat row
// start and the tap limit.
struct RowCtx {
  int64_t lk, ob, base, lim;
};

// Taps are present below the key length, inside the input, and below the
// last tap any output window uses (4*NB - 1).
__device__ __forceinline__ void set_tap_limit(const PoolArgs& a, RowCtx& c) {
  const int64_t lim = c.lk < (a.numel - c.base) ? c.lk : (a.numel - c.base);
  c.lim = lim < 4 * a.NB ? lim : 4 * a.NB;
}

__device__ __forceinline__ RowCtx row_ctx(const PoolArgs& a, int64_t row, int64_t t) {
  const int b = find_sequence(a.cu_q, a.B, t);
  RowCtx c{0, 0, row * a.F, 0};
  if (b >= 0) {
    c.lk = static_cast<int64_t>(a.cu_k[b + 1] - a.cu_k[b]) + a.cache[b];
    // 0 <= t - cu_q[b] < 2^31: a 32-bit division (a 64-bit one is a long
    // emulated sequence)
    c.ob = static_cast<uint32_t>(t - a.cu_q[b]) / static_cast<uint32_t>(a.block_size);
  }
  set_tap_limit(a, c);
  return c;
}

// The taps of one lane: v = taps 4*n0 .. 4*n0+15, and below = tap 4*n0-1
// (loaded by lane 0 only; the other lanes take it from the lane below).
struct Taps {
  float v[16];
  float below;
};

// Issue the loads of a lane's taps for outputs n0..n0+3 (n0 = 256*chunk + 4*lane).
template <typename T, bool kVec>
__device__ __forceinline__ void load_taps(const PoolArgs& a, const RowCtx& c, int64_t chunk, Taps& tp) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t n0 = chunk * 256 + 4 * lane;
  const int64_t p0 = 4 * n0;
  float* v = tp.v;
  // Taps of this lane below the limit.  A lane straddling it still loads
  // whole vectors when they lie inside the input (pool_taps masks the taps
  // past the limit, so nothing here waits for the loads): only at the
  // input's very end does a lane load tap by tap.
  const int64_t avail = c.lim - p0;
  const bool in_alloc = c.base + p0 + 15 < a.numel;
  if (kVec && avail > 0 && (avail >= 16 || in_alloc)) {
    Vec16<T>::load(a.in, c.base + p0, v);
  } else if (avail > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      v[j] = (p0 + j < c.lim) ? Elem<T>::load(a.in, c.base + p0 + j) : -INFINITY;
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = -INFINITY;
  }
  tp.below = -INFINITY;
  if (lane == 0) {
    const int64_t pe = p0 - 1;
    if (pe >= 0 && pe < c.lim) tp.below = Elem<T>::load(a.in, c.base + pe);
  }
}

// Pooled outputs n0..n0+3 of a row from the lane's taps.
__device__ __forceinline__ void pool_taps(const PoolArgs& a, const RowCtx& c, int64_t chunk,
                                          const Taps& tp, float* r) {
  const int lane = threadIdx.x & (kWave - 1);
  // 32-bit arithmetic: block indices, the key length and the token's block
  // are below 2^31 (int32 sequence offsets), and lim <= 4*NB.
  const int32_t n0 = static_cast<int32_t>(chunk) * 256 + 4 * lane;
  const int32_t lim = static_cast<int32_t>(c.lim);
  const int32_t lk = static_cast<int32_t>(c.lk < INT32_MAX ? c.lk : INT32_MAX);
  const int32_t ob = static_cast<int32_t>(c.ob);
  const int32_t avail = lim - 4 * n0;
  float v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) v[j] = tp.v[j];
  if (avail < 16) {
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = j < avail ? v[j] : -INFINITY;
  }
  const float prev = wave_shr1(v[15], tp.below);  // tap 4*n0-1
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int32_t n = n0 + e;
    const float first = e == 0 ? prev : v[4 * e - 1];
    const float m = fmaxf(fmaxf(first, v[4 * e]),
                          fmaxf(fmaxf(v[4 * e + 1], v[4 * e + 2]), v[4 * e + 3]));
    // The window 4n-1 .. 4n+3 (from tap 0) holds a tap below lk.
    const bool any = lk > (n > 0 ? 4 * n - 1 : 0);
    const bool force = n < a.init_blocks || (ob >= n && ob - n <= a.local_blocks);
    r[e] = force ? INFINITY : (any ? m : -INFINITY);
  }
}

// Pooled outputs n0..n0+3 (n0 = 256*chunk + 4*lane) of a row.
template <typename T, bool kVec>
__device__ __forceinline__ void pool4(const PoolArgs& a, const RowCtx& c, int64_t chunk, float* r) {
  Taps tp;
  load_taps<T, kVec>(a, c, chunk, tp);
  pool_taps(a, c, chunk, tp, r);
}

template <typename T, bool kVec>
__device__ __forceinline__ void store_pooled(const PoolArgs& a, int64_t row, int64_t n0, const float* r) {
  if (n0 >= a.NB) return;
  const int64_t o = row * a.NB + n0;
  if (kVec && n0 + 3 < a.NB) {
    store4<T>(a.out, o, r);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (n0 + e < a.NB) Elem<T>::store(a.out, o + e, r[e]);
  }
}

// The (token, chunk) unit of a wave: blockIdx.y is the head and the waves of
// blockIdx.x run over the Tq*n_chunks units of that head (below 2^31, checked
// by the launcher), so a unit's token needs at most a 32-bit division.
struct Unit {
  int64_t row, t, chunk;  // row = h*Tq + t
  bool ok;
};
__device__ __forceinline__ Unit pool_unit(const PoolArgs& a) {
  const uint32_t v = blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave);
  const uint32_t nc = static_cast<uint32_t>(a.n_chunks);
  const uint32_t t = nc == 1 ? v : v / nc;
  Unit u;
  u.t = t;
  u.chunk = v - t * nc;
  u.row = static_cast<int64_t>(blockIdx.y) * a.Tq + t;
  u.ok = t < a.Tq;
  return u;
}

template <typename T, bool kVec>
__global__ __launch_bounds__(256) void maxpool_p4_kernel(PoolArgs a) {
  const Unit un = pool_unit(a);
  if (!un.ok) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = un.row, chunk = un.chunk;
  const RowCtx c = row_ctx(a, row, un.t);
  float r[4];
  pool4<T, kVec>(a, c, chunk, r);
  store_pooled<T, kVec>(a, row, chunk * 256 + 4 * lane, r);
}

// ------------------------------------------------------- fused block top-k
// The selection the pipeline makes from the pooled scores, fused into the
// pool: one wave per (head, token) row pools all NB blocks into registers
// (the P == 4 path above; optionally storing them) and writes the row's top K
// block ids under the order (score descending, block id ascending), sorted
// ascending, with -1 for a selected block whose score is -inf and for the
// slots past NB -- the -1 entries first.
//
// Selection: scores map to order-preserving unsigned keys; a threshold is
// built bit by bit from the top (each step a ballot count of the keys at or
// above a candidate) until it is the K-th largest key or exactly K keys lie
// at or above it; keys above it are taken, and of the keys equal to it the
// ones with the lowest block ids, by a running rank.
// Raw buffer resources: loads past `bytes` read 0 (the range check is per
// 4-byte word).
constexpr uint32_t kBufferFlags = 0x00020000;  // gfx9 raw buffer resource word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           static_cast<int>(kBufferFlags));
}

constexpr int kTopkMaxChunks = 16;  // NB <= 4096 (64 keys per lane)
constexpr uint32_t kKeyNegInf = 0x007fffffu;  // order_key(-inf)
constexpr uint32_t kKeyPosInf = 0xff800000u;  // order_key(+inf)
constexpr int kTopkShortList = 1024;  // keys between the bounds kept per wave (16 a lane)
constexpr int kTopkListCap = 640;     // (score, id) pairs of topk_select_list's wave list

// LDS words of each wave of a 256-thread block: topk_select_list's list of
// score bits and block ids (reused afterwards for its bitmaps), which also
// holds topk_select's short list; none with one chunk a row, where the search
// counts the keys in registers.
template <int NCH>
constexpr int topk_list_len() { return NCH >= 2 ? 2 * kTopkListCap : 1; }
static_assert(2 * kTopkListCap >= kTopkShortList, "the short list shares the wave's LDS");

// Order-preserving unsigned key of a score; -0.0 maps to +0.0's key, since
// the two are equal scores (ties, taken in ascending block id).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t b = __float_as_uint(f);
  b = b == 0x80000000u ? 0u : b;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
// The score of a key order_key returns.
__device__ __forceinline__ float key_score(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Wave-wide max / min (wave-uniform results): DPP within each 16-lane row
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror),
// then the four rows' results through readlane.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t rows4_u32(uint32_t v, int r) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 16 * r));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  return max(max(rows4_u32(v, 0), rows4_u32(v, 1)), max(rows4_u32(v, 2), rows4_u32(v, 3)));
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<0xB1>(v));
  v = min(v, dpp_u32<0x4E>(v));
  v = min(v, dpp_u32<0x141>(v));
  v = min(v, dpp_u32<0x140>(v));
  return min(min(rows4_u32(v, 0), rows4_u32(v, 1)), min(rows4_u32(v, 2), rows4_u32(v, 3)));
}

// Lanes below this one whose bit is set in mask.
__device__ __forceinline__ int32_t lanes_below(uint64_t mask) {
  return static_cast<int32_t>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}

// Inclusive sum over the wave's lanes (lane 0 first): DPP shifts within each
// 16-lane row, then each row's total carried into the rows after it.
template <int CTRL, int RM>
__device__ __forceinline__ uint32_t dpp_or0(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, RM, 0xF, false));
}
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t x) {
  x += dpp_or0<0x111, 0xF>(x);  // row_shr:1
  x += dpp_or0<0x112, 0xF>(x);  // row_shr:2
  x += dpp_or0<0x114, 0xF>(x);  // row_shr:4
  x += dpp_or0<0x118, 0xF>(x);  // row_shr:8
  x += dpp_or0<0x142, 0xA>(x);  // row_bcast:15 into rows 1 and 3
  x += dpp_or0<0x143, 0xC>(x);  // row_bcast:31 into rows 2 and 3
  return x;
}

// The threshold search over a short list of `total` keys in LDS, NS of them
// a lane (total <= 64*NS; the slots past it hold key 0, below every
// candidate): bits `top`..0 of tau, each kept when at least K keys (the
// list's count plus n_inf) lie at or above the candidate, stopping at a
// candidate past `lo` with exactly K.  Every key above the final tau is in
// the list or +inf, and every key equal to it is in the list, so the list
// also gives n_gt (keys > tau, with the n_inf ones) and n_eq (keys == tau).
template <int NS>
__device__ __forceinline__ uint32_t list_search(const uint32_t* list, int32_t total, int top,
                                                uint32_t tau, int32_t n_inf, int32_t K,
                                                uint32_t lo, int32_t& n_gt, int32_t& n_eq) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t sk[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int idx = i * kWave + lane;
    sk[i] = idx < total ? list[idx] : 0u;
  }
  for (int bit = top; bit >= 0; --bit) {
    const uint32_t cand = tau | (1u << bit);
    int32_t n = n_inf;
#pragma unroll
    for (int i = 0; i < NS; ++i) n += __popcll(__ballot(sk[i] >= cand));
    if (n >= K) tau = cand;
    if (n == K && cand > lo) break;
  }
  n_gt = n_inf;
  n_eq = 0;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    n_gt += __popcll(__ballot(sk[i] > tau));
    n_eq += __popcll(__ballot(sk[i] == tau));
  }
  return tau;
}

// The top K of a row's keys (blocks n = 256*ch + 4*lane + e; key 0, below
// every real key, past NB) into orow.  `list` is the wave's short list in LDS
// (kTopkShortList keys; unused with one chunk).
template <int NCH>
__device__ __forceinline__ void topk_select(const uint32_t (&key)[NCH][4], int32_t NB, int32_t K,
                                            int32_t* orow, uint32_t* list) {
  const int lane = threadIdx.x & (kWave - 1);
  auto count_ge = [&](uint32_t cand) -> int32_t {
    int32_t n = 0;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) n += __popcll(__ballot(key[ch][e] >= cand));
    return n;
  };
  auto count_eq = [&](uint32_t cand) -> int32_t {
    int32_t n = 0;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) n += __popcll(__ballot(key[ch][e] == cand));
    return n;
  };
  uint32_t tau = 0;     // the K-th largest key (0 when every block is taken)
  int32_t need_eq = 0;  // blocks with key == tau to take, lowest ids first
  int32_t neg = 0;      // taken blocks scoring -inf
  int32_t n_eq = -1;    // blocks with key == tau, when the short list counted them
  if (NB > K) {
    // Bounds on tau that fix its high bits: while fewer than K blocks are
    // forced to +inf, tau is at most the largest finite key; and for K <= 64
    // it is at least the smallest of the lanes' largest finite keys (64
    // distinct keys lie at or above it).  tau shares every bit above the
    // highest bit where the two differ, so the search starts there.  With
    // one chunk (four keys a lane) the bounds cost more than the steps they
    // save (measured, with the reductions on ds_bpermute and on DPP alike).
    int top = 31;
    bool searched = false;
    int32_t n_gt = 0;  // keys > tau, from the short list
    const int32_t n_inf = NCH >= 2 && K <= kWave ? count_ge(kKeyPosInf) : K;
    if (n_inf < K) {
      uint32_t lmax = 0;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t k = key[ch][e] < kKeyPosInf ? key[ch][e] : 0u;
          lmax = k > lmax ? k : lmax;
        }
      const uint32_t hi = wave_max_u32(lmax), lo = wave_min_u32(lmax);
      if (lo == hi) {
        top = -1;  // tau == hi
        tau = hi;
      } else {
        top = 31 - __builtin_clz(lo ^ hi);
        tau = hi & ~((2u << top) - 1u);  // the shared bits above `top`
        // Only keys in [lo, hi] (and the +inf ones, counted apart) can be at
        // or above a candidate past lo: when at most kTopkShortList of them
        // exist they go to a per-wave list in LDS, and the search counts
        // that list -- at most sixteen keys a lane instead of 4*NCH.  At or below lo
        // the list undercounts, but still holds at least 64 >= K keys, so
        // the `>= K` decision stands; only the exact-K stop waits for a
        // candidate past lo.
        int32_t mine = 0;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
          for (int e = 0; e < 4; ++e) mine += (key[ch][e] >= lo && key[ch][e] <= hi) ? 1 : 0;
        const int32_t incl = static_cast<int32_t>(wave_incl_sum(static_cast<uint32_t>(mine)));
        const int32_t total = __builtin_amdgcn_readlane(incl, kWave - 1);
        if (total <= kTopkShortList) {
          int32_t pos = incl - mine;
#pragma unroll
          for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (key[ch][e] >= lo && key[ch][e] <= hi) list[pos++] = key[ch][e];
          // Every step counts only the list's occupied slots: a search over
          // ceil(total/64) keys a lane (cfg5's real rows: 205-701 keys).
          switch ((total + kWave - 1) / kWave) {
#define TOPK_NS(N) \
  case N: tau = list_search<N>(list, total, top, tau, n_inf, K, lo, n_gt, n_eq); break;
            TOPK_NS(1) TOPK_NS(2) TOPK_NS(3) TOPK_NS(4) TOPK_NS(5) TOPK_NS(6) TOPK_NS(7)
            TOPK_NS(8) TOPK_NS(9) TOPK_NS(10) TOPK_NS(11) TOPK_NS(12) TOPK_NS(13) TOPK_NS(14)
            TOPK_NS(15) TOPK_NS(16)
#undef TOPK_NS
            default: break;  // total >= 1: hi is a key of the list
          }
          searched = true;
        }
      }
    }
    // A candidate with exactly K keys at or above it decides the selection
    // (keys >= it); the lower bits are then not needed, and the tie rule
    // below takes every key equal to it.
    // Unrolled over the 32 bits (with one chunk, top is 31 at compile time):
    // each step is its compares and counts, the tau update and one exit
    // branch, with no loop counter or combined exit condition.
    if (!searched) {
#pragma unroll
      for (int bit = 31; bit >= 0; --bit) {
        if (bit > top) continue;
        const uint32_t cand = tau | (1u << bit);
        const int32_t n = count_ge(cand);
        if (n >= K) tau = cand;
        if (n == K) break;
      }
    }
    need_eq = K - (searched ? n_gt : tau == 0xffffffffu ? 0 : count_ge(tau + 1));
    neg = tau == kKeyNegInf ? need_eq : 0;
  } else {
    neg = count_ge(kKeyNegInf) - count_ge(kKeyNegInf + 1);
  }
  int32_t lead = (NB < K ? K - NB : 0) + neg;  // -1 slots, first
  lead = lead < K ? lead : K;
  for (int32_t j = lane; j < lead; j += kWave) orow[j] = -1;
  int32_t out_pos = lead, eq_seen = 0;
  // The keys of chunk ch with take[e] set go to the next output slots, in
  // block-id order.
  auto emit = [&](int ch, const bool (&take)[4]) {
    uint64_t m_take[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) m_take[e] = __ballot(take[e]);
    int32_t pos = out_pos;
#pragma unroll
    for (int e = 0; e < 4; ++e) pos += lanes_below(m_take[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (take[e] && pos < K) orow[pos] = 256 * ch + 4 * lane + e;
      pos += take[e] ? 1 : 0;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) out_pos += __popcll(m_take[e]);
  };
  // Usually every key equal to tau is taken (ties at the threshold are rare)
  // or none is: a key is then taken by its compares alone, without the
  // running rank of the equal keys below.
  if (need_eq == 0 || (n_eq >= 0 ? n_eq : count_eq(tau)) == need_eq) {
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      bool take[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k = key[ch][e];
        take[e] = (k > tau || (need_eq > 0 && k == tau)) && k != kKeyNegInf;
      }
      emit(ch, take);
    }
    return;
  }
  // Ranked output: the equal keys are taken by ascending id, need_eq of them.
  // A chunk holding no equal key still to rank (none at all, or need_eq
  // taken already) takes the keys above tau by their compares alone.
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    bool eq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) eq[e] = key[ch][e] == tau;
    bool take[4];
    if (eq_seen >= need_eq || __ballot(eq[0] || eq[1] || eq[2] || eq[3]) == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) take[e] = key[ch][e] > tau && key[ch][e] != kKeyNegInf;
      emit(ch, take);
      continue;
    }
    uint64_t m_eq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) m_eq[e] = __ballot(eq[e]);
    int32_t eq_rank = eq_seen;  // equal keys at lower block ids
#pragma unroll
    for (int e = 0; e < 4; ++e) eq_rank += lanes_below(m_eq[e]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool sel = key[ch][e] > tau || (eq[e] && eq_rank < need_eq);
      eq_rank += eq[e] ? 1 : 0;
      take[e] = sel && key[ch][e] != kKeyNegInf;
    }
    emit(ch, take);
#pragma unroll
    for (int e = 0; e < 4; ++e) eq_seen += __popcll(m_eq[e]);
  }
}

// ----------------------------------------- list selection (two chunks or more)
// For rows of two or more chunks and K <= 64, the selection of topk_select
// over a list instead of the 4*NCH keys a lane.  The K-th largest score is at
// least lo, the smallest of the lanes' largest scores (64 scores lie at or
// above it), so every score >= lo goes, with its block id, to a per-wave list
// in LDS (cfg5's real pooled rows: 202-704 of 2112 blocks, measured on the CPU
// from the oracle's rows; past kTopkListCap, lo is first raised by steps of
// the threshold search over the lane's scores), and the threshold search, the
// tie rule and the output run over its entries alone -- ceil(total/64) a
// lane.  The output
// needs no sort: the taken blocks are marked in a bitmap of the row (64
// blocks a lane), and an entry's slot is the number of taken blocks below it.
// Equal scores still to rank (fewer taken than tied) are ranked the same way
// through a bitmap of the tied blocks.  Scores past NB are -inf here: they
// rank after every real -inf block (higher ids), so they are taken only where
// a real -inf block would be too, and a taken -inf block is written as -1
// whatever its id.

// Bits of the 64-bit word (lo, hi) below bit b.
__device__ __forceinline__ int32_t bits_below(uint32_t lo, uint32_t hi, int b) {
  const uint64_t w = (static_cast<uint64_t>(hi) << 32) | lo;
  return __popcll(w & ((uint64_t(1) << b) - 1u));
}
__device__ __forceinline__ void lds_or(uint32_t* p, uint32_t bit) {
  __hip_atomic_fetch_or(p, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}

// The list holds `total` entries, entry i's score bits at lds[i] and block id
// at lds[kTopkListCap + i]; NS = ceil(total / 64).  Every key of the row >= lo
// is in the list, and at least K keys are.
template <int NS>
__device__ __forceinline__ void list_select(uint32_t* lds, int32_t total, uint32_t lo, int32_t K,
                                            int32_t* orow) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t sk[NS];
  int32_t sid[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const int idx = i * kWave + lane;  // < NS*64 <= kTopkListCap: inside the list
    const uint32_t b = lds[idx], id = lds[kTopkListCap + idx];
    sk[i] = idx < total ? order_key(__uint_as_float(b)) : 0u;  // key 0: below every candidate
    sid[i] = idx < total ? static_cast<int32_t>(id) : 0;
  }
  auto count = [&](auto pred) -> int32_t {
    int32_t n = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) n += __popcll(__ballot(pred(sk[i])));
    return n;
  };
  // tau: the K-th largest key.  With K or more +inf scores it is +inf;
  // otherwise the list holds a finite key >= lo, hi (the largest one) >= lo,
  // and tau in [lo, hi] shares every bit above the highest bit where they
  // differ (hi == lo: lo is a key, and tau).
  uint32_t tau = kKeyPosInf;
  int top = -1;
  if (count([](uint32_t k) { return k == kKeyPosInf; }) < K) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < NS; ++i) m = (sk[i] < kKeyPosInf && sk[i] > m) ? sk[i] : m;
    const uint32_t hi = wave_max_u32(m);
    if (hi == lo) {
      tau = lo;
    } else {
      top = 31 - __builtin_clz(lo ^ hi);
      tau = hi & ~((2u << top) - 1u);
    }
  }
  // Below lo the list undercounts but still holds >= K keys, so the `>= K`
  // decisions stand.  Exactly K list keys at or above a candidate are the K
  // largest of the row even below lo (every key >= the K-th largest, ties
  // included, is >= lo and in the list), so the exact-K stop needs no bound.
  // The candidate bit is a mask shifted down each step, cleared by the stop:
  // one scalar loop condition.
  for (uint32_t b = top < 0 ? 0u : 1u << top; b != 0u;) {
    const uint32_t cand = tau | b;
    const int32_t n = count([cand](uint32_t k) { return k >= cand; });
    if (n >= K) tau = cand;
    b = n == K ? 0u : b >> 1;
  }
  const int32_t need_eq = K - count([tau](uint32_t k) { return k > tau; });  // >= 0
  const bool neg = tau == kKeyNegInf;  // the tied blocks score -inf: -1 slots, first
  const int32_t n_eq = need_eq > 0 && !neg ? count([tau](uint32_t k) { return k == tau; }) : 0;
  const bool rank_eq = need_eq > 0 && need_eq < n_eq;
  bool take[NS];
#pragma unroll
  for (int i = 0; i < NS; ++i)
    take[i] = sk[i] > tau || (sk[i] == tau && need_eq > 0 && !neg && !rank_eq);

  // The list has been read into registers: its LDS now holds the bitmaps.
  uint32_t* bm = lds;          // taken blocks: bit n % 32 of word n / 32
  uint32_t* before = lds + 128;  // taken blocks below lane l's 64 blocks
  __builtin_amdgcn_wave_barrier();
  bm[2 * lane] = 0u;
  bm[2 * lane + 1] = 0u;
  if (rank_eq) {
    uint32_t* em = lds + 192;   // tied blocks
    uint32_t* eb = lds + 320;   // tied blocks below lane l's 64 blocks
    em[2 * lane] = 0u;
    em[2 * lane + 1] = 0u;
#pragma unroll
    for (int i = 0; i < NS; ++i)
      if (sk[i] == tau) lds_or(em + (sid[i] >> 5), 1u << (sid[i] & 31));
    __builtin_amdgcn_wave_barrier();
    const int32_t c = __popc(em[2 * lane]) + __popc(em[2 * lane + 1]);
    eb[lane] = wave_incl_sum(c) - c;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (sk[i] == tau) {
        const int L = sid[i] >> 6;
        take[i] = static_cast<int32_t>(eb[L]) + bits_below(em[2 * L], em[2 * L + 1], sid[i] & 63) < need_eq;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NS; ++i)
    if (take[i]) lds_or(bm + (sid[i] >> 5), 1u << (sid[i] & 31));
  __builtin_amdgcn_wave_barrier();
  const int32_t c = __popc(bm[2 * lane]) + __popc(bm[2 * lane + 1]);
  before[lane] = wave_incl_sum(c) - c;
  __builtin_amdgcn_wave_barrier();
  const int32_t lead = neg ? need_eq : 0;
  if (lane < lead) orow[lane] = -1;
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    if (take[i]) {
      const int L = sid[i] >> 6;
      // lead + the taken blocks is K; the bound only keeps NaN scores (outside
      // the contract) inside the row.
      const int32_t slot = lead + static_cast<int32_t>(before[L]) + bits_below(bm[2 * L], bm[2 * L + 1], sid[i] & 63);
      if (slot < K) orow[slot] = sid[i];
    }
  }
}

// Builds the list from the lane's scores v (block 256*ch + 4*lane + e; -inf
// past NB) and selects from it; false, with nothing written, when no
// threshold puts K to kTopkListCap scores at or above it.
template <int NCH>
__device__ __forceinline__ bool topk_select_list(const float (&v)[NCH][4], int32_t K, int32_t* orow,
                                                 uint32_t* lds) {
  const int lane = threadIdx.x & (kWave - 1);
  // The lane's largest score from the scores' bits as integers: the largest
  // of them when a score has the sign bit clear, else the smallest (sign and
  // magnitude order negative scores the other way round).
  int32_t imax = INT32_MIN, imin = INT32_MAX;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int32_t b = __float_as_int(v[ch][e]);
      imax = b > imax ? b : imax;
      imin = b < imin ? b : imin;
    }
  uint32_t lo = wave_min_u32(order_key(__int_as_float(imax >= 0 ? imax : imin)));
  // Scores >= lo go to the list slot by slot ((ch, e) in turn, lanes in
  // order within a slot); false when a chunk would pass the cap.
  uint32_t total = 0;  // wave-uniform
  auto build = [&](float lo_score) -> bool {
    total = 0;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      bool in[4];
      uint64_t m[4];
      uint32_t n = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        in[e] = v[ch][e] >= lo_score;
        m[e] = __ballot(in[e]);
        n += static_cast<uint32_t>(__popcll(m[e]));
      }
      if (total + n > kTopkListCap) return false;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (in[e]) {
          const uint32_t pos = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m[e] >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m[e]), total));
          lds[pos] = __float_as_uint(v[ch][e]);
          lds[kTopkListCap + pos] = static_cast<uint32_t>(256 * ch + 4 * lane + e);
        }
        total += static_cast<uint32_t>(__popcll(m[e]));
      }
    }
    return true;
  };
  if (!build(key_score(lo))) {
    // More than kTopkListCap scores >= lo: raise lo by the threshold search
    // over the lane's scores, from the bits lo and the largest finite key
    // share, to the first candidate with K to kTopkListCap scores at or
    // above it, and build the list again.  Rows where no such candidate
    // exists (ties past the cap) take topk_select.
    uint32_t m = 0;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k = order_key(v[ch][e]);
        m = (k < kKeyPosInf && k > m) ? k : m;
      }
    const uint32_t hi = wave_max_u32(m);
    if (hi <= lo) return false;
    const int top = 31 - __builtin_clz(lo ^ hi);
    uint32_t tau = hi & ~((2u << top) - 1u);
    bool found = false;
    for (uint32_t b = 1u << top; b != 0u;) {
      const uint32_t cand = tau | b;
      const float cs = key_score(cand);
      int32_t n = 0;
#pragma unroll
      for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
        for (int e = 0; e < 4; ++e) n += __popcll(__ballot(v[ch][e] >= cs));
      if (n >= K) {
        tau = cand;
        found = n <= kTopkListCap;
      }
      b = found ? 0u : b >> 1;
    }
    if (!found) return false;
    lo = tau;
    if (!build(key_score(lo))) return false;
  }
  __builtin_amdgcn_wave_barrier();
  switch ((total + kWave - 1) / kWave) {
#define TOPK_LIST(N) \
  case N: list_select<N>(lds, static_cast<int32_t>(total), lo, K, orow); return true;
    TOPK_LIST(1) TOPK_LIST(2) TOPK_LIST(3) TOPK_LIST(4) TOPK_LIST(5)
    TOPK_LIST(6) TOPK_LIST(7) TOPK_LIST(8) TOPK_LIST(9) TOPK_LIST(10)
#undef TOPK_LIST
    default: return false;  // no score >= lo: NaN scores
  }
}
static_assert(kTopkListCap == 10 * kWave, "list_select is instantiated for 1..10 entries a lane");

// The selection of a row whose lane holds scores v (block 256*ch + 4*lane +
// e, -inf past NB): the list selection when it applies, else topk_select.
// topk_select takes the -inf past NB as blocks of the row (NCH*256 of them):
// they rank after every real block, so they are taken only where a real -inf
// block would be, and -- -inf -- are written as -1 like those; the -1 count
// K - NB of slots past a short row comes out the same.
template <int NCH>
__device__ __forceinline__ void select_row(const float (&v)[NCH][4], int32_t K, int32_t* orow,
                                           uint32_t* lds) {
  if constexpr (NCH >= 2) {
    if (K <= kWave && topk_select_list<NCH>(v, K, orow, lds)) return;
  }
  uint32_t key[NCH][4];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) key[ch][e] = order_key(v[ch][e]);
  topk_select<NCH>(key, 256 * NCH, K, orow, lds);
}

template <int NCH>
__global__ __launch_bounds__(256) void maxpool_topk_kernel(PoolArgs a, int32_t* topk, int32_t K,
                                                           int32_t store) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + (threadIdx.x / kWave);
  if (t >= a.Tq) return;  // wave-uniform
  const int64_t row = static_cast<int64_t>(blockIdx.y) * a.Tq + t;  // blockIdx.y: the head
  const int lane = threadIdx.x & (kWave - 1);
  const RowCtx c = row_ctx(a, row, t);
  const int32_t NB = static_cast<int32_t>(a.NB);
  __shared__ uint32_t lds[4][topk_list_len<NCH>()];  // one per wave of the 256-thread block
  float v[NCH][4];
  if constexpr (NCH == 1) {
    float r[4];
    pool4<float, true>(a, c, 0, r);
    if (store) store_pooled<float, true>(a, row, 4 * lane, r);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[0][e] = 4 * lane + e < NB ? r[e] : -INFINITY;
  } else {
    // Rows of several chunks: chunk ch+1's taps are loaded while chunk ch is
    // pooled (two tap buffers), so a row's loads overlap instead of waiting
    // chunk by chunk.  Every chunk is four 16-byte buffer loads a lane over
    // the row's taps below lim: the range check is per 4-byte word, so the
    // words past lim read 0 (masked to -inf by pool_taps) and no branch
    // separates the loads.  Lane 0's tap 4*n0-1 is the previous chunk's last
    // tap, from lane 63.
    // The row's start and limit are wave-uniform: readfirstlane lets the
    // compiler keep the resource in scalar registers.
    const uint64_t row_addr = reinterpret_cast<uint64_t>(static_cast<const float*>(a.in) + c.base);
    const uint64_t ra = (static_cast<uint64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(row_addr >> 32))) << 32) |
                        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(row_addr)));
    const int32_t lim = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(c.lim));  // <= 4*NB
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(reinterpret_cast<const float*>(ra), static_cast<uint32_t>(lim) * 4u);
    float tb[2][16];
    auto issue = [&](int ch, float (&d)[16]) {
      const int off = 4 * (1024 * ch + 16 * lane);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * j, 0, 0));
        d[4 * j] = x.x; d[4 * j + 1] = x.y; d[4 * j + 2] = x.z; d[4 * j + 3] = x.w;
      }
    };
    issue(0, tb[0]);
    float carry = -INFINITY;  // tap 1024*ch - 1, for lane 0
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      if (ch + 1 < NCH) issue(ch + 1, tb[(ch + 1) & 1]);
      Taps tp;
#pragma unroll
      for (int j = 0; j < 16; ++j) tp.v[j] = tb[ch & 1][j];
      tp.below = carry;
      float r[4];
      pool_taps(a, c, ch, tp, r);
      carry = 1024 * ch + 1023 < lim
                  ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tp.v[15]), 63))
                  : -INFINITY;
      if (store) store_pooled<float, true>(a, row, ch * 256 + 4 * lane, r);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[ch][e] = 256 * ch + 4 * lane + e < NB ? r[e] : -INFINITY;
    }
  }
  select_row<NCH>(v, K, topk + row * K, lds[threadIdx.x >> 6]);
}

// The same selection over rows already pooled (the fused stage-1 + max-pool
// output): one wave per row of `pooled` ([rows, row_stride] fp32, NB blocks
// a row), lane l holding blocks 256*ch + 4l .. +3 as in the fused kernel, so
// the ids are the ones maxpool_topk_kernel writes for the same pooled row.
template <int NCH, bool kVec>
__global__ __launch_bounds__(256) void topk_rows_kernel(const float* pooled, int64_t rows,
                                                        int64_t row_stride, int32_t NB,
                                                        int32_t* topk, int32_t K) {
  // The wave's row, wave-uniform for the compiler (readfirstlane): the
  // branches on per-row values below are scalar branches.
  const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) +
                      __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (row >= rows) return;
  const int lane = threadIdx.x & (kWave - 1);
  const float* src = pooled + row * row_stride;
  __shared__ uint32_t lds[4][topk_list_len<NCH>()];
  // Every chunk's loads are issued before any is used: one 16-byte buffer
  // load a lane and chunk over the row's NB scores (four 4-byte loads for
  // rows not 16-byte aligned), with no branch between them: the range check
  // is per 4-byte word, so the words past NB read 0 (replaced by -inf).
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, static_cast<uint32_t>(NB) * 4u);
  float v[NCH][4];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int32_t n0 = 256 * ch + 4 * lane;
    if constexpr (kVec) {  // 16-byte aligned rows
      const f32x4 x = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 4 * n0, 0, 0));
      v[ch][0] = x.x; v[ch][1] = x.y; v[ch][2] = x.z; v[ch][3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        v[ch][e] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 4 * (n0 + e), 0, 0));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[ch][e] = n0 + e < NB ? v[ch][e] : -INFINITY;
  }
  select_row<NCH>(v, K, topk + row * K, lds[threadIdx.x >> 6]);
}

// Rows of more than 4096 blocks (contexts past 262 144 tokens), past the
// registers of a wave: one workgroup of kThreads threads per row (256 for up
// to 8192 blocks, 1024 above), thread j holding blocks j*M .. j*M+M-1 --
// contiguous, so thread order is block-id order and every rank the output
// needs is a workgroup prefix sum.  The selection is topk_select's (order
// (score descending, id ascending), the K-th key built bit by bit, keys
// equal to it taken by ascending id, -1 first for selected -inf blocks and
// for slots past NB); each count is summed over the workgroup through LDS.
constexpr int kTopkLongMaxBlocks = 32 * 1024;  // M <= 32 keys a thread, 1024 threads

// Sum of v over the workgroup's W waves (every thread gets it).  red holds
// two slots per wave, used alternately: a call's writes cannot overtake the
// previous call's reads, which every thread finished before that call's
// barrier.
template <int W>
__device__ __forceinline__ int32_t long_sum(int32_t v, int32_t (*red)[W], int& par) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int32_t w = __builtin_amdgcn_readlane(static_cast<int32_t>(wave_incl_sum(static_cast<uint32_t>(v))), kWave - 1);
  if (lane == 0) red[par][wave] = w;
  __syncthreads();
  int32_t s = 0;
#pragma unroll
  for (int i = 0; i < W; i += 4) {
    const i32x4 r = *reinterpret_cast<const i32x4*>(&red[par][i]);
    s += (r.x + r.y) + (r.z + r.w);
  }
  par ^= 1;
  return s;
}

// Largest and smallest of v over the workgroup (every thread gets both);
// the same two-slot scheme as long_sum.
template <int W>
__device__ __forceinline__ void long_max_min(uint32_t vmax, uint32_t vmin, uint32_t (*red)[2 * W],
                                             int& par, uint32_t& hi, uint32_t& lo) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const uint32_t a = wave_max_u32(vmax), b = wave_min_u32(vmin);
  if (lane == 0) {
    red[par][wave] = a;
    red[par][W + wave] = b;
  }
  __syncthreads();
  hi = 0u;
  lo = 0xffffffffu;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    hi = max(hi, red[par][i]);
    lo = min(lo, red[par][W + i]);
  }
  par ^= 1;
}

// Exclusive prefix sum of v over the workgroup's threads in thread order.
template <int W>
__device__ __forceinline__ int32_t long_excl_scan(int32_t v, int32_t (*red)[W], int& par) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x & (kWave - 1);
  const int32_t incl = static_cast<int32_t>(wave_incl_sum(static_cast<uint32_t>(v)));
  if (lane == kWave - 1) red[par][wave] = incl;
  __syncthreads();
  int32_t before = 0;
#pragma unroll
  for (int i = 0; i < W; ++i) before += i < wave ? red[par][i] : 0;
  par ^= 1;
  return before + incl - v;
}

template <int M, int kThreads, bool kVec>
__global__ __launch_bounds__(kThreads) void topk_long_kernel(const float* pooled, int64_t row_stride,
                                                             int32_t NB, int32_t* topk, int32_t K) {
  constexpr int W = kThreads / kWave;
  static_assert(W % 4 == 0, "wave counts are summed four at a time");
  __shared__ __align__(16) int32_t red[2][W];
  __shared__ uint32_t red_mm[2][2 * W];
  int par = 0, par_mm = 0;
  const int64_t row = blockIdx.x;
  const int j = threadIdx.x;
  const int32_t n0 = j * M;  // this thread's first block
  const float* src = pooled + row * row_stride + n0;
  uint32_t key[M];
  if (kVec && n0 + M <= NB) {
#pragma unroll
    for (int i = 0; i < M; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + i);
      key[i] = order_key(v.x);
      key[i + 1] = order_key(v.y);
      key[i + 2] = order_key(v.z);
      key[i + 3] = order_key(v.w);
    }
  } else {
    // Scalar loads at indices clamped into the row (the last block), so every
    // load is unconditional; keys past NB are 0, below every real key.
    const int32_t last = NB - 1 - n0;  // negative for a thread past the row's end
#pragma unroll
    for (int i = 0; i < M; ++i) {
      const float v = src[i < last ? i : last];
      key[i] = i <= last ? order_key(v) : 0u;
    }
  }
  auto count = [&](auto pred) -> int32_t {
    int32_t n = 0;
#pragma unroll
    for (int i = 0; i < M; ++i) n += pred(key[i]) ? 1 : 0;
    return n;
  };
  uint32_t tau = 0;     // the K-th largest key (0 when every block is taken)
  int32_t need_eq = 0;  // blocks with key == tau to take, lowest ids first
  int32_t neg = 0;      // taken blocks scoring -inf
  if (NB > K) {
    // The counts are workgroup-uniform, so every thread takes the same
    // branch.  Bounds on tau fix its high bits, as in topk_select: while
    // fewer than K blocks are +inf, tau is at most the largest finite key,
    // and when at least K threads hold blocks, at least the smallest of
    // their largest keys (distinct keys, one a thread).
    int top = 31;
    const int32_t holders = (NB + M - 1) / M;  // threads holding a block
    if (K <= holders && long_sum<W>(count([&](uint32_t k) { return k >= kKeyPosInf; }), red, par) < K) {
      uint32_t tmax = 0;
#pragma unroll
      for (int i = 0; i < M; ++i) tmax = max(tmax, key[i] < kKeyPosInf ? key[i] : 0u);
      uint32_t hi, lo;
      long_max_min<W>(tmax, n0 < NB ? tmax : 0xffffffffu, red_mm, par_mm, hi, lo);
      if (lo == hi) {
        top = -1;  // tau == hi
        tau = hi;
      } else {
        top = 31 - __builtin_clz(lo ^ hi);
        tau = hi & ~((2u << top) - 1u);  // the shared bits above `top`
      }
    }
    for (int bit = top; bit >= 0; --bit) {
      const uint32_t cand = tau | (1u << bit);
      const int32_t n = long_sum<W>(count([&](uint32_t k) { return k >= cand; }), red, par);
      if (n >= K) tau = cand;
      if (n == K) break;
    }
    const int32_t gt = tau == 0xffffffffu ? 0 : long_sum<W>(count([&](uint32_t k) { return k > tau; }), red, par);
    need_eq = K - gt;
    neg = tau == kKeyNegInf ? need_eq : 0;
  } else {
    neg = long_sum<W>(count([&](uint32_t k) { return k == kKeyNegInf; }), red, par);
  }
  int32_t lead = (NB < K ? K - NB : 0) + neg;  // -1 slots, first
  lead = lead < K ? lead : K;
  int32_t* orow = topk + row * K;
  for (int32_t i = j; i < lead; i += kThreads) orow[i] = -1;
  // Keys equal to tau still to take go by ascending id: the thread's rank
  // among them is the equal keys of the threads before it.
  const bool rank_eq = need_eq > 0 && tau != kKeyNegInf;
  int32_t eq_rank = rank_eq ? long_excl_scan<W>(count([&](uint32_t k) { return k == tau; }), red, par) : 0;
  bool take[M];
  int32_t n_take = 0;
#pragma unroll
  for (int i = 0; i < M; ++i) {
    const bool eq = key[i] == tau;
    take[i] = (key[i] > tau || (rank_eq && eq && eq_rank < need_eq)) && key[i] != kKeyNegInf;
    eq_rank += eq ? 1 : 0;
    n_take += take[i] ? 1 : 0;
  }
  int32_t pos = lead + long_excl_scan<W>(n_take, red, par);
#pragma unroll
  for (int i = 0; i < M; ++i) {
    if (take[i] && pos < K) orow[pos] = n0 + i;
    pos += take[i] ? 1 : 0;
  }
}

// General path: any P >= 1 (window of P+1 taps, padding 1); one output per lane.
template <typename T>
__global__ __launch_bounds__(256) void maxpool_generic_kernel(PoolArgs a) {
  const Unit un = pool_unit(a);
  if (!un.ok) return;  // wave-uniform
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = un.row, chunk = un.chunk, t = un.t;
  const int b = find_sequence(a.cu_q, a.B, t);
  int64_t lk = 0, ob = 0;
  if (b >= 0) {
    lk = static_cast<int64_t>(a.cu_k[b + 1] - a.cu_k[b]) + a.cache[b];
    ob = static_cast<uint32_t>(t - a.cu_q[b]) / static_cast<uint32_t>(a.block_size);
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
  // One wave per (token, chunk) unit; blockIdx.y is the head.
  const int64_t units = a.Tq * a.n_chunks;
  if (units >= (int64_t{1} << 31) || a.H > 65535)
    UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, "max_pooling_1d_varlen: too many rows (H=%lld, Tq=%lld)",
              (long long)a.H, (long long)a.Tq);
  const dim3 blocks(static_cast<unsigned>((units + threads / kWave - 1) / (threads / kWave)),
                    static_cast<unsigned>(a.H));
  if (a.P == 4) {
    const dim3 blocks4 = blocks;
    // Vector loads need 16-byte aligned taps (F a multiple of 16 bytes' worth of
    // elements), vector stores 16/8-byte aligned output runs (NB % 4 == 0).
    const bool vec = (reinterpret_cast<uintptr_t>(a.in) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                     ((a.F * (int64_t)sizeof(T)) % 16) == 0 && (a.NB % 4) == 0;
    if (vec)
      hipLaunchKernelGGL((maxpool_p4_kernel<T, true>), blocks4, dim3(threads), 0, s, a);
    else
      hipLaunchKernelGGL((maxpool_p4_kernel<T, false>), blocks4, dim3(threads), 0, s, a);
  } else {
    hipLaunchKernelGGL((maxpool_generic_kernel<T>), blocks, dim3(threads), 0, s, a);
  }
  return check_launch("max_pooling_1d_varlen");
}

int launch_topk(const PoolArgs& a, int32_t* topk, int32_t K, int32_t store, hipStream_t s) {
  const int nch = static_cast<int>((a.NB + 255) / 256);
  // One wave per row: the token on blockIdx.x (four a workgroup), the head on blockIdx.y.
  if (a.Tq >= (int64_t{1} << 31) || a.H > 65535)
    UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, "max_pooling_1d_varlen_topk: too many rows (H=%lld, Tq=%lld)",
              (long long)a.H, (long long)a.Tq);
  const dim3 g(static_cast<unsigned>((a.Tq + 3) / 4), static_cast<unsigned>(a.H)), b(256);
  switch (nch) {
#define UNUM_TOPK_CASE(N) \
    case N: hipLaunchKernelGGL((maxpool_topk_kernel<N>), g, b, 0, s, a, topk, K, store); break;
    UNUM_TOPK_CASE(1) UNUM_TOPK_CASE(2) UNUM_TOPK_CASE(3) UNUM_TOPK_CASE(4)
    UNUM_TOPK_CASE(5) UNUM_TOPK_CASE(6) UNUM_TOPK_CASE(7) UNUM_TOPK_CASE(8)
    UNUM_TOPK_CASE(9) UNUM_TOPK_CASE(10) UNUM_TOPK_CASE(11) UNUM_TOPK_CASE(12)
    UNUM_TOPK_CASE(13) UNUM_TOPK_CASE(14) UNUM_TOPK_CASE(15) UNUM_TOPK_CASE(16)
#undef UNUM_TOPK_CASE
    default: UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "max_pooling_1d_varlen_topk: %lld blocks (max %d)",
                       (long long)a.NB, kTopkMaxChunks * 256);
  }
  return check_launch("max_pooling_1d_varlen_topk");
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case UNUM_DTYPE_F32: return launch_pool<float>(a, s);
    case UNUM_DTYPE_BF16: return launch_pool<__bf16>(a, s);
    case UNUM_DTYPE_F16: return launch_pool<_Float16>(a, s);
    default: UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "max_pooling_1d_varlen: unsupported dtype %d", dtype);
  }
}

extern "C" int unum_max_pooling_1d_varlen_topk(const void* input, int64_t input_numel,
                                               const int32_t* cu_seqlens_q,
                                               const int32_t* cu_seqlens_k,
                                               const int32_t* cache_lens, void* pooled,
                                               int32_t* topk_idx, int64_t H, int64_t Tq,
                                               int64_t B, int64_t flat_stride,
                                               int64_t num_blocks, int32_t block_size,
                                               int32_t stride, int32_t local_blocks,
                                               int32_t init_blocks, int32_t topk, void* stream) {
  using namespace unum;
  clear_error();
  UNUM_REQUIRE(H >= 0 && Tq >= 0 && B >= 0 && num_blocks >= 0 && flat_stride >= 0,
               "max_pooling_1d_varlen_topk: negative size");
  UNUM_REQUIRE(topk >= 1, "max_pooling_1d_varlen_topk: topk=%d", topk);
  UNUM_REQUIRE(block_size > 0 && stride > 0 && block_size / stride == 4,
               "max_pooling_1d_varlen_topk: block_size / stride must be 4 (got %d / %d)",
               block_size, stride);
  UNUM_REQUIRE(num_blocks <= kTopkMaxChunks * 256,
               "max_pooling_1d_varlen_topk: %lld blocks exceed %d", (long long)num_blocks,
               kTopkMaxChunks * 256);
  if (H == 0 || Tq == 0) return UNUM_OK;
  UNUM_REQUIRE(num_blocks >= 1, "max_pooling_1d_varlen_topk: no blocks");
  UNUM_REQUIRE(input && topk_idx && cu_seqlens_q && cu_seqlens_k && cache_lens,
               "max_pooling_1d_varlen_topk: null pointer");
  UNUM_REQUIRE(B >= 1, "max_pooling_1d_varlen_topk: cu_seqlens must hold at least 2 entries");
  UNUM_REQUIRE(H * Tq * flat_stride <= input_numel,
               "max_pooling_1d_varlen_topk: flat row stride %lld times H*Tq=%lld rows exceeds "
               "the input's %lld elements",
               (long long)flat_stride, (long long)(H * Tq), (long long)input_numel);
  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(input) & 15) == 0 && (flat_stride % 4) == 0,
               "max_pooling_1d_varlen_topk: input rows must be 16-byte aligned");
  UNUM_REQUIRE(pooled == nullptr ||
                   ((reinterpret_cast<uintptr_t>(pooled) & 15) == 0 && (num_blocks % 4) == 0),
               "max_pooling_1d_varlen_topk: the pooled output needs 16-byte aligned rows "
               "(num_blocks %% 4 == 0)");
  PoolArgs a;
  a.in = input;
  a.numel = input_numel;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.cache = cache_lens;
  a.out = pooled;
  a.H = H;
  a.Tq = Tq;
  a.B = B;
  a.F = flat_stride;
  a.NB = num_blocks;
  a.block_size = block_size;
  a.P = 4;
  a.local_blocks = local_blocks;
  a.init_blocks = init_blocks;
  a.n_chunks = (num_blocks + 255) / 256;
  return launch_topk(a, topk_idx, topk, pooled != nullptr ? 1 : 0, static_cast<hipStream_t>(stream));
}

extern "C" int unum_topk_blocks(const float* pooled, int64_t rows, int64_t row_stride,
                                int64_t num_blocks, int32_t* topk_idx, int32_t topk,
                                void* stream) {
  using namespace unum;
  clear_error();
  UNUM_REQUIRE(rows >= 0 && num_blocks >= 0 && row_stride >= num_blocks,
               "topk_blocks: bad sizes (rows=%lld, row_stride=%lld, num_blocks=%lld)",
               (long long)rows, (long long)row_stride, (long long)num_blocks);
  UNUM_REQUIRE(topk >= 1, "topk_blocks: topk=%d", topk);
  UNUM_REQUIRE(num_blocks <= kTopkLongMaxBlocks, "topk_blocks: %lld blocks exceed %d",
               (long long)num_blocks, kTopkLongMaxBlocks);
  if (rows == 0) return UNUM_OK;
  UNUM_REQUIRE(num_blocks >= 1, "topk_blocks: no blocks");
  UNUM_REQUIRE(pooled && topk_idx, "topk_blocks: null pointer");
  const int64_t grid = (rows + 3) / 4;
  UNUM_REQUIRE(grid <= INT32_MAX, "topk_blocks: too many rows (%lld)", (long long)rows);
  const bool vec = (reinterpret_cast<uintptr_t>(pooled) & 15) == 0 && (row_stride % 4) == 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_blocks > kTopkMaxChunks * 256) {
    // A workgroup per row: 256 threads of 32 blocks up to 8192 blocks, then
    // 1024 threads of 16 or 32.
    UNUM_REQUIRE(rows <= INT32_MAX, "topk_blocks: too many rows (%lld)", (long long)rows);
    const dim3 gl(static_cast<unsigned>(rows));
    const int32_t nbl = static_cast<int32_t>(num_blocks);
#define UNUM_TOPK_LONG(M, TH)                                                                          \
    if (vec)                                                                                           \
      hipLaunchKernelGGL((topk_long_kernel<M, TH, true>), gl, dim3(TH), 0, s, pooled, row_stride, nbl, \
                         topk_idx, topk);                                                              \
    else                                                                                               \
      hipLaunchKernelGGL((topk_long_kernel<M, TH, false>), gl, dim3(TH), 0, s, pooled, row_stride, nbl, \
                         topk_idx, topk)
    if (num_blocks <= 32 * 256)
      UNUM_TOPK_LONG(32, 256);
    else if (num_blocks <= 16 * 1024)
      UNUM_TOPK_LONG(16, 1024);
    else
      UNUM_TOPK_LONG(32, 1024);
#undef UNUM_TOPK_LONG
    return check_launch("topk_blocks");
  }
  const int nch = static_cast<int>((num_blocks + 255) / 256);
  const dim3 g(static_cast<unsigned>(grid)), b(256);
  const int32_t NB = static_cast<int32_t>(num_blocks);
  switch (nch) {
#define UNUM_TOPK_ROWS_CASE(N)                                                                       \
    case N:                                                                                          \
      if (vec)                                                                                       \
        hipLaunchKernelGGL((topk_rows_kernel<N, true>), g, b, 0, s, pooled, rows, row_stride, NB,    \
                           topk_idx, topk);                                                          \
      else                                                                                           \
        hipLaunchKernelGGL((topk_rows_kernel<N, false>), g, b, 0, s, pooled, rows, row_stride, NB,   \
                           topk_idx, topk);                                                          \
      break;
    UNUM_TOPK_ROWS_CASE(1) UNUM_TOPK_ROWS_CASE(2) UNUM_TOPK_ROWS_CASE(3) UNUM_TOPK_ROWS_CASE(4)
    UNUM_TOPK_ROWS_CASE(5) UNUM_TOPK_ROWS_CASE(6) UNUM_TOPK_ROWS_CASE(7) UNUM_TOPK_ROWS_CASE(8)
    UNUM_TOPK_ROWS_CASE(9) UNUM_TOPK_ROWS_CASE(10) UNUM_TOPK_ROWS_CASE(11) UNUM_TOPK_ROWS_CASE(12)
    UNUM_TOPK_ROWS_CASE(13) UNUM_TOPK_ROWS_CASE(14) UNUM_TOPK_ROWS_CASE(15) UNUM_TOPK_ROWS_CASE(16)
#undef UNUM_TOPK_ROWS_CASE
    default: UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "topk_blocks: %lld blocks", (long long)num_blocks);
  }
  return check_launch("topk_blocks");
}
