// infllmv2_attn_stage1: InfLLM-v2 stage-1 block scores on gfx950.
//
// Reference semantics: the exported Triton v2 kernel and wrapper
// (src/unum_ops/infllm_v2/infllmv2_attn_stage1_triton_v2.py:20-228).  For token
// t of sequence b and kv group g with G = Hq/Hkv query heads:
//   s_i[j]  = scale * q[t, gG+i] . k[cu_k[b]+j, g]      (bf16 in, fp32 accumulate)
//   vis     = causal ? clamp(tdiv(lq-15,16) + Lk - tdiv(Lq-15,16), 0, Lk) : Lk
//   out[g,t,j] = sum_i softmax_{j<vis}(s_i)[j]  for j < vis, 0 elsewhere,
// and an all-zero row when vis == 0 or Lk <= 0 (the reference's NaN scrub).
//
// MFMA path (G == 16, D == 128): one wave owns one (token, group) row.  The
// 16 heads of the group are the M dimension of v_mfma_f32_16x16x32_bf16, 16
// compressed keys are N, and D = 128 is four K = 32 steps; the query fragment
// stays in registers for the whole row.  In the 16x16 accumulator layout lane
// l holds heads 4*(l/16)+r (r < 4) of key l%16, so
//   * per-head max / sum over keys  = in-lane over tiles, then across the 16
//     lanes of a lane group;
//   * per-key sum over heads        = in-lane over r, then across the 4 groups.
// Rows with at most kTiles*16 visible keys keep every score tile in registers
// and take the exact max before a single exp per score (one pass over K).
// Longer rows run the reference's two passes (online max/sum, then recompute
// and normalise) over register chunks of kTiles tiles.  Tiles past the causal
// limit are skipped entirely.  exp is exp2 with log2(e) folded into the scale.
#include "common.h"

namespace unum {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct Stage1Args {
  const __bf16* q;
  int64_t q_st, q_sh;
  const __bf16* k;
  int64_t k_st, k_sh;
  const int32_t* cu_q;
  const int32_t* cu_k;
  void* out;
  int64_t B, Tq, Tk;
  int32_t Hq, Hkv, G, D;
  int64_t out_cols;
  float scale_log2;  // softmax scale * log2(e)
  int32_t causal;
};

// Fused max-pool (kernels instantiated with kPool): pooled [Hkv, Tq, nb] fp32
// of each row's own scores, as max_pooling_1d_varlen computes it with block
// 64 / stride 16 and a flat row stride of out_cols.  Kept apart from
// Stage1Args so the unfused kernels do not carry its fields.
struct Stage1Pool {
  float* pooled;
  int32_t nb;
  int32_t init_blocks, local_blocks;
  int32_t write_scores;     // 0: the scores are not stored
};

__device__ __forceinline__ int32_t tdiv16(int32_t a) {  // truncating a / 16
  return a / 16;  // C++ integer division truncates toward zero
}

struct RowInfo {
  int64_t ks;  // first compressed key of the sequence
  int32_t lk;  // keys of the sequence
  int32_t vis; // visible keys of this token
};

// Sequence lookup for token t (wave-uniform): one vector load of cu_q and a
// ballot.  Returns vis = 0 when the row must be all zero.
__device__ __forceinline__ RowInfo row_info(const Stage1Args& a, int64_t t) {
  const int lane = threadIdx.x & (kWave - 1);
  int count = 0;
  for (int64_t base = 0; base <= a.B; base += kWave) {
    const int64_t i = base + lane;
    const bool le = (i <= a.B) && (a.cu_q[i] <= t);
    count += __popcll(__ballot(le));
  }
  RowInfo r{0, 0, 0};
  const int b = count - 1;
  if (b < 0 || b >= a.B) return r;
  const int32_t qs = a.cu_q[b], qe = a.cu_q[b + 1];
  if (t >= qe) return r;
  const int32_t ks = a.cu_k[b], ke = a.cu_k[b + 1];
  const int32_t lk = ke - ks;
  if (lk <= 0) return r;
  int32_t vis = lk;
  if (a.causal) {
    const int32_t lq = static_cast<int32_t>(t) - qs;
    const int32_t Lq = qe - qs;
    vis = tdiv16(lq - 15) + lk - tdiv16(Lq - 16 + 1);
    vis = vis < 0 ? 0 : (vis > lk ? lk : vis);
  }
  // Keys at or past the output's columns are dropped (in no denominator), as
  // on every other path.
  vis = vis < a.out_cols ? vis : static_cast<int32_t>(a.out_cols);
  r.ks = ks;
  r.lk = lk;
  r.vis = vis;
  return r;
}

// Keys of a sequence (first key ks, lk keys) that a buffer descriptor may
// cover: none when ks is negative, never past the end of k, and at most
// out_cols -- the columns past it are not computed, and the cap keeps the
// descriptor's byte range ((keys-1)*k_st + D)*2 inside 32 bits on every path
// that checks (out_cols + chunk)*k_st*2 < 2^31.  Whatever cu_seqlens_k holds,
// no load reads outside k.
__device__ __forceinline__ int64_t readable_keys(const Stage1Args& a, int64_t ks, int64_t lk) {
  if (ks < 0 || ks >= a.Tk) return 0;
  int64_t n = lk < a.Tk - ks ? lk : a.Tk - ks;
  n = n < a.out_cols ? n : a.out_cols;
  return n > 0 ? n : 0;
}

// Score stores are non-temporal: nothing re-reads the rows, and keeping them
// out of the caches measured about 6% faster on the prefill shape.
template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) {
  __builtin_nontemporal_store(v, p);
}
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* p, float v) {
  __builtin_nontemporal_store(f32_to_bf16_bits(v), p);
}

// Zero [from, out_cols) of a row; lanes write consecutive elements.
template <typename OutT>
__device__ __forceinline__ void zero_tail(OutT* orow, int64_t from, int64_t out_cols,
                                          int lane = threadIdx.x & (kWave - 1)) {
  for (int64_t j = from + lane; j < out_cols; j += kWave) store_out<OutT>(orow + j, 0.f);
}

__device__ __forceinline__ float wave_max16(float v) {  // over the 16 lanes of a group
  v = fmaxf(v, __shfl_xor(v, 1));
  v = fmaxf(v, __shfl_xor(v, 2));
  v = fmaxf(v, __shfl_xor(v, 4));
  v = fmaxf(v, __shfl_xor(v, 8));
  return v;
}
__device__ __forceinline__ float wave_sum16(float v) {
  v += __shfl_xor(v, 1);
  v += __shfl_xor(v, 2);
  v += __shfl_xor(v, 4);
  v += __shfl_xor(v, 8);
  return v;
}
__device__ __forceinline__ float group_sum4(float v) {  // across the 4 lane groups
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Raw buffer resources: loads past `bytes` read 0 and stores past it are
// dropped by the hardware range check.
constexpr uint32_t kBufferFlags = 0x00020000;  // gfx9 raw buffer resource word 3

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           static_cast<int>(kBufferFlags));
}
constexpr int kDropOffset = 0x7fffffff;  // an offset past every range: the store is dropped
constexpr int kStoreNT = 2;              // buffer store cache policy: non-temporal

// Buffer stores take every offset in the vector operand: the hardware range
// check covers it, not the scalar offset.  Row stores use one descriptor per
// row, so the range also stops a row's last chunk at the row end.
template <typename OutT>
__device__ __forceinline__ void buffer_store_out(__amdgpu_buffer_rsrc_t r, int off, float v) {
  if constexpr (sizeof(OutT) == 4) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kStoreNT);
  } else {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v), r, off, 0, kStoreNT);
  }
}

// Fused max-pool of one 64-key quad of a row's scores (lane = key - key0):
// block n = key0/4 + lane/4 takes the taps 4n-1 .. 4n+3 that lie below lk
// (the -1 tap is the previous quad's last key, `carry`); +inf when forced
// (n < init_blocks or n <= ob <= n + local_blocks), -inf when no tap is
// present -- max_pooling_1d_varlen with block 64 / stride 16.  Lanes 4i store
// block i (nothing is stored when `drop`); `carry` becomes this quad's last tap.
__device__ __forceinline__ void pool_quad(const Stage1Pool& a, __amdgpu_buffer_rsrc_t prs,
                                          int32_t key0, int32_t lk, int32_t ob, float o,
                                          float& carry, bool drop,
                                          int lane = threadIdx.x & (kWave - 1)) {
  const float x = key0 + lane < lk ? o : -INFINITY;
  float m = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)));
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
  const float left = wave_shr1(x, carry);
  const int32_t n = (key0 >> 2) + (lane >> 2);
  const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
  const float blk = force ? INFINITY : fmaxf(m, left);
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(blk), prs,
                                        (lane & 3) == 0 && !drop ? n * 4 : kDropOffset, 0, kStoreNT);
  carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), kWave - 1));
}

// Pooled blocks past the computed columns (first = the first such block,
// 4*first the first column not computed): those columns hold zero scores
// below lk (keys the row does not see), so a block with a tap there pools to
// at least 0; the first block's tap 4*first-1 is the last computed column,
// `carry` (-inf at or past lk).  A block with no tap below lk is -inf.
__device__ __forceinline__ void pool_tail(const Stage1Pool& a, __amdgpu_buffer_rsrc_t prs,
                                          int32_t first, int32_t lk, int32_t ob, float carry,
                                          int lane = threadIdx.x & (kWave - 1)) {
  for (int64_t n = first + lane; n < a.nb; n += kWave) {
    const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
    const bool zero_tap = n == first ? 4 * n < lk : 4 * n - 1 < lk;
    const float v = fmaxf(n == first ? carry : -INFINITY, zero_tap ? 0.f : -INFINITY);
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(force ? INFINITY : v), prs,
                                          static_cast<int>(n * 4), 0, kStoreNT);
  }
}



// The LDS-resident kernel pools a row's quads into its wave's LDS slot of
// blocks (lanes 4i of quad qd write block 16qd + i) and stores the row's
// pooled blocks at the end, each store a run of 64 consecutive blocks (256
// bytes): the quads' own 64-byte stores, half a 128-byte line each, wrote
// back about 1.4 times the pooled bytes.  `row` is the wave's slot (LDS
// writes and reads of one wave complete in order, so no barrier is needed).
__device__ __forceinline__ void pool_quad_lds(const Stage1Pool& a, float* row, int32_t key0,
                                              int32_t lk, int32_t ob, float o, float& carry,
                                              int lane) {
  const float x = key0 + lane < lk ? o : -INFINITY;
  float m = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)));
  m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
  const float left = wave_shr1(x, carry);
  const int32_t n = (key0 >> 2) + (lane >> 2);
  const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
  if ((lane & 3) == 0) row[n] = force ? INFINITY : fmaxf(m, left);
  carry = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), kWave - 1));
}

// Blocks [first, end) of the slot for quads whose scores are all zero
// (past the row's visible keys): block n takes its taps from zero columns,
// present below lk, and the first block its -1 tap from the last computed
// column, `carry` -- the values pool_quad_lds gives such quads, without their
// lane moves.
__device__ __forceinline__ void pool_zero_lds(const Stage1Pool& a, float* row, int32_t first,
                                              int32_t end, int32_t lk, int32_t ob, float carry,
                                              int lane) {
  for (int32_t n = first + lane; n < end; n += kWave) {
    const bool force = n < a.init_blocks || (ob >= n && ob <= n + a.local_blocks);
    const bool zero_tap = n == first ? 4 * n < lk : 4 * n - 1 < lk;
    const float v = fmaxf(n == first ? carry : -INFINITY, zero_tap ? 0.f : -INFINITY);
    row[n] = force ? INFINITY : v;
  }
}

// Blocks [0, nblk) of the slot to the pooled row (the descriptor's range
// drops blocks at or past the row's nb).
__device__ __forceinline__ void pool_flush_lds(__amdgpu_buffer_rsrc_t prs, const float* row,
                                               int32_t nblk, int lane) {
  for (int32_t j = lane; j < nblk; j += kWave)
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(row[j]), prs, j * 4, 0, kStoreNT);
}

// Pooled row of a token outside every sequence: no taps, block of the token 0.
__device__ __forceinline__ void orphan_pool_row(const Stage1Pool& p, int64_t row,
                                                int lane = threadIdx.x & (kWave - 1)) {
  pool_tail(p, make_rsrc(p.pooled + row * p.nb, static_cast<uint32_t>(p.nb * 4)), 0, 0, 0, -INFINITY,
            lane);
}

// ---------------------------------------------------------------- MFMA path
constexpr int kD = 128;      // head dim of the MFMA path
constexpr int kG = 16;       // heads per group of the MFMA path
constexpr int kTiles = 32;   // 16-key tiles held in registers (512 keys)

struct Frag {
  bf16x8 v[kD / 32];
};

__device__ __forceinline__ Frag load_q_frag(const Stage1Args& a, int64_t t, int g,
                                            int lane = threadIdx.x & (kWave - 1)) {
  const __bf16* p = a.q + t * a.q_st + static_cast<int64_t>(g * kG + (lane & 15)) * a.q_sh +
                    8 * (lane >> 4);
  Frag f;
#pragma unroll
  for (int c = 0; c < kD / 32; ++c) f.v[c] = *reinterpret_cast<const bf16x8*>(p + 32 * c);
  return f;
}

// Whether key j of a sequence whose first key is row ks of k is read: the
// rule of every path (the buffer-descriptor paths through readable_keys) --
// a sequence starting outside [0, Tk) reads no key, and keys at rows past
// the end of k read none; a key not read scores as a zero key.
__device__ __forceinline__ bool key_inside(const Stage1Args& a, int64_t ks, int64_t j) {
  return ks >= 0 && ks < a.Tk && ks + j < a.Tk;
}

// Score tile: keys [16*jt, 16*jt+16) of the sequence (clamped to stay in the
// sequence; masked by the caller).  Returns raw q.k (fp32).
__device__ __forceinline__ f32x4 score_tile(const Stage1Args& a, const Frag& qf,
                                            const RowInfo& ri, int g, int jt) {
  const int lane = threadIdx.x & (kWave - 1);
  int32_t j = 16 * jt + (lane & 15);
  j = j < ri.lk ? j : ri.lk - 1;
  const bool inside = key_inside(a, ri.ks, j);
  const int64_t row = inside ? ri.ks + j : 0;  // never read outside k, whatever cu_seqlens_k holds
  const __bf16* p = a.k + row * a.k_st + static_cast<int64_t>(g) * a.k_sh + 8 * (lane >> 4);
  bf16x8 kb[kD / 32];
#pragma unroll
  for (int c = 0; c < kD / 32; ++c) {
    const i32x4 v = *reinterpret_cast<const i32x4*>(p + 32 * c);
    kb[c] = __builtin_bit_cast(bf16x8, inside ? v : i32x4{0, 0, 0, 0});
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < kD / 32; ++c)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf.v[c], kb[c], acc, 0, 0, 0);
  return acc;
}

// Scale into the log2 domain and mask keys >= vis of tile jt to -inf.
__device__ __forceinline__ f32x4 scale_mask(f32x4 s, float c, int jt, int32_t vis) {
  const int lane = threadIdx.x & (kWave - 1);
  const bool ok = 16 * jt + (lane & 15) < vis;
  f32x4 r;
  r.x = ok ? s.x * c : -INFINITY;
  r.y = ok ? s.y * c : -INFINITY;
  r.z = ok ? s.z * c : -INFINITY;
  r.w = ok ? s.w * c : -INFINITY;
  return r;
}

template <typename OutT>
__global__ __launch_bounds__(256) void stage1_mfma_kernel(Stage1Args a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int g = blockIdx.y;
  if (t >= a.Tq) return;  // wave-uniform
  OutT* orow = static_cast<OutT*>(a.out) + (static_cast<int64_t>(g) * a.Tq + t) * a.out_cols;
  const RowInfo ri = row_info(a, t);
  if (ri.vis <= 0) {
    zero_tail<OutT>(orow, 0, a.out_cols);
    return;
  }
  const Frag qf = load_q_frag(a, t, g);
  const float c = a.scale_log2;
  const int nt = (ri.vis + 15) >> 4;   // visible tiles
  const int grp = lane >> 4;

  if (nt <= kTiles) {
    // ---- one pass: all visible tiles in registers
    f32x4 s[kTiles];
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int jt = 0; jt < kTiles; ++jt) {
      if (jt < nt) {
        s[jt] = scale_mask(score_tile(a, qf, ri, g, jt), c, jt, ri.vis);
        m[0] = fmaxf(m[0], s[jt].x);
        m[1] = fmaxf(m[1], s[jt].y);
        m[2] = fmaxf(m[2], s[jt].z);
        m[3] = fmaxf(m[3], s[jt].w);
      }
    }
    float l[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m[r] = wave_max16(m[r]);
      l[r] = 0.f;
    }
#pragma unroll
    for (int jt = 0; jt < kTiles; ++jt) {
      if (jt < nt) {
        s[jt].x = __builtin_amdgcn_exp2f(s[jt].x - m[0]);
        s[jt].y = __builtin_amdgcn_exp2f(s[jt].y - m[1]);
        s[jt].z = __builtin_amdgcn_exp2f(s[jt].z - m[2]);
        s[jt].w = __builtin_amdgcn_exp2f(s[jt].w - m[3]);
        l[0] += s[jt].x;
        l[1] += s[jt].y;
        l[2] += s[jt].z;
        l[3] += s[jt].w;
      }
    }
    float inv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) inv[r] = 1.f / wave_sum16(l[r]);
    const int nq = (nt + 3) >> 2;  // runs of 4 tiles
#pragma unroll
    for (int qd = 0; qd < kTiles / 4; ++qd) {
      if (qd < nq) {
        float mine = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int jt = 4 * qd + u;
          float o = 0.f;
          if (jt < nt) {
            o = group_sum4(s[jt].x * inv[0] + s[jt].y * inv[1] + s[jt].z * inv[2] +
                           s[jt].w * inv[3]);
          }
          mine = (grp == u) ? o : mine;
        }
        const int64_t j = 64 * qd + lane;
        if (j < a.out_cols) store_out<OutT>(orow + j, mine);
      }
    }
    zero_tail<OutT>(orow, 64 * static_cast<int64_t>(nq), a.out_cols);
    return;
  }

  // ---- two passes over register chunks of kTiles tiles
  float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  float l[4] = {0.f, 0.f, 0.f, 0.f};
  for (int base = 0; base < nt; base += kTiles) {
    f32x4 s[kTiles];
    float cm[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
      const int jt = base + u;
      if (jt < nt) {
        s[u] = scale_mask(score_tile(a, qf, ri, g, jt), c, jt, ri.vis);
        cm[0] = fmaxf(cm[0], s[u].x);
        cm[1] = fmaxf(cm[1], s[u].y);
        cm[2] = fmaxf(cm[2], s[u].z);
        cm[3] = fmaxf(cm[3], s[u].w);
      }
    }
    float nm[4], sub[4], add[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      nm[r] = fmaxf(m[r], cm[r]);
      sub[r] = (nm[r] == -INFINITY) ? 0.f : nm[r];  // all keys so far masked: exps are 0
      add[r] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < kTiles; ++u) {
      const int jt = base + u;
      if (jt < nt) {
        add[0] += __builtin_amdgcn_exp2f(s[u].x - sub[0]);
        add[1] += __builtin_amdgcn_exp2f(s[u].y - sub[1]);
        add[2] += __builtin_amdgcn_exp2f(s[u].z - sub[2]);
        add[3] += __builtin_amdgcn_exp2f(s[u].w - sub[3]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // A lane whose keys so far are all masked keeps m = -inf, l = 0.
      const float scale_old = (m[r] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m[r] - nm[r]);
      l[r] = l[r] * scale_old + add[r];
      m[r] = nm[r];
    }
  }
  // Combine the per-lane partial stats across the 16 lanes of a group.
  float bias[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float M = wave_max16(m[r]);
    const float part = (m[r] == -INFINITY) ? 0.f : l[r] * __builtin_amdgcn_exp2f(m[r] - M);
    const float L = wave_sum16(part);
    bias[r] = M + __log2f(L);  // p = exp2(s - bias)
  }
  for (int base = 0; base < nt; base += kTiles) {
    const int nq = (((nt - base) < kTiles ? (nt - base) : kTiles) + 3) >> 2;
#pragma unroll
    for (int qd = 0; qd < kTiles / 4; ++qd) {
      if (qd < nq) {
        float mine = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int jt = base + 4 * qd + u;
          float o = 0.f;
          if (jt < nt) {
            const f32x4 sv = scale_mask(score_tile(a, qf, ri, g, jt), c, jt, ri.vis);
            o = group_sum4(__builtin_amdgcn_exp2f(sv.x - bias[0]) +
                           __builtin_amdgcn_exp2f(sv.y - bias[1]) +
                           __builtin_amdgcn_exp2f(sv.z - bias[2]) +
                           __builtin_amdgcn_exp2f(sv.w - bias[3]));
          }
          mine = (grp == u) ? o : mine;
        }
        const int64_t j = 16 * static_cast<int64_t>(base) + 64 * qd + lane;
        if (j < a.out_cols) store_out<OutT>(orow + j, mine);
      }
    }
  }
  zero_tail<OutT>(orow, 64 * static_cast<int64_t>((nt + 3) >> 2), a.out_cols);
}

// ------------------------------------------------------------- generic path
// Any G and D: one wave per (token, group); q of the group staged in LDS as
// fp32; lanes stride over keys; per-head stats are reduced across the wave.
template <typename OutT>
__global__ __launch_bounds__(64) void stage1_generic_kernel(Stage1Args a) {
  extern __shared__ float smem[];  // q[G*D] then stats[2*G]
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x;
  const int g = blockIdx.y;
  const int G = a.G, D = a.D;
  OutT* orow = static_cast<OutT*>(a.out) + (static_cast<int64_t>(g) * a.Tq + t) * a.out_cols;
  const RowInfo ri = row_info(a, t);
  if (ri.vis <= 0) {
    zero_tail<OutT>(orow, 0, a.out_cols);
    return;
  }
  float* qs = smem;
  float* st = smem + G * D;
  for (int i = lane; i < G * D; i += kWave) {
    const int h = i / D, d = i - h * D;
    qs[i] = static_cast<float>(a.q[t * a.q_st + static_cast<int64_t>(g * G + h) * a.q_sh + d]);
  }
  __syncthreads();
  const float c = a.scale_log2;
  auto score = [&](int h, int32_t j) -> float {
    if (!key_inside(a, ri.ks, j)) return 0.f;  // a key outside k scores as a zero key
    const __bf16* kp = a.k + (ri.ks + j) * a.k_st + static_cast<int64_t>(g) * a.k_sh;
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc += qs[h * D + d] * static_cast<float>(kp[d]);
    return acc * c;
  };
  for (int h = 0; h < G; ++h) {
    float m = -INFINITY, l = 0.f;
    for (int32_t j = lane; j < ri.vis; j += kWave) {
      const float s = score(h, j);
      const float nm = fmaxf(m, s);
      l = l * ((m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - nm)) +
          __builtin_amdgcn_exp2f(s - nm);
      m = nm;
    }
    float M = m;
    for (int o = 1; o < kWave; o <<= 1) M = fmaxf(M, __shfl_xor(M, o));
    float part = (m == -INFINITY) ? 0.f : l * __builtin_amdgcn_exp2f(m - M);
    for (int o = 1; o < kWave; o <<= 1) part += __shfl_xor(part, o);
    if (lane == 0) st[h] = M + __log2f(part);
    __syncthreads();
  }
  const int32_t wr = ri.vis < a.out_cols ? ri.vis : static_cast<int32_t>(a.out_cols);
  for (int32_t j = lane; j < wr; j += kWave) {
    float o = 0.f;
    for (int h = 0; h < G; ++h) o += __builtin_amdgcn_exp2f(score(h, j) - st[h]);
    store_out<OutT>(orow + j, o);
  }
  zero_tail<OutT>(orow, wr, a.out_cols);
}

// ------------------------------- row segments, shared by the workgroup paths
// Rows (group, token) of the batch in the order sequence, group, token
// zig-zag; a workgroup's contiguous range of that order is cut into segments
// of one (sequence, group) each (or of tokens outside every sequence).  The
// LDS-resident kernel that walks them is further below.
constexpr int kLdsTiles = 32;                    // 512 keys
constexpr int kLdsUnits = kLdsTiles * 4 * kWave; // bf16x8 units: 128 KiB

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// Reductions over the 16 lanes of a lane group (one head's keys of a tile):
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float grp_max16(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}
__device__ __forceinline__ float grp_sum16(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}

enum SegKind { kSeq = 0, kOrphan = 1, kSkip = 2 };

struct Segment {
  int64_t end;   // first row after the segment
  int64_t k0;    // zig-zag position of the first row (sequence segments)
  int32_t kind;  // SegKind
  int32_t b, g;
  int32_t qs, lq_len, ks, lk;
  int64_t rlo, t0, nt_orphan;  // orphan segments: first row, first token, token count
};

// Rows are r in [0, Hkv*Tq): sequence b owns [Hkv*cu_q[b], Hkv*cu_q[b+1]),
// group-major inside; rows before Hkv*cu_q[0] / after Hkv*cu_q[B] belong to
// tokens outside every sequence (all-zero rows).
__device__ Segment find_segment(const Stage1Args& a, int64_t r, int64_t r_end,
                                int lane = threadIdx.x & (kWave - 1)) {
  int count = 0;
  for (int64_t base = 0; base <= a.B; base += kWave) {
    const int64_t i = base + lane;
    const bool le = (i <= a.B) && (static_cast<int64_t>(a.cu_q[i]) * a.Hkv <= r);
    count += __popcll(__ballot(le));
  }
  Segment s;
  s.kind = kSkip;
  s.b = -1;
  s.g = 0;
  s.k0 = 0;
  s.qs = s.lq_len = s.ks = s.lk = 0;
  s.rlo = s.t0 = 0;
  s.nt_orphan = 1;
  const int b = count - 1;
  const int64_t first = static_cast<int64_t>(a.cu_q[0]) * a.Hkv;
  const int64_t last = static_cast<int64_t>(a.cu_q[a.B]) * a.Hkv;
  if (b < 0 || r >= last || first < 0) {
    // Orphan rows: tokens [0, cu_q[0]) or [cu_q[B], Tq), group-major.
    const bool pre = b < 0;
    const int64_t tlo = pre ? 0 : a.cu_q[a.B];
    const int64_t thi = pre ? a.cu_q[0] : a.Tq;
    const int64_t rlo = pre ? 0 : last;
    const int64_t n = thi - tlo;
    s.kind = n > 0 ? kOrphan : kSkip;
    s.rlo = rlo;
    s.t0 = tlo;
    s.nt_orphan = n > 0 ? n : 1;
    const int64_t rhi = rlo + a.Hkv * s.nt_orphan;
    s.end = rhi < r_end ? rhi : r_end;
    if (s.end <= r) s.end = r + 1;
    return s;
  }
  const int32_t qs = a.cu_q[b], qe = a.cu_q[b + 1];
  const int32_t Lq = qe - qs;
  const int64_t off = r - static_cast<int64_t>(qs) * a.Hkv;
  if (Lq <= 0 || off < 0) {  // malformed cu_seqlens_q: skip one row, write nothing
    s.end = r + 1;
    return s;
  }
  s.kind = kSeq;
  s.b = b;
  s.g = static_cast<int32_t>(off / Lq);
  s.k0 = off - static_cast<int64_t>(s.g) * Lq;
  s.qs = qs;
  s.lq_len = Lq;
  s.ks = a.cu_k[b];
  s.lk = a.cu_k[b + 1] - s.ks;
  const int64_t seg_hi = static_cast<int64_t>(qs) * a.Hkv + static_cast<int64_t>(s.g + 1) * Lq;
  s.end = seg_hi < r_end ? seg_hi : r_end;
  if (s.end <= r) s.end = r + 1;
  // A sequence reaching outside [0, Tq) (malformed cu_seqlens_q) is skipped,
  // so no token indexes past q or the output.
  if (qs < 0 || qe > a.Tq) s.kind = kSkip;
  return s;
}

__device__ __forceinline__ int64_t zigzag(int64_t k, int64_t L) {
  return (k & 1) ? (L - 1 - (k >> 1)) : (k >> 1);
}

template <typename OutT>
__device__ __forceinline__ void zero_row_vec(OutT* orow, int64_t from, int64_t cols,
                                             int lane = threadIdx.x & (kWave - 1)) {
  if constexpr (sizeof(OutT) == 4) {
    if ((cols & 3) == 0 && (from & 3) == 0) {
      for (int64_t j = from + 4 * lane; j < cols; j += 4 * kWave)
        __builtin_nontemporal_store(f32x4{0.f, 0.f, 0.f, 0.f}, reinterpret_cast<f32x4*>(orow + j));
      return;
    }
  }
  zero_tail<OutT>(orow, from, cols, lane);
}

// ------------------------------------------------- pieces of the streaming path
// The tokens of each (sequence, group) cut into blocks of R, numbered
// sequence-major: sequence b owns Hkv*ceil(Lq_b/R) consecutive pieces, group-
// major inside.  A workgroup finds its piece with a wave-level prefix sum over
// cu_seqlens_q, 64 sequences per step; so no piece straddles two sequences.
// Workgroups past the last piece zero the rows of tokens outside every
// sequence.  A sequence reaching outside [0, Tq) (malformed cu_seqlens_q) has
// its pieces skipped, so no token indexes past q or the output.
constexpr int kStExtraGroups = 32;  // workgroups beyond the piece bound, for those rows

struct Piece {
  int32_t kind;        // SegKind
  int32_t b, g;
  int32_t qs, lq_len;  // the sequence's first token and length (the causal rule uses it)
  int32_t ks, lk;      // its first compressed key and key count
  int32_t t0, n;       // the piece's first token within the sequence, and its token count
  int64_t extra, n_extra;  // kOrphan: this workgroup's index among those past the pieces
};

// Grid size: Hkv*(ceil(Tq/R) + B) bounds the piece count of a well-formed batch.
__host__ __device__ inline int64_t piece_grid(int64_t Hkv, int64_t Tq, int64_t B, int R) {
  return Hkv * ((Tq + R - 1) / R + B) + kStExtraGroups;
}

__device__ Piece find_piece(const Stage1Args& a, int64_t p, int R) {
  const int lane = threadIdx.x & (kWave - 1);
  Piece s{};
  s.kind = kSkip;
  s.n = 1;
  int64_t before = 0;
  for (int64_t base = 0; base < a.B; base += kWave) {
    const int64_t b = base + lane;
    int32_t cnt = 0;
    if (b < a.B) {
      const int32_t L = a.cu_q[b + 1] - a.cu_q[b];
      cnt = L > 0 ? static_cast<int32_t>(a.Hkv) * ((L + R - 1) / R) : 0;
    }
    int32_t incl = cnt;  // inclusive prefix over the 64 lanes
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int32_t v = __shfl_up(incl, d);
      incl += lane >= d ? v : 0;
    }
    const int32_t total = __builtin_amdgcn_readfirstlane(__shfl(incl, kWave - 1));
    if (p < before + total) {
      const uint64_t m = __ballot(before + incl > p);
      const int l = static_cast<int>(__builtin_ctzll(m));
      // Wave-uniform: the values below live in scalar registers.
      const int64_t start = before + __builtin_amdgcn_readfirstlane(__shfl(incl - cnt, l));
      const int32_t bb = static_cast<int32_t>(base + l);
      const int32_t qs = a.cu_q[bb], qe = a.cu_q[bb + 1];
      const int32_t L = qe - qs, nj = (L + R - 1) / R;
      const int32_t off = static_cast<int32_t>(p - start);
      s.b = bb;
      s.g = off / nj;
      s.t0 = (off - s.g * nj) * R;
      s.n = L - s.t0 < R ? L - s.t0 : R;
      s.qs = qs;
      s.lq_len = L;
      s.ks = a.cu_k[bb];
      s.lk = a.cu_k[bb + 1] - s.ks;
      s.kind = (qs >= 0 && qe <= a.Tq) ? kSeq : kSkip;
      return s;
    }
    before += total;
  }
  s.kind = kOrphan;
  s.extra = p - before;
  s.n_extra = static_cast<int64_t>(gridDim.x) - before;
  return s;
}

// Zero the rows of tokens outside every sequence -- [0, cu_q[0]) and
// [cu_q[B], Tq), every group -- striding over the workgroups past the pieces.
template <typename OutT, bool kPool>
__device__ void zero_orphan_rows(const Stage1Args& a, const Stage1Pool& pp, const Piece& pc, int W) {
  const int wave = static_cast<int>(threadIdx.x >> 6);
  const int64_t lo = a.cu_q[0] < 0 ? 0 : (a.cu_q[0] > a.Tq ? a.Tq : a.cu_q[0]);
  int64_t hi = a.cu_q[a.B] < lo ? lo : a.cu_q[a.B];
  hi = hi > a.Tq ? a.Tq : hi;
  const int64_t n_tok = lo + (a.Tq - hi);  // tokens before lo and from hi on
  const int64_t n_rows = a.Hkv * n_tok;
  for (int64_t r = pc.extra * W + wave; r < n_rows; r += pc.n_extra * W) {
    const int64_t g = r / n_tok, i = r - g * n_tok;
    const int64_t t = i < lo ? i : hi + (i - lo);
    if (!kPool || pp.write_scores)
      zero_row_vec<OutT>(static_cast<OutT*>(a.out) + (g * a.Tq + t) * a.out_cols, 0, a.out_cols);
    if constexpr (kPool) orphan_pool_row(pp, g * a.Tq + t);
  }
}

// ------------------------------------------------------ K-streaming path
// For rows longer than the LDS-resident path holds (Kp > 512: long contexts,
// decode against a large cache).  A workgroup of W waves owns a piece of up
// to W*TW consecutive tokens of one (sequence, group); wave w computes the
// tokens TW*w .. TW*w+TW-1, so every K fragment read from LDS feeds TW score
// MFMAs.  K streams through a ring of NB LDS buffers (whole key rows per
// load, laid out as StreamRead describes), CT*16 keys at a time, loaded by
// buffer-to-LDS loads NB-1 chunks ahead of the one being computed, with one
// barrier per chunk.  Whole rows run eight waves; key splits (below) run four
// or eight with a third of the LDS, so that several workgroups share a CU
// (measured 40% faster on decode batches; eight waves measured faster on long
// rows).
//
// The reference's two passes, with the VALU work per score kept to an fma, an
// exp and one more op:
//   pass 1: l += exp2(c*s - c*mref) per (lane, head), where mref is a per-lane
//           reference taken from the first quad's exact max and moved only when
//           a quad's sum of exponentials exceeds 2^64 (the quad is then redone
//           against its exact max, so nothing overflows); the lanes' (mref, l)
//           are combined at the end into bias = c*max + log2(sum);
//   pass 2: p = exp2(c*s - bias) is already normalised; the sum over the 16
//           heads runs on the matrix core (an f16 MFMA against a 0/1 pattern)
//           and each 64-key quad is stored with one buffer store per token.
// Every quad of a streamed chunk is computed (keys past the visible range are
// masked to 0), and stores past the row are dropped by the buffer range check,
// so each chunk issues the same memory operations and waits stay exact.
constexpr float kStLimit = 18446744073709551616.f;  // 2^64
// Tokens sharing each K fragment: three (fewer LDS reads per MFMA) measured
// no faster on long rows and slower on decode batches.
constexpr int kStTokensPerWave = 2;
// Whole rows: waves per workgroup, 16-key tiles per chunk, ring depth
// (96 KiB of LDS, one workgroup per CU).
constexpr int kStWaves = 8, kStChunkTiles = 8, kStRing = 3;
// Key splits: 48 KiB of LDS and at most 168 VGPRs, so three workgroups share
// a CU.
constexpr int kStSplitWaves = 4, kStSplitTiles = 4, kStSplitRing = 3;
// Batches of long sequences (at least 16 new tokens each on average) run the
// key splits with eight waves: pieces of 16 tokens share each K chunk (cfg5
// measured 7 % faster); short ones keep four (cfg4 measured 20 % slower with
// eight: half as many pieces, fewer workgroups at once).
constexpr int kStSplitWavesWide = 8;
__host__ __device__ inline int split_waves(int64_t Tq, int64_t B) {
  return Tq >= 16 * B ? kStSplitWavesWide : kStSplitWaves;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void* lds_void_ptr;
constexpr int kDeadOffset = 0x7ffffff0;  // past every K range (< 2^31): reads zero

// Buffer-to-LDS load of chunk `ch` (keys CT*16*ch ..) of the piece's K block
// into `buf`: wave w issues the loads f = w, w+W, ... (four whole key rows
// each), each writing one 1 KiB run of LDS by one buffer_load ... lds.  Keys past the readable range, and every key of
// a chunk that is not `live` (past the piece), read as zero through the
// buffer range check, so every chunk issues the same loads.  The loads are
// issued from inline assembly: the compiler cannot tell the ring's buffers
// apart and would otherwise wait for every pending load before each LDS read
// of the chunk being computed; the kernel waits for them itself.
template <int W, int CT>
__device__ __forceinline__ void stream_dma(__amdgpu_buffer_rsrc_t kr, int64_t k_st, int ch, bool live,
                                           const bf16x8* buf, int wave) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < CT * 4 / W; ++i) {
    // Load f of the chunk: whole 256-byte rows of keys 4(f%4) .. 4(f%4)+3 of
    // tile f/4, lane l taking 16-byte piece (l%16) ^ n of key n = 4(f%4) +
    // l/16 (n counted within the tile), into units f*64 + l (see StreamRead).
    const int f = wave + i * W;
    const int n = 4 * (f & 3) + (lane >> 4);
    const int key = CT * 16 * ch + 16 * (f >> 2) + n;
    const int piece = (lane & 15) ^ n;
    const int off = live ? static_cast<int>((static_cast<int64_t>(key) * k_st + 8 * piece) * 2) : kDeadOffset;
    const int m0 = __builtin_amdgcn_readfirstlane(
        static_cast<int>(reinterpret_cast<uintptr_t>((lds_void_ptr)(buf + f * kWave))));
    // M0 holds the LDS destination; the compiler's value of M0 is restored.
    int saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\tbuffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(m0), "v"(off), "s"(kr)
        : "memory");
  }
}

// A chunk's layout in LDS: tile t (16 keys) takes units t*256 .. t*256+255,
// unit 64*(n/4) + 16*(n%4) + (P ^ n) holding the 16-byte piece P (elements
// 8P .. 8P+7) of key n of the tile.  Each load above then reads whole key
// rows (a row of one group is 256 contiguous bytes; the 64-byte pieces of
// 16 keys a fragment needs measured 2.4x slower to stream), and the MFMA B
// fragment (tile t, column block cc) -- lane L wants piece 4cc + L/16 of key
// L%16 -- reads unit t*256 + off[cc]: the 16 lanes of a read group hit 16
// distinct 16-byte bank groups.
struct StreamRead {
  int off[kD / 32];
};
__device__ __forceinline__ StreamRead stream_read_offsets() {
  const int lane = threadIdx.x & (kWave - 1);
  const int n = lane & 15;
  StreamRead r;
#pragma unroll
  for (int cc = 0; cc < kD / 32; ++cc) r.off[cc] = 64 * (n >> 2) + 16 * (n & 3) + ((4 * cc + (lane >> 4)) ^ n);
  return r;
}

// Wait until at most N of this wave's vector memory operations are pending
// (they complete in issue order), then join the workgroup barrier.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt is six bits");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

// The wait before chunk k (0-based) of a pass: the chunk's loads are done
// once at most Base + min(k, D) * S operations are pending -- the loads of
// the D-1 chunks issued after it (Base) and the S stores of each chunk
// computed since it was issued (at most D of them).
template <int Base, int S, int D>
__device__ __forceinline__ void chunk_wait(int k) {
  if constexpr (S == 0) {
    vm_wait_barrier<Base>();
  } else if constexpr (D == 0) {
    vm_wait_barrier<Base>();
  } else {
    if (k >= D)
      vm_wait_barrier<Base + D * S>();
    else
      chunk_wait<Base, S, D - 1>(k);
  }
}

// Scores of quad qd (keys 64*qd .. +63 of the chunk in `buf`) for TW tokens.
template <int TW>
__device__ __forceinline__ void stream_scores(const bf16x8* buf, int qd, const StreamRead& rd,
                                              const Frag (&qf)[TW], f32x4 (&acc)[TW][4]) {
  int qbase = qd * 16 * kWave;
  asm volatile("" : "+v"(qbase));
  const bf16x8* kq = buf + qbase;  // fragment (tile u, cc) at kq[u * 256 + rd.off[cc]]
  bf16x8 cur[4], nxt[4];
#pragma unroll
  for (int k = 0; k < TW; ++k)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[k][u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < 4; ++u) cur[u] = kq[u * 4 * kWave + rd.off[0]];
#pragma unroll
  for (int cc = 0; cc < kD / 32; ++cc) {
    if (cc + 1 < kD / 32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) nxt[u] = kq[u * 4 * kWave + rd.off[cc + 1]];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int k = 0; k < TW; ++k)
        acc[k][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf[k].v[cc], cur[u], acc[k][u], 0, 0, 0);
    if (cc + 1 < kD / 32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) cur[u] = nxt[u];
    }
  }
}

// Key splits (kSplit != 0): for rows with few tokens and many keys (decode
// against a long cache) one workgroup per 16-row piece leaves most of the
// GPU idle, so the keys are split too.  kSplit == 1 runs the first pass over
// one split (blockIdx.y) and writes each (row, head)'s log2-sum-exp of the
// split, c*max + log2(sum), to `ws`; kSplit == 2 combines a row's splits into
// the bias and runs the second pass over its split, writing that split's
// columns.  The two launches are the reference's two passes.  With the pool
// fused (second pass only), a split's first block takes its -1 tap from the
// previous split's last column: the split first computes the chunk before
// its own, storing nothing, to carry that column in.
struct Stage1Split {
  float* ws;        // [pieces][n_splits][16 rows][16 heads]
  int32_t* pieces;  // [pieces][kPieceInts]: each piece as the first pass found it
  int32_t chunks;   // 256-key chunks per split
  int32_t n_splits;
};

// A piece as stored between the two key-split launches: the first pass's
// split-0 workgroup of each piece writes what find_piece returned, and the
// second pass reads it back with one load instead of searching cu_seqlens
// again behind the first pass's traffic.
constexpr int kPieceInts = 12;

__device__ __forceinline__ void store_piece(int32_t* dst, const Piece& pc) {
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t v[kPieceInts] = {pc.kind, pc.b, pc.g, pc.qs, pc.lq_len, pc.ks, pc.lk, pc.t0, pc.n,
                                 static_cast<int32_t>(pc.extra), static_cast<int32_t>(pc.n_extra), 0};
#pragma unroll
  for (int i = 0; i < kPieceInts; ++i)
    if (lane == i) dst[i] = v[i];
}

__device__ __forceinline__ Piece load_piece(const int32_t* src) {
  const i32x4 a = *reinterpret_cast<const i32x4*>(src);
  const i32x4 b = *reinterpret_cast<const i32x4*>(src + 4);
  const i32x4 c = *reinterpret_cast<const i32x4*>(src + 8);
  Piece pc{};
  pc.kind = __builtin_amdgcn_readfirstlane(a[0]);
  pc.b = __builtin_amdgcn_readfirstlane(a[1]);
  pc.g = __builtin_amdgcn_readfirstlane(a[2]);
  pc.qs = __builtin_amdgcn_readfirstlane(a[3]);
  pc.lq_len = __builtin_amdgcn_readfirstlane(b[0]);
  pc.ks = __builtin_amdgcn_readfirstlane(b[1]);
  pc.lk = __builtin_amdgcn_readfirstlane(b[2]);
  pc.t0 = __builtin_amdgcn_readfirstlane(b[3]);
  pc.n = __builtin_amdgcn_readfirstlane(c[0]);
  pc.extra = __builtin_amdgcn_readfirstlane(c[1]);
  pc.n_extra = __builtin_amdgcn_readfirstlane(c[2]);
  return pc;
}

// Key splits: workgroup x of a split's row of workgroups runs piece
// pair_slot(x) -- pieces 2i and 2i+1 of each run of 16 go to workgroups 8
// apart, which the dispatcher, dealing workgroups to the 8 XCDs in turn,
// places on one XCD at about the same time.  With two kv groups every
// sequence's pieces start at an even index, so the two pieces of a
// (sequence, group) of 9-16 tokens stream its keys through one L2 instead of
// two (the grid's row is a multiple of 16, so this is a permutation).
__device__ __forceinline__ int64_t pair_slot(int64_t x) {
  const int64_t r = x & 15;
  return (x - r) + 2 * (r & 7) + (r >> 3);
}

template <typename OutT, int W, int TW, int CT, int NB, bool kPool, int kSplit>
__global__ __launch_bounds__(W* kWave) void stage1_stream_kernel(Stage1Args a, Stage1Pool pp,
                                                                 Stage1Split sp) {
  static_assert(!(kPool && kSplit == 1), "the first pass writes no scores to pool");
  static_assert((CT * 4) % W == 0, "every wave loads the same number of K fragments");
  static_assert(NB >= 2, "a ring of at least two chunks");
  __shared__ bf16x8 kbuf[NB][CT * 4 * kWave];
  constexpr int kAhead = NB - 1;                             // chunks in flight
  constexpr int kLoads = CT * 4 / W;                         // loads per wave and chunk
  constexpr int kStores = TW * (CT / 4) * (kPool ? 2 : 1);   // pass-2 stores per chunk
  // Wave-uniform by construction; readfirstlane lets the compiler keep the
  // per-token rows and store descriptors in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & (kWave - 1);
  const float c = a.scale_log2;  // > 0 on this path
  constexpr int R = W * TW;
  // Head-sum pattern: A row m has ones at the k-slots of the heads of tile
  // u = m/4 (tiles 0,1 in wa, tiles 2,3 in wb), so lane group u of the result
  // holds tile u's per-key head sum.
  f16x8 wa, wb;
  {
    const int m = lane & 15;
    const _Float16 one = static_cast<_Float16>(1.f), z = static_cast<_Float16>(0.f);
    const _Float16 a0 = m < 4 ? one : z, a1 = (m >= 4 && m < 8) ? one : z;
    const _Float16 b0 = (m >= 8 && m < 12) ? one : z, b1 = m >= 12 ? one : z;
    wa = f16x8{a0, a0, a0, a0, a1, a1, a1, a1};
    wb = f16x8{b0, b0, b0, b0, b1, b1, b1, b1};
  }
  const uint32_t row_bytes = static_cast<uint32_t>(a.out_cols * sizeof(OutT));
  const StreamRead rd = stream_read_offsets();

  const int split = kSplit ? static_cast<int>(blockIdx.y) : 0;
  const int64_t pid = kSplit ? pair_slot(blockIdx.x) : static_cast<int64_t>(blockIdx.x);
  constexpr int kChunkKeys = CT * 16;
  Piece sg;
  if constexpr (kSplit == 2) {
    sg = load_piece(sp.pieces + pid * kPieceInts);
  } else {
    sg = find_piece(a, pid, R);
    if (kSplit == 1 && split == 0 && threadIdx.x < kWave)
      store_piece(sp.pieces + pid * kPieceInts, sg);
  }
  if (sg.kind == kOrphan && kSplit != 1 && split == 0) zero_orphan_rows<OutT, kPool>(a, pp, sg, W);
  if (sg.kind == kSeq) {
    const int64_t n = sg.n;
    // Piece: tokens lq = t0 .. t0+n-1 of sequence b, group g (n <= R).
    int32_t lq[TW], vis[TW];
    bool own[TW];
    auto vis_of = [&](int32_t q) -> int32_t {
      int32_t v = sg.lk;
      if (a.causal) {
        v = tdiv16(q - 15) + sg.lk - tdiv16(sg.lq_len - 16 + 1);
        v = v < 0 ? 0 : (v > sg.lk ? sg.lk : v);
      }
      return v < a.out_cols ? v : static_cast<int32_t>(a.out_cols);
    };
    int32_t vis_min = INT32_MAX;
    // Wave w owns tokens TW*w .. TW*w+TW-1 of the piece: in a piece of fewer
    // than R tokens the last waves own none and skip their scores (they still
    // issue every load, barrier and -- dropped -- store, so the waits stay
    // exact).
#pragma unroll
    for (int k = 0; k < TW; ++k) {
      const int64_t i = static_cast<int64_t>(TW) * wave + k;
      own[k] = i < n;
      lq[k] = static_cast<int32_t>(sg.t0 + (own[k] ? i : n - 1));
      vis[k] = vis_of(lq[k]);
      vis_min = vis[k] < vis_min ? vis[k] : vis_min;
    }
    // Causal visibility grows with the token, so the piece's last token sees
    // the most keys.
    const int32_t kv_hi = vis_of(static_cast<int32_t>(sg.t0 + n - 1));
    const int nch = (kv_hi + kChunkKeys - 1) / kChunkKeys;
    // Chunks of this launch: all of them, or those of this key split.
    const int ch_lo = kSplit ? (split * sp.chunks < nch ? split * sp.chunks : nch) : 0;
    const int ch_hi = kSplit ? (ch_lo + sp.chunks < nch ? ch_lo + sp.chunks : nch) : nch;
    // The first chunk streamed: with the pool, a later split starts one
    // chunk early to carry in the previous split's last column.
    const int ch_first = kPool && kSplit == 2 && ch_lo > 0 && ch_hi > ch_lo ? ch_lo - 1 : ch_lo;
    // Workspace row of token k: the row it is computed for (a repeated
    // token reads the row of the one it repeats).
    const bool active = own[0];  // wave-uniform
    auto ws_row = [&](int k) -> int64_t {
      const int64_t i = own[k] ? static_cast<int64_t>(TW) * wave + k : n - 1;
      return ((pid * sp.n_splits) * R + i) * 16;
    };
    Frag qf[TW];
#pragma unroll
    for (int k = 0; k < TW; ++k) qf[k] = load_q_frag(a, sg.qs + lq[k], sg.g);

    // K block of (sequence, group): keys [0, keys_ok) are readable.
    const int64_t keys_ok = readable_keys(a, sg.ks, sg.lk);
    const __bf16* kbase = a.k + (keys_ok > 0 ? static_cast<int64_t>(sg.ks) * a.k_st : 0) +
                          static_cast<int64_t>(sg.g) * a.k_sh;
    const uint32_t k_bytes = keys_ok > 0 ? static_cast<uint32_t>(((keys_ok - 1) * a.k_st + kD) * 2) : 0u;
    const __amdgpu_buffer_rsrc_t kr = make_rsrc(kbase, k_bytes);

    float nb[TW][4];  // pass-2 bias: p = exp2(c*s + nb)
    [[maybe_unused]] float carry_out[TW];  // fused pool: each token's last tap so far
#pragma unroll
    for (int k = 0; k < TW; ++k) carry_out[k] = -INFINITY;
    for (int pass = kSplit == 2 ? 1 : 0; pass < (kSplit == 1 ? 1 : 2) && ch_hi > ch_lo; ++pass) {
      float mref[TW][4], mc[TW][4], l[TW][4];
#pragma unroll
      for (int k = 0; k < TW; ++k)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          mref[k][rr] = -INFINITY;
          mc[k][rr] = 0.f;
          l[k][rr] = 0.f;
        }
      // Per-token row descriptors: their ranges drop stores past the row
      // end, and every store of a token this wave computes but does not own
      // (and the scores when they are not wanted).
      __amdgpu_buffer_rsrc_t orsrc[TW];
      [[maybe_unused]] __amdgpu_buffer_rsrc_t prsrc[TW];
#pragma unroll
      for (int k = 0; k < TW; ++k) {
        const int64_t row = static_cast<int64_t>(sg.g) * a.Tq + sg.qs + lq[k];
        orsrc[k] = make_rsrc(static_cast<OutT*>(a.out) + row * a.out_cols,
                             own[k] && (!kPool || pp.write_scores) ? row_bytes : 0u);
        if constexpr (kPool)
          prsrc[k] = make_rsrc(pp.pooled + row * pp.nb, own[k] ? static_cast<uint32_t>(pp.nb * 4) : 0u);
      }
      __syncthreads();  // the previous user of kbuf is done
#pragma unroll
      for (int i = 0; i < kAhead; ++i)
        stream_dma<W, CT>(kr, a.k_st, ch_first + i, ch_first + i < ch_hi, kbuf[i], wave);
      if constexpr (kSplit == 2) {
        // Combine the splits' log2-sum-exps of each (row, head): lane group g
        // reads heads 4g..4g+3 of the splits that hold visible keys.
        const int64_t split_stride = static_cast<int64_t>(R) * 16;
#pragma unroll
        for (int k = 0; k < TW; ++k) {
          const int ns = (vis[k] + sp.chunks * kChunkKeys - 1) / (sp.chunks * kChunkKeys);
          const float* src = sp.ws + ws_row(k) + 4 * (lane >> 4);
          float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
          float sum[4] = {0.f, 0.f, 0.f, 0.f};
          for (int t0 = 0; t0 < ns; t0 += 4) {  // four splits' loads in flight at once
            f32x4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
              v[u] = t0 + u < ns ? *reinterpret_cast<const f32x4*>(src + (t0 + u) * split_stride)
                                 : f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float vv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) {
                const float nm = fmaxf(m[rr], vv[rr]);
                if (nm != -INFINITY) {
                  sum[rr] = sum[rr] * __builtin_amdgcn_exp2f(m[rr] - nm) +
                            __builtin_amdgcn_exp2f(vv[rr] - nm);
                  m[rr] = nm;
                }
              }
            }
          }
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            nb[k][rr] = sum[rr] > 0.f ? -(m[rr] + __builtin_amdgcn_logf(sum[rr])) : -INFINITY;
        }
      }
      // Take the queries (and split sums) here, while the first chunks load:
      // the compiler does not count the ring's loads, so its own wait for
      // them would otherwise come after the next chunk's loads are issued.
#pragma unroll
      for (int k = 0; k < TW; ++k)
        asm volatile("" : : "v"(qf[k].v[0]), "v"(qf[k].v[1]), "v"(qf[k].v[2]), "v"(qf[k].v[3]));
      for (int ch = ch_first; ch < ch_hi; ++ch) {
        const int kc = ch - ch_first;
        const bool carry_only = ch < ch_lo;  // the pool's carry chunk: nothing stored
        if (pass == 0)
          chunk_wait<(kAhead - 1) * kLoads, 0, kAhead>(kc);
        else
          chunk_wait<(kAhead - 1) * kLoads, kStores, kAhead>(kc);
        // Every wave is past chunk ch-1, whose buffer takes chunk ch+kAhead.
        stream_dma<W, CT>(kr, a.k_st, ch + kAhead, ch + kAhead < ch_hi, kbuf[(kc + kAhead) % NB], wave);
        const bf16x8* buf = kbuf[kc % NB];
#pragma unroll
        for (int qd = 0; qd < CT / 4; ++qd) {
          f32x4 acc[TW][4];
          if (active) stream_scores<TW>(buf, qd, rd, qf, acc);
          const int key0 = kChunkKeys * ch + 64 * qd;  // first key of the quad
          const bool masked = key0 + 64 > vis_min;              // wave-uniform
          if (pass == 0 && active) {
            if (masked) {
#pragma unroll
              for (int k = 0; k < TW; ++k)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  const bool ok = key0 + 16 * u + (lane & 15) < vis[k];
                  acc[k][u].x = ok ? acc[k][u].x : -INFINITY;
                  acc[k][u].y = ok ? acc[k][u].y : -INFINITY;
                  acc[k][u].z = ok ? acc[k][u].z : -INFINITY;
                  acc[k][u].w = ok ? acc[k][u].w : -INFINITY;
                }
            }
            if (ch == ch_lo && qd == 0) {  // the reference: the first quad's exact max
#pragma unroll
              for (int k = 0; k < TW; ++k) {
                float q4[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) q4[rr] = -INFINITY;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  q4[0] = fmaxf(q4[0], acc[k][u].x);
                  q4[1] = fmaxf(q4[1], acc[k][u].y);
                  q4[2] = fmaxf(q4[2], acc[k][u].z);
                  q4[3] = fmaxf(q4[3], acc[k][u].w);
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                  mref[k][rr] = q4[rr];
                  mc[k][rr] = q4[rr] == -INFINITY ? 0.f : -c * q4[rr];
                }
              }
            }
            float le[TW][4];
            bool big = false;
#pragma unroll
            for (int k = 0; k < TW; ++k) {
              // The quad's four exponentials per (lane, head), summed as a
              // tree; one compare of the largest sum checks them all.
              float e[4][4];
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                e[u][0] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].x, c, mc[k][0]));
                e[u][1] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].y, c, mc[k][1]));
                e[u][2] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].z, c, mc[k][2]));
                e[u][3] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].w, c, mc[k][3]));
              }
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) le[k][rr] = (e[0][rr] + e[1][rr]) + (e[2][rr] + e[3][rr]);
              const float m = fmaxf(fmaxf(le[k][0], le[k][1]), fmaxf(le[k][2], le[k][3]));
              big |= !(m <= kStLimit);
            }
            if (__builtin_amdgcn_ballot_w64(big) != 0) {
              // Rare: a quad far above the reference.  Move the reference of
              // the affected (lane, head) to the quad's exact max and redo it.
#pragma unroll
              for (int k = 0; k < TW; ++k) {
                float q4[4];
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) q4[rr] = -INFINITY;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  q4[0] = fmaxf(q4[0], acc[k][u].x);
                  q4[1] = fmaxf(q4[1], acc[k][u].y);
                  q4[2] = fmaxf(q4[2], acc[k][u].z);
                  q4[3] = fmaxf(q4[3], acc[k][u].w);
                }
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                  if (!(le[k][rr] <= kStLimit)) {
                    const float nm = fmaxf(mref[k][rr], q4[rr]);
                    l[k][rr] *= __builtin_amdgcn_exp2f((mref[k][rr] - nm) * c);
                    mref[k][rr] = nm;
                    mc[k][rr] = -c * nm;
                    float e = 0.f;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                      const float sv = rr == 0 ? acc[k][u].x : rr == 1 ? acc[k][u].y
                                     : rr == 2 ? acc[k][u].z : acc[k][u].w;
                      e += __builtin_amdgcn_exp2f(__builtin_fmaf(sv, c, mc[k][rr]));
                    }
                    le[k][rr] = e;
                  }
                }
              }
            }
#pragma unroll
            for (int k = 0; k < TW; ++k)
#pragma unroll
              for (int rr = 0; rr < 4; ++rr) l[k][rr] += le[k][rr];
          } else if (pass != 0) {
#pragma unroll
            for (int k = 0; k < TW; ++k) {
              f32x4 o = {0.f, 0.f, 0.f, 0.f};
              if (active) {
                f32x4 p[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  p[u].x = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].x, c, nb[k][0]));
                  p[u].y = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].y, c, nb[k][1]));
                  p[u].z = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].z, c, nb[k][2]));
                  p[u].w = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[k][u].w, c, nb[k][3]));
                }
                if (masked) {
#pragma unroll
                  for (int u = 0; u < 4; ++u) {
                    const bool ok = key0 + 16 * u + (lane & 15) < vis[k];
                    p[u].x = ok ? p[u].x : 0.f;
                    p[u].y = ok ? p[u].y : 0.f;
                    p[u].z = ok ? p[u].z : 0.f;
                    p[u].w = ok ? p[u].w : 0.f;
                  }
                }
                // f16 packs (rounded toward zero: one instruction per pair).
                uint32_t pk[8];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  pk[2 * u] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[u].x, p[u].y));
                  pk[2 * u + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p[u].z, p[u].w));
                }
                const f16x8 b01 = __builtin_bit_cast(f16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
                const f16x8 b23 = __builtin_bit_cast(f16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
                o = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, b01, o, 0, 0, 0);
                o = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, b23, o, 0, 0, 0);
              }
              buffer_store_out<OutT>(orsrc[k],
                                     carry_only ? kDropOffset : (key0 + lane) * static_cast<int>(sizeof(OutT)),
                                     o.x);
              if constexpr (kPool)
                pool_quad(pp, prsrc[k], key0, sg.lk, lq[k] >> 6, o.x, carry_out[k], carry_only);
            }
          }
        }
      }
      if (pass == 0) {
        // Combine the lanes' (reference, sum) into the row bias.
#pragma unroll
        for (int k = 0; k < TW; ++k)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float M = grp_max16(mref[k][rr]);
            const float part = mref[k][rr] == -INFINITY ? 0.f
                               : l[k][rr] * __builtin_amdgcn_exp2f((mref[k][rr] - M) * c);
            const float L = grp_sum16(part);
            nb[k][rr] = L > 0.f ? -(M * c + __builtin_amdgcn_logf(L)) : -INFINITY;
          }
        if constexpr (kSplit == 1) {
          // This split's log2-sum-exp per (row, head): lane 16g + rr (rr < 4)
          // writes head 4g + rr -- one store per head slot, so nb stays in
          // registers (a lane-dependent pick among nb[k][0..3] would be
          // lowered to a dynamically indexed stack array).
          const int j = lane & 15;
#pragma unroll
          for (int k = 0; k < TW; ++k) {
            float* dst = sp.ws + ws_row(k) + static_cast<int64_t>(split) * R * 16 + 4 * (lane >> 4);
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const float v = nb[k][rr];  // -inf: no visible key, log2-sum-exp -inf
              if (own[k] && j == rr) dst[rr] = v == -INFINITY ? -INFINITY : -v;
            }
          }
        }
      }
    }
    // Columns past the streamed chunks (of this split's columns); the split
    // sums of rows with no visible key in a split are not written: the
    // second pass reads only the splits below a row's visible count.
#pragma unroll
    for (int k = 0; k < TW; ++k) {
      if (kSplit != 1 && own[k]) {
        const int64_t row = static_cast<int64_t>(sg.g) * a.Tq + sg.qs + lq[k];
        int64_t done = static_cast<int64_t>(nch) * kChunkKeys;
        int64_t end = a.out_cols;
        if constexpr (kSplit == 2) {
          const int64_t s0 = static_cast<int64_t>(split) * sp.chunks * kChunkKeys;
          const int64_t s1 = s0 + static_cast<int64_t>(sp.chunks) * kChunkKeys;
          done = done > s0 ? done : s0;
          end = s1 < end ? s1 : end;
        }
        if ((!kPool || pp.write_scores) && done < end)
          zero_row_vec<OutT>(static_cast<OutT*>(a.out) + row * a.out_cols, done, end);
        if constexpr (kPool) {
          // Blocks past the computed columns belong to the split whose chunks
          // end them (the first split when no chunk runs); the last computed
          // column's tap is carried only when a chunk ran.
          const bool tail_here = ch_hi > ch_lo ? ch_hi == nch : split == 0;
          if (tail_here)
            pool_tail(pp, make_rsrc(pp.pooled + row * pp.nb, static_cast<uint32_t>(pp.nb * 4)),
                      nch * kChunkKeys / 4, sg.lk, lq[k] >> 6, nch > 0 ? carry_out[k] : -INFINITY);
        }
      }
    }
  }
  // No buffer-to-LDS load may still be writing when the workgroup's LDS is
  // released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// --------------------------------------------- LDS-resident K, pipelined rows
// For sequences with at most kLdsTiles*16 = 512 compressed keys (the "32K"
// prefill shapes).  One persistent workgroup of twelve waves per CU keeps the
// whole compressed K of a (sequence, group) in LDS -- 128 KiB in MFMA
// B-fragment order, filled by buffer-to-LDS loads -- and each wave computes
// whole (token, group) rows, each row's queries loaded at its start (the
// other waves of the SIMD cover the wait).  Every row reads 16 KiB of K fragments
// from LDS per 64-key quad, and the LDS delivers more bytes per clock the
// more waves issue reads: twelve waves (three per SIMD, at most 168 VGPRs)
// measured faster than eight (which leave room for more registers) and than
// sixteen (which spill).
//
// Softmax with one exp per score: the exponentials are taken against each
// head's max over the row's first 16 keys (a reference, not the row max; the
// key holding it has exponential 1, so every per-head sum is at least 1) and
// kept in registers as f16 (rounded toward zero) until the row is done.  The
// per-head sums and the final head sum both run on the matrix core: every
// half-quad's f16 pack is multiplied by a 0/1 head selector into a per-head
// accumulator, and at the end by the heads' 1/sum weights into the output.
// Every exponential is positive, so a head's sum bounds each of its values:
// one check per row -- every head's sum at most 2^14 -- proves that no f16
// value overflowed and that every weight is a normal f16.  A row that fails
// it (a later key far above the first 16) is redone against its exact max,
// where the sums lie in [1, 512].
//
// Work split: the (group, token) rows of the batch are ordered by sequence,
// then group, then token in zig-zag order (0, L-1, 1, L-2, ...), and each
// workgroup takes one contiguous range of that order.  A range therefore
// touches one or two (sequence, group) K blocks -- loaded once -- and its
// causal work is balanced; wave w takes the row pairs (2w, 2w+1), (2w+24,
// 2w+25), ... of a segment, each pair one short and one long row.
constexpr int kRowSumLimit = 16384;  // 2^14: 1/sum is a normal f16
constexpr int kRowWaves = 12;        // 768 threads: three waves per SIMD

// K block of (sequence, group) -> LDS in fragment order (tiles [0, ntl)):
// unit ((jt*4 + cc)*64 + l) = k[ks + 16*jt + l%16][g][32*cc + 8*(l/16) .. +8].
// Keys past the sequence (or past k) read as zero through the buffer range.
template <int kWaves>
__device__ __forceinline__ void row_k_issue(const Stage1Args& a, bf16x8* kt, const Segment& sg,
                                            int ntl, int wave, int lane = threadIdx.x & (kWave - 1)) {
  int64_t keys_ok = readable_keys(a, sg.ks, sg.lk);
  keys_ok = keys_ok < 16 * ntl ? keys_ok : 16 * ntl;
  const __bf16* kb = a.k + (keys_ok > 0 ? static_cast<int64_t>(sg.ks) * a.k_st : 0) +
                     static_cast<int64_t>(sg.g) * a.k_sh;
  const uint32_t bytes = keys_ok > 0 ? static_cast<uint32_t>(((keys_ok - 1) * a.k_st + kD) * 2) : 0u;
  const __amdgpu_buffer_rsrc_t kr = make_rsrc(kb, bytes);
  for (int f = wave; f < 4 * ntl; f += kWaves) {
    const int jt = f >> 2, cc = f & 3;
    const int key = 16 * jt + (lane & 15);
    const int off = static_cast<int>((static_cast<int64_t>(key) * a.k_st + 32 * cc + 8 * (lane >> 4)) * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void_ptr)(kt + f * kWave), 16, off, 0, 0, 0);
  }
}

typedef __attribute__((address_space(3))) const bf16x8 lds_bf16x8;

// The LDS key block as seen by one lane: fragment f at lo[f*64] for f < 64
// and at hi[(f-64)*64] above, so every fragment's address is a base register
// plus an immediate below 64 KiB (the ds_read offset field).  hi is opaque
// to the compiler, which would otherwise keep one address register per
// fragment of the upper half.
struct KView {
  lds_bf16x8* lo;
  lds_bf16x8* hi;
};

__device__ __forceinline__ KView make_kview(const bf16x8* kt) {
  const int lane = threadIdx.x & (kWave - 1);
  KView v;
  v.lo = (lds_bf16x8*)(kt) + lane;  // generic -> LDS address space
  v.hi = v.lo + 64 * kWave;
  asm volatile("" : "+v"(v.hi));
  return v;
}

// Raw scores of half j (quad j/2, tiles 2(j%2) and 2(j%2)+1) of one row: the
// half's eight K fragments are read from LDS at once (they return in order,
// so each MFMA waits only for its own), then two interleaved accumulation
// chains over the four K = 32 steps.
__device__ __forceinline__ void row_half_mfma(KView kv, int j, const Frag& qf, f32x4 (&acc)[2]) {
  const int f0 = (j >> 1) * 16 + (j & 1) * 8;  // first fragment of the half
  lds_bf16x8* kq = f0 < 64 ? kv.lo + f0 * kWave : kv.hi + (f0 - 64) * kWave;  // (u, cc) at kq[(4u+cc)*64]
  bf16x8 kf[kD / 32][2];
#pragma unroll
  for (int cc = 0; cc < kD / 32; ++cc)
#pragma unroll
    for (int u = 0; u < 2; ++u) kf[cc][u] = kq[(4 * u + cc) * kWave];
#pragma unroll
  for (int u = 0; u < 2; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cc = 0; cc < kD / 32; ++cc)
#pragma unroll
    for (int u = 0; u < 2; ++u)
      acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf.v[cc], kf[cc][u], acc[u], 0, 0, 0);
}

__device__ __forceinline__ uint32_t pk_f16(float x, float y) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(x, y));
}

// Per-head max of a quad's raw scores (kMasked: over keys < vis), into m.
template <bool kMasked>
__device__ __forceinline__ void row_quad_max(const f32x4 (&sa)[2], const f32x4 (&sb)[2], int key0,
                                             int32_t vis, float (&m)[4]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const f32x4& s = t < 2 ? sa[t] : sb[t - 2];
    // key0 + 16t + lane%16 < vis, as a lane index against a scalar limit
    const bool ok = !kMasked || (lane & 15) < __builtin_amdgcn_readfirstlane(vis - key0 - 16 * t);
    m[0] = fmaxf(m[0], ok ? s.x : -INFINITY);
    m[1] = fmaxf(m[1], ok ? s.y : -INFINITY);
    m[2] = fmaxf(m[2], ok ? s.z : -INFINITY);
    m[3] = fmaxf(m[3], ok ? s.w : -INFINITY);
  }
}

// Exponentials p = exp2(c*s + mc) of half j (zeroed for keys >= vis when
// kMasked) -> pw[j/2][j%2] as the f16 pack in the B layout of the head-sum
// MFMA (tile 0's four heads, then tile 1's), and their per-head sums into
// lsum: with A = `sel` (row m has ones at the k-slots of head m in both
// tiles), D[head][n] adds the head's two values of key column n.  Summed over
// the row, lane group g holds heads 4g..4g+3 per key column; a 16-lane sum
// finishes the per-head sums.
template <bool kMasked, int kOutQ>
__device__ __forceinline__ void row_stage_exp(int j, const f32x4 (&s)[2], float c,
                                              const float (&mc)[4], int32_t vis, f16x8 sel,
                                              f16x8 (&pw)[kOutQ][2], f32x4& lsum) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t pk[4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u].x, c, mc[0]));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u].y, c, mc[1]));
    const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u].z, c, mc[2]));
    const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u].w, c, mc[3]));
    pk[2 * u] = pk_f16(p0, p1);
    pk[2 * u + 1] = pk_f16(p2, p3);
    if constexpr (kMasked) {  // the lane's key: one mask for all four heads (two packs)
      const bool ok = (lane & 15) < __builtin_amdgcn_readfirstlane(vis - 32 * j - 16 * u);
      pk[2 * u] = ok ? pk[2 * u] : 0u;
      pk[2 * u + 1] = ok ? pk[2 * u + 1] : 0u;
    }
  }
  const f16x8 v = __builtin_bit_cast(f16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
  pw[j >> 1][j & 1] = v;
  lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, v, lsum, 0, 0, 0);
}

// The exponentials of a row's visible halves (half j = keys 32j..32j+31) into
// pw, their per-head sums into lsum.  Software pipeline over halves: stage j
// issues the score MFMAs of half j and exponentiates half j-1 in one basic
// block, so the matrix core and the VALU work side by side; halves 0 and 1
// (quad 0) are exponentiated together at stage 2, after (first) the
// reference max mc is taken from quad 0 -- otherwise mc is given.  Only the
// quad holding the causal limit is masked.  Accumulators alternate between
// two register sets (quad 0 has its own).
template <int kOutQ>
__device__ __forceinline__ void row_pipeline(KView kl, const Frag& qf, int32_t vis, int nq,
                                             bool first, float c, float (&mc)[4], f16x8 sel,
                                             f16x8 (&pw)[kOutQ][2], f32x4& lsum) {
  const int nq_full = vis >> 6;  // quads with every key visible
  lsum = f32x4{0.f, 0.f, 0.f, 0.f};
  f32x4 q0a[2], q0b[2], buf[2][2];
  row_half_mfma(kl, 0, qf, q0a);
  row_half_mfma(kl, 1, qf, q0b);
  const bool m0 = nq_full < 1;  // quad 0 masked (wave-uniform)
  if (first) {
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    if (m0)
      row_quad_max<true>(q0a, q0b, 0, vis, m);
    else
      row_quad_max<false>(q0a, q0b, 0, vis, m);
#pragma unroll
    for (int r = 0; r < 4; ++r) mc[r] = -c * grp_max16(m[r]);
  }
  // stage 2: half 2 (quad 1) with the exponentials of quad 0
  if (nq > 1) {
    row_half_mfma(kl, 2, qf, buf[0]);
    row_stage_exp<false, kOutQ>(0, q0a, c, mc, vis, sel, pw, lsum);
    row_stage_exp<false, kOutQ>(1, q0b, c, mc, vis, sel, pw, lsum);
  } else {
    row_stage_exp<true, kOutQ>(0, q0a, c, mc, vis, sel, pw, lsum);
    row_stage_exp<true, kOutQ>(1, q0b, c, mc, vis, sel, pw, lsum);
  }
  // stage j >= 3: half j's MFMAs with half j-1's exponentials; the stage
  // after the last half exponentiates it alone (masked: the row ends there).
#pragma unroll
  for (int j = 3; j <= 2 * kOutQ; ++j) {
    if (j < 2 * nq) {
      row_half_mfma(kl, j, qf, buf[j & 1]);
      if (j - 1 >= 2 * nq_full)
        row_stage_exp<true, kOutQ>(j - 1, buf[(j - 1) & 1], c, mc, vis, sel, pw, lsum);
      else
        row_stage_exp<false, kOutQ>(j - 1, buf[(j - 1) & 1], c, mc, vis, sel, pw, lsum);
    } else if (j == 2 * nq) {
      row_stage_exp<true, kOutQ>(j - 1, buf[(j - 1) & 1], c, mc, vis, sel, pw, lsum);
    }
  }
}

// Normalise, sum over the 16 heads on the matrix core and store one row: for
// tiles u of a quad, B = the tile's f16 exponentials (lane (key n, group g)
// holds heads 4g..4g+3 -- the accumulator layout of the score MFMA is the B
// layout with heads as the reduction index), A = 1/sum of those heads placed
// on rows 4u..4u+3.  Two K = 32 MFMAs (tiles 0,1 then 2,3, accumulated)
// leave every lane of group u holding the output of tile u for key l%16,
// i.e. the quad's 64 outputs in lane order.  The row is written by exactly
// kOutQ 64-column stores: quads [0, nq) computed, the rest zeros.
// Fused max-pool of one row (kernels instantiated with kPool): the pooled
// row's descriptor, the sequence's key count and the token's 64-token block.
struct RowPool {
  __amdgpu_buffer_rsrc_t prs;
  int32_t lk;
  int32_t ob;
  float* slot;  // the wave's LDS slot of pooled blocks (16 * kOutQ floats)
};

template <typename OutT, int kOutQ, int N, bool kPool>
__device__ __forceinline__ void row_store(OutT* orow, const float (&L)[4], const f16x8 (&pw)[N][2],
                                          int nq, const Stage1Pool& pp, const RowPool& rp) {
  const int lane = threadIdx.x & (kWave - 1);
  f16x8 wa, wb;
  {
    // The four weights as two f16 pairs (rounded to nearest: truncation would
    // bias every row's sum low), placed whole dwords at a time: lanes of A
    // row m hold them in the slots of tile m/4.
    uint32_t wh[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) wh[r] = f32_to_f16_bits(__builtin_amdgcn_rcpf(L[r]));
    const uint32_t w01 = wh[0] | (wh[1] << 16), w23 = wh[2] | (wh[3] << 16);
    const int t = (lane & 15) >> 2;  // the tile of this lane's A row
    wa = __builtin_bit_cast(f16x8, u32x4{t == 0 ? w01 : 0u, t == 0 ? w23 : 0u,
                                         t == 1 ? w01 : 0u, t == 1 ? w23 : 0u});
    wb = __builtin_bit_cast(f16x8, u32x4{t == 2 ? w01 : 0u, t == 2 ? w23 : 0u,
                                         t == 3 ? w01 : 0u, t == 3 ? w23 : 0u});
  }
  [[maybe_unused]] float ov[kOutQ];  // fused pool: the row's outputs, pooled once pw is dead
#pragma unroll
  for (int qd = 0; qd < kOutQ; ++qd) {
    float o = 0.f;
    if (qd < N && qd < nq) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, pw[qd < N ? qd : 0][0], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, pw[qd < N ? qd : 0][1], acc, 0, 0, 0);
      o = acc.x;
    }
    if (!kPool || pp.write_scores) store_out<OutT>(orow + 64 * qd + lane, o);
    if constexpr (kPool) ov[qd] = o;
  }
  if constexpr (kPool) {
    // The quads past nq hold zero scores: pooled like the stored row.  Blocks
    // past the row's columns have no tap below lk (lk <= out_cols).  The lane
    // index is opaque here, so the pool's per-lane offsets are computed here
    // rather than hoisted out of the row loop (they would stay live across
    // every row and push its registers into spills).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    float carry = -INFINITY;
#pragma unroll
    for (int qd = 0; qd < kOutQ; ++qd)
      if (qd < N && qd < nq) pool_quad_lds(pp, rp.slot, 64 * qd, rp.lk, rp.ob, ov[qd], carry, ln);
    // The quads past nq hold zero scores.
    if (nq < kOutQ) {
      pool_zero_lds(pp, rp.slot, 16 * nq, 16 * kOutQ, rp.lk, rp.ob, carry, ln);
      carry = 64 * kOutQ - 1 < rp.lk ? 0.f : -INFINITY;
    }
    pool_flush_lds(rp.prs, rp.slot, 16 * kOutQ, ln);
    pool_tail(pp, rp.prs, 16 * kOutQ, rp.lk, rp.ob, carry, ln);
  }
}

// Per-head sums of a row from the accumulated selector MFMAs; false when one
// exceeds 2^14 (the first-tile reference was too low for f16).
__device__ __forceinline__ bool row_sums(const f32x4& lsum, float (&L)[4]) {
  const float lv[4] = {lsum.x, lsum.y, lsum.z, lsum.w};
#pragma unroll
  for (int r = 0; r < 4; ++r) L[r] = grp_sum16(lv[r]);
  // One compare of the largest sum (an overflow to inf fails it too).
  const float m = fmaxf(fmaxf(L[0], L[1]), fmaxf(L[2], L[3]));
  return __builtin_amdgcn_ballot_w64(!(m <= static_cast<float>(kRowSumLimit))) == 0;
}

// A row of exactly NQ visible quads, as one straight-line block: the scores,
// the exponentials against a per-head reference and their per-head sums,
// quad by quad (the compiler interleaves one quad's MFMAs with the previous
// quad's exponentials); only the last quad is masked.  The reference is each
// head's max over the visible keys of tile 0 (keys 0..15, one 16-lane
// reduction per head), so every per-head sum is at least the exponential of
// that key, 1.  Measured on cfg3 against the 64-key quad max (more VALU per
// row): 123-126 us against 130-132 on flat scores, 129-133 against 128-130
// with peaky keys (x8).  Key 0 alone was no faster on flat scores and 70 %
// slower on peaky ones, where a fifth of the rows fail the 2^14 check below.
// Returns false, having stored nothing, when the row needs its exact max.
template <typename OutT, int NQ, int kOutQ, bool kPool>
__device__ __forceinline__ bool row_fast(KView kl, const Frag& qf, int32_t vis, float c, f16x8 sel,
                                         OutT* orow, const Stage1Pool& pp, const RowPool& rp) {
  f16x8 pw[NQ][2];
  f32x4 lsum = {0.f, 0.f, 0.f, 0.f};
  float mc[4];
  {
    f32x4 sa[2], sb[2];
    row_half_mfma(kl, 0, qf, sa);
    row_half_mfma(kl, 1, qf, sb);
    {
      const int lane = threadIdx.x & (kWave - 1);
      // Keys of tile 0 at or past vis only exist in rows of one quad.
      const bool ok = NQ > 1 || (lane & 15) < vis;
      mc[0] = -c * grp_max16(ok ? sa[0].x : -INFINITY);
      mc[1] = -c * grp_max16(ok ? sa[0].y : -INFINITY);
      mc[2] = -c * grp_max16(ok ? sa[0].z : -INFINITY);
      mc[3] = -c * grp_max16(ok ? sa[0].w : -INFINITY);
    }
    row_stage_exp<NQ == 1, NQ>(0, sa, c, mc, vis, sel, pw, lsum);
    row_stage_exp<NQ == 1, NQ>(1, sb, c, mc, vis, sel, pw, lsum);
  }
#pragma unroll
  for (int qd = 1; qd < NQ; ++qd) {
    f32x4 sa[2], sb[2];
    if (qd == NQ - 1) {
      // The last quad: its second half only when a key of it is visible.
      const bool both = vis > 64 * qd + 32;  // wave-uniform
      row_half_mfma(kl, 2 * qd, qf, sa);
      if (both) row_half_mfma(kl, 2 * qd + 1, qf, sb);
      row_stage_exp<true, NQ>(2 * qd, sa, c, mc, vis, sel, pw, lsum);
      if (both)
        row_stage_exp<true, NQ>(2 * qd + 1, sb, c, mc, vis, sel, pw, lsum);
      else
        pw[qd][1] = f16x8{};
    } else {
      row_half_mfma(kl, 2 * qd, qf, sa);
      row_half_mfma(kl, 2 * qd + 1, qf, sb);
      row_stage_exp<false, NQ>(2 * qd, sa, c, mc, vis, sel, pw, lsum);
      row_stage_exp<false, NQ>(2 * qd + 1, sb, c, mc, vis, sel, pw, lsum);
    }
  }
  float L[4];
  if (!row_sums(lsum, L)) return false;
  row_store<OutT, kOutQ, NQ, kPool>(orow, L, pw, NQ, pp, rp);
  return true;
}

// One (token, group) row with the whole key block in LDS.  kOutQ = out_cols/64
// is a compile-time count: the row is written by exactly kOutQ 64-column
// stores (computed quads, then zeros).  A row of nq visible quads runs the
// straight-line row_fast<nq>; a row whose first-tile reference fails runs
// the general pipeline against its exact max.
template <typename OutT, int kOutQ, bool kPool>
__device__ __forceinline__ void lds_row(const Stage1Args& a, const Stage1Pool& pp, KView kl,
                                        const Segment& sg, int32_t lq, const Frag& qf, f16x8 sel,
                                        float* pslot) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(sg.g) * a.Tq + sg.qs + lq;
  OutT* orow = static_cast<OutT*>(a.out) + row * a.out_cols;
  RowPool rp{};
  if constexpr (kPool)
    rp = RowPool{make_rsrc(pp.pooled + row * pp.nb, static_cast<uint32_t>(pp.nb * 4)), sg.lk, lq >> 6,
                 pslot};
  int32_t vis = sg.lk;
  if (a.causal) {
    vis = tdiv16(lq - 15) + sg.lk - tdiv16(sg.lq_len - 16 + 1);
    vis = vis < 0 ? 0 : (vis > sg.lk ? sg.lk : vis);
  }
  vis = vis < 64 * kOutQ ? vis : 64 * kOutQ;  // keys past the output row are not written
  vis = __builtin_amdgcn_readfirstlane(vis);   // wave-uniform: scalar branches below
  const int nq = (vis + 63) >> 6;              // 64-key quads; 0 when nothing is visible
  const float c = a.scale_log2;                // > 0 on this path
  if (nq == 0) {
#pragma unroll
    for (int qd = 0; qd < kOutQ; ++qd)
      if (!kPool || pp.write_scores) store_out<OutT>(orow + 64 * qd + lane, 0.f);
    if constexpr (kPool) {
      int ln = lane;  // opaque: see row_store
      asm volatile("" : "+v"(ln));
      pool_zero_lds(pp, rp.slot, 0, 16 * kOutQ, rp.lk, rp.ob, -INFINITY, ln);
      pool_flush_lds(rp.prs, rp.slot, 16 * kOutQ, ln);
      pool_tail(pp, rp.prs, 16 * kOutQ, rp.lk, rp.ob, 64 * kOutQ - 1 < rp.lk ? 0.f : -INFINITY, ln);
    }
    return;
  }
  bool done = false;
  switch (nq) {
#define UNUM_ROW_CASE(N) \
    case N: if constexpr (N <= kOutQ) done = row_fast<OutT, N, kOutQ, kPool>(kl, qf, vis, c, sel, orow, pp, rp); break;
    UNUM_ROW_CASE(1) UNUM_ROW_CASE(2) UNUM_ROW_CASE(3) UNUM_ROW_CASE(4)
    UNUM_ROW_CASE(5) UNUM_ROW_CASE(6) UNUM_ROW_CASE(7) UNUM_ROW_CASE(8)
#undef UNUM_ROW_CASE
    default: break;
  }
  if (done) return;
  // Rare: the exact row max from a pass over the scores alone, then the
  // exponentials against it (every per-head sum then lies in [1, 512]).
  float mc[4];
  {
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int qd = 0; qd < kOutQ; ++qd) {
      if (qd < nq) {
        f32x4 sa[2], sb[2];
        row_half_mfma(kl, 2 * qd, qf, sa);
        row_half_mfma(kl, 2 * qd + 1, qf, sb);
        row_quad_max<true>(sa, sb, 64 * qd, vis, mx);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) mc[r] = -c * grp_max16(mx[r]);
  }
  f16x8 pw[kOutQ][2];
  f32x4 lsum;
  row_pipeline<kOutQ>(kl, qf, vis, nq, false, c, mc, sel, pw, lsum);
  float L[4];
  row_sums(lsum, L);
  row_store<OutT, kOutQ, kOutQ, kPool>(orow, L, pw, nq, pp, rp);
}

template <typename OutT, int kOutQ, bool kPool>
__global__ __launch_bounds__(kRowWaves* kWave) void stage1_lds_kernel(Stage1Args a, int64_t n_rows,
                                                                       Stage1Pool pp) {
  __shared__ bf16x8 kt[kLdsUnits];                             // 128 KiB
  // Fused pool: each wave's row of pooled blocks, stored whole (6 KiB).
  __shared__ float pool_slots[kPool ? kRowWaves * 16 * kOutQ : 1];
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & (kWave - 1);
  const KView kl = make_kview(kt);
  float* pslot = kPool ? pool_slots + wave * 16 * kOutQ : nullptr;
  // Per-head sum selector (A operand): row m has ones at the k-slots of head
  // m in both tiles, i.e. lane (m, g) at j with 4g + j%4 == m.
  f16x8 sel;
  {
    const int m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      sel[jj] = static_cast<_Float16>(4 * g + (jj & 3) == m ? 1.f : 0.f);
  }
  const int64_t r_begin = n_rows * blockIdx.x / gridDim.x;
  const int64_t r_end = n_rows * (blockIdx.x + 1) / gridDim.x;
  for (int64_t r = r_begin; r < r_end;) {
    // The lane index is opaque to the compiler inside each segment, so the
    // segment-level per-lane addresses (sequence lookup, K block loads,
    // query loads, orphan rows) are computed here rather than hoisted out of
    // the loop, where they stayed live across every row and spilled.
    int sl = lane;
    asm volatile("" : "+v"(sl));
    const Segment sg = find_segment(a, r, r_end, sl);
    const int64_t n = sg.end - r;
    __syncthreads();  // the previous segment is done with kt
    // Wave w takes the row pairs (2w, 2w+1), (2w+24, 2w+25), ... of the
    // segment: in zig-zag order each pair is one short and one long causal
    // row, so the waves get equal work without a shared counter.
    auto my_row = [&](int64_t j) -> int64_t { return (j >> 1) * (2 * kRowWaves) + 2 * wave + (j & 1); };
    if (sg.kind == kOrphan) {
      for (int64_t j = 0; my_row(j) < n; ++j) {
        const int64_t rel = r + my_row(j) - sg.rlo;
        const int64_t g = rel / sg.nt_orphan, t = sg.t0 + rel % sg.nt_orphan;
        if (g < a.Hkv && t < a.Tq) {
          if (!kPool || pp.write_scores)
            zero_row_vec<OutT>(static_cast<OutT*>(a.out) + (g * a.Tq + t) * a.out_cols, 0, a.out_cols,
                               sl);
          if constexpr (kPool) orphan_pool_row(pp, g * a.Tq + t, sl);
        }
      }
      r = sg.end;
      continue;
    }
    if (sg.kind != kSeq) {
      r = sg.end;
      continue;
    }
    if (sg.lk > 0) {
      int ntl = 4 * ((sg.lk + 63) >> 6);
      ntl = ntl < 4 * kOutQ ? ntl : 4 * kOutQ;
      row_k_issue<kRowWaves>(a, kt, sg, ntl, wave, sl);
    }
    const bool any = my_row(0) < n;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // kt is filled
    if (!any) {
      r = sg.end;
      continue;
    }
    // Each row's queries load at its start.  Loading the next row's a row
    // ahead (16 registers held through the row) measured the same on cfg3 and
    // 3 % slower with the fused pool, and pushed the eight-quad instances
    // into 12-52 B/lane of scratch under the 168-register cap.
    for (int64_t j = 0; my_row(j) < n; ++j) {
      const int32_t lq = static_cast<int32_t>(zigzag(sg.k0 + my_row(j), sg.lq_len));
      const Frag qf = load_q_frag(a, sg.qs + lq, sg.g, sl);
      lds_row<OutT, kOutQ, kPool>(a, pp, kl, sg, lq, qf, sel, pslot);
    }
    r = sg.end;
  }
}

// ------------------------------------------------------------- decode rows
// For batches of about one new token per sequence (decode) over rows of at
// most kDecMaxKeys keys: one workgroup of eight waves per (token, group) row,
// the waves splitting the row's visible quads evenly.  A wave loads its keys
// straight from global memory into registers (a quad's sixteen B fragments,
// the next quad's loads issued before the current quad's MFMAs) and keeps
// the row's f16 exponentials in LDS (128 KiB at most), as the resident
// kernel keeps them in registers: one pass over the keys, then the waves
// combine their per-head (reference, sum) and head-sum their exponentials
// with weights 2^(c*mref - c*max) / sum.  No token slot repeats a token and
// no workspace is needed.
constexpr int kDecWaves = 8;
constexpr int kDecMaxKeys = 4096;  // longer rows take the streaming path

struct QuadK {
  bf16x8 f[4][4];  // [16-key tile u][32-column block cc]
};

// The sixteen K fragments of quad qd (keys 64*qd ..) of this lane; keys past
// the readable range read as zero.
__device__ __forceinline__ void dec_load(__amdgpu_buffer_rsrc_t kr, int64_t k_st, int qd, QuadK& k) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int key = 64 * qd + 16 * u + (lane & 15);
      const int off = static_cast<int>((static_cast<int64_t>(key) * k_st + 32 * cc + 8 * (lane >> 4)) * 2);
      k.f[u][cc] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0));
    }
}

__device__ __forceinline__ void dec_scores(const QuadK& k, const Frag& qf, f32x4 (&acc)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int cc = 0; cc < 4; ++cc)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qf.v[cc], k.f[u][cc], acc[u], 0, 0, 0);
}

// Exponentials of quad qd of a decode row against the per-head reference mc
// (keys at or past vis zeroed), packed to f16 in the B layout of the head-sum
// MFMA (tiles 0,1 in v[0], tiles 2,3 in v[1]); their per-head sums go into
// lsum through the 0/1 head selector `sel`.
__device__ __forceinline__ void dec_exps(const f32x4 (&acc)[4], int key0, int32_t vis, float c,
                                         const float (&mc)[4], f16x8 sel, f16x8 (&v)[2],
                                         f32x4& lsum) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t pk[8];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[u].x, c, mc[0]));
    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[u].y, c, mc[1]));
    const float p2 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[u].z, c, mc[2]));
    const float p3 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[u].w, c, mc[3]));
    const bool ok = key0 + 16 * u + (lane & 15) < vis;
    pk[2 * u] = ok ? pk_f16(p0, p1) : 0u;
    pk[2 * u + 1] = ok ? pk_f16(p2, p3) : 0u;
  }
  v[0] = __builtin_bit_cast(f16x8, u32x4{pk[0], pk[1], pk[2], pk[3]});
  v[1] = __builtin_bit_cast(f16x8, u32x4{pk[4], pk[5], pk[6], pk[7]});
  lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, v[0], lsum, 0, 0, 0);
  lsum = __builtin_amdgcn_mfma_f32_16x16x32_f16(sel, v[1], lsum, 0, 0, 0);
}

// Per head of the lane's group, the masked max of quad scores (acc) into m.
__device__ __forceinline__ void dec_quad_max(const f32x4 (&acc)[4], int key0, int32_t vis,
                                             float (&m)[4]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const bool ok = key0 + 16 * u + (lane & 15) < vis;
    m[0] = fmaxf(m[0], ok ? acc[u].x : -INFINITY);
    m[1] = fmaxf(m[1], ok ? acc[u].y : -INFINITY);
    m[2] = fmaxf(m[2], ok ? acc[u].z : -INFINITY);
    m[3] = fmaxf(m[3], ok ? acc[u].w : -INFINITY);
  }
}

// One pass of a wave over its quads [q_lo, q_hi) of a decode row: the f16
// exponentials against mc into the workgroup's LDS row, their per-head sums
// into lsum.  With kFirst, mc is first taken from the wave's first quad (its
// exact max over the 16 lanes of each head, so one reference per head).
template <bool kFirst>
__device__ __forceinline__ void dec_pass(__amdgpu_buffer_rsrc_t kr, int64_t k_st, const Frag& qf,
                                         int q_lo, int q_hi, int32_t vis, float c, float (&mc)[4],
                                         f16x8 sel, f16x8 (*erow)[2 * kWave], f32x4& lsum) {
  const int lane = threadIdx.x & (kWave - 1);
  lsum = f32x4{0.f, 0.f, 0.f, 0.f};
  QuadK kc, kn;
  if (q_lo < q_hi) dec_load(kr, k_st, q_lo, kc);
  for (int qd = q_lo; qd < q_hi; ++qd) {
    if (qd + 1 < q_hi) dec_load(kr, k_st, qd + 1, kn);
    f32x4 acc[4];
    dec_scores(kc, qf, acc);
    if (kFirst && qd == q_lo) {
      float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      dec_quad_max(acc, 64 * qd, vis, m);
#pragma unroll
      for (int r = 0; r < 4; ++r) mc[r] = -c * grp_max16(m[r]);  // a quad of the row has a visible key
    }
    f16x8 v[2];
    dec_exps(acc, 64 * qd, vis, c, mc, sel, v, lsum);
    erow[qd][lane] = v[0];
    erow[qd][kWave + lane] = v[1];
    kc = kn;
  }
}

template <typename OutT>
__global__ __launch_bounds__(kDecWaves* kWave) void stage1_decode_kernel(Stage1Args a) {
  __shared__ f16x8 erow[kDecMaxKeys / 64][2 * kWave];  // the row's f16 exponentials: 128 KiB
  __shared__ float part_max[kDecWaves][kG];  // per wave and head: c * reference
  __shared__ float part_sum[kDecWaves][kG];  // the sum of exp2 against it
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & (kWave - 1);
  const float c = a.scale_log2;  // > 0 on this path
  const Piece pc = find_piece(a, blockIdx.x, 1);
  if (pc.kind == kOrphan) zero_orphan_rows<OutT, false>(a, Stage1Pool{}, pc, kDecWaves);
  if (pc.kind != kSeq) return;  // workgroup-uniform
  int32_t vis = pc.lk;
  if (a.causal) {
    vis = tdiv16(pc.t0 - 15) + pc.lk - tdiv16(pc.lq_len - 16 + 1);
    vis = vis < 0 ? 0 : (vis > pc.lk ? pc.lk : vis);
  }
  vis = vis < a.out_cols ? vis : static_cast<int32_t>(a.out_cols);
  const int nq = (vis + 63) >> 6;
  const int q_lo = nq * wave / kDecWaves, q_hi = nq * (wave + 1) / kDecWaves;
  const int64_t row = static_cast<int64_t>(pc.g) * a.Tq + pc.qs + pc.t0;
  OutT* orow = static_cast<OutT*>(a.out) + row * a.out_cols;
  // K block of (sequence, group): keys [0, keys_ok) are readable.
  const int64_t keys_ok = readable_keys(a, pc.ks, pc.lk);
  const __bf16* kbase = a.k + (keys_ok > 0 ? static_cast<int64_t>(pc.ks) * a.k_st : 0) +
                        static_cast<int64_t>(pc.g) * a.k_sh;
  const __amdgpu_buffer_rsrc_t kr =
      make_rsrc(kbase, keys_ok > 0 ? static_cast<uint32_t>(((keys_ok - 1) * a.k_st + kD) * 2) : 0u);
  const Frag qf = load_q_frag(a, pc.qs + pc.t0, pc.g);
  // Per-head sum selector (A operand): row m has ones at the k-slots of head
  // m in both tiles of a half.
  f16x8 sel;
  {
    const int m = lane & 15, g = lane >> 4;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) sel[jj] = static_cast<_Float16>(4 * g + (jj & 3) == m ? 1.f : 0.f);
  }

  // One pass over the keys: f16 exponentials against the exact max of the
  // wave's first quad, kept in LDS.  Every head's sum at most 2^14 proves
  // that no f16 value overflowed; a wave that fails it (a later key far
  // above its first quad) redoes its quads against their exact max.
  float mc[4];
  f32x4 lsum;
  dec_pass<true>(kr, a.k_st, qf, q_lo, q_hi, vis, c, mc, sel, erow, lsum);
  float L[4];
  if (q_lo < q_hi && !row_sums(lsum, L)) {
    float m[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    QuadK kc;
    for (int qd = q_lo; qd < q_hi; ++qd) {
      dec_load(kr, a.k_st, qd, kc);
      f32x4 acc[4];
      dec_scores(kc, qf, acc);
      dec_quad_max(acc, 64 * qd, vis, m);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) mc[r] = -c * grp_max16(m[r]);
    dec_pass<false>(kr, a.k_st, qf, q_lo, q_hi, vis, c, mc, sel, erow, lsum);
    row_sums(lsum, L);
  }
  // The row's per-head (max, sum) over the waves.
  if ((lane & 15) == 0) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      part_max[wave][4 * (lane >> 4) + rr] = q_lo < q_hi ? -mc[rr] : -INFINITY;
      part_sum[wave][4 * (lane >> 4) + rr] = q_lo < q_hi ? L[rr] : 0.f;
    }
  }
  __syncthreads();
  if (q_lo < q_hi) {
    // Head-sum weights of this wave's exponentials: 2^(c*mref - c*max) / sum
    // for the heads of the lane's group, placed as in the resident kernel.
    uint32_t wh[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int h = 4 * (lane >> 4) + rr;
      float Mg = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) Mg = fmaxf(Mg, part_max[w][h]);
      float Lg = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w)
        Lg += part_max[w][h] == -INFINITY ? 0.f : part_sum[w][h] * __builtin_amdgcn_exp2f(part_max[w][h] - Mg);
      wh[rr] = f32_to_f16_bits(__builtin_amdgcn_exp2f(-mc[rr] - Mg) * __builtin_amdgcn_rcpf(Lg));
    }
    const uint32_t w01 = wh[0] | (wh[1] << 16), w23 = wh[2] | (wh[3] << 16);
    const int t = (lane & 15) >> 2;  // the tile of this lane's A row
    const f16x8 wa = __builtin_bit_cast(f16x8, u32x4{t == 0 ? w01 : 0u, t == 0 ? w23 : 0u,
                                                     t == 1 ? w01 : 0u, t == 1 ? w23 : 0u});
    const f16x8 wb = __builtin_bit_cast(f16x8, u32x4{t == 2 ? w01 : 0u, t == 2 ? w23 : 0u,
                                                     t == 3 ? w01 : 0u, t == 3 ? w23 : 0u});
    const __amdgpu_buffer_rsrc_t orsrc =
        make_rsrc(orow, static_cast<uint32_t>(a.out_cols * sizeof(OutT)));
    for (int qd = q_lo; qd < q_hi; ++qd) {
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, erow[qd][lane], o, 0, 0, 0);
      o = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, erow[qd][kWave + lane], o, 0, 0, 0);
      buffer_store_out<OutT>(orsrc, (64 * qd + lane) * static_cast<int>(sizeof(OutT)), o.x);
    }
  }
  // Columns past the visible quads, spread over the waves.
  for (int64_t j = static_cast<int64_t>(nq) * 64 + threadIdx.x; j < a.out_cols; j += kDecWaves * kWave)
    store_out<OutT>(orow + j, 0.f);
}

enum Stage1Path { kPathLds, kPathStream, kPathRowMfma, kPathGeneric };

template <typename OutT>
Stage1Path stage1_path(const Stage1Args& a) {
  const bool aligned = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(a.k) & 15) == 0 && (a.q_st % 8) == 0 &&
                       (a.q_sh % 8) == 0 && (a.k_st % 8) == 0 && (a.k_sh % 8) == 0;
  const bool mfma = a.G == kG && a.D == kD && aligned;
  if (mfma && a.out_cols <= kLdsTiles * 16 && (a.out_cols % 64) == 0 && a.scale_log2 > 0.f)
    return kPathLds;
  if (mfma && a.scale_log2 > 0.f && a.k_st >= kD &&
      (a.out_cols + kStChunkTiles * 16) * a.k_st * 2 < (int64_t{1} << 31) &&
      a.out_cols * static_cast<int64_t>(sizeof(OutT)) < (int64_t{1} << 31))
    return kPathStream;
  return mfma ? kPathRowMfma : kPathGeneric;
}

// Decode batches (at most two new tokens per sequence on average, rows of at
// most kDecMaxKeys keys) run stage1_decode_kernel on the streaming path.
inline bool decode_batch(const Stage1Args& a) {
  return a.Tq <= 2 * a.B && a.out_cols <= kDecMaxKeys &&
         (a.out_cols + 64) * a.k_st * 2 < (int64_t{1} << 31) &&
         piece_grid(a.Hkv, a.Tq, a.B, 1) <= INT32_MAX;
}

// Key-split plan of the streaming path: pieces of 2W tokens (W waves of two,
// W from split_waves) times splits of `chunks` 64-key chunks, about six workgroups per CU in
// all against the piece bound (measured on decode batches: four left CUs
// idle, eight and more spent more on combining the splits; pieces of 4
// tokens measured slower);
// the workspace holds one float per (piece, split, row, head), then each
// piece's kPieceInts lookup result.  A plan of one split runs the whole-row
// kernel instead.
struct SplitPlan {
  int64_t pieces;
  int32_t chunks, n_splits;
  int64_t bytes;
};

SplitPlan split_plan(int64_t Hkv, int64_t Tq, int64_t B, int64_t out_cols) {
  const int R = split_waves(Tq, B) * kStTokensPerWave;
  constexpr int64_t kChunkKeys = kStSplitTiles * 16;
  SplitPlan p{};
  p.pieces = (piece_grid(Hkv, Tq, B, R) + 15) / 16 * 16;  // whole runs of 16 for pair_slot
  const int64_t out_chunks = (out_cols + kChunkKeys - 1) / kChunkKeys;
  const int64_t target = 6 * static_cast<int64_t>(num_cus());
  int64_t chunks = (out_chunks * p.pieces + target - 1) / target;
  chunks = chunks < 1 ? 1 : chunks;
  const int64_t n_splits = out_chunks > 0 ? (out_chunks + chunks - 1) / chunks : 0;
  p.chunks = static_cast<int32_t>(chunks);
  p.n_splits = static_cast<int32_t>(n_splits < 65535 ? n_splits : 0);
  p.bytes = p.n_splits >= 2 ? p.pieces * (p.n_splits * R * 16 * static_cast<int64_t>(sizeof(float)) +
                                          kPieceInts * static_cast<int64_t>(sizeof(int32_t)))
                            : 0;
  return p;
}

// The two key-split launches (per-split sums, then the scores -- and with
// kPool the pooled blocks -- of each split).
template <typename OutT, bool kPool>
int launch_split(const Stage1Args& a, const Stage1Pool& pp, const SplitPlan& plan, void* ws,
                 hipStream_t s) {
  constexpr int kTW = kStTokensPerWave;
  // The workspace: the split sums, then the pieces (split_plan's bytes).
  const int64_t R = split_waves(a.Tq, a.B) * kStTokensPerWave;
  float* sums = static_cast<float*>(ws);
  int32_t* pieces = reinterpret_cast<int32_t*>(sums + plan.pieces * plan.n_splits * R * 16);
  const Stage1Split sp{sums, pieces, plan.chunks, plan.n_splits};
  const dim3 grid(static_cast<unsigned>(plan.pieces), static_cast<unsigned>(plan.n_splits));
  const char* op = kPool ? "infllmv2_attn_stage1_maxpool" : "infllmv2_attn_stage1";
  if (split_waves(a.Tq, a.B) == kStSplitWavesWide) {
    constexpr int W = kStSplitWavesWide;
    hipLaunchKernelGGL((stage1_stream_kernel<OutT, W, kTW, kStSplitTiles, kStSplitRing, false, 1>),
                       grid, dim3(W * kWave), 0, s, a, pp, sp);
    const int st = check_launch(op);
    if (st != UNUM_OK) return st;
    hipLaunchKernelGGL((stage1_stream_kernel<OutT, W, kTW, kStSplitTiles, kStSplitRing, kPool, 2>),
                       grid, dim3(W * kWave), 0, s, a, pp, sp);
  } else {
    constexpr int W = kStSplitWaves;
    hipLaunchKernelGGL((stage1_stream_kernel<OutT, W, kTW, kStSplitTiles, kStSplitRing, false, 1>),
                       grid, dim3(W * kWave), 0, s, a, pp, sp);
    const int st = check_launch(op);
    if (st != UNUM_OK) return st;
    hipLaunchKernelGGL((stage1_stream_kernel<OutT, W, kTW, kStSplitTiles, kStSplitRing, kPool, 2>),
                       grid, dim3(W * kWave), 0, s, a, pp, sp);
  }
  return check_launch(op);
}

// The LDS-resident kernel: one persistent workgroup per CU, instantiated per
// output quads (out_cols / 64 of 1..8).
template <typename OutT, bool kPool>
void launch_lds(const Stage1Args& a, const Stage1Pool& pp, int64_t n_rows, hipStream_t s) {
  int64_t grid = (n_rows + kRowWaves - 1) / kRowWaves;
  const int64_t cus = num_cus();
  grid = grid < cus ? grid : cus;
  const dim3 g(static_cast<unsigned>(grid)), b(kRowWaves * kWave);
  switch (a.out_cols / 64) {
#define UNUM_LDS_CASE(N) \
    case N: hipLaunchKernelGGL((stage1_lds_kernel<OutT, N, kPool>), g, b, 0, s, a, n_rows, pp); break;
    UNUM_LDS_CASE(1) UNUM_LDS_CASE(2) UNUM_LDS_CASE(3) UNUM_LDS_CASE(4)
    UNUM_LDS_CASE(5) UNUM_LDS_CASE(6) UNUM_LDS_CASE(7)
#undef UNUM_LDS_CASE
    default: hipLaunchKernelGGL((stage1_lds_kernel<OutT, 8, kPool>), g, b, 0, s, a, n_rows, pp); break;
  }
}

template <typename OutT, bool kPool>
int launch_stage1(const Stage1Args& a, const Stage1Pool& pp, void* ws, int64_t ws_bytes,
                  hipStream_t s) {
  const Stage1Path path = stage1_path<OutT>(a);
  // The pool is fused into the K-streaming and LDS-resident kernels (the MFMA
  // paths); other shapes run the two ops.
  if (kPool && path != kPathStream && path != kPathLds)
    UNUM_FAIL(UNUM_ERR_UNSUPPORTED,
              "infllmv2_attn_stage1_maxpool: fused only on the MFMA paths: G=16, D=128, "
              "16-byte aligned q/k and a positive scale (got G=%d, D=%d, %lld columns)",
              a.G, a.D, (long long)a.out_cols);
  const int64_t n_rows = static_cast<int64_t>(a.Hkv) * a.Tq;
  if (path == kPathStream && piece_grid(a.Hkv, a.Tq, a.B, kStSplitWaves * kStTokensPerWave) > INT32_MAX)
    UNUM_FAIL(UNUM_ERR_INVALID_ARGUMENT, "infllmv2_attn_stage1: %lld tokens and %lld sequences are too many",
              (long long)a.Tq, (long long)a.B);
  if (kPool && path == kPathLds) {
    launch_lds<OutT, kPool>(a, pp, n_rows, s);
  } else if constexpr (kPool) {
    // Key splits when the caller gave the workspace they need, else whole rows.
    const SplitPlan plan = split_plan(a.Hkv, a.Tq, a.B, a.out_cols);
    if (plan.n_splits >= 2 && ws != nullptr && ws_bytes >= plan.bytes)
      return launch_split<OutT, true>(a, pp, plan, ws, s);
    constexpr int kTW = kStTokensPerWave;
    const int64_t grid = piece_grid(a.Hkv, a.Tq, a.B, kStWaves * kTW);
    hipLaunchKernelGGL((stage1_stream_kernel<OutT, kStWaves, kTW, kStChunkTiles, kStRing, true, 0>),
                       dim3(static_cast<unsigned>(grid)), dim3(kStWaves * kWave), 0, s, a, pp,
                       Stage1Split{});
  } else if (path == kPathLds) {
    launch_lds<OutT, false>(a, pp, n_rows, s);
  } else if (path == kPathStream && decode_batch(a)) {
    // Decode batches (at most two new tokens per sequence on average): one
    // workgroup per row, the waves splitting its keys.
    hipLaunchKernelGGL(stage1_decode_kernel<OutT>,
                       dim3(static_cast<unsigned>(piece_grid(a.Hkv, a.Tq, a.B, 1))),
                       dim3(kDecWaves * kWave), 0, s, a);
  } else if (path == kPathStream) {
    constexpr int kTW = kStTokensPerWave;
    const SplitPlan plan = split_plan(a.Hkv, a.Tq, a.B, a.out_cols);
    if (plan.n_splits >= 2 && ws != nullptr && ws_bytes >= plan.bytes) {
      return launch_split<OutT, false>(a, pp, plan, ws, s);
    } else {
      hipLaunchKernelGGL((stage1_stream_kernel<OutT, kStWaves, kTW, kStChunkTiles, kStRing, false, 0>),
                         dim3(static_cast<unsigned>(piece_grid(a.Hkv, a.Tq, a.B, kStWaves * kTW))),
                         dim3(kStWaves * kWave), 0, s, a, pp, Stage1Split{});
    }
  } else if (path == kPathRowMfma) {
    const dim3 grid(static_cast<unsigned>((a.Tq + 3) / 4), static_cast<unsigned>(a.Hkv));
    hipLaunchKernelGGL(stage1_mfma_kernel<OutT>, grid, dim3(256), 0, s, a);
  } else {
    const size_t lds = (static_cast<size_t>(a.G) * a.D + 2 * a.G) * sizeof(float);
    if (lds > 64 * 1024)
      UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "infllmv2_attn_stage1: G*D=%d too large", a.G * a.D);
    const dim3 grid(static_cast<unsigned>(a.Tq), static_cast<unsigned>(a.Hkv));
    hipLaunchKernelGGL(stage1_generic_kernel<OutT>, grid, dim3(64), lds, s, a);
  }
  return check_launch("infllmv2_attn_stage1");
}

}  // namespace
}  // namespace unum

extern "C" int64_t unum_infllmv2_attn_stage1_workspace_size(int64_t B, int64_t Tq, int64_t Hq,
                                                            int64_t Hkv, int64_t D,
                                                            int64_t max_seqlen_k) {
  using namespace unum;
  // Only the streaming path (G = 16, D = 128, rows over 512 keys) splits keys.
  if (Tq <= 0 || Hkv <= 0 || Hq != kG * Hkv || D != kD || max_seqlen_k <= 0) return 0;
  const int64_t out_cols = (max_seqlen_k + 127) / 128 * 128;
  if (out_cols <= kLdsTiles * 16) return 0;
  // Decode batches (Tq <= 2B, at most 4096 columns) run the one-workgroup-a-row
  // kernel in plain stage 1 and leave the workspace unused; the fused
  // stage-1 + max-pool entry splits their keys with it.
  return split_plan(Hkv, Tq, B, out_cols).bytes;
}

namespace unum {
namespace {
// Validation and argument packing shared by both entry points.
int stage1_args(Stage1Args& a, const void* q, int64_t q_stride_t, int64_t q_stride_h,
                const void* k, int64_t k_stride_t, int64_t k_stride_h,
                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, void* out, int64_t B,
                int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
                int64_t max_seqlen_k, int64_t out_cols, float scale, int32_t causal,
                const char* op) {
  UNUM_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0 && D > 0 && out_cols >= 0,
               "%s: bad sizes (B=%lld Tq=%lld Tk=%lld Hq=%lld Hkv=%lld D=%lld)", op,
               (long long)B, (long long)Tq, (long long)Tk, (long long)Hq, (long long)Hkv,
               (long long)D);
  UNUM_REQUIRE(Hq % Hkv == 0, "%s: Hq=%lld not a multiple of Hkv=%lld", op, (long long)Hq,
               (long long)Hkv);
  UNUM_REQUIRE(max_seqlen_k <= out_cols, "%s: max_seqlen_k=%lld exceeds the %lld output columns",
               op, (long long)max_seqlen_k, (long long)out_cols);
  a = Stage1Args{};
  if (Tq == 0 || out_cols == 0) return 1;  // nothing to launch
  UNUM_REQUIRE(q && k && cu_seqlens_q && cu_seqlens_k, "%s: null pointer", op);
  UNUM_REQUIRE(B >= 1, "%s: cu_seqlens must hold at least 2 entries", op);
  UNUM_REQUIRE(Tk >= 1, "%s: empty k", op);
  UNUM_REQUIRE(Tq <= INT32_MAX && Hkv <= 65535, "%s: size exceeds grid", op);
  a.q = static_cast<const __bf16*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k = static_cast<const __bf16*>(k);
  a.k_st = k_stride_t;
  a.k_sh = k_stride_h;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.out = out;
  a.B = B;
  a.Tq = Tq;
  a.Tk = Tk;
  a.Hq = (int32_t)Hq;
  a.Hkv = (int32_t)Hkv;
  a.G = (int32_t)(Hq / Hkv);
  a.D = (int32_t)D;
  a.out_cols = out_cols;
  a.scale_log2 = scale * kLog2e;
  a.causal = causal;
  return 0;
}
}  // namespace
}  // namespace unum

extern "C" int unum_infllmv2_attn_stage1(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                         const void* k, int64_t k_stride_t, int64_t k_stride_h,
                                         const int32_t* cu_seqlens_q,
                                         const int32_t* cu_seqlens_k, void* out,
                                         int32_t out_dtype, int64_t B, int64_t Tq, int64_t Tk,
                                         int64_t Hq, int64_t Hkv, int64_t D,
                                         int64_t max_seqlen_k, int64_t out_cols, float scale,
                                         int32_t causal, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
  using namespace unum;
  clear_error();
  Stage1Args a;
  const int st = stage1_args(a, q, q_stride_t, q_stride_h, k, k_stride_t, k_stride_h,
                             cu_seqlens_q, cu_seqlens_k, out, B, Tq, Tk, Hq, Hkv, D,
                             max_seqlen_k, out_cols, scale, causal, "infllmv2_attn_stage1");
  if (st != 0) return st < 0 ? st : UNUM_OK;
  UNUM_REQUIRE(out, "infllmv2_attn_stage1: null output");
  if (out_dtype != UNUM_DTYPE_F32 && out_dtype != UNUM_DTYPE_BF16)
    UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "infllmv2_attn_stage1: unsupported out dtype %d", out_dtype);
  int dev = 0;
  const int sd = launch_device(stream, "infllmv2_attn_stage1", &dev);
  if (sd != UNUM_OK) return sd;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == UNUM_DTYPE_F32)
    return launch_stage1<float, false>(a, Stage1Pool{}, workspace, workspace_bytes, s);
  return launch_stage1<uint16_t, false>(a, Stage1Pool{}, workspace, workspace_bytes, s);
}

extern "C" int unum_infllmv2_attn_stage1_maxpool(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
    int64_t k_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, void* scores,
    float* pooled, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
    int64_t max_seqlen_k, int64_t out_cols, float scale, int32_t causal, int64_t num_blocks,
    int32_t local_blocks, int32_t init_blocks, void* workspace, int64_t workspace_bytes,
    void* stream) {
  using namespace unum;
  clear_error();
  const char* op = "infllmv2_attn_stage1_maxpool";
  UNUM_REQUIRE(num_blocks >= 0, "%s: num_blocks=%lld", op, (long long)num_blocks);
  UNUM_REQUIRE(num_blocks <= (int64_t{1} << 28) && out_cols <= (int64_t{1} << 28),
               "%s: rows too long", op);
  Stage1Args a;
  const int st = stage1_args(a, q, q_stride_t, q_stride_h, k, k_stride_t, k_stride_h,
                             cu_seqlens_q, cu_seqlens_k, scores, B, Tq, Tk, Hq, Hkv, D,
                             max_seqlen_k, out_cols, scale, causal, op);
  if (st < 0) return st;
  if (Tq == 0 || num_blocks == 0) return UNUM_OK;
  UNUM_REQUIRE(pooled, "%s: null pooled output", op);
  UNUM_REQUIRE(out_cols > 0, "%s: out_cols must be positive", op);
  Stage1Pool pp;
  pp.pooled = pooled;
  pp.nb = static_cast<int32_t>(num_blocks);
  pp.init_blocks = init_blocks;
  pp.local_blocks = local_blocks;
  pp.write_scores = scores != nullptr;
  int dev = 0;
  const int sd = launch_device(stream, op, &dev);
  if (sd != UNUM_OK) return sd;
  return launch_stage1<float, true>(a, pp, workspace, workspace_bytes,
                                    static_cast<hipStream_t>(stream));
}

// ------------------------------------------------ stage 1 without allocation
// The key-split workspace of unum_infllmv2_attn_stage1 held in a file-scope
// device array, for callers that cannot allocate.  Each device that loads the
// library holds its own copy of the array until the process ends.  In host
// code `scratch` names a host-side stand-in: the kernels take the device
// address that hipGetSymbolAddress returns for the current device, resolved
// once per device on the first call there.
namespace unum {
namespace {
constexpr int64_t kScratchBytes = int64_t{4} << 20;  // 4 MiB per device
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device `dev`'s address of `scratch` (dev is the current device), or
// nullptr (with the error set).
void* scratch_ptr(int dev, const char* op) {
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("%s: device index %d out of range", op, dev);
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", op, dev,
              hipGetErrorString(e));
    return nullptr;
  }
  // Racing first calls on one device store the same address.
  g_scratch_ptr[dev].store(p, std::memory_order_release);
  return p;
}
}  // namespace
}  // namespace unum

extern "C" int unum_infllmv2_attn_stage1_noalloc(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k, int64_t k_stride_t,
    int64_t k_stride_h, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, void* out,
    int32_t out_dtype, int64_t B, int64_t Tq, int64_t Tk, int64_t Hq, int64_t Hkv, int64_t D,
    int64_t max_seqlen_k, int64_t out_cols, float scale, int32_t causal, void* stream) {
  using namespace unum;
  clear_error();
  const char* op = "infllmv2_attn_stage1_noalloc";
  Stage1Args a;
  const int st = stage1_args(a, q, q_stride_t, q_stride_h, k, k_stride_t, k_stride_h,
                             cu_seqlens_q, cu_seqlens_k, out, B, Tq, Tk, Hq, Hkv, D,
                             max_seqlen_k, out_cols, scale, causal, op);
  if (st != 0) return st < 0 ? st : UNUM_OK;
  UNUM_REQUIRE(out, "%s: null output", op);
  UNUM_REQUIRE(out_dtype == UNUM_DTYPE_F32 || out_dtype == UNUM_DTYPE_BF16,
               "%s: unsupported out dtype %d", op, out_dtype);
  // The workspace the plain entry point would split keys with; none for the
  // paths that do not split (rows of at most 512 keys, decode batches).
  const bool splits = out_dtype == UNUM_DTYPE_F32 ? stage1_path<float>(a) == kPathStream
                                                  : stage1_path<uint16_t>(a) == kPathStream;
  const int64_t need = splits && !decode_batch(a) ? split_plan(a.Hkv, a.Tq, a.B, a.out_cols).bytes : 0;
  if (need > kScratchBytes)
    UNUM_FAIL(UNUM_ERR_WORKSPACE,
              "%s: this problem splits its keys over %lld bytes of workspace, more than the "
              "%lld-byte device scratch array; call unum_infllmv2_attn_stage1 with a workspace",
              op, (long long)need, (long long)kScratchBytes);
  int dev = 0;
  const int sd = launch_device(stream, op, &dev);
  if (sd != UNUM_OK) return sd;
  void* ws = nullptr;
  if (need > 0) {
    ws = scratch_ptr(dev, op);
    if (ws == nullptr) return UNUM_ERR_LAUNCH;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (out_dtype == UNUM_DTYPE_F32)
    return launch_stage1<float, false>(a, Stage1Pool{}, ws, need > 0 ? kScratchBytes : 0, s);
  return launch_stage1<uint16_t, false>(a, Stage1Pool{}, ws, need > 0 ? kScratchBytes : 0, s);
}
