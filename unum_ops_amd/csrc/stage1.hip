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
  r.ks = ks;
  r.lk = lk;
  r.vis = vis;
  return r;
}

template <typename OutT>
__device__ __forceinline__ void store_out(OutT* p, float v);
template <>
__device__ __forceinline__ void store_out<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_out<uint16_t>(uint16_t* p, float v) {
  *p = f32_to_bf16_bits(v);
}

// Zero [from, out_cols) of a row; lanes write consecutive elements.
template <typename OutT>
__device__ __forceinline__ void zero_tail(OutT* orow, int64_t from, int64_t out_cols) {
  const int lane = threadIdx.x & (kWave - 1);
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

// ---------------------------------------------------------------- MFMA path
constexpr int kD = 128;      // head dim of the MFMA path
constexpr int kG = 16;       // heads per group of the MFMA path
constexpr int kTiles = 32;   // 16-key tiles held in registers (512 keys)

struct Frag {
  bf16x8 v[kD / 32];
};

__device__ __forceinline__ Frag load_q_frag(const Stage1Args& a, int64_t t, int g) {
  const int lane = threadIdx.x & (kWave - 1);
  const __bf16* p = a.q + t * a.q_st + static_cast<int64_t>(g * kG + (lane & 15)) * a.q_sh +
                    8 * (lane >> 4);
  Frag f;
#pragma unroll
  for (int c = 0; c < kD / 32; ++c) f.v[c] = *reinterpret_cast<const bf16x8*>(p + 32 * c);
  return f;
}

// Score tile: keys [16*jt, 16*jt+16) of the sequence (clamped to stay in the
// sequence; masked by the caller).  Returns raw q.k (fp32).
__device__ __forceinline__ f32x4 score_tile(const Stage1Args& a, const Frag& qf,
                                            const RowInfo& ri, int g, int jt) {
  const int lane = threadIdx.x & (kWave - 1);
  int32_t j = 16 * jt + (lane & 15);
  j = j < ri.lk ? j : ri.lk - 1;
  int64_t row = ri.ks + j;
  row = row < a.Tk ? row : a.Tk - 1;  // never read outside k, whatever cu_seqlens_k holds
  row = row < 0 ? 0 : row;
  const __bf16* p = a.k + row * a.k_st + static_cast<int64_t>(g) * a.k_sh + 8 * (lane >> 4);
  bf16x8 kb[kD / 32];
#pragma unroll
  for (int c = 0; c < kD / 32; ++c) kb[c] = *reinterpret_cast<const bf16x8*>(p + 32 * c);
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
    int64_t row = ri.ks + j;
    row = row < a.Tk ? row : a.Tk - 1;
    row = row < 0 ? 0 : row;
    const __bf16* kp = a.k + row * a.k_st + static_cast<int64_t>(g) * a.k_sh;
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

template <typename OutT>
int launch_stage1(const Stage1Args& a, hipStream_t s) {
  const bool aligned = (reinterpret_cast<uintptr_t>(a.q) & 15) == 0 &&
                       (reinterpret_cast<uintptr_t>(a.k) & 15) == 0 && (a.q_st % 8) == 0 &&
                       (a.q_sh % 8) == 0 && (a.k_st % 8) == 0 && (a.k_sh % 8) == 0;
  if (a.G == kG && a.D == kD && aligned) {
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

extern "C" int64_t unum_infllmv2_attn_stage1_workspace_size(int64_t, int64_t, int64_t,
                                                            int64_t, int64_t, int64_t) {
  return 0;
}

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
  (void)workspace;
  (void)workspace_bytes;
  clear_error();
  UNUM_REQUIRE(B >= 0 && Tq >= 0 && Tk >= 0 && Hq > 0 && Hkv > 0 && D > 0 && out_cols >= 0,
               "infllmv2_attn_stage1: bad sizes (B=%lld Tq=%lld Tk=%lld Hq=%lld Hkv=%lld D=%lld)",
               (long long)B, (long long)Tq, (long long)Tk, (long long)Hq, (long long)Hkv,
               (long long)D);
  UNUM_REQUIRE(Hq % Hkv == 0, "infllmv2_attn_stage1: Hq=%lld not a multiple of Hkv=%lld",
               (long long)Hq, (long long)Hkv);
  UNUM_REQUIRE(max_seqlen_k <= out_cols,
               "infllmv2_attn_stage1: max_seqlen_k=%lld exceeds the %lld output columns",
               (long long)max_seqlen_k, (long long)out_cols);
  if (Tq == 0 || out_cols == 0) return UNUM_OK;
  UNUM_REQUIRE(q && k && out && cu_seqlens_q && cu_seqlens_k, "infllmv2_attn_stage1: null pointer");
  UNUM_REQUIRE(B >= 1, "infllmv2_attn_stage1: cu_seqlens must hold at least 2 entries");
  UNUM_REQUIRE(Tk >= 1, "infllmv2_attn_stage1: empty k");
  UNUM_REQUIRE(Tq <= INT32_MAX && Hkv <= 65535, "infllmv2_attn_stage1: size exceeds grid");
  Stage1Args a;
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
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (out_dtype) {
    case UNUM_DTYPE_F32: return launch_stage1<float>(a, s);
    case UNUM_DTYPE_BF16: return launch_stage1<uint16_t>(a, s);
    default:
      UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "infllmv2_attn_stage1: unsupported out dtype %d", out_dtype);
  }
}
