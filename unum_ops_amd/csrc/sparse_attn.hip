// Stage-2 sparse attention over the block table's KV slots, on gfx950.
//
// For token t and kv head h (G = 16 query heads per kv head, D = 128), the
// keys are the entries (t, h, 64k + o) of get_block_table's output
// (src/unum_ops/sparse_kernel_extension/get_table_torch.py:4-44,
// get_table_triton.py:6-67): entry p = topk_idx[h, t, k]*64 + o (wrapping
// int32) is attended when 0 <= p < seqlen_q[b] and p < token_pos_in_bs[t]
// (b = token_to_bs[t] in [0, B)), and its KV row is the slot
// Hkv * block_table[b, min(p, L-1)] + h -- row `slot` of the cache viewed as
// [-1, D], i.e. token slot block_table[b, p], head h of a [num_blocks,
// block_size, Hkv, D] cache -- or, given a precomputed slot table, that
// table's entry.  Rows outside the cache are not attended.  Then
//   out[t, h*16 + i] = softmax_j(scale * q[t, h*16+i] . K[row_j]) @ V[rows]
// (0 when no entry is attended).  The reference's consumer of the table is an
// NPU paged-attention operator (test/test_pa.py:48-71); this is its
// arithmetic on the slots the table lists.
//
// One wave per (t, h).  The block ids give, with no table access, which
// 16-key stages (a quarter of a 64-entry block) can hold an attended entry:
// a quarter is live when its first position lies in [0, lim).  Each live
// stage then takes three loads in flight, kRing stages apart: the 64 bytes
// of the table that name its 16 rows, its 16 K rows and 16 V rows (8 KiB;
// ordinary loads, so the compiler's waits are exact), and its arithmetic.
// No per-entry table is kept in LDS (a wave uses a 4 KiB V buffer); the
// launch sets the LDS per workgroup to hold eight waves per CU, the
// occupancy at which the gathers, which bound the kernel, ran fastest.
// Per stage:
//   * S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (keys as M, heads as N), so a
//     lane holds four keys of one head: the online-softmax state (max, sum)
//     is one head per lane and needs no transposes;
//   * the scores are scaled before the max and the key mask, so any scale
//     (zero and negative ones too) gives the softmax of the scaled scores;
//   * P^T, as it stands in the accumulator layout, is the B operand of
//     v_mfma_f32_16x16x16_bf16 for O^T += V^T P^T, taken as two bf16 terms
//     (P to about 2^-15); the V rows go to a 4 KiB LDS buffer and come back
//     as V^T fragments through ds_read_b64_tr_b16 (transposing reads);
//   * the running max moves only when a stage's max exceeds it by more than
//     8 (log2 units), so the O^T rescale is rare; exponentials stay <= 2^8.
#include "common.h"

namespace unum {
namespace {

constexpr float kSaLog2e = 1.4426950408889634f;
constexpr int kSaD = 128;          // head dim
constexpr int kSaG = 16;           // query heads per kv head
constexpr int kSaStageKeys = 16;   // keys per pipeline stage
// Stages in flight per wave (register sets of 33 VGPRs).
constexpr int kSaRing = 3;
// LDS each workgroup (one wave) takes, the 4 KiB V buffer included: 20 KiB
// holds a CU at eight waves.  The gathers bound the kernel and their rate
// depends on how many waves share a CU's caches; measured on the cfg5 / cfg4
// selections with the gather calibration below and this kernel: 12 waves per
// CU (the register limit) 1960 / 323 us, 8 waves 1835 / 322 us, 6 waves
// 2055 / 322 us, 5 and 4 waves 1884 / 560 us.
constexpr int kSaLdsBytes = 20 * 1024;
constexpr int kSaVBytes = kSaStageKeys * kSaD * 2;  // a stage's V rows
constexpr int kSaMaxBlocks = 64;   // K <= 64 (one block id per lane)
constexpr float kSaRescale = 8.f;  // lazy-rescale threshold (log2 units)

// 256 zero bytes: the K and V "row" of every entry that is not attended, so
// each stage issues the same loads (masked keys then score 0 and carry P = 0
// against a V of zeros); also the table "entries" of a stage past the last.
__device__ __align__(256) uint32_t sa_zero_row[64];

struct SaArgs {
  const __bf16* q;
  int64_t q_st, q_sh;
  const char* kc;
  const char* vc;
  int64_t row_bytes;   // bytes between consecutive cache rows
  int64_t n_rows;      // rows of the cache viewed as [-1, D]
  const int32_t* idx;
  int64_t i_sh, i_st, i_sk;
  const int32_t* bt;   // [B, L] (fused slots), or null
  int64_t bt_sb;
  const int32_t* slots;  // [T, Hkv, K*64] slot table, or null
  const int32_t* tok_bs;
  const int32_t* pos;
  const int32_t* slen;
  int32_t pos_n, slen_n;
  void* out;           // [T, Hkv*16, 128] contiguous (u32 [T, Hkv, 64] for the gather calibration)
  int32_t T, Hkv, K, B, L;
  float c;             // softmax scale * log2(e)
};

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 sa_lds_i16x4;

// Max / sum of v over the lanes l and l^16 (l^32): v_permlane16_swap
// (v_permlane32_swap) with v in both operands returns each lane's value and
// its partner's, one in each result.
__device__ __forceinline__ float sa_max_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sa_max_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sa_sum_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sa_sum_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The selection of one (t, h): lane k holds block id k (-1 past K), the
// position limit min(seqlen_q[b], token_pos_in_bs[t]) (0 when t has no
// sequence), and the base of the table the rows come from -- the slot
// table's (t, h) row, or block_table's row b.
struct SaSel {
  int32_t lane_id;
  int32_t lim;
  int32_t h;
  const int32_t* tab;
};

// The live stages: bit k of mq set when quarter q of block k (positions
// p0 .. p0+15, p0 = id*64 + 16q wrapping int32) can hold an attended entry,
// i.e. p0 lies in [0, lim).  p0 is a multiple of 16, so p0 >= 0 puts every
// position of the quarter in [0, 2^31) and p0 < 0 puts none there.  Four
// scalar words, not an array, so that no index into them is a runtime value.
struct SaStages {
  uint64_t m0, m1, m2, m3;
};

__device__ __forceinline__ SaStages sa_live(const SaSel& sel) {
  const uint32_t base = static_cast<uint32_t>(sel.lane_id) * 64u;
  auto live = [&](uint32_t q) {
    const int32_t p0 = static_cast<int32_t>(base + 16u * q);
    return p0 >= 0 && p0 < sel.lim;
  };
  return SaStages{__ballot(live(0)), __ballot(live(1)), __ballot(live(2)), __ballot(live(3))};
}

// The next live stage, 4k + q, in ascending order (-1 if none); clears it.
__device__ __forceinline__ int sa_pop(SaStages& m) {
  const uint64_t any = m.m0 | m.m1 | m.m2 | m.m3;
  if (any == 0) return -1;
  const int k = __builtin_ctzll(any);
  const uint64_t bit = 1ull << k;
  if (m.m0 & bit) { m.m0 &= ~bit; return 4 * k; }
  if (m.m1 & bit) { m.m1 &= ~bit; return 4 * k + 1; }
  if (m.m2 & bit) { m.m2 &= ~bit; return 4 * k + 2; }
  m.m3 &= ~bit;
  return 4 * k + 3;
}

// Position of this lane's entry of stage sg (lane l: entry 16q + l%16 of
// block k), wrapping int32.
__device__ __forceinline__ int32_t sa_pos(const SaSel& sel, int sg) {
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t id = __builtin_amdgcn_readlane(sel.lane_id, sg >> 2);
  return static_cast<int32_t>(static_cast<uint32_t>(id) * 64u +
                              static_cast<uint32_t>(16 * (sg & 3) + (lane & 15)));
}

// The table entry naming this lane's row of stage sg: the slot table's
// entry, or block_table[b, min(max(p, 0), L-1)] (the clamp only matters for
// entries that are not attended or at p >= L); the zero row past the last
// stage.  One 64-byte run per stage (lanes l and l+16 read the same word).
template <bool kTable>
__device__ __forceinline__ int32_t sa_table(const SaArgs& a, const SaSel& sel, int sg) {
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t* p;
  if (sg < 0) {
    p = reinterpret_cast<const int32_t*>(sa_zero_row);
  } else if constexpr (kTable) {
    p = sel.tab + 16 * sg + (lane & 15);  // entry 64k + 16q + l%16
  } else {
    int32_t pc = sa_pos(sel, sg);
    pc = pc < 0 ? 0 : (pc > a.L - 1 ? a.L - 1 : pc);
    p = sel.tab + pc;
  }
  return *p;
}

// A stage in flight: this lane's K and V chunks of its key (lane l gathers
// key l%16, 16-byte chunks 4i + l/16, i < 4 -- for K exactly the A operand
// of the score MFMA, chunk 4cc + g of key m) and the stage's mask of
// attended keys (bit j: key j; lanes 0..15 gather keys 0..15).
struct SaStage {
  bf16x8 k[4];
  bf16x8 v[4];
  uint32_t mask;
};

// Issue the gathers of stage sg, whose table entry for this lane is `tv`
// (ordinary loads: the compiler waits for each stage's loads exactly where
// they are used).  A key that is not attended -- position at or past the
// limit, row outside the cache -- gathers the zero row, and so does every
// key when sg < 0 (no stage left): every call issues the same eight loads,
// so on every path through the ring the same number of loads follows each
// set and the compiler's wait before using a set stays a partial one.
template <bool kTable>
__device__ __forceinline__ void sa_issue(const SaArgs& a, const SaSel& sel, int sg, int32_t tv,
                                         SaStage& st) {
  const int lane = threadIdx.x & (kWave - 1);
  int32_t row = -1;
  if (sg >= 0) {
    const int32_t r = kTable ? tv
                             : static_cast<int32_t>(static_cast<uint32_t>(a.Hkv) * static_cast<uint32_t>(tv) +
                                                    static_cast<uint32_t>(sel.h));
    row = sa_pos(sel, sg) < sel.lim && r >= 0 && r < a.n_rows ? r : -1;  // the stage is live: p >= 0
  }
  const uint64_t col = static_cast<uint64_t>(16 * (lane >> 4));
  const char *kp, *vp;
  if (row >= 0) {
    const uint64_t off = static_cast<uint64_t>(row) * static_cast<uint64_t>(a.row_bytes) + col;
    kp = a.kc + off;
    vp = a.vc + off;
  } else {
    kp = vp = reinterpret_cast<const char*>(sa_zero_row) + col;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) st.k[i] = *reinterpret_cast<const bf16x8*>(kp + 64 * i);
#pragma unroll
  for (int i = 0; i < 4; ++i) st.v[i] = *reinterpret_cast<const bf16x8*>(vp + 64 * i);
  st.mask = static_cast<uint32_t>(__ballot(row >= 0) & 0xFFFFull);
}

// The (t, h) selection of this workgroup: block ids one per lane (one load,
// complete before the ring's loads are issued), the limit and the table row.
template <bool kTable>
__device__ __forceinline__ SaSel sa_select(const SaArgs& a, int t, int h) {
  const int lane = threadIdx.x & (kWave - 1);
  SaSel sel;
  sel.h = h;
  sel.lim = 0;
  sel.tab = nullptr;
  const int32_t b = a.tok_bs[t];
  if (b >= 0 && b < a.B) {
    const int32_t sl = a.slen[a.slen_n == 1 ? 0 : b];
    const int32_t ps = a.pos[a.pos_n == 1 ? 0 : t];
    sel.lim = sl < ps ? sl : ps;  // <= 0: nothing is attended
    sel.tab = kTable ? a.slots + (static_cast<int64_t>(t) * a.Hkv + h) * (static_cast<int64_t>(a.K) * 64)
                     : a.bt + static_cast<int64_t>(b) * a.bt_sb;
  }
  const int32_t* idx_t = a.idx + static_cast<int64_t>(h) * a.i_sh + static_cast<int64_t>(t) * a.i_st;
  sel.lane_id = lane < a.K && sel.tab != nullptr ? idx_t[static_cast<int64_t>(lane) * a.i_sk] : -1;
  return sel;
}

// The pipeline shared by the attention kernel and the gather calibration:
// slot j of a ring of kRing holds the gathers of stage sr[j] and the table
// entry of the stage after it in that slot, st[j].  Every step computes the
// oldest stage, issues the gathers of the stage whose table entry has
// arrived and loads the table entry kRing stages further on, so a table load
// leads its gathers, and the gathers their arithmetic, by kRing stages.  The
// stages are walked in order, so the first slot left empty ends the walk.
template <bool kTable, int kRing, typename Compute>
__device__ __forceinline__ void sa_walk(const SaArgs& a, const SaSel& sel, SaStages stages,
                                        Compute&& compute) {
  SaStage r[kRing];
  int sr[kRing], st[kRing];
  int32_t tv[kRing];
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    st[j] = sa_pop(stages);
    tv[j] = sa_table<kTable>(a, sel, st[j]);
  }
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    sr[j] = st[j];
    sa_issue<kTable>(a, sel, sr[j], tv[j], r[j]);
    st[j] = sa_pop(stages);
    tv[j] = sa_table<kTable>(a, sel, st[j]);
  }
  for (bool more = true; more;) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      if (more && sr[j] >= 0) {
        compute(r[j]);
        sr[j] = st[j];
        sa_issue<kTable>(a, sel, sr[j], tv[j], r[j]);
        st[j] = sa_pop(stages);
        tv[j] = sa_table<kTable>(a, sel, st[j]);
      } else {
        more = false;
      }
    }
  }
}

template <typename OutT>
__device__ __forceinline__ void sa_store4(OutT* p, f32x4 v);
template <>
__device__ __forceinline__ void sa_store4<float>(float* p, f32x4 v) {
  *reinterpret_cast<f32x4*>(p) = v;
}
template <>
__device__ __forceinline__ void sa_store4<uint16_t>(uint16_t* p, f32x4 v) {
  const uint32_t lo = f32_to_bf16_bits(v.x) | (static_cast<uint32_t>(f32_to_bf16_bits(v.y)) << 16);
  const uint32_t hi = f32_to_bf16_bits(v.z) | (static_cast<uint32_t>(f32_to_bf16_bits(v.w)) << 16);
  *reinterpret_cast<uint2*>(p) = make_uint2(lo, hi);
}

template <typename OutT, bool kTable, int kRing>
__global__ __launch_bounds__(kWave) void sparse_attn_kernel(SaArgs a) {
  __shared__ __align__(16) char vst[kSaVBytes];
  const int lane = threadIdx.x;
  const int t = blockIdx.x, h = blockIdx.y;
  const SaSel sel = sa_select<kTable>(a, t, h);

  // Query fragments, the B operand of S^T = K Q^T: lane (head n, g) holds
  // q[t, 16h + n, 32cc + 8g .. +8].
  bf16x8 qf[4];
  {
    const __bf16* qp = a.q + static_cast<int64_t>(t) * a.q_st +
                       static_cast<int64_t>(kSaG * h + (lane & 15)) * a.q_sh + 8 * (lane >> 4);
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qf[cc] = *reinterpret_cast<const bf16x8*>(qp + 32 * cc);
  }
  // The compiler's own loads (ids, queries) complete here, before the ring's
  // loads are issued: a wait of its own for them placed inside the loop would
  // drain the ring on every stage.
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) asm volatile("" : : "v"(qf[cc]));
  asm volatile("" : : "v"(sel.lane_id));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const SaStages stages = sa_live(sel);

  // Per-lane constants of the stage computation.
  const int g = lane >> 4;
  // V chunk i of this lane's key goes to byte 1024*i + vput of vst, which
  // puts chunk c of key k at 1024*(c/4) + 16*(16*(c%4) + (k ^ 4*((c%4)&1))):
  // the transposing reads below then hit no bank twice.
  const int vput = 16 * (lane ^ (4 * (g & 1)));
  // V^T fragment (dims 16dt + 4(s%4) .. +3 of key 4g + s/4, s = lane%16):
  // byte 1024*(dt/2) + 512*(dt%2) + vread of vst.
  const int s = lane & 15;
  const int vkey = 4 * g + (s >> 2);
  const int vbit = (s >> 1) & 1;
  const int vread = 256 * vbit + 16 * (vkey ^ (4 * vbit)) + 8 * (s & 1);

  float m_run = -INFINITY;  // running max of this lane's head's scaled scores
  float l_run = 0.f;        // sum of exp2 against it over this lane's keys
  f32x4 o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float c = a.c;

  auto compute = [&](const SaStage& st) {
    if (st.mask == 0) return;  // every row of the stage outside the cache (wave-uniform)
    // V rows to LDS for the transposing reads
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<bf16x8*>(vst + 1024 * i + vput) = st.v[i];
    // scores S^T (keys 4g + r of the stage, head lane%16), scaled first: the
    // max and the exponentials below then hold for any sign of the scale
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(st.k[cc], qf[cc], acc, 0, 0, 0);
    float x0 = acc.x * c, x1 = acc.y * c, x2 = acc.z * c, x3 = acc.w * c;
    if (st.mask != 0xFFFFu) {  // keys of the stage not attended -> -inf (wave-uniform test)
      const uint32_t mb = st.mask >> (4 * g);
      x0 = (mb & 1u) ? x0 : -INFINITY;
      x1 = (mb & 2u) ? x1 : -INFINITY;
      x2 = (mb & 4u) ? x2 : -INFINITY;
      x3 = (mb & 8u) ? x3 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(x0, x1), fmaxf(x2, x3));
    mx = sa_max_x32(sa_max_x16(mx));  // finite: the stage has an attended key
    if (__ballot(mx > m_run + kSaRescale) != 0) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        o[dt].x *= alpha;
        o[dt].y *= alpha;
        o[dt].z *= alpha;
        o[dt].w *= alpha;
      }
      m_run = m_new;
    }
    // exponentials (0 for -inf scores); m_run is finite after the first stage
    const float p0 = __builtin_amdgcn_exp2f(x0 - m_run);
    const float p1 = __builtin_amdgcn_exp2f(x1 - m_run);
    const float p2 = __builtin_amdgcn_exp2f(x2 - m_run);
    const float p3 = __builtin_amdgcn_exp2f(x3 - m_run);
    l_run += (p0 + p1) + (p2 + p3);
    // P^T as two bf16 terms: hi = P truncated to bf16, lo = the exact residual
    // P - hi truncated to bf16, so hi + lo carries P to about 2^-15 (one bf16
    // P alone, 2^-9, left the numerator off the fp32 sum l_run by up to 0.2 %
    // of the attended values' magnitude).  A byte permute packs two values'
    // upper halves into one dword.
    const uint32_t u0 = __float_as_uint(p0), u1 = __float_as_uint(p1);
    const uint32_t u2 = __float_as_uint(p2), u3 = __float_as_uint(p3);
    const uint32_t w0 = __float_as_uint(p0 - __uint_as_float(u0 & 0xffff0000u));
    const uint32_t w1 = __float_as_uint(p1 - __uint_as_float(u1 & 0xffff0000u));
    const uint32_t w2 = __float_as_uint(p2 - __uint_as_float(u2 & 0xffff0000u));
    const uint32_t w3 = __float_as_uint(p3 - __uint_as_float(u3 & 0xffff0000u));
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const i16x4 pb = __builtin_bit_cast(i16x4, u32x2{__builtin_amdgcn_perm(u1, u0, 0x07060302u),
                                                     __builtin_amdgcn_perm(u3, u2, 0x07060302u)});
    const i16x4 pl = __builtin_bit_cast(i16x4, u32x2{__builtin_amdgcn_perm(w1, w0, 0x07060302u),
                                                     __builtin_amdgcn_perm(w3, w2, 0x07060302u)});
    // O^T += V^T P^T, one 16-dim tile at a time
    sa_lds_i16x4* vb = (sa_lds_i16x4*)(vst + vread);
    i16x4 vf[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      vf[dt] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (sa_lds_i16x4*)((__attribute__((address_space(3))) char*)vb + 1024 * (dt >> 1) + 512 * (dt & 1)));
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[dt], pb, o[dt], 0, 0, 0);
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf[dt], pl, o[dt], 0, 0, 0);
  };
  sa_walk<kTable, kRing>(a, sel, stages, compute);

  // ---- normalise and store: lane (head n, g) holds dims 16dt + 4g + r
  const float l_tot = sa_sum_x32(sa_sum_x16(l_run));
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  OutT* orow = static_cast<OutT*>(a.out) +
               (static_cast<int64_t>(t) * a.Hkv * kSaG + kSaG * h + (lane & 15)) * kSaD + 4 * g;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    f32x4 v = o[dt];
    v.x *= inv;
    v.y *= inv;
    v.z *= inv;
    v.w *= inv;
    sa_store4<OutT>(orow + 16 * dt, v);
  }
}

// Calibration of the gather rate (a measurement tool, not part of the
// attention): the same live stages, table entries and row checks, with every
// attended K and V row read once, coalesced -- lane l = 16r + s reads the
// 16-byte chunk s of the rows of keys 4r + i (i < 4), so 16 lanes read one
// 256-byte row -- kRing stages in flight, and no arithmetic but an XOR of
// the gathered words into a checksum, written per (t, h, lane) to a u32
// [T, Hkv, 64] output.  Its time is the floor the gathers alone set for a
// selection (the coalesced pattern measured 5 % faster than the attention
// kernel's fragment-order gathers on cfg5, at the same eight waves per CU).
struct SaRows {
  i32x4 k[4];
  i32x4 v[4];
};

// Table entries of keys 4r + i of stage sg (r = lane/16).
template <bool kTable>
__device__ __forceinline__ void sa_co_table(const SaArgs& a, const SaSel& sel, int sg, int32_t (&tv)[4]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = 4 * (lane >> 4) + i;  // entry of the quarter
    const int32_t* p;
    if (sg < 0) {
      p = reinterpret_cast<const int32_t*>(sa_zero_row);
    } else if constexpr (kTable) {
      p = sel.tab + 16 * sg + o;
    } else {
      const int32_t id = __builtin_amdgcn_readlane(sel.lane_id, sg >> 2);
      int32_t pc = static_cast<int32_t>(static_cast<uint32_t>(id) * 64u + static_cast<uint32_t>(16 * (sg & 3) + o));
      pc = pc < 0 ? 0 : (pc > a.L - 1 ? a.L - 1 : pc);
      p = sel.tab + pc;
    }
    tv[i] = *p;
  }
}

template <bool kTable>
__device__ __forceinline__ void sa_co_issue(const SaArgs& a, const SaSel& sel, int sg,
                                            const int32_t (&tv)[4], SaRows& st) {
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t col = static_cast<uint64_t>(16 * (lane & 15));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int32_t row = -1;
    if (sg >= 0) {
      const int32_t id = __builtin_amdgcn_readlane(sel.lane_id, sg >> 2);
      const int32_t p = static_cast<int32_t>(static_cast<uint32_t>(id) * 64u +
                                             static_cast<uint32_t>(16 * (sg & 3) + 4 * (lane >> 4) + i));
      const int32_t r = kTable ? tv[i]
                               : static_cast<int32_t>(static_cast<uint32_t>(a.Hkv) * static_cast<uint32_t>(tv[i]) +
                                                      static_cast<uint32_t>(sel.h));
      row = p < sel.lim && r >= 0 && r < a.n_rows ? r : -1;
    }
    const char *kp, *vp;
    if (row >= 0) {
      const uint64_t off = static_cast<uint64_t>(row) * static_cast<uint64_t>(a.row_bytes) + col;
      kp = a.kc + off;
      vp = a.vc + off;
    } else {
      kp = vp = reinterpret_cast<const char*>(sa_zero_row) + col;
    }
    st.k[i] = *reinterpret_cast<const i32x4*>(kp);
    st.v[i] = *reinterpret_cast<const i32x4*>(vp);
  }
}

template <bool kTable, int kRing>
__global__ __launch_bounds__(kWave) void sparse_gather_kernel(SaArgs a) {
  const int lane = threadIdx.x;
  const int t = blockIdx.x, h = blockIdx.y;
  const SaSel sel = sa_select<kTable>(a, t, h);
  asm volatile("" : : "v"(sel.lane_id));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  SaStages stages = sa_live(sel);
  uint32_t x = 0;
  SaRows r[kRing];
  int sr[kRing], st[kRing];
  int32_t tv[kRing][4];
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    st[j] = sa_pop(stages);
    sa_co_table<kTable>(a, sel, st[j], tv[j]);
  }
#pragma unroll
  for (int j = 0; j < kRing; ++j) {
    sr[j] = st[j];
    sa_co_issue<kTable>(a, sel, sr[j], tv[j], r[j]);
    st[j] = sa_pop(stages);
    sa_co_table<kTable>(a, sel, st[j], tv[j]);
  }
  for (bool more = true; more;) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) {
      if (more && sr[j] >= 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const i32x4 kv = r[j].k[i] ^ r[j].v[i];
          x ^= static_cast<uint32_t>(kv.x ^ kv.y ^ kv.z ^ kv.w);
        }
        sr[j] = st[j];
        sa_co_issue<kTable>(a, sel, sr[j], tv[j], r[j]);
        st[j] = sa_pop(stages);
        sa_co_table<kTable>(a, sel, st[j], tv[j]);
      } else {
        more = false;
      }
    }
  }
  static_cast<uint32_t*>(a.out)[(static_cast<int64_t>(t) * a.Hkv + h) * kWave + lane] = x;
}

}  // namespace
}  // namespace unum

namespace unum {
namespace {

// Validation and argument block shared by the attention entry point and the
// gather calibration (q, out and the scale are set by the caller).
int sa_args(SaArgs& a, const char* op, const void* key_cache, const void* value_cache,
            int64_t kv_row_stride, int64_t n_rows, const int32_t* topk_idx, int64_t topk_stride_h,
            int64_t topk_stride_t, int64_t topk_stride_k, const int32_t* block_table,
            int64_t bt_stride_b, const int32_t* slots, const int32_t* token_to_bs,
            const int32_t* token_pos_in_bs, int64_t pos_numel, const int32_t* seqlen_q,
            int64_t seqlen_numel, int64_t T, int64_t Hkv, int64_t K, int64_t B, int64_t L) {
  UNUM_REQUIRE(K <= kSaMaxBlocks, "%s: at most %d blocks per token (K=%lld)", op, kSaMaxBlocks,
               (long long)K);
  UNUM_REQUIRE(key_cache && value_cache && topk_idx && token_to_bs && token_pos_in_bs && seqlen_q,
               "%s: null pointer", op);
  UNUM_REQUIRE(slots || (block_table && B >= 1 && L >= 1),
               "%s: a block table (B, L >= 1) or a slot table is required", op);
  UNUM_REQUIRE(pos_numel == 1 || pos_numel == T, "%s: token_pos_in_bs has %lld entries (T=%lld)",
               op, (long long)pos_numel, (long long)T);
  UNUM_REQUIRE(seqlen_numel == 1 || seqlen_numel >= B, "%s: seqlen_q has %lld entries (B=%lld)", op,
               (long long)seqlen_numel, (long long)B);
  UNUM_REQUIRE(n_rows >= 0 && kv_row_stride >= kSaD && (kv_row_stride % 8) == 0,
               "%s: cache rows must be D elements or more apart, in multiples of 8 (stride %lld)",
               op, (long long)kv_row_stride);
  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(key_cache) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(value_cache) & 15) == 0,
               "%s: the caches must be 16-byte aligned", op);
  UNUM_REQUIRE(T <= INT32_MAX && Hkv <= 65535 && n_rows <= INT32_MAX && B <= INT32_MAX &&
                   L <= INT32_MAX,
               "%s: size exceeds the kernel's index range", op);
  a.kc = static_cast<const char*>(key_cache);
  a.vc = static_cast<const char*>(value_cache);
  a.row_bytes = kv_row_stride * 2;
  a.n_rows = n_rows;
  a.idx = topk_idx;
  a.i_sh = topk_stride_h;
  a.i_st = topk_stride_t;
  a.i_sk = topk_stride_k;
  a.bt = block_table;
  a.bt_sb = bt_stride_b;
  a.slots = slots;
  a.tok_bs = token_to_bs;
  a.pos = token_pos_in_bs;
  a.slen = seqlen_q;
  a.pos_n = static_cast<int32_t>(pos_numel);
  a.slen_n = static_cast<int32_t>(seqlen_numel == 1 ? 1 : 2);
  a.T = static_cast<int32_t>(T);
  a.Hkv = static_cast<int32_t>(Hkv);
  a.K = static_cast<int32_t>(K);
  a.B = static_cast<int32_t>(B);
  a.L = static_cast<int32_t>(L);
  return UNUM_OK;
}

}  // namespace
}  // namespace unum

extern "C" int unum_sparse_paged_attention(
    const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* key_cache,
    const void* value_cache, int64_t kv_row_stride, int64_t n_rows, const int32_t* topk_idx,
    int64_t topk_stride_h, int64_t topk_stride_t, int64_t topk_stride_k,
    const int32_t* block_table, int64_t bt_stride_b, const int32_t* slots,
    const int32_t* token_to_bs, const int32_t* token_pos_in_bs, int64_t pos_numel,
    const int32_t* seqlen_q, int64_t seqlen_numel, void* out, int32_t out_dtype, int64_t T,
    int64_t Hq, int64_t Hkv, int64_t D, int64_t K, int64_t B, int64_t L, float scale,
    void* stream) {
  using namespace unum;
  clear_error();
  const char* op = "sparse_paged_attention";
  UNUM_REQUIRE(T >= 0 && Hq > 0 && Hkv > 0 && D > 0 && K >= 0 && B >= 0 && L >= 0,
               "%s: bad sizes (T=%lld Hq=%lld Hkv=%lld D=%lld K=%lld B=%lld L=%lld)", op,
               (long long)T, (long long)Hq, (long long)Hkv, (long long)D, (long long)K,
               (long long)B, (long long)L);
  if (T == 0) return UNUM_OK;
  if (Hq != kSaG * Hkv || D != kSaD)
    UNUM_FAIL(UNUM_ERR_UNSUPPORTED, "%s: needs 16 query heads per kv head and D = 128 (got Hq=%lld, "
              "Hkv=%lld, D=%lld)", op, (long long)Hq, (long long)Hkv, (long long)D);
  UNUM_REQUIRE(q && out, "%s: null pointer", op);
  UNUM_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15) == 0 && (q_stride_t % 8) == 0 &&
                   (q_stride_h % 8) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0,
               "%s: q and out must be 16-byte aligned (q strides multiples of 8)", op);
  UNUM_REQUIRE(out_dtype == UNUM_DTYPE_BF16 || out_dtype == UNUM_DTYPE_F32,
               "%s: unsupported out dtype %d", op, out_dtype);
  SaArgs a{};
  const int st = sa_args(a, op, key_cache, value_cache, kv_row_stride, n_rows, topk_idx,
                         topk_stride_h, topk_stride_t, topk_stride_k, block_table, bt_stride_b,
                         slots, token_to_bs, token_pos_in_bs, pos_numel, seqlen_q, seqlen_numel,
                         T, Hkv, K, B, L);
  if (st != UNUM_OK) return st;
  a.q = static_cast<const __bf16*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.out = out;
  a.c = scale * kSaLog2e;
  const dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(Hkv));
  hipStream_t s = static_cast<hipStream_t>(stream);
#define UNUM_SA_LAUNCH(OutT, kTab) \
  hipLaunchKernelGGL((sparse_attn_kernel<OutT, kTab, kSaRing>), grid, dim3(kWave), \
                     kSaLdsBytes - kSaVBytes, s, a)
  if (out_dtype == UNUM_DTYPE_BF16) {
    if (slots)
      UNUM_SA_LAUNCH(uint16_t, true);
    else
      UNUM_SA_LAUNCH(uint16_t, false);
  } else {
    if (slots)
      UNUM_SA_LAUNCH(float, true);
    else
      UNUM_SA_LAUNCH(float, false);
  }
#undef UNUM_SA_LAUNCH
  return check_launch(op);
}

extern "C" int unum_sparse_gather_calibrate(
    const void* key_cache, const void* value_cache, int64_t kv_row_stride, int64_t n_rows,
    const int32_t* topk_idx, int64_t topk_stride_h, int64_t topk_stride_t, int64_t topk_stride_k,
    const int32_t* block_table, int64_t bt_stride_b, const int32_t* slots,
    const int32_t* token_to_bs, const int32_t* token_pos_in_bs, int64_t pos_numel,
    const int32_t* seqlen_q, int64_t seqlen_numel, uint32_t* out, int64_t T, int64_t Hkv,
    int64_t K, int64_t B, int64_t L, void* stream) {
  using namespace unum;
  clear_error();
  const char* op = "sparse_gather_calibrate";
  UNUM_REQUIRE(T >= 0 && Hkv > 0 && K >= 0 && B >= 0 && L >= 0,
               "%s: bad sizes (T=%lld Hkv=%lld K=%lld B=%lld L=%lld)", op, (long long)T,
               (long long)Hkv, (long long)K, (long long)B, (long long)L);
  if (T == 0) return UNUM_OK;
  UNUM_REQUIRE(out, "%s: null pointer", op);
  SaArgs a{};
  const int st = sa_args(a, op, key_cache, value_cache, kv_row_stride, n_rows, topk_idx,
                         topk_stride_h, topk_stride_t, topk_stride_k, block_table, bt_stride_b,
                         slots, token_to_bs, token_pos_in_bs, pos_numel, seqlen_q, seqlen_numel,
                         T, Hkv, K, B, L);
  if (st != UNUM_OK) return st;
  a.out = out;
  const dim3 grid(static_cast<unsigned>(T), static_cast<unsigned>(Hkv));
  hipStream_t s = static_cast<hipStream_t>(stream);
  // eight waves per CU, as the attention kernel
  if (slots)
    hipLaunchKernelGGL((sparse_gather_kernel<true, kSaRing>), grid, dim3(kWave), kSaLdsBytes, s, a);
  else
    hipLaunchKernelGGL((sparse_gather_kernel<false, kSaRing>), grid, dim3(kWave), kSaLdsBytes, s, a);
  return check_launch(op);
}
