// Decode attention building blocks shared by the split-K decode kernels and the
// fused decode step: the query of one (sequence, head), one key block streamed
// into an online-softmax state, and the (o, m, l) partial of a wavefront.
//
// One wavefront handles one key block: 16 lanes per 256-byte key row (4 rows per
// load instruction), the K and V loads of a 64-key slice all issued before the
// first use, row sums by DPP, softmax in base 2.  Lane group g = lane / 16 keeps
// its own o[8] (dims 8 (lane % 16) .. +7) under a wavefront-wide running max.
#pragma once

#include "dash_common.h"

namespace dash {

constexpr int kDcMaxK = 16;       // routed slots of the fused decode step
constexpr int kDcMaxSlots = 64;   // routed slots of dash_attn_decode (one per lane)
constexpr int kDcMaxSplit = 64;

struct DecodeArgs {
  const bf16* q; int64_t q_sb, q_sh;
  const bf16* k; const bf16* v;
  int64_t k_sb, k_sh, k_st, k_sp;
  int64_t v_sb, v_sh, v_st, v_sp;
  const int32_t* table; int64_t table_stride; int page;
  const int32_t* lens; const int32_t* q_pos;
  const int32_t* idx; const uint8_t* valid; const float* bias; int K;
  void* out; int out_bf16; int64_t o_sb, o_sh;
  float* lse; int64_t lse_sb, lse_sh;
  float* part;                   // [B*H*nsplit, D + 2]: o[D], m, l
  int S, H, bs, lw, nsplit;
  int piece;                     // keys per window piece of the fused decode step
  float scale_log2e;
};

// Where the rows of one round trip (keys jb .. jl, jl - jb < ROWS <= 32) live: row j
// is at element offset (j - rb < page ? o0 : o1) + (j - rb) * st.  With a block table
// the entries of the at most two pages those keys touch (every page holds at least
// 32 keys: block sizes are 32 or multiples of 64 and pages hold whole blocks) are read
// once, as scalar loads, before any row load is issued; a table read per row made
// each row load wait for its own table read, and so for every row load before it.
struct DcRows {
  int rb;
  int64_t k0, k1, v0, v1;
};

__device__ __forceinline__ DcRows dc_rows(const DecodeArgs& a, int b, int jb, int jl) {
  DcRows r;
  if (a.table) {
    const int bu = __builtin_amdgcn_readfirstlane(b);
    const int pg = __builtin_amdgcn_readfirstlane(jb) / a.page;
    r.rb = pg * a.page;
    const int32_t* tr = a.table + (int64_t)bu * a.table_stride + pg;
    const int p0 = tr[0];
    const int p1 = __builtin_amdgcn_readfirstlane(jl) >= r.rb + a.page ? tr[1] : p0;
    r.k0 = (int64_t)p0 * a.k_sp;
    r.v0 = (int64_t)p0 * a.v_sp;
    r.k1 = (int64_t)p1 * a.k_sp - (int64_t)a.page * a.k_st;
    r.v1 = (int64_t)p1 * a.v_sp - (int64_t)a.page * a.v_st;
  } else {
    r.rb = 0;                            // one base: the page test picks either
    r.k0 = r.k1 = (int64_t)b * a.k_sb;
    r.v0 = r.v1 = (int64_t)b * a.v_sb;
  }
  return r;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
  return v;
}

// The key range of one decode query: window (qp - lw, qp] and window blocks.
struct DcSpan {
  int len, qp, ls, lo, nblk, w0, n_win;
};

__device__ __forceinline__ DcSpan dc_span(const DecodeArgs& a, int b) {
  DcSpan s;
  s.len = a.lens ? min(max(a.lens[b], 0), a.S) : a.S;
  s.qp = a.q_pos ? min(a.q_pos[b], s.len - 1) : s.len - 1;   // at most the last cached token
  s.ls = s.qp - a.lw + 1;
  s.lo = max(s.ls, 0);
  s.nblk = s.len > 0 ? (s.len + a.bs - 1) / a.bs : 0;
  s.w0 = s.lo / a.bs;
  s.n_win = (s.len > 0 && s.qp >= 0) ? s.qp / a.bs - s.w0 + 1 : 0;
  return s;
}

// Online-softmax state of one wavefront.
struct DcState {
  bf16x2 qp2[4];                 // this lane's 8 query dims
  int g, dl;                     // lane group (key row within 4) and first dim
  float m_run, l_run, o[8];
};

__device__ __forceinline__ void dc_init(DcState& st, const DecodeArgs& a, int b, int h, int lane) {
  st.g = lane >> 4;
  st.dl = (lane & 15) * 8;
  const bf16x8 qv8 = *(const bf16x8*)(a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + st.dl);
#pragma unroll
  for (int e = 0; e < 4; ++e) { st.qp2[e][0] = qv8[2 * e]; st.qp2[e][1] = qv8[2 * e + 1]; }
  st.m_run = -INFINITY;
  st.l_run = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) st.o[e] = 0.f;
}

// The K and V rows of one round trip: ROWS keys from jb, ROWS / 4 loads of each per
// lane (16 lanes per 256-byte row, 4 rows per load).
template <int ROWS>
struct DcRound {
  bf16x8 k[ROWS / 4], v[ROWS / 4];
};

// Issue the loads of the round trip of keys jb .. (rows past j1 - 1 repeat it).  A
// decode step reads each K/V row once, so the loads are non-temporal: streamed rows
// then do not displace the partials and index data the step reads back (12-layer paged
// step 971 -> 869 us).
template <int ROWS>
__device__ __forceinline__ void dc_issue(DcRound<ROWS>& rd, const DcState& st, const DecodeArgs& a,
                                         int b, int h, int jb, int j1) {
  static_assert(ROWS <= 32, "the rows of a round trip touch at most two table pages");
  const bf16* kh = a.k + (int64_t)h * a.k_sh;
  const bf16* vh = a.v + (int64_t)h * a.v_sh;
  const int jl = min(jb + ROWS, j1) - 1;   // last key; later rows repeat it
  const DcRows rw = dc_rows(a, b, jb, jl);
#pragma unroll
  for (int t = 0; t < ROWS / 4; ++t) {
    const int r = min(jb + 4 * t + st.g, jl) - rw.rb;
    rd.k[t] = __builtin_nontemporal_load((const bf16x8*)(kh + (r < a.page ? rw.k0 : rw.k1) + (int64_t)r * a.k_st + st.dl));
  }
#pragma unroll
  for (int t = 0; t < ROWS / 4; ++t) {
    const int r = min(jb + 4 * t + st.g, jl) - rw.rb;
    rd.v[t] = __builtin_nontemporal_load((const bf16x8*)(vh + (r < a.page ? rw.v0 : rw.v1) + (int64_t)r * a.v_st + st.dl));
  }
}

// Online-softmax update of the state with the round trip of keys jb .. (of a routed
// block, with log2 bias blog, or of the window).
template <int ROWS>
__device__ __forceinline__ void dc_consume(DcState& st, const DcRound<ROWS>& rd, const DecodeArgs& a,
                                           const DcSpan& sp, int jb, int j1, bool routed, float blog) {
  constexpr int NT = ROWS / 4;
  float s[NT];
  float mloc = -INFINITY;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      bf16x2 kk;
      kk[0] = rd.k[t][2 * e];
      kk[1] = rd.k[t][2 * e + 1];
      acc = __builtin_amdgcn_fdot2_f32_bf16(st.qp2[e], kk, acc, false);
    }
    acc = row16_sum(acc);
    const int key = jb + 4 * t + st.g;
    bool ok = key < j1;
    ok = ok && (routed ? (key < sp.ls) : (key >= sp.lo && key <= sp.qp));
    s[t] = ok ? acc * a.scale_log2e + blog : -INFINITY;
    mloc = fmaxf(mloc, s[t]);
  }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, kWave));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
  const float m_new = fmaxf(st.m_run, mloc);
  const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
  const float alpha = fast_exp2(st.m_run - m_use);
  st.l_run *= alpha;
#pragma unroll
  for (int e = 0; e < 8; ++e) st.o[e] *= alpha;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const float p = fast_exp2(s[t] - m_use);
    st.l_run += p;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.o[e] = fmaf(p, bf2f(rd.v[t][e]), st.o[e]);
  }
  st.m_run = m_new;
}

// Stream keys [j0, j1) (of a routed block, with log2 bias blog, or of the window)
// into the state, ROWS keys per round trip, every load of a round trip issued before
// the first use.
template <int ROWS>
__device__ __forceinline__ void dc_keys(DcState& st, const DecodeArgs& a, int b, int h,
                                        const DcSpan& sp, int j0, int j1, bool routed, float blog) {
  for (int jb = j0; jb < j1; jb += ROWS) {
    DcRound<ROWS> rd;
    dc_issue<ROWS>(rd, st, a, b, h, jb, j1);
    __builtin_amdgcn_sched_barrier(0);
    dc_consume<ROWS>(st, rd, a, sp, jb, j1, routed, blog);
  }
}

// Stream key block cu (a routed block with log2 bias blog, or a window block);
// blocks of at most 32 keys take one 32-row round trip.
template <int ROWS = 64>
__device__ __forceinline__ void dc_block(DcState& st, const DecodeArgs& a, int b, int h,
                                         const DcSpan& sp, int cu, bool routed, float blog) {
  const int j0 = cu * a.bs, j1 = min((cu + 1) * a.bs, sp.len);
  if (ROWS > 32 && a.bs <= 32)
    dc_keys<32>(st, a, b, h, sp, j0, j1, routed, blog);
  else
    dc_keys<ROWS>(st, a, b, h, sp, j0, j1, routed, blog);
}

// Sum the four lane groups (they share m_run) and store the wavefront's partial
// (o[D], m, l) at part.
template <int D>
__device__ __forceinline__ void dc_store_partial(DcState& st, float* part, int lane) {
  st.l_run += __shfl_xor(st.l_run, 16, kWave);
  st.l_run += __shfl_xor(st.l_run, 32, kWave);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    st.o[e] += __shfl_xor(st.o[e], 16, kWave);
    st.o[e] += __shfl_xor(st.o[e], 32, kWave);
  }
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) part[st.dl + e] = st.o[e];
  }
  if (lane == 0) { part[D] = st.m_run; part[D + 1] = st.l_run; }
}

// Routed blocks of sequence b, by the lanes of one wavefront (lanes < K load the
// slots): valid, remote (keys below the window), first occurrence, in slot order,
// into sRC / sRB (log2 bias).  sTmp holds kWave ints.  Returns their count.  The
// caller's barrier (sync) orders the LDS accesses between lanes.
template <typename Sync>
__device__ __forceinline__ int dc_routed(const DecodeArgs& a, int b, const DcSpan& sp, int lane,
                                         int* sTmp, int* sRC, float* sRB, Sync sync) {
  int c = -1;
  float bl = 0.f;
  bool keep = false;
  if (lane < a.K && sp.len > 0) {
    const int64_t o = (int64_t)b * a.K + lane;
    c = a.idx[o];
    keep = c >= 0 && c < sp.nblk && c * a.bs < sp.ls && (!a.valid || a.valid[o] != 0);
    bl = a.bias[o] * 1.4426950408889634f;
  }
  sTmp[lane] = keep ? c : -1;
  sync();
  if (keep)
    for (int j = 0; j < lane; ++j) keep &= (sTmp[j] != c);
  const uint64_t mask = __ballot(keep);
  if (keep) {
    const int pos = __popcll(mask & ((1ull << lane) - 1ull));
    sRC[pos] = c;
    sRB[pos] = bl;
  }
  sync();
  return __popcll(mask);
}

// Log-sum-exp merge of n partials (lane i holds the (m, l) of partial i, i < n)
// by one wavefront; part_at(s) gives partial s's o[D].  Writes out and lse.
template <int D, typename PartAt>
__device__ __forceinline__ void dc_merge(const DecodeArgs& a, int b, int h, int lane, int n,
                                         float ms, float lsum, float* sW, PartAt part_at) {
  // every partial's o (n <= 64, in groups of eight, the last group's surplus
  // loads repeating partial n - 1) is loaded before the weights are known, so
  // the merge waits on memory once
  float2 ov[kWave];
  if (n > 0) {
#pragma unroll
    for (int g = 0; g < kWave / 8; ++g)
      if (8 * g < n) {
#pragma unroll
        for (int u = 0; u < 8; ++u) ov[8 * g + u] = *(const float2*)(part_at(min(8 * g + u, n - 1)) + lane * 2);
      }
  }
  const float M = wave_max(ms);
  const float Mu = (M == -INFINITY) ? 0.f : M;
  const float w = lane < n ? fast_exp2(ms - Mu) : 0.f;
  const float L = wave_sum(lsum * w);
  sW[lane] = w;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float inv = L > 0.f ? 1.f / L : 0.f;
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int g = 0; g < kWave / 8; ++g)
    if (8 * g < n) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float wu = 8 * g + u < n ? sW[8 * g + u] : 0.f;
        acc0 += ov[8 * g + u].x * wu;
        acc1 += ov[8 * g + u].y * wu;
      }
    }
  const int64_t off = (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + lane * 2;
  if (a.out_bf16) {
    bf16x2 r;
    r[0] = (bf16)(acc0 * inv);
    r[1] = (bf16)(acc1 * inv);
    *(bf16x2*)((bf16*)a.out + off) = r;
  } else {
    *(float2*)((float*)a.out + off) = make_float2(acc0 * inv, acc1 * inv);
  }
  if (a.lse && lane == 0)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh] =
        L > 0.f ? (M + log2f(L)) * 0.6931471805599453f : -INFINITY;
}

}  // namespace dash
