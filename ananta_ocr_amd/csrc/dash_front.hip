// Fused router front end for bf16 hidden states: index q/k projection (one bf16
// MFMA GEMM against the q_proj / k_proj weights), nan_to_num of the hidden states,
// Gemma RMSNorm, RoPE and the finiteness guards (modeling_deepseekv2.py:336-348,
// dash_attention.py:680-700), and for stage 0 "head_cls" the block summaries k_bar
// (dash_attention.py:863-888 / modeling_deepseekv2.py:362-379), in one launch.
//
// One work-group of four wavefronts per 64 token rows of one sequence.  Wavefront
// w computes side w / 2 (0: q, 1: k) for index dims 32 (w % 2) + [0, 32) and
// 64 + 32 (w % 2) + [0, 32): the two halves that RoPE's rotate_half pairs, so the
// rotation needs no exchange.  The hidden states stream through a four-stage LDS
// ring filled by direct loads; the weights come pre-packed in the MFMA operand
// order, so that every weight load of a wavefront is one contiguous 1 KB read.  The
// projection stays in the MFMA accumulators through the norm, RoPE and k_bar
// pooling; row reductions are reduce-scatters across the 32 lanes of a row group
// plus one exchange between the two wavefronts of a side.
#include <climits>
#include <type_traits>

#include "dash_common.h"

namespace dash {

constexpr int kFrRows = 64;       // token rows per work-group
constexpr int kFrKc = 64;         // hidden columns per staged chunk
constexpr int kFrD = 128;         // index dim
constexpr int kFrStage = kFrRows * kFrKc / 8;   // 16-byte granules of a hidden-state stage

struct FrontArgs {
  const bf16* hs; int64_t hs_sb, hs_st; int B, S, hid;
  const bf16* w;                              // packed weights (front_pack_kernel)
  const bf16* wq; const bf16* wk;             // the same weights, [128, hid] each
  const float* wq_n; const float* wk_n; float eps;
  const void* cos; const void* sin; int cs_bf16, cs_lds; int64_t cs_sb, cs_st;
  const float* head_cls; int bs; float inv_sqrt_d;
  float* iq; int64_t iq_sb;
  float* ik; int64_t ik_sb;
  float* kbar; int64_t kb_sb;
  int ntiles;
};

struct FrontSmem {
  uint16_t cs[2][kFrRows * kFrD];             // 32 KB: bf16 cos / sin rows of the tile
  float part[2][2][kFrRows];                  // [side][wavefront half][row] partial sums
  float r[4][kFrRows];                        // per wavefront: 1/rms of each row
  float wgt[kFrRows];                         // k_bar weights of the tile's rows
  float fix[4][64];                           // per wavefront: a recomputed projection row
  uint32_t bad[2];                            // rows whose projection is not finite
};

__device__ __forceinline__ float fr_rb16(float x) { return (float)(bf16)x; }
__device__ __forceinline__ float fr_finite(float x) {
  return (fabsf(x) <= 3.402823466e38f) ? x : 0.f;
}

// nan_to_num(nan/inf -> 0) of the two bf16 halves of a word
__device__ __forceinline__ uint32_t fr_sanitize2(uint32_t x) {
  const uint32_t lo = x & 0xffffu, hi = x >> 16;
  const uint32_t l2 = ((lo & 0x7f80u) == 0x7f80u) ? 0u : lo;
  const uint32_t h2 = ((hi & 0x7f80u) == 0x7f80u) ? 0u : hi;
  return l2 | (h2 << 16);
}
__device__ __forceinline__ bf16x8 fr_sanitize8(uint4 v) {
  v.x = fr_sanitize2(v.x); v.y = fr_sanitize2(v.y);
  v.z = fr_sanitize2(v.z); v.w = fr_sanitize2(v.w);
  return __builtin_bit_cast(bf16x8, v);
}

// v_cndmask with a constant lane mask: mask bit set -> b, else a.  An explicit
// instruction, so that the selects of the reduce-scatter below stay selects of
// registers (the compiler otherwise turns them into indexed reads of the array).
__device__ __forceinline__ float fr_sel(float a, float b, uint64_t mask) {
  float r;
  asm volatile("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "s"(mask));
  return r;
}

// Sum over the 32 lanes of each wavefront half of 32 values per lane: afterwards
// lane l holds the half's total of value l % 32.  Both lanes of an exchange add
// the same two operands, so every total is formed by one fixed tree.
__device__ __forceinline__ float fr_reduce_scatter32(float (&v)[32]) {
  constexpr uint64_t kUp[5] = {0xFFFF0000FFFF0000ull, 0xFF00FF00FF00FF00ull, 0xF0F0F0F0F0F0F0F0ull,
                               0xCCCCCCCCCCCCCCCCull, 0xAAAAAAAAAAAAAAAAull};
#pragma unroll
  for (int s = 0; s < 5; ++s) {
    const int d = 16 >> s, n = 32 >> s;
#pragma unroll
    for (int k = 0; k < n / 2; ++k) {
      const float lo = v[k], hi = v[k + n / 2];
      const float send = fr_sel(hi, lo, kUp[s]);     // lanes with bit d send the lower half
      const float keep = fr_sel(lo, hi, kUp[s]);
      v[k] = keep + __shfl_xor(send, d, kWave);
    }
  }
  return v[0];
}

// tile row of accumulator element i of m-tile mt for a lane of half h
__device__ __forceinline__ int fr_row(int mt, int i, int h) {
  return 32 * mt + 8 * (i >> 2) + 4 * h + (i & 3);
}

// hidden-state stage layout in LDS: row r's 16-byte piece p at granule r*8 + (p ^ ((r >> 1) & 7))
__device__ __forceinline__ int fr_aslot(int r, int p) { return r * 8 + (p ^ ((r >> 1) & 7)); }

template <int N>
__device__ __forceinline__ void fr_wait_vm() {
  // vmcnt(N): this wavefront has at most N vector-memory operations outstanding
  // (vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at their maxima)
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// Waits until at most n vector-memory operations are outstanding, for the counts
// the projection loop can produce (each one an immediate).
__device__ __forceinline__ void fr_wait_vm_n(int n) {
  switch (n) {
    case 0: fr_wait_vm<0>(); break;
    case 2: fr_wait_vm<2>(); break;
    case 4: fr_wait_vm<4>(); break;
    case 8: fr_wait_vm<8>(); break;
    case 10: fr_wait_vm<10>(); break;
    case 12: fr_wait_vm<12>(); break;
    case 16: fr_wait_vm<16>(); break;
    case 18: fr_wait_vm<18>(); break;
    default: fr_wait_vm<20>(); break;
  }
}

__global__ __launch_bounds__(256, 2) void router_front_kernel(FrontArgs a) {
#pragma clang fp contract(off)
  __shared__ FrontSmem sm;
  // the hidden-state ring: four stages, each its own LDS object, so that reads of
  // one stage do not wait for the direct loads into another
  __shared__ uint4 sH0[kFrStage], sH1[kFrStage], sH2[kFrStage], sH3[kFrStage];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int side = wv >> 1, part = wv & 1;
  const int m32 = lane & 31, half = lane >> 5;
  const int b = blockIdx.x / a.ntiles, tile = blockIdx.x % a.ntiles;
  const int t0 = tile * kFrRows;
  if (tid == 0) sm.bad[0] = sm.bad[1] = 0u;

  // bf16 cos / sin rows of the tile, straight into LDS (first in the load queue)
  if (a.cs_lds) {
#pragma unroll
    for (int arr = 0; arr < 2; ++arr) {
      const uint16_t* src = (const uint16_t*)(arr ? a.sin : a.cos) + (int64_t)b * a.cs_sb;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int g = u * 256 + wv * 64 + lane, row = g >> 4, piece = g & 15;
        const uint16_t* p = src + (int64_t)min(t0 + row, a.S - 1) * a.cs_st + 8 * piece;
        __builtin_amdgcn_global_load_lds(
            (const void*)p, (__attribute__((address_space(3))) void*)&sm.cs[arr][(u * 256 + wv * 64) * 8],
            16, 0, 0);
      }
    }
  }

  // ---------------------------------------------------------------- projection
  // this lane's weight rows (B operand): dims d0 = 32 part + m32 and d1 = d0 + 64;
  // the packed weights hold, per chunk and wavefront, the 8 operand pieces of every
  // lane back to back (1 KB per piece index: one coalesced load)
  const int d0 = 32 * part + m32, d1 = d0 + 64;
  const bf16* wp = a.w + (int64_t)wv * 8 * 512 + lane * 8;
  // direct loads of a stage: granule g = u*256 + 64 wv + lane holds row g / 8's
  // piece (g % 8) ^ ((row >> 1) % 8); rows past the sequence repeat its last row
  const bf16* hsrc[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int g = u * 256 + wv * 64 + lane, row = g >> 3, p = (g & 7) ^ ((row >> 1) & 7);
    hsrc[u] = a.hs + (int64_t)b * a.hs_sb + (int64_t)min(t0 + row, a.S - 1) * a.hs_st + 8 * p;
  }
  const int nch = a.hid / kFrKc;
  auto dma_h = [&](uint4* stage, int c) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(hsrc[u] + c * kFrKc),
                                       (__attribute__((address_space(3))) void*)(stage + u * 256 + wv * 64),
                                       16, 0, 0);
  };
  uint4 wA[4][2], wB[4][2], wC[4][2];
  auto load_w = [&](uint4 (&dst)[4][2], int c) {
    const bf16* src = wp + (int64_t)c * 4 * 8 * 512;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      dst[s][0] = *(const uint4*)(src + (2 * s) * 512);
      dst[s][1] = *(const uint4*)(src + (2 * s + 1) * 512);
    }
  };
  floatx16 acc[2][2];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][nt][i] = 0.f;
  auto compute = [&](const uint4 (&wr)[4][2], const uint4* stage) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 a0 = __builtin_bit_cast(bf16x8, stage[fr_aslot(m32, 2 * s + half)]);
      const bf16x8 a1 = __builtin_bit_cast(bf16x8, stage[fr_aslot(32 + m32, 2 * s + half)]);
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, wr[s][0]);
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, wr[s][1]);
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, b1, acc[1][1], 0, 0, 0);
    }
  };
  // Vector-memory operations of this wavefront issued after the stage of chunk c:
  // the prologue issues W(0), W(1) (8 each), then the stages of chunks 0, 1, 2 (2
  // each); step k issues W(k+2) and then the stage of chunk k+3, when they exist.
  auto ops_after_stage = [&](int c) {
    int n = 0;
    if (c <= 2)
      n += 2 * max(0, min(2, nch - 1) - c);
    for (int k = max(0, c - 2); k < c; ++k) n += (k + 2 < nch ? 8 : 0) + (k + 3 < nch ? 2 : 0);
    return n;
  };
  // Step c: chunk c's stage has landed (each wavefront waits for its own direct
  // loads, then the barrier), the weights of chunk c+2 and the stage of chunk c+3
  // are requested, chunk c is multiplied.
  auto step = [&](int c, auto hs_tag, auto w_tag) {
    constexpr int HS = decltype(hs_tag)::value, WS = decltype(w_tag)::value;
    uint4* const cur = HS == 0 ? sH0 : (HS == 1 ? sH1 : (HS == 2 ? sH2 : sH3));
    uint4* const nxt = HS == 0 ? sH3 : (HS == 1 ? sH0 : (HS == 2 ? sH1 : sH2));   // chunk c+3
    fr_wait_vm_n(ops_after_stage(c));
    __syncthreads();
    if (c + 2 < nch) load_w(WS == 0 ? wC : (WS == 1 ? wA : wB), c + 2);
    if (c + 3 < nch) dma_h(nxt, c + 3);
    compute(WS == 0 ? wA : (WS == 1 ? wB : wC), cur);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  load_w(wA, 0);
  if (nch > 1) load_w(wB, 1);
  dma_h(sH0, 0);
  if (nch > 1) dma_h(sH1, 1);
  if (nch > 2) dma_h(sH2, 2);
  for (int c = 0; c < nch; c += 12) {
    step(c, I0{}, I0{});
    if (c + 1 < nch) step(c + 1, I1{}, I1{});
    if (c + 2 < nch) step(c + 2, I2{}, I2{});
    if (c + 3 < nch) step(c + 3, I3{}, I0{});
    if (c + 4 < nch) step(c + 4, I0{}, I1{});
    if (c + 5 < nch) step(c + 5, I1{}, I2{});
    if (c + 6 < nch) step(c + 6, I2{}, I0{});
    if (c + 7 < nch) step(c + 7, I3{}, I1{});
    if (c + 8 < nch) step(c + 8, I0{}, I2{});
    if (c + 9 < nch) step(c + 9, I1{}, I0{});
    if (c + 10 < nch) step(c + 10, I2{}, I1{});
    if (c + 11 < nch) step(c + 11, I3{}, I2{});
  }

  // ---------------------------------------------------------------- non-finite rows
  // The GEMM multiplies the hidden states as they are; a non-finite value in a row
  // makes every projection of that row non-finite.  Such rows (and rows that
  // overflow) are recomputed from the hidden states with nan/inf -> 0, which is
  // the reference's nan_to_num ahead of the projection.
  {
    uint32_t bad_lo = 0, bad_hi = 0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool bad = !(fabsf(acc[mt][0][i]) <= 3.402823466e38f) ||
                         !(fabsf(acc[mt][1][i]) <= 3.402823466e38f);
        const uint64_t m = __ballot(bad);
        const uint32_t r0 = (uint32_t)fr_row(mt, i, 0), r1 = (uint32_t)fr_row(mt, i, 1);
        if ((uint32_t)m) { if (r0 < 32) bad_lo |= 1u << r0; else bad_hi |= 1u << (r0 - 32); }
        if ((uint32_t)(m >> 32)) { if (r1 < 32) bad_lo |= 1u << r1; else bad_hi |= 1u << (r1 - 32); }
      }
    if (lane == 0 && (bad_lo | bad_hi)) {
      atomicOr(&sm.bad[0], bad_lo);
      atomicOr(&sm.bad[1], bad_hi);
    }
  }
  __syncthreads();
  {
    uint64_t bad = ((uint64_t)sm.bad[1] << 32) | sm.bad[0];
    if (a.S - t0 < 64) bad &= (1ull << (a.S - t0)) - 1ull;      // rows past the sequence
    while (bad) {
      const int r = __builtin_ctzll(bad);
      bad &= bad - 1ull;
      // lane: dim d0 (half 0) or d1 (half 1) of this wavefront's side
      const bf16* hrow = a.hs + (int64_t)b * a.hs_sb + (int64_t)(t0 + r) * a.hs_st;
      const bf16* wrow = (side ? a.wk : a.wq) + (int64_t)(half ? d1 : d0) * a.hid;
      float dot = 0.f;
      for (int k = 0; k < a.hid; k += 8) {
        const bf16x8 hv = fr_sanitize8(*(const uint4*)(hrow + k));
        const bf16x8 wv8 = *(const bf16x8*)(wrow + k);
#pragma unroll
        for (int e = 0; e < 8; ++e) dot = dot + (float)hv[e] * (float)wv8[e];
      }
      sm.fix[wv][lane] = dot;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float f0 = sm.fix[wv][m32], f1 = sm.fix[wv][32 + m32];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (fr_row(mt, i, half) == r) { acc[mt][0][i] = f0; acc[mt][1][i] = f1; }
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---------------------------------------------------------------- norm + RoPE
  // the bf16 projection (the linear layer's output dtype), non-finite -> 0
  float v[32];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float x0 = fr_finite(fr_rb16(acc[mt][0][i]));
      const float x1 = fr_finite(fr_rb16(acc[mt][1][i]));
      acc[mt][0][i] = x0;
      acc[mt][1][i] = x1;
      v[16 * mt + i] = x0 * x0 + x1 * x1;
    }
  const int my_row = fr_row(m32 >> 4, m32 & 15, half);
  sm.part[side][part][my_row] = fr_reduce_scatter32(v);
  __syncthreads();
  {
    const float ss = (sm.part[side][0][my_row] + sm.part[side][1][my_row]);
    sm.r[wv][my_row] = rsqrtf(ss * (1.0f / kFrD) + a.eps);
  }
  __syncthreads();
  {
    const float* wn = side ? a.wk_n : a.wq_n;
    const float g0 = (1.0f + wn[d0]), g1 = (1.0f + wn[d1]);
    const bool bf = a.cs_bf16 != 0;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = fr_row(mt, i, half);
        const float r = sm.r[wv][row];
        float y0 = fminf(fmaxf((acc[mt][0][i] * r), -kActClamp), kActClamp);
        float y1 = fminf(fmaxf((acc[mt][1][i] * r), -kActClamp), kActClamp);
        y0 = fr_rb16(fminf(fmaxf((y0 * g0), -kActClamp), kActClamp));
        y1 = fr_rb16(fminf(fmaxf((y1 * g1), -kActClamp), kActClamp));
        if (a.cos) {
          float c0, c1, s0, s1;
          if (a.cs_lds) {
            c0 = __uint_as_float((uint32_t)sm.cs[0][row * kFrD + d0] << 16);
            c1 = __uint_as_float((uint32_t)sm.cs[0][row * kFrD + d1] << 16);
            s0 = __uint_as_float((uint32_t)sm.cs[1][row * kFrD + d0] << 16);
            s1 = __uint_as_float((uint32_t)sm.cs[1][row * kFrD + d1] << 16);
          } else {
            const int64_t o = (int64_t)b * a.cs_sb + (int64_t)min(t0 + row, a.S - 1) * a.cs_st;
            if (bf) {
              c0 = (float)((const bf16*)a.cos)[o + d0]; c1 = (float)((const bf16*)a.cos)[o + d1];
              s0 = (float)((const bf16*)a.sin)[o + d0]; s1 = (float)((const bf16*)a.sin)[o + d1];
            } else {
              c0 = ((const float*)a.cos)[o + d0]; c1 = ((const float*)a.cos)[o + d1];
              s0 = ((const float*)a.sin)[o + d0]; s1 = ((const float*)a.sin)[o + d1];
            }
          }
          // rotate_half: dim d0 (< 64) takes -y[d1], dim d1 takes y[d0]
          float p0 = (y0 * c0), p1 = (y1 * c1);
          float q0 = (-y1 * s0), q1 = (y0 * s1);
          if (bf) { p0 = fr_rb16(p0); p1 = fr_rb16(p1); q0 = fr_rb16(q0); q1 = fr_rb16(q1); }
          y0 = (p0 + q0);
          y1 = (p1 + q1);
          if (bf) { y0 = fr_rb16(y0); y1 = fr_rb16(y1); }
        }
        acc[mt][0][i] = fr_finite(y0);
        acc[mt][1][i] = fr_finite(y1);
      }
  }

  // ---------------------------------------------------------------- k_bar
  if (a.head_cls) {
    if (side == 1) {
      const float h0 = a.head_cls[d0], h1 = a.head_cls[d1];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[16 * mt + i] = acc[mt][0][i] * h0 + acc[mt][1][i] * h1;
      sm.part[1][part][my_row] = fr_reduce_scatter32(v);
    }
    __syncthreads();
    if (wv == 2) {
      // softmax over the valid rows of each block (bs = 32: lanes of a half; 64: all)
      const int row = lane;
      const bool ok = t0 + row < a.S;
      const float lg = fminf(fmaxf((sm.part[1][0][row] + sm.part[1][1][row]) * a.inv_sqrt_d,
                                   -kActClamp), kActClamp);
      float m = ok ? lg : -INFINITY;
#pragma unroll
      for (int k = 16; k >= 1; k >>= 1) m = fmaxf(m, __shfl_xor(m, k, kWave));
      if (a.bs == 64) m = fmaxf(m, __shfl_xor(m, 32, kWave));
      const float e = ok ? expf(lg - m) : 0.f;
      float den = e;
#pragma unroll
      for (int k = 16; k >= 1; k >>= 1) den += __shfl_xor(den, k, kWave);
      if (a.bs == 64) den += __shfl_xor(den, 32, kWave);
      sm.wgt[row] = ok ? e / fmaxf(den, 1e-6f) : 0.f;
    }
    __syncthreads();
    if (side == 1) {
      float s[2][2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          float acc_s = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i)
            acc_s = acc_s + sm.wgt[fr_row(mt, i, half)] * acc[mt][nt][i];
          s[mt][nt] = (acc_s + __shfl_xor(acc_s, 32, kWave));
        }
      if (half == 0) {
        float* kb = a.kbar + (int64_t)b * a.kb_sb;
        if (a.bs == 32) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt)
            if (t0 + 32 * mt < a.S) {
              float* o = kb + (int64_t)(t0 / 32 + mt) * kFrD;
              o[d0] = fr_finite(s[mt][0]);
              o[d1] = fr_finite(s[mt][1]);
            }
        } else {
          float* o = kb + (int64_t)(t0 / 64) * kFrD;
          o[d0] = fr_finite((s[0][0] + s[1][0]));
          o[d1] = fr_finite((s[0][1] + s[1][1]));
        }
      }
    }
  }
  // outputs: idx_q / idx_k rows
  {
    float* dst = side ? a.ik : a.iq;
    const int64_t dsb = side ? a.ik_sb : a.iq_sb;
    if (dst) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = t0 + fr_row(mt, i, half);
          if (t < a.S) {
            float* o = dst + (int64_t)b * dsb + (int64_t)t * kFrD;
            o[d0] = acc[mt][0][i];
            o[d1] = acc[mt][1][i];
          }
        }
    }
  }
}

// Packed weights: for chunk c (64 hidden columns), wavefront w, k-step s and
// n-tile nt, a 1 KB block whose 16-byte piece l is lane l's B operand:
// row (w / 2 ? k_proj : q_proj)[64 nt + 32 (w % 2) + l % 32],
// columns 64 c + 16 s + 8 (l / 32) + [0, 8).
__global__ __launch_bounds__(256) void front_pack_kernel(const bf16* __restrict__ wq,
                                                         const bf16* __restrict__ wk, int hid,
                                                         bf16* __restrict__ out) {
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;     // 16-byte piece
  if (p >= (int64_t)hid * 32) return;
  const int l = (int)(p & 63);
  int64_t rest = p >> 6;
  const int nt = (int)(rest & 1); rest >>= 1;
  const int s = (int)(rest & 3); rest >>= 2;
  const int w = (int)(rest & 3);
  const int c = (int)(rest >> 2);
  const int row = 64 * nt + 32 * (w & 1) + (l & 31);
  const int k = 64 * c + 16 * s + 8 * (l >> 5);
  const bf16* src = ((w >> 1) ? wk : wq) + (int64_t)row * hid + k;
  *(uint4*)(out + p * 8) = *(const uint4*)src;
}

}  // namespace dash

namespace {
inline int front_launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? dash::kOk : (int)e;
}
}  // namespace

extern "C" int dash_router_front_pack_weights(const void* w_q, const void* w_k, int hidden,
                                              void* w_pack, void* stream) {
  using namespace dash;
  if (!w_q || !w_k || !w_pack || hidden <= 0) return kErrInvalid;
  if (hidden % kFrKc != 0) return kErrUnsupported;
  if ((uintptr_t)w_q % 16 != 0 || (uintptr_t)w_k % 16 != 0 || (uintptr_t)w_pack % 16 != 0)
    return kErrUnsupported;
  const int64_t pieces = (int64_t)hidden * 32;
  hipLaunchKernelGGL(front_pack_kernel, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16*)w_q, (const bf16*)w_k, hidden,
                     (bf16*)w_pack);
  return front_launch_status();
}

extern "C" int dash_router_front(const void* hs, int64_t hs_sb, int64_t hs_st, int B, int S,
                                 int hidden, const void* w_pack, const void* w_q,
                                 const void* w_k, const float* wq_norm, const float* wk_norm,
                                 float eps, const void* cos, const void* sin, int cs_bf16,
                                 int64_t cs_sb, int64_t cs_st, const float* head_cls,
                                 int block_size, float inv_sqrt_d, float* idx_q, int64_t iq_sb,
                                 float* idx_k, int64_t ik_sb, float* kbar, int64_t kb_sb,
                                 int nblk_cap, void* stream) {
  using namespace dash;
  if (!hs || !w_pack || !w_q || !w_k || !wq_norm || !wk_norm || B < 0 || S < 0 || hidden <= 0)
    return kErrInvalid;
  if ((cos == nullptr) != (sin == nullptr)) return kErrInvalid;
  if (hidden % kFrKc != 0) return kErrUnsupported;
  if (hs_st % 8 != 0 || hs_sb % 8 != 0 || (uintptr_t)hs % 16 != 0 || (uintptr_t)w_pack % 16 != 0 ||
      (uintptr_t)w_q % 16 != 0 || (uintptr_t)w_k % 16 != 0)
    return kErrUnsupported;
  if (head_cls) {
    if (block_size != 32 && block_size != 64) return kErrUnsupported;
    if (!kbar) return kErrInvalid;
    if (nblk_cap < (S + block_size - 1) / block_size || kb_sb < (int64_t)nblk_cap * kFrD)
      return kErrInvalid;
  } else if (kbar) {
    return kErrInvalid;
  }
  if (idx_q && iq_sb < (int64_t)S * kFrD) return kErrInvalid;
  if (idx_k && ik_sb < (int64_t)S * kFrD) return kErrInvalid;
  if (B == 0 || S == 0) return kOk;
  FrontArgs a;
  a.hs = (const bf16*)hs; a.hs_sb = hs_sb; a.hs_st = hs_st; a.B = B; a.S = S; a.hid = hidden;
  a.w = (const bf16*)w_pack; a.wq = (const bf16*)w_q; a.wk = (const bf16*)w_k;
  a.wq_n = wq_norm; a.wk_n = wk_norm; a.eps = eps;
  a.cos = cos; a.sin = sin; a.cs_bf16 = cs_bf16; a.cs_sb = cs_sb; a.cs_st = cs_st;
  // bf16 cos / sin with 16-byte aligned rows go through LDS
  a.cs_lds = cos && cs_bf16 && cs_st % 8 == 0 && cs_sb % 8 == 0 &&
             (uintptr_t)cos % 16 == 0 && (uintptr_t)sin % 16 == 0;
  a.head_cls = head_cls; a.bs = block_size; a.inv_sqrt_d = inv_sqrt_d;
  a.iq = idx_q; a.iq_sb = iq_sb; a.ik = idx_k; a.ik_sb = ik_sb;
  a.kbar = kbar; a.kb_sb = kb_sb;
  a.ntiles = (S + kFrRows - 1) / kFrRows;
  const int64_t grid = (int64_t)B * a.ntiles;
  if (grid > 0x7fffffff) return kErrUnsupported;
  hipLaunchKernelGGL(router_front_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     a);
  return front_launch_status();
}
