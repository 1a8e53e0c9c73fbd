// DASH router kernels: stage-0 block summaries, block scores and 1.5-entmax
// routing.  Written for gfx950 (wave64).
//
//   kbar_kernel        k_bar = softmax(k.head_cls/sqrt(d)) pooling per key block
//                      (dash_attention.py:851-888, modeling_deepseekv2.py:362-377)
//   scores_kernel      z = clamp(q.k_bar/sqrt(d)), remote-block mask
//                      (modeling_deepseekv2.py:378-386)
//   blockmax_kernel    indexer stage-0: per-block max of q.k over non-local keys
//                      (modeling_deepseekv2.py:387-400, sparse_gather_triton.py:395-428)
//   route_kernel       top-M selection + 1.5-entmax + top-K + centred log-prior bias
//                      (modeling_deepseekv2.py:309-333, dash_attention.py:615-662)

#include "dash_common.h"

#include <atomic>
#include <mutex>
#include "dash_decode_unit.h"

namespace dash {

// ---------------------------------------------------------------------------
// k_bar: one work-group (256 threads) per (key block, sequence).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void kbar_kernel(
    const float* __restrict__ idx_k, SeqLayout lay, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ lens, const float* __restrict__ head_cls, int S, int d,
    int bs, int tail_only, float inv_sqrt_d, float* __restrict__ kbar, int64_t kb_sb) {
  __shared__ float s_aw[256];
  __shared__ float s_red[2];
  const int b = blockIdx.y;
  const int len = seq_length(cu, lens, b, S);
  if (len <= 0) return;
  const int c = tail_only ? (len - 1) / bs : (int)blockIdx.x;
  const int t0 = c * bs;
  if (t0 >= len) return;
  const int n = min(bs, len - t0);
  const int lane = wave_lane();
  const int wv = threadIdx.x / kWave;

  // per-token logits aw_j = clamp((k_j . head_cls) / sqrt(d), +-1e4)
  for (int j = wv; j < n; j += 4) {
    const float* kr = idx_k + lay.row(b, t0 + j);
    float acc = 0.f;
    for (int i = lane; i < d; i += kWave) acc += kr[i] * head_cls[i];
    acc = wave_sum(acc);
    if (lane == 0) s_aw[j] = fminf(fmaxf(acc * inv_sqrt_d, -kActClamp), kActClamp);
  }
  __syncthreads();
  if (threadIdx.x < kWave) {
    float m = -INFINITY;
    for (int j = lane; j < n; j += kWave) m = fmaxf(m, s_aw[j]);
    m = wave_max(m);
    float sum = 0.f;
    for (int j = lane; j < n; j += kWave) sum += expf(s_aw[j] - m);
    sum = wave_sum(sum);
    if (lane == 0) { s_red[0] = m; s_red[1] = fmaxf(sum, 1e-6f); }
  }
  __syncthreads();
  const float m = s_red[0], den = s_red[1];
  for (int j = threadIdx.x; j < n; j += blockDim.x) s_aw[j] = expf(s_aw[j] - m) / den;
  __syncthreads();
  for (int i = threadIdx.x; i < d; i += blockDim.x) {
    float acc = 0.f;
    for (int j = 0; j < n; ++j) acc += s_aw[j] * idx_k[lay.row(b, t0 + j) + i];
    if (!(fabsf(acc) <= 3.402823466e38f)) acc = 0.f;   // nan_to_num(nan/inf -> 0)
    kbar[(int64_t)b * kb_sb + (int64_t)c * d + i] = acc;
  }
}

// ---------------------------------------------------------------------------
// k_bar for d = 128 and blocks of at most 64 keys: the block's key rows are
// staged once in LDS with every load in flight together, then read twice (the
// logits, with four lanes per key, and the weighted sum, with eight key groups
// per dimension quad).  Same results as kbar_kernel up to summation order.
// ---------------------------------------------------------------------------
constexpr int kKbD = 128;
constexpr int kKbMaxBs = 64;

__global__ __launch_bounds__(256) void kbar128_kernel(
    const float* __restrict__ idx_k, SeqLayout lay, const int32_t* __restrict__ cu,
    const int32_t* __restrict__ lens, const float* __restrict__ head_cls, int S, int bs,
    int tail_only, float inv_sqrt_d, float* __restrict__ kbar, int64_t kb_sb) {
  __shared__ float4 s_k[kKbMaxBs][kKbD / 4 + 1];
  __shared__ float s_w[kKbMaxBs];
  __shared__ float4 s_part[8][kKbD / 4];
  const int b = blockIdx.y;
  const int len = seq_length(cu, lens, b, S);
  if (len <= 0) return;
  const int c = tail_only ? (len - 1) / bs : (int)blockIdx.x;
  const int t0 = c * bs;
  if (t0 >= len) return;
  const int n = min(bs, len - t0);
  const int tid = threadIdx.x, lane = wave_lane();

  // stage: 8 float4 per thread, all issued before the first LDS write
  float4 buf[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int e = tid + 256 * u, j = e / 32, f = e % 32;
    buf[u] = j < n ? reinterpret_cast<const float4*>(idx_k + lay.row(b, t0 + j))[f]
                   : make_float4(0.f, 0.f, 0.f, 0.f);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int e = tid + 256 * u;
    s_k[e / 32][e % 32] = buf[u];
  }
  __syncthreads();

  // logits: key j = tid / 4, lanes 4j..4j+3 take float4 columns q, q+4, ..., q+28
  {
    const int j = tid / 4, q = tid % 4;
    const float4* hc = reinterpret_cast<const float4*>(head_cls);
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 kv = s_k[j][q + 4 * u], h = hc[q + 4 * u];
      acc += kv.x * h.x + kv.y * h.y + kv.z * h.z + kv.w * h.w;
    }
    acc += __shfl_xor(acc, 1, kWave);
    acc += __shfl_xor(acc, 2, kWave);
    if (q == 0 && j < n) s_w[j] = fminf(fmaxf(acc * inv_sqrt_d, -kActClamp), kActClamp);
  }
  __syncthreads();
  // softmax over the n logits (wave 0), weights left in s_w
  if (tid < kWave) {
    const float x = lane < n ? s_w[lane] : -INFINITY;
    const float m = wave_max(x);
    const float e = lane < n ? expf(x - m) : 0.f;
    const float den = fmaxf(wave_sum(e), 1e-6f);
    if (lane < n) s_w[lane] = e / den;
  }
  __syncthreads();
  // weighted sum: group g = tid / 32 takes keys g, g+8, ...; f = float4 column
  {
    const int g = tid / 32, f = tid % 32;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = g; j < n; j += 8) {
      const float w = s_w[j];
      const float4 kv = s_k[j][f];
      acc.x += w * kv.x; acc.y += w * kv.y; acc.z += w * kv.z; acc.w += w * kv.w;
    }
    s_part[g][f] = acc;
  }
  __syncthreads();
  if (tid < kKbD) {
    const float* sp = reinterpret_cast<const float*>(&s_part[0][0]);
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 8; ++g) acc += sp[g * kKbD + tid];
    if (!(fabsf(acc) <= 3.402823466e38f)) acc = 0.f;   // nan_to_num(nan/inf -> 0)
    kbar[(int64_t)b * kb_sb + (int64_t)c * kKbD + tid] = acc;
  }
}

// ---------------------------------------------------------------------------
// head_cls block scores: 64 query rows x 64 key blocks per work-group, fp32 FMA.
// Tiles whose blocks are all beyond every row's causal limit only write the
// sentinel.  VEC: d % 16 == 0 and 16-byte aligned rows, staged with float4 loads
// one k-slice ahead.
// ---------------------------------------------------------------------------
constexpr int kScTile = 64;
constexpr int kScK = 16;
constexpr int kScPad = kScTile + 4;

template <bool VEC>
__global__ __launch_bounds__(256) void scores_kernel(
    const float* __restrict__ idx_q, SeqLayout lay_q, const int32_t* __restrict__ cu_q,
    int Lq, const int32_t* __restrict__ q_pos, const float* __restrict__ kbar, int64_t kb_sb,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ lens_k, int S, int d,
    int bs, int local_blocks, int nblk_cap, float inv_sqrt_d, float* __restrict__ z,
    int64_t z_stride) {
  __shared__ __align__(16) float sq[kScK][kScPad];
  __shared__ __align__(16) float sk[kScK][kScPad];
  const int b = blockIdx.z;
  const int nq = cu_q ? (cu_q[b + 1] - cu_q[b]) : Lq;
  const int r0 = blockIdx.x * kScTile;
  const int c0 = blockIdx.y * kScTile;
  if (r0 >= nq) return;
  const int klen = seq_length(cu_k, lens_k, b, S);
  const int nblk_b = (klen + bs - 1) / bs;
  const int tid = threadIdx.x;
  const int tx = tid % 16, ty = tid / 16;

  int lim[4];
  int my_max = INT_MIN;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty * 4 + i;
    lim[i] = INT_MIN;
    if (r < nq) {
      const int pos = q_pos ? q_pos[token_row(cu_q, b, r, Lq)] : r;
      lim[i] = (pos >= 0 ? pos / bs : -((-pos + bs - 1) / bs)) - local_blocks;
      my_max = max(my_max, lim[i]);
    }
  }
  if (!__syncthreads_or(c0 <= my_max && c0 < nblk_b)) {
    for (int e = tid; e < kScTile * kScTile; e += 256) {
      const int r = r0 + e / kScTile, c = c0 + e % kScTile;
      if (r < nq && c < nblk_cap) z[token_row(cu_q, b, r, Lq) * z_stride + c] = kScoreNeg;
    }
    return;
  }

  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;

  const int srr = tid / 4, skq = tid % 4;   // VEC staging: row srr, dims 4*skq..+3
  const bool q_ok = r0 + srr < nq, k_ok = c0 + srr < nblk_cap;
  const float* qrow = q_ok ? idx_q + lay_q.row(b, r0 + srr) + 4 * skq : nullptr;
  const float* krow = k_ok ? kbar + (int64_t)b * kb_sb + (int64_t)(c0 + srr) * d + 4 * skq
                           : nullptr;
  float4 qn = make_float4(0.f, 0.f, 0.f, 0.f), kn = qn;
  if (VEC) {
    if (q_ok) qn = *reinterpret_cast<const float4*>(qrow);
    if (k_ok) kn = *reinterpret_cast<const float4*>(krow);
  }
  for (int k0 = 0; k0 < d; k0 += kScK) {
    if (VEC) {
      sq[4 * skq + 0][srr] = qn.x; sq[4 * skq + 1][srr] = qn.y;
      sq[4 * skq + 2][srr] = qn.z; sq[4 * skq + 3][srr] = qn.w;
      sk[4 * skq + 0][srr] = kn.x; sk[4 * skq + 1][srr] = kn.y;
      sk[4 * skq + 2][srr] = kn.z; sk[4 * skq + 3][srr] = kn.w;
      if (k0 + kScK < d) {
        if (q_ok) qn = *reinterpret_cast<const float4*>(qrow + k0 + kScK);
        if (k_ok) kn = *reinterpret_cast<const float4*>(krow + k0 + kScK);
      }
    } else {
      for (int e = tid; e < kScTile * kScK; e += 256) {
        const int rr = e / kScK, kk = e % kScK;
        const int r = r0 + rr, c = c0 + rr, dd = k0 + kk;
        float qv = 0.f, kv = 0.f;
        if (r < nq && dd < d) qv = idx_q[lay_q.row(b, r) + dd];
        if (c < nblk_cap && dd < d) kv = kbar[(int64_t)b * kb_sb + (int64_t)c * d + dd];
        sq[kk][rr] = qv;
        sk[kk][rr] = kv;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kScK; ++kk) {
      const float4 a = *reinterpret_cast<const float4*>(&sq[kk][ty * 4]);
      const float4 bb = *reinterpret_cast<const float4*>(&sk[kk][tx * 4]);
      const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + ty * 4 + i;
    if (r >= nq) continue;
    const int64_t row = token_row(cu_q, b, r, Lq);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = c0 + tx * 4 + j;
      if (c >= nblk_cap) continue;
      float v = kScoreNeg;
      if (c <= lim[i] && c < nblk_b) {
        v = acc[i][j] * inv_sqrt_d;
        v = fminf(fmaxf(v, -kActClamp), kActClamp);
      }
      z[row * z_stride + c] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Block scores for d = 128 on the matrix cores.  Every fp32 operand is split into
// three bf16 parts x = x_h + x_m + x_l (each part the round-to-nearest of what the
// previous ones leave; together they hold the 24-bit significand), and q.k is
// the fp32-accumulated sum of the six products with x_i y_j for i + j <= 2
// (h = 0, m = 1, l = 2); the dropped ones are below 2^-24 of the product, so the
// result is an fp32-accurate dot product.  A work-group covers 128 query rows x 64
// blocks: the 64 k_bar rows are split once into three swizzled LDS planes (16-byte
// chunk c of block row n at slot c ^ (n % 16)), and each wavefront multiplies its
// 32 rows, split in registers 8 dims at a time, with v_mfma_f32_32x32x16_bf16.
// Tiles beyond every row's causal limit only write the sentinel.
// ---------------------------------------------------------------------------
constexpr int kSmRows = 128, kSmBlk = 64;

__device__ __forceinline__ void split3(float x, __bf16& h, __bf16& m, __bf16& l) {
  h = (__bf16)x;
  const float r1 = x - (float)h;
  m = (__bf16)r1;
  l = (__bf16)(r1 - (float)m);
}

__global__ __launch_bounds__(256) void scores_mfma_kernel(
    const float* __restrict__ idx_q, SeqLayout lay_q, const int32_t* __restrict__ cu_q, int Lq,
    const int32_t* __restrict__ q_pos, const float* __restrict__ kbar, int64_t kb_sb,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ lens_k, int S, int bs,
    int local_blocks, int nblk_cap, float inv_sqrt_d, float* __restrict__ z, int64_t z_stride) {
  __shared__ __attribute__((aligned(16))) bf16 sK[3][kSmBlk * 128];
  __shared__ int sLim[kSmRows];
  const int b = blockIdx.z;
  const int nq = cu_q ? (cu_q[b + 1] - cu_q[b]) : Lq;
  const int r0 = blockIdx.x * kSmRows;
  const int c0 = blockIdx.y * kSmBlk;
  if (r0 >= nq) return;
  const int klen = seq_length(cu_k, lens_k, b, S);
  const int nblk_b = (klen + bs - 1) / bs;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  int my_max = INT_MIN;
  if (tid < kSmRows) {
    const int r = r0 + tid;
    int lim = INT_MIN;
    if (r < nq) {
      const int pos = q_pos ? q_pos[token_row(cu_q, b, r, Lq)] : r;
      lim = (pos >= 0 ? pos / bs : -((-pos + bs - 1) / bs)) - local_blocks;
    }
    sLim[tid] = lim;
    my_max = lim;
  }
  if (!__syncthreads_or(c0 <= my_max && c0 < nblk_b)) {
    for (int e = tid; e < kSmRows * kSmBlk; e += 256) {
      const int r = r0 + e / kSmBlk, c = c0 + e % kSmBlk;
      if (r < nq && c < nblk_cap) z[token_row(cu_q, b, r, Lq) * z_stride + c] = kScoreNeg;
    }
    return;
  }
  // this wavefront's 32 query rows: lane (m, half) holds dims 16 kk + 8 half .. +7;
  // its 64 dims are loaded now, in flight during the k_bar split
  const int mrow = lane & 31, half = lane >> 5;
  const int rq = min(r0 + wv * 32 + mrow, nq - 1);
  const float* qr = idx_q + lay_q.row(b, rq) + 8 * half;
  float4 qv[16];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    qv[2 * kk] = *(const float4*)(qr + 16 * kk);
    qv[2 * kk + 1] = *(const float4*)(qr + 16 * kk + 4);
  }
  // the 64 k_bar rows, split into the three planes (rows past nblk_cap are zero)
  float4 kv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = (tid + 256 * j) * 4;          // element of the 64 x 128 tile
    const int n = e / 128, k = e % 128;
    kv[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c0 + n < nblk_cap) kv[j] = *(const float4*)(kbar + (int64_t)b * kb_sb + (int64_t)(c0 + n) * 128 + k);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int e = (tid + 256 * j) * 4;
    const int n = e / 128, k = e % 128;
    const float4 v = kv[j];
    const float xs[4] = {v.x, v.y, v.z, v.w};
    bf16x4 ph, pm, pl;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      __bf16 h, m, l;
      split3(xs[u], h, m, l);
      ph[u] = h; pm[u] = m; pl[u] = l;
    }
    const int off = n * 128 + (((k >> 3) ^ (n & 15)) << 3) + (k & 7);
    *(bf16x4*)(&sK[0][off]) = ph;
    *(bf16x4*)(&sK[1][off]) = pm;
    *(bf16x4*)(&sK[2][off]) = pl;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(qv[i].x), "+v"(qv[i].y), "+v"(qv[i].z), "+v"(qv[i].w));
  floatx16 acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.f;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const float4 qa = qv[2 * kk], qb = qv[2 * kk + 1];
    const float xs[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    bf16x8 ah, am, al;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      __bf16 h, m, l;
      split3(xs[u], h, m, l);
      ah[u] = h; am[u] = m; al[u] = l;
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int n = t * 32 + mrow;
      const int off = n * 128 + (((2 * kk + half) ^ (n & 15)) << 3);
      const bf16x8 bh = *(const bf16x8*)(&sK[0][off]);
      const bf16x8 bm = *(const bf16x8*)(&sK[1][off]);
      const bf16x8 bl = *(const bf16x8*)(&sK[2][off]);
      // smallest terms first
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bm, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(am, bh, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bm, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc[t], 0, 0, 0);
    }
  }
  // C layout: lane l holds block column l % 32 of each 32-block tile, rows
  // 8 (i / 4) + 4 (l / 32) + i % 4.  The wavefront's 32 x 64 scores pass through
  // its 8 KB of the (now idle) k_bar planes, so that each store writes four whole
  // 256-byte row pieces.
  __syncthreads();                         // every wavefront is done with the planes
  float* const so = (float*)&sK[0][0] + wv * 32 * kSmBlk;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int cl = t * 32 + mrow, c = c0 + cl;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = 8 * (i >> 2) + 4 * half + (i & 3);
      float v = kScoreNeg;
      if (c <= sLim[wv * 32 + rr] && c < nblk_b)
        v = fminf(fmaxf(acc[t][i] * inv_sqrt_d, -kActClamp), kActClamp);
      so[rr * kSmBlk + cl] = v;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int cq = (lane & 15) * 4;          // four columns per lane
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int rr = 4 * k + (lane >> 4);
    const int r = r0 + wv * 32 + rr;
    const float4 v = *(const float4*)(so + rr * kSmBlk + cq);
    if (r < nq) {
      float* zr = z + token_row(cu_q, b, r, Lq) * z_stride + c0 + cq;
      if (c0 + cq + 3 < nblk_cap && ((uintptr_t)zr & 15) == 0) {
        *(float4*)zr = v;
      } else {
        const float vs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c0 + cq + u < nblk_cap) zr[u] = vs[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Indexer stage-0 block scores: per-block max of q.k_j over keys j < ls(t)
// (ls = pos - LW + 1), optionally j >= seg[t].  mode 0: torch form (clamp to
// +-1e4, SCORE_NEG for empty blocks); mode 1: fused-kernel form (no clamp,
// -inf for empty blocks).  One work-group per (64 query rows, key block).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void blockmax_kernel(
    const float* __restrict__ q, SeqLayout lay_q, int C, const int32_t* __restrict__ pos,
    const int32_t* __restrict__ seg, int64_t ps_sb, const float* __restrict__ k,
    SeqLayout lay_k, int Sk, int d, int bs, int lw, int nblk, int mode,
    float* __restrict__ out, int64_t o_sb, int64_t o_sc) {
  __shared__ float sq[kScK][kScTile + 1];
  __shared__ float sk[kScK][kScTile + 1];
  __shared__ float smax[kScTile][17];
  const int b = blockIdx.z;
  const int r0 = blockIdx.x * kScTile;
  const int c = blockIdx.y;
  if (r0 >= C) return;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  const float empty = mode == 0 ? kScoreNeg : -INFINITY;
  float best[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) best[i] = -INFINITY;
  int lsr[4], sgr[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = min(r0 + ty * 4 + i, C - 1);
    const int p = pos[(int64_t)b * ps_sb + r];
    lsr[i] = max(p - lw + 1, 0);
    sgr[i] = seg ? seg[(int64_t)b * ps_sb + r] : 0;
  }
  for (int j0 = c * bs; j0 < min((c + 1) * bs, Sk); j0 += kScTile) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    const int jend = min(min((c + 1) * bs, Sk), j0 + kScTile);
    for (int k0 = 0; k0 < d; k0 += kScK) {
      for (int e = threadIdx.x; e < kScTile * kScK; e += 256) {
        const int rr = e / kScK, kk = e % kScK;
        const int r = r0 + rr, j = j0 + rr, dd = k0 + kk;
        sq[kk][rr] = (r < C && dd < d) ? q[lay_q.row(b, r) + dd] : 0.f;
        sk[kk][rr] = (j < jend && dd < d) ? k[lay_k.row(b, j) + dd] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kScK; ++kk) {
        float a[4], bb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = sq[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) bb[j] = sk[kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], bb[j], acc[i][j]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = j0 + tx * 4 + j;
        if (key < jend && key < lsr[i] && key >= sgr[i]) {
          float v = acc[i][j];
          if (mode == 0) v = fminf(fmaxf(v, -kActClamp), kActClamp);
          best[i] = fmaxf(best[i], v);
        }
      }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) smax[ty * 4 + i][tx] = best[i];
  __syncthreads();
  if (threadIdx.x < kScTile) {
    const int r = r0 + threadIdx.x;
    if (r < C) {
      float m = -INFINITY;
      for (int j = 0; j < 16; ++j) m = fmaxf(m, smax[threadIdx.x][j]);
      out[(int64_t)b * o_sb + (int64_t)r * o_sc + c] = (m == -INFINITY) ? empty : m;
    }
  }
}

// ---------------------------------------------------------------------------
// Routing: one wavefront per query row.
// ---------------------------------------------------------------------------
constexpr int kMaxM = 16;


// 1.5-entmax over M values sorted in descending order follows the fp32 sequence
// of dash_attention.py:623-647 on the CPU: X = (x - max)/2, cumsums accumulated in
// double and rounded to fp32, every other operation a single correctly rounded fp32
// operation (no contraction).  The kernels below hold entry m on lane m, each lane
// forming its own prefix sums in the serial order, so the result is the serial one
// bit for bit.

// Order-preserving key of a finite float: larger value -> larger key; -0 and +0
// share a key (they compare equal).
__device__ __forceinline__ uint32_t ord_key(float x) {
  const uint32_t b = x == 0.f ? 0u : __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int lane_prefix(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
}

// DPP controls: quad_perm [1,0,3,2] and [2,3,0,1]; row_ror 4 and 8.
#define DASH_DPP(v, c) ((uint32_t)__builtin_amdgcn_mov_dpp((int)(v), c, 0xf, 0xf, false))
__device__ __forceinline__ uint32_t quad_max_u32(uint32_t v) {
  v = max(v, DASH_DPP(v, 0xB1));
  return max(v, DASH_DPP(v, 0x4E));
}
// For values uniform within each quad: min / max over the wavefront, uniform.
__device__ __forceinline__ uint32_t wave_min_of_quads(uint32_t v) {
  v = min(v, DASH_DPP(v, 0x124));
  v = min(v, DASH_DPP(v, 0x128));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return min(min(a, b), min(c, d));
}
__device__ __forceinline__ uint32_t wave_max_of_quads(uint32_t v) {
  v = max(v, DASH_DPP(v, 0x124));
  v = max(v, DASH_DPP(v, 0x128));
  const uint32_t a = __builtin_amdgcn_readlane(v, 0), b = __builtin_amdgcn_readlane(v, 16);
  const uint32_t c = __builtin_amdgcn_readlane(v, 32), d = __builtin_amdgcn_readlane(v, 48);
  return max(max(a, b), max(c, d));
}
#undef DASH_DPP

// Largest T with #{keys >= T} >= M over the wavefront's keys (NV per lane, 0 =
// absent), given a lower bound t_lo with #{keys >= t_lo} >= M and the maximum
// key t_hi.  T shares the bits above the highest bit where t_lo and t_hi differ;
// the rest is found two bits per step with ballots.
template <int NV>
__device__ __forceinline__ uint32_t kth_key(const uint32_t (&h)[NV], int M, uint32_t t_lo,
                                            uint32_t t_hi) {
  const uint32_t diff = t_lo ^ t_hi;
  int nb = diff ? 32 - __clz(diff) : 0;
  uint32_t T = nb >= 32 ? 0u : (t_lo & ~((1u << nb) - 1u));
  auto count = [&](uint32_t t) {
    int n = 0;
#pragma unroll
    for (int i = 0; i < NV; ++i) n += __popcll(__ballot(h[i] >= t));
    return n;
  };
  while (nb >= 2) {
    nb -= 2;
    const uint32_t c3 = T | (3u << nb), c2 = T | (2u << nb), c1 = T | (1u << nb);
    const int n3 = count(c3), n2 = count(c2), n1 = count(c1);
    T = n3 >= M ? c3 : n2 >= M ? c2 : n1 >= M ? c1 : T;
    if (n3 == M || n2 == M || n1 == M) return T;
  }
  if (nb == 1) {
    const uint32_t c1 = T | 1u;
    if (count(c1) >= M) T = c1;
  }
  return T;
}

// Routing: work-groups of four wavefronts own 8 consecutive score rows, two per
// wavefront (more rows per wavefront lengthen each wavefront's serial chain; one
// row leaves three quarters of the lanes idle in phase 2).
//  Phase 1, one row at a time over the whole wavefront: every entry gets the
//  64-bit key  ord_key(x) << 32 | (0xffff - block id) << 1 | candidate  whose
//  descending order is (value desc, block id asc).  The top-M set is found
//  exactly without sorting:
//   * t0 = min over the 16 residue classes (block id mod 16) of the class
//     maximum.  At least 16 >= M entries reach t0, so the top M are among the
//     entries >= t0; these (at most 64, one per lane) are compacted in block-id
//     order and the M-th largest value key T among them is found by bisection
//     over its 32 bits with ballots;
//   * rows with more than 64 entries >= t0 (ties, e.g. fewer than 16 remote
//     blocks) run the same bisection over all their entries.
//  The entries above T and the lowest-id entries at T form the set, parked in
//  LDS.
//  Phase 2, each wavefront for its own rows, 16 lanes per row: rank sort of the M
//  keys, 1.5-entmax with entry m on lane m, first K, centred log-prior bias.
constexpr int kRtRowsPerWave = 2;
constexpr int kRtWaves = 4;
constexpr int kRtRows = kRtRowsPerWave * kRtWaves;

__device__ __forceinline__ float ord_key_inv(uint32_t h) {
  return __uint_as_float((h & 0x80000000u) ? (h & 0x7fffffffu) : ~h);
}

// Phase 1 for one row held by one wavefront: entry c = lane + 64 i has value key
// hi[i] (0: no entry) and candidate flag cb[i]; the M largest 64-bit keys
// hi << 32 | (0xffff - c) << 1 | cb (value descending, block id ascending) are
// written to sel[0 .. M) in no particular order.  s_cand: 64 entries of this
// wavefront's LDS.  Every lane of the wavefront calls it.
template <int NPL>
__device__ __forceinline__ void route_row_topm(const uint32_t (&hi)[NPL], const uint8_t (&cb)[NPL],
                                               int M, uint64_t* s_cand, uint64_t* sel) {
  const int lane = wave_lane();
  uint32_t cmx = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) cmx = max(cmx, hi[i]);
  // classes = lane quads (16 of them, all non-empty once the row has >= 61 entries):
  // t0 = the smallest class maximum (0 if a class is empty), kmax = the row maximum
  cmx = quad_max_u32(cmx);
  const uint32_t t0 = wave_min_of_quads(cmx);
  const uint32_t kmax = wave_max_of_quads(cmx);
  int nc = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool pass = hi[i] != 0u && hi[i] >= t0;
    const uint64_t mask = __ballot(pass);
    const int slot = nc + lane_prefix(mask);
    const int c = lane + kWave * i;
    if (pass && slot < kWave)
      s_cand[slot] = ((uint64_t)hi[i] << 32) | ((uint32_t)(0xffff - c) << 1) | cb[i];
    nc += __popcll(mask);
  }
  if (M == 0) {
  } else if (nc <= kWave) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint64_t mine = lane < nc ? s_cand[lane] : 0ull;
    const uint32_t h[1] = {(uint32_t)(mine >> 32)};
    const uint32_t T = kth_key<1>(h, M, t0, kmax);
    const int need_eq = M - __popcll(__ballot(h[0] > T));
    const bool eq = h[0] == T && lane < nc;
    const bool take = h[0] > T || (eq && lane_prefix(__ballot(eq)) < need_eq);
    const uint64_t mt = __ballot(take);
    if (take) sel[lane_prefix(mt)] = mine;
  } else {
    const uint32_t T = kth_key<NPL>(hi, M, t0, kmax);
    int n_gt = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) n_gt += __popcll(__ballot(hi[i] > T));
    const int need_eq = M - n_gt;
    int taken = 0, eq_seen = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const bool eq = hi[i] == T;
      const uint64_t meq = __ballot(eq);
      const bool take = hi[i] > T || (eq && eq_seen + lane_prefix(meq) < need_eq);
      const uint64_t mt = __ballot(take);
      const int c = lane + kWave * i;
      if (take)
        sel[taken + lane_prefix(mt)] = ((uint64_t)hi[i] << 32) | ((uint32_t)(0xffff - c) << 1) | cb[i];
      taken += __popcll(mt);
      eq_seen += __popcll(meq);
    }
  }
}

// Routing slots published inside one launch (the fused decode step).  Slot s of the
// routing is two 64-bit words, each with its top bit set: the block id + 1 (16 bits)
// and the valid flag (bit 16), and the bias bits.  They are stored and read as
// relaxed atomics at agent scope, which every work-group of the device sees
// coherently without a fence; a word holds the value it marks as published, so no
// ordering between words is needed.  The words are zero between steps: zeroed
// workspace before the first step, and the step's last launch zeroes the words it
// published.
constexpr uint64_t kPubBit = 1ull << 63;
__device__ __forceinline__ void publish_slot(uint64_t* pub, int64_t slot, int c, bool valid,
                                             float bias) {
  __hip_atomic_store(pub + 2 * slot, kPubBit | ((uint64_t)valid << 16) | (uint64_t)((uint32_t)(c + 1) & 0xffffu),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(pub + 2 * slot + 1, kPubBit | (uint64_t)__float_as_uint(bias), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

// Phase 2 of the inference routing for one row per 16-lane group (lane m = entry
// m): the row's M <= 16 selected keys sel[0..M) (any order; sorted in place) are
// ranked, then 1.5-entmax with entry m on lane m (each lane forms its prefix sums
// in the serial order, so the result is the serial one bit for bit), first K,
// centred log-prior bias; writes idx / bias / valid row `row` (Kout slots), and with
// pub also publishes them (publish_slot).  Every lane of the wavefront
// calls it (wavefront barriers inside).
__device__ __forceinline__ void route_finish(uint64_t* sel, int M, bool row_ok, int64_t row,
                                             float floor_p, float inv_sigma, int K, int Kout,
                                             int32_t* __restrict__ idx_out,
                                             float* __restrict__ bias_out,
                                             uint8_t* __restrict__ valid_out,
                                             uint64_t* pub = nullptr) {
#pragma clang fp contract(off)
  const int lane = wave_lane();
  const int m = lane & 15, gbase = lane & ~15;
  const uint64_t key = m < M ? sel[m] : 0ull;
  int rank = 0;
#pragma unroll
  for (int j = 0; j < kMaxM; ++j) {
    const uint64_t kj = row_ok ? sel[j] : 0ull;
    rank += (j < M && kj > key) ? 1 : 0;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (m < M) sel[rank] = key;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint64_t ks = m < M ? sel[m] : 0ull;           // entry m of the descending order
  const uint32_t kh = (uint32_t)(ks >> 32), kl = (uint32_t)ks;
  const float xv = m < M ? ord_key_inv(kh) : 0.f;
  const int sel_id = 0xffff - (int)((kl >> 1) & 0xffff);
  const bool sel_c = (kl & 1u) != 0;
  const float x0 = __shfl(xv, gbase, kWave);
  const float X = __fdiv_rn(__fsub_rn(xv, x0), 2.0f);
  double cs = 0.0, cs2 = 0.0;
#pragma unroll
  for (int j = 0; j < kMaxM; ++j) {
    const float Xj = __shfl(X, gbase + j, kWave);
    if (j <= m) {
      cs += (double)Xj;
      cs2 += (double)__fmul_rn(Xj, Xj);
    }
  }
  const int Me = max(M, 1);                  // entmax over at least one entry
  float tau = 0.f;
  bool sup = false;
  if (m < Me) {
    const float rho = (float)(m + 1);
    const float mean = __fdiv_rn((float)cs, rho);
    const float mean_sq = __fdiv_rn((float)cs2, rho);
    const float ss = __fmul_rn(rho, __fsub_rn(mean_sq, __fmul_rn(mean, mean)));
    const float delta = __fdiv_rn(__fsub_rn(1.0f, ss), rho);
    const float delta_nz = delta > 0.f ? delta : 0.f;
    tau = __fsub_rn(mean, __fsqrt_rn(delta_nz));
    sup = tau <= X;
  }
  const uint32_t grp = (uint32_t)(__ballot(sup) >> gbase) & 0xffffu;
  const int support = max(__popc(grp), 1);
  const float tau_star = __shfl(tau, gbase + support - 1, kWave);
  const float tt = __fsub_rn(X, tau_star);
  const float cc = tt > 0.f ? tt : 0.f;
  const float prior = m < M ? __fmul_rn(cc, cc) : 0.f;
  const float logp = logf(fmaxf(prior, floor_p));
  const int Kp = max(1, min(K, M));
  // mean log-prior of the kept candidate slots, summed in slot order
  const uint32_t keep = (uint32_t)(__ballot(m < Kp && m < M && sel_c) >> gbase) & 0xffffu;
  float musum = 0.f;
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < kMaxM; ++j) {
    const float lj = __shfl(logp, gbase + j, kWave);
    if ((keep >> j) & 1u) { musum += lj; ++cnt; }
  }
  const float mu = musum / (float)max(cnt, 1);
  if (!row_ok) return;
  int32_t* io = idx_out + row * Kout;
  float* bo = bias_out + row * Kout;
  uint8_t* vo = valid_out ? valid_out + row * Kout : nullptr;
  if (m < Kout) {
    const bool in = m < Kp && m < M;
    const bool va = in && sel_c;
    io[m] = in ? sel_id : -1;
    bo[m] = va ? (logp - mu) * inv_sigma : 0.f;
    if (vo) vo[m] = va ? 1 : 0;
    if (pub) publish_slot(pub, row * Kout + m, in ? sel_id : -1, vo ? va : true,
                          va ? (logp - mu) * inv_sigma : 0.f);
  }
  for (int mm = kMaxM + m; mm < Kout; mm += kMaxM) {
    io[mm] = -1;
    bo[mm] = 0.f;
    if (vo) vo[mm] = 0;
    if (pub) publish_slot(pub, row * Kout + mm, -1, false, 0.f);
  }
}

template <int NPL>
__global__ __launch_bounds__(kRtWaves * kWave) void route_kernel(
    const float* __restrict__ z, int64_t z_stride, int rows, int nblk_cols,
    const int32_t* __restrict__ row_nblk, const uint8_t* __restrict__ cand_in,
    int64_t cand_stride, float idx_scale, float floor_p, float inv_sigma, int K, int topm,
    int Kout, int32_t* __restrict__ idx_out, float* __restrict__ bias_out,
    uint8_t* __restrict__ valid_out) {
  __shared__ uint64_t s_cand[kRtWaves][kWave];
  __shared__ uint64_t s_sel[kRtRows][kMaxM];
  __shared__ int s_M[kRtRows];
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
  const int wg_row0 = blockIdx.x * kRtRows;
  const int row0 = wg_row0 + wv * kRtRowsPerWave;
  const int nrow = max(0, min(kRtRowsPerWave, rows - row0));

  // Score loads are unconditional (column clamped into the row).  For rows of up
  // to 512 blocks the loads of all of this wavefront's rows are issued together
  // up front; wider rows load one row at a time.
  constexpr bool kAllRows = NPL <= 8;
  constexpr int kBuf = kAllRows ? kRtRowsPerWave : 1;
  float zb[kBuf][NPL];
  int nb_rows[kBuf];
  auto fetch = [&](int slot, int row) {
    const float* zr = z + (int64_t)row * z_stride;
#pragma unroll
    for (int i = 0; i < NPL; ++i) zb[slot][i] = zr[min(lane + kWave * i, nblk_cols - 1)];
    nb_rows[slot] = row_nblk ? row_nblk[row] : nblk_cols;
  };
  if (kAllRows) {
#pragma unroll
    for (int rr = 0; rr < kBuf; ++rr)
      if (rr < nrow) fetch(rr, row0 + rr);
  }
#pragma unroll
  for (int rr = 0; rr < kRtRowsPerWave; ++rr) {
    if (rr >= nrow) break;
    const int sr = wv * kRtRowsPerWave + rr;   // row slot in the work-group
    const int row = row0 + rr;
    const int bs_ = kAllRows ? rr : 0;
    if (!kAllRows) fetch(0, row);
    float zv[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) zv[i] = zb[bs_][i];
    const int nn = nb_rows[bs_];
    const int nblk = max(0, min(__builtin_amdgcn_readfirstlane(nn), nblk_cols));
    uint8_t cb[NPL];
    if (cand_in) {
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        cb[i] = cand_in[(int64_t)row * cand_stride + min(lane + kWave * i, nblk_cols - 1)];
    }
    bool any_cand = false;
    if (cand_in) {
#pragma unroll
      for (int i = 0; i < NPL; ++i)
        any_cand |= (lane + kWave * i < nblk) && zv[i] > kScoreNeg * 0.5f && cb[i] != 0;
    }
    // rows without any candidate fall back to every remote block
    const bool use_cand = cand_in && __any(any_cand);
    uint32_t hi[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = lane + kWave * i;
      const bool remote = (c < nblk) && (zv[i] > kScoreNeg * 0.5f);
      const bool cd = use_cand ? (remote && cb[i] != 0) : remote;
      float x = cd ? zv[i] * idx_scale : kEntmaxNeg;
      if (!(fabsf(x) <= 3.402823466e38f)) x = kEntmaxNeg;
      // candidate flag in bit 0 of the key: only block ids break ties, never it
      hi[i] = c < nblk ? ord_key(x) : 0u;
      cb[i] = cd ? 1 : 0;
    }
    const int M = nblk == 0 ? 0 : (topm > 0 ? max(1, min(topm, nblk)) : nblk);
    route_row_topm<NPL>(hi, cb, M, s_cand[wv], s_sel[sr]);
    if (lane == 0) s_M[sr] = M;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // ---- phase 2: each wavefront finishes its own rows, 16 lanes per row ----
  {
    const int gi = lane >> 4;
    const bool row_ok = gi < nrow;
    const int sr = wv * kRtRowsPerWave + gi;
    route_finish(s_sel[sr], row_ok ? s_M[sr] : 0, row_ok, row0 + gi, floor_p, inv_sigma, K, Kout,
                 idx_out, bias_out, valid_out);
  }
}

// ---------------------------------------------------------------------------
// Training routing (dash_attention.py:906-960): one wavefront per score row.
//   x = cand ? z idx_scale : -1e4 (non-finite -> -1e4), over the row's nblk blocks;
//   prior = 1.5-entmax(x) over the whole row (dash_attention.py:638-647):
//     X = (x - max)/2, prior = max(X - tau, 0)^2 with sum(prior) = 1; tau by
//     bisection in double, then exactly from the support's sums (the sort-threshold
//     closed form at the support size);
//   the K' = max(1, min(K, nblk)) largest of the masked prior (non-candidates at -1),
//     ties to the lower block id; valid = candidate;
//   bias = valid ? clamp((log(max(p, floor)) - mean over valid) / sigma, +-1e4) : 0.
// The row maximum and tau are kept for the backward, which recomputes the prior.
// ---------------------------------------------------------------------------
constexpr int kTrWaves = 4;
constexpr int kTrMaxK = 64;

struct TrainRow {
  int nb;
  float xmax;
};

// x of the row's columns c = lane + 64 i (entries past nb: -inf) and candidate flags.
template <int NPL>
__device__ __forceinline__ TrainRow train_row_inputs(const float* z, int64_t z_stride, int row,
                                                     int nblk, const int32_t* row_nblk,
                                                     const uint8_t* cand_in, int64_t cand_stride,
                                                     float idx_scale, float (&x)[NPL],
                                                     bool (&cd)[NPL]) {
  const int lane = wave_lane();
  TrainRow r;
  r.nb = row_nblk ? max(0, min(row_nblk[row], nblk)) : nblk;
  float zv[NPL];
  uint8_t cb[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = min(lane + kWave * i, nblk - 1);
    zv[i] = z[(int64_t)row * z_stride + c];
    cb[i] = cand_in ? cand_in[(int64_t)row * cand_stride + c] : 1;
  }
  bool any_cand = false;
  if (cand_in) {
#pragma unroll
    for (int i = 0; i < NPL; ++i)
      any_cand |= (lane + kWave * i < r.nb) && zv[i] > kScoreNeg * 0.5f && cb[i] != 0;
  }
  const bool use_cand = cand_in && __any(any_cand);
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + kWave * i;
    const bool remote = c < r.nb && zv[i] > kScoreNeg * 0.5f;
    cd[i] = use_cand ? (remote && cb[i] != 0) : remote;
    float xv = cd[i] ? zv[i] * idx_scale : kEntmaxNeg;
    if (!(fabsf(xv) <= 3.402823466e38f)) xv = kEntmaxNeg;
    x[i] = c < r.nb ? xv : -INFINITY;
    mx = fmaxf(mx, x[i]);
  }
  r.xmax = wave_max(mx);
  return r;
}

// tau of the 1.5-entmax of X = (x - xmax)/2 over the live entries (max X = 0).
template <int NPL>
__device__ __forceinline__ float train_tau(const float (&x)[NPL], float xmax) {
#pragma clang fp contract(off)
  float X[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) X[i] = __fdiv_rn(__fsub_rn(x[i], xmax), 2.0f);   // -inf stays
  double lo = -1.0, hi = 0.0;               // f(-1) >= 1 (the maximum contributes 1), f(0) = 0
  // The root stays in [lo, hi).  Once no entry lies in (lo, hi], every point of the
  // bracket has the support {X > lo}, the one the 48 steps would end on, and the
  // closed form below gives the same threshold: the bisection stops there.
  for (int it = 0; it < 48; ++it) {
    bool inside = false;
#pragma unroll
    for (int i = 0; i < NPL; ++i) inside |= ((double)X[i] > lo) & ((double)X[i] <= hi);
    if (!__any(inside)) break;
    const double mid = 0.5 * (lo + hi);
    double f = 0.0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const double d = (double)X[i] - mid;
      if (d > 0.0) f += d * d;
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) f += __shfl_xor(f, m, kWave);
    if (f >= 1.0) lo = mid; else hi = mid;
  }
  const double t0 = 0.5 * (lo + hi);
  double n = 0.0, s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int i = 0; i < NPL; ++i)
    if ((double)X[i] > t0) { n += 1.0; s1 += X[i]; s2 += (double)X[i] * X[i]; }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    n += __shfl_xor(n, m, kWave);
    s1 += __shfl_xor(s1, m, kWave);
    s2 += __shfl_xor(s2, m, kWave);
  }
  const double mean = s1 / n, msq = s2 / n;
  const double delta = (1.0 - n * (msq - mean * mean)) / n;
  return (float)(mean - sqrt(delta > 0.0 ? delta : 0.0));
}

__device__ __forceinline__ float train_prior(float x, float xmax, float tau) {
#pragma clang fp contract(off)
  const float X = __fdiv_rn(__fsub_rn(x, xmax), 2.0f);
  const float t = __fsub_rn(X, tau);
  return t > 0.f ? __fmul_rn(t, t) : 0.f;
}

template <int NPL>
__global__ __launch_bounds__(kTrWaves * kWave) void train_route_kernel(
    const float* __restrict__ z, int64_t z_stride, int rows, int nblk,
    const int32_t* __restrict__ row_nblk, const uint8_t* __restrict__ cand_in,
    int64_t cand_stride, float idx_scale, float floor_p, float inv_sigma, int K, int Kout,
    int by_x, int topm, int32_t* __restrict__ idx_out, float* __restrict__ bias_out,
    uint8_t* __restrict__ valid_out, float* __restrict__ topv_out, float2* __restrict__ stat_out) {
  __shared__ uint64_t s_sel[kTrWaves][kTrMaxK];
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
  const int row = blockIdx.x * kTrWaves + wv;
  if (row >= rows) return;
  float x[NPL];
  bool cd[NPL];
  const TrainRow tr = train_row_inputs<NPL>(z, z_stride, row, nblk, row_nblk, cand_in, cand_stride,
                                            idx_scale, x, cd);
  int32_t* io = idx_out + (int64_t)row * Kout;
  float* bo = bias_out + (int64_t)row * Kout;
  if (tr.nb == 0) {
    for (int m = lane; m < Kout; m += kWave) {
      io[m] = -1; bo[m] = 0.f;
      if (valid_out) valid_out[(int64_t)row * Kout + m] = 0;
      if (topv_out) topv_out[(int64_t)row * Kout + m] = -1.f;
    }
    if (lane == 0 && stat_out) stat_out[row] = make_float2(0.f, 0.f);
    return;
  }
  uint32_t hkey[NPL];
  uint32_t kmx = 0;
  int Mp = tr.nb;
  if (by_x) {
    // inference: entries ranked by x (ties to the lower id); the entmax runs over
    // the top M' = max(1, min(topm, nb)) of them (all nb when topm <= 0)
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      hkey[i] = lane + kWave * i < tr.nb ? ord_key(x[i]) : 0u;
      kmx = max(kmx, hkey[i]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) kmx = max(kmx, (uint32_t)__shfl_xor((int)kmx, m, kWave));
    if (topm > 0 && topm < tr.nb) {
      Mp = topm;
      const uint32_t TM = kth_key<NPL>(hkey, Mp, 1u, kmx);
      int gt = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) gt += __popcll(__ballot(hkey[i] > TM));
      int eq_seen = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const bool eq = hkey[i] == TM;
        const uint64_t meq = __ballot(eq);
        const bool in = hkey[i] > TM || (eq && eq_seen + lane_prefix(meq) < Mp - gt);
        if (!in) x[i] = -INFINITY;               // outside the top M': not in the entmax
        eq_seen += __popcll(meq);
      }
    }
  }
  const float tau = train_tau<NPL>(x, tr.xmax);
  if (!by_x) {
    // training: candidates by masked prior, non-candidates at -1, absent entries 0
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = lane + kWave * i;
      const float sp = cd[i] ? train_prior(x[i], tr.xmax, tau) : -1.f;
      hkey[i] = c < tr.nb ? ord_key(sp) : 0u;
      kmx = max(kmx, hkey[i]);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) kmx = max(kmx, (uint32_t)__shfl_xor((int)kmx, m, kWave));
  }
  const int Kp = max(1, min(min(K, kTrMaxK), Mp));
  const uint32_t T = kth_key<NPL>(hkey, Kp, by_x ? 1u : ord_key(-1.f), kmx);
  int n_gt = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) n_gt += __popcll(__ballot(hkey[i] > T));
  const int need_eq = Kp - n_gt;
  int taken = 0, eq_seen = 0;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const bool eq = hkey[i] == T;
    const uint64_t meq = __ballot(eq);
    const bool take = hkey[i] > T || (eq && eq_seen + lane_prefix(meq) < need_eq);
    const uint64_t mt = __ballot(take);
    const int c = lane + kWave * i;
    if (take)
      s_sel[wv][taken + lane_prefix(mt)] =
          ((uint64_t)hkey[i] << 32) | ((uint32_t)(0xffff - c) << 1) | (cd[i] ? 1u : 0u);
    taken += __popcll(mt);
    eq_seen += __popcll(meq);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // rank of lane m's entry among the Kp selected: its output slot
  const uint64_t key = lane < Kp ? s_sel[wv][lane] : 0ull;
  int rank = 0;
  for (int j = 0; j < Kp; ++j) rank += s_sel[wv][j] > key ? 1 : 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < Kp) s_sel[wv][rank] = key;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // lane m holds slot m
  const uint64_t ks = lane < Kp ? s_sel[wv][lane] : 0ull;
  float v = -1.f;
  if (lane < Kp) {
    v = ord_key_inv((uint32_t)(ks >> 32));
    if (by_x) v = train_prior(v, tr.xmax, tau);       // the key held x: its prior
  }
  const int c = 0xffff - (int)(((uint32_t)ks >> 1) & 0xffff);
  const bool va = lane < Kp && (ks & 1ull) != 0;
  const float logp = logf(fmaxf(v, floor_p));
  // mean log-prior of the valid slots, summed in slot order
  const uint64_t vm = __ballot(va);
  float musum = 0.f;
  int cnt = 0;
  for (int j = 0; j < Kp; ++j)
    if ((vm >> j) & 1ull) {
      musum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(logp), j));
      ++cnt;
    }
  const float mu = musum / (float)max(cnt, 1);
  for (int m = lane; m < Kout; m += kWave) {
    const bool in = m < Kp;
    const bool mv = in && va;                  // m == lane when in (Kp <= 64)
    io[m] = in ? c : -1;
    const float bv = (logp - mu) * inv_sigma;
    bo[m] = mv ? (by_x ? bv : fminf(fmaxf(bv, -kActClamp), kActClamp)) : 0.f;
    if (valid_out) valid_out[(int64_t)row * Kout + m] = mv ? 1 : 0;
    if (topv_out) topv_out[(int64_t)row * Kout + m] = in ? v : -1.f;
  }
  if (lane == 0 && stat_out) stat_out[row] = make_float2(tr.xmax, tau);
}

// Backward of train_route_kernel for one row: the bias gradient of the valid slots
// through the centred log-prior (d logp_j = (g_j - mean over valid g)/sigma, g the
// bias gradient where the clamp passes it; d p_j = d logp_j / p_j where p_j >= floor),
// scattered to the prior's columns; the 1.5-entmax backward (dash_attention.py:650-658:
// dX = dY sqrt(Y) - q sqrt(Y), q = sum(dY sqrt(Y)) / sum(sqrt(Y))) on the recomputed
// prior; dz = dX idx_scale on candidates, 0 elsewhere.
template <int NPL>
__global__ __launch_bounds__(kTrWaves * kWave) void train_route_bwd_kernel(
    const float* __restrict__ z, int64_t z_stride, int rows, int nblk,
    const int32_t* __restrict__ row_nblk, const uint8_t* __restrict__ cand_in,
    int64_t cand_stride, float idx_scale, float floor_p, float inv_sigma, int Kout,
    const int32_t* __restrict__ idx, const uint8_t* __restrict__ valid,
    const float* __restrict__ topv, const float2* __restrict__ stat,
    const float* __restrict__ dbias, float* __restrict__ dz, int64_t dz_stride) {
  __shared__ float s_dy[kTrWaves][64 * NPL];
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
  const int row = blockIdx.x * kTrWaves + wv;
  if (row >= rows) return;
  float x[NPL];
  bool cd[NPL];
  const TrainRow tr = train_row_inputs<NPL>(z, z_stride, row, nblk, row_nblk, cand_in, cand_stride,
                                            idx_scale, x, cd);
  float* dzr = dz + (int64_t)row * dz_stride;
  const float2 st = stat[row];
#pragma unroll
  for (int i = 0; i < NPL; ++i) s_dy[wv][lane + kWave * i] = 0.f;
  // slot gradients, lane m = slot m (Kout <= 64)
  const int64_t so = (int64_t)row * Kout;
  const bool in = lane < Kout;
  const int ci = in ? idx[so + lane] : -1;
  const bool va = in && valid[so + lane] != 0 && ci >= 0 && ci < tr.nb;
  const float v = in ? topv[so + lane] : 0.f;
  const float logp = logf(fmaxf(v, floor_p));
  const uint64_t vm = __ballot(va);
  float musum = 0.f;
  int cnt = 0;
  for (int j = 0; j < Kout && j < kWave; ++j)
    if ((vm >> j) & 1ull) {
      musum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(logp), j));
      ++cnt;
    }
  const float mu = musum / (float)max(cnt, 1);
  const float bv = (logp - mu) * inv_sigma;
  const float g = (va && bv >= -kActClamp && bv <= kActClamp) ? dbias[so + lane] : 0.f;
  const float gsum = wave_sum(g);
  const float dlogp = va ? (g - gsum / (float)max(cnt, 1)) * inv_sigma : 0.f;
  // the prior's gradient passes _sanitize_grad (dash_attention.py:607-613, hooked at :1046):
  // non-finite -> 0, clamped to +-1e4
  float dv = (va && v >= floor_p) ? dlogp / v : 0.f;
  dv = (fabsf(dv) <= 3.402823466e38f) ? fminf(fmaxf(dv, -kGradClamp), kGradClamp) : 0.f;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (va) s_dy[wv][ci] = dv;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // entmax backward on the recomputed prior
  float gp[NPL], dx[NPL];
  float sg = 0.f, sdx = 0.f;
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + kWave * i;
    const float y = c < tr.nb ? train_prior(x[i], st.x, st.y) : 0.f;
    gp[i] = sqrtf(y);
    dx[i] = (c < tr.nb ? s_dy[wv][c] : 0.f) * gp[i];
    sg += gp[i];
    sdx += dx[i];
  }
  sg = wave_sum(sg);
  sdx = wave_sum(sdx);
  const float qv = sdx / fmaxf(sg, 1e-12f);
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int c = lane + kWave * i;
    if (c < nblk) dzr[c] = (c < tr.nb && cd[i]) ? (dx[i] - qv * gp[i]) * idx_scale : 0.f;
  }
}

}  // namespace dash

// ---------------------------------------------------------------------------
// C entry points
// ---------------------------------------------------------------------------
namespace {
inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? dash::kOk : (int)e;
}
}  // namespace

extern "C" int dash_kbar(const float* idx_k, int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
                         const int32_t* cu_seqlens, const int32_t* seq_lens,
                         const int32_t* block_table, int64_t table_stride, int page_size,
                         const float* head_cls, int B, int S, int d, int block_size,
                         int tail_only, float* kbar, int64_t kb_sb, int nblk_cap,
                         void* stream) {
  using namespace dash;
  if (!idx_k || !head_cls || !kbar || B < 0 || S < 0 || d <= 0) return kErrInvalid;
  if (block_size <= 0 || block_size > 256) return kErrUnsupported;
  if (block_table && page_size <= 0) return kErrInvalid;
  if (B == 0 || nblk_cap == 0) return kOk;
  SeqLayout lay{cu_seqlens, block_table, table_stride, ik_sb, ik_sp, ik_st, page_size};
  dim3 grid(tail_only ? 1 : nblk_cap, B);
  const bool aligned = ((uintptr_t)idx_k % 16 == 0) && ((uintptr_t)head_cls % 16 == 0) &&
                       ik_sb % 4 == 0 && ik_st % 4 == 0 && ik_sp % 4 == 0;
  if (d == kKbD && block_size <= kKbMaxBs && aligned) {
    hipLaunchKernelGGL(kbar128_kernel, grid, dim3(256), 0, (hipStream_t)stream, idx_k, lay,
                       cu_seqlens, seq_lens, head_cls, S, block_size, tail_only,
                       (float)(1.0 / sqrt((double)d)), kbar, kb_sb);
    return launch_status();
  }
  hipLaunchKernelGGL(kbar_kernel, grid, dim3(256), 0, (hipStream_t)stream, idx_k, lay,
                     cu_seqlens, seq_lens, head_cls, S, d, block_size, tail_only,
                     (float)(1.0 / sqrt((double)d)), kbar, kb_sb);
  return launch_status();
}

extern "C" int dash_block_scores(const float* idx_q, int64_t iq_sb, int64_t iq_st,
                                 const int32_t* cu_q, int Lq, const int32_t* q_pos,
                                 const float* kbar, int64_t kb_sb, int nblk_cap,
                                 const int32_t* cu_k, const int32_t* lens_k, int S, int B,
                                 int d, int block_size, int local_blocks, float* z,
                                 int64_t z_stride, void* stream) {
  using namespace dash;
  if (!idx_q || !kbar || !z || B < 0 || Lq < 0 || d <= 0 || nblk_cap < 0) return kErrInvalid;
  if (block_size <= 0) return kErrInvalid;
  if (B == 0 || Lq == 0 || nblk_cap == 0) return kOk;
  SeqLayout lay{cu_q, nullptr, 0, iq_sb, 0, iq_st, 1};
  dim3 grid((Lq + kScTile - 1) / kScTile, (nblk_cap + kScTile - 1) / kScTile, B);
  const bool vec = d % kScK == 0 && (uintptr_t)idx_q % 16 == 0 && (uintptr_t)kbar % 16 == 0 &&
                   iq_sb % 4 == 0 && iq_st % 4 == 0 && kb_sb % 4 == 0;
  if (vec && d == 128) {
    dim3 g2((Lq + kSmRows - 1) / kSmRows, (nblk_cap + kSmBlk - 1) / kSmBlk, B);
    hipLaunchKernelGGL(scores_mfma_kernel, g2, dim3(256), 0, (hipStream_t)stream, idx_q, lay, cu_q,
                       Lq, q_pos, kbar, kb_sb, cu_k, lens_k, S, block_size, local_blocks, nblk_cap,
                       (float)(1.0 / sqrt((double)d)), z, z_stride);
    return launch_status();
  }
  auto kern = vec ? scores_kernel<true> : scores_kernel<false>;
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, (hipStream_t)stream, idx_q, lay, cu_q,
                     Lq, q_pos, kbar, kb_sb, cu_k, lens_k, S, d, block_size, local_blocks,
                     nblk_cap, (float)(1.0 / sqrt((double)d)), z, z_stride);
  return launch_status();
}

extern "C" int dash_block_max_score(const float* q, int64_t q_sb, int64_t q_st, int C,
                                    const int32_t* pos, const int32_t* seg, int64_t ps_sb,
                                    const float* k, int64_t k_sb, int64_t k_st, int Sk, int B,
                                    int d, int block_size, int local_window, int nblk, int mode,
                                    float* out, int64_t o_sb, int64_t o_sc, void* stream) {
  using namespace dash;
  if (!q || !pos || !k || !out || B < 0 || C < 0 || d <= 0 || nblk < 0) return kErrInvalid;
  if (block_size <= 0 || (mode != 0 && mode != 1)) return kErrInvalid;
  if (B == 0 || C == 0 || nblk == 0) return kOk;
  SeqLayout lq{nullptr, nullptr, 0, q_sb, 0, q_st, 1};
  SeqLayout lk{nullptr, nullptr, 0, k_sb, 0, k_st, 1};
  dim3 grid((C + kScTile - 1) / kScTile, nblk, B);
  hipLaunchKernelGGL(blockmax_kernel, grid, dim3(256), 0, (hipStream_t)stream, q, lq, C, pos,
                     seg, ps_sb, k, lk, Sk, d, block_size, max(1, local_window), nblk, mode,
                     out, o_sb, o_sc);
  return launch_status();
}

extern "C" int dash_route(const float* z, int64_t z_stride, int rows, int nblk_cols,
                          const int32_t* row_nblk, const uint8_t* cand, int64_t cand_stride,
                          float idx_scale, float floor_p, float sigma, int K, int topm,
                          int Kout, int32_t* idx, float* bias, uint8_t* valid,
                          void* stream) {
  using namespace dash;
  if (!z || !idx || !bias || rows < 0 || nblk_cols < 0) return kErrInvalid;
  if (topm < 1 || topm > kMaxM) {
    // wider entmax (topm > 16, or the whole row for topm <= 0): one row per wavefront
    if (K < 1 || Kout < 1) return kErrInvalid;
    const int Mw = topm > 0 ? std::min(topm, std::max(nblk_cols, 1)) : std::max(nblk_cols, 1);
    if (Kout < std::min(K, Mw)) return kErrInvalid;
    if (K > kTrMaxK || Kout > kTrMaxK) return kErrUnsupported;
    if (z_stride < nblk_cols || (cand && cand_stride < nblk_cols)) return kErrInvalid;
    if (nblk_cols > 64 * 32) return kErrUnsupported;
    if (rows == 0) return kOk;
    if (nblk_cols == 0) return kErrInvalid;
    const float inv_s = (float)(1.0 / (double)sigma);
    dim3 g((rows + kTrWaves - 1) / kTrWaves);
    hipStream_t s0 = (hipStream_t)stream;
    const int np = (nblk_cols + 63) / 64;
#define DASH_WROUTE(N)                                                                            \
  hipLaunchKernelGGL(train_route_kernel<N>, g, dim3(kTrWaves * kWave), 0, s0, z, z_stride, rows,    \
                     nblk_cols, row_nblk, cand, cand_stride, idx_scale, floor_p, inv_s, K, Kout, 1, \
                     topm, idx, bias, valid, (float*)nullptr, (float2*)nullptr)
    if (np <= 1) DASH_WROUTE(1);
    else if (np <= 2) DASH_WROUTE(2);
    else if (np <= 4) DASH_WROUTE(4);
    else if (np <= 8) DASH_WROUTE(8);
    else if (np <= 16) DASH_WROUTE(16);
    else DASH_WROUTE(32);
#undef DASH_WROUTE
    return launch_status();
  }
  if (K < 1 || Kout < 1) return kErrInvalid;
  if (Kout < std::min(K, std::min(topm, std::max(nblk_cols, 1)))) return kErrInvalid;
  if (nblk_cols > 64 * 32) return kErrUnsupported;
  if (rows == 0) return kOk;
  if (nblk_cols == 0) return kErrInvalid;   // top-M of an empty row
  const float inv_sigma = (float)(1.0 / (double)sigma);
  dim3 grid((rows + kRtRows - 1) / kRtRows);
  hipStream_t st = (hipStream_t)stream;
  const int npl = (nblk_cols + 63) / 64;
#define DASH_ROUTE(N)                                                                       \
  hipLaunchKernelGGL(route_kernel<N>, grid, dim3(kRtWaves * kWave), 0, st, z, z_stride, rows, \
                     nblk_cols, row_nblk, cand, cand_stride, idx_scale, floor_p, inv_sigma, \
                     K, topm, Kout, idx, bias, valid)
  if (npl <= 1) DASH_ROUTE(1);
  else if (npl <= 2) DASH_ROUTE(2);
  else if (npl <= 4) DASH_ROUTE(4);
  else if (npl <= 8) DASH_ROUTE(8);
  else if (npl <= 16) DASH_ROUTE(16);
  else DASH_ROUTE(32);
#undef DASH_ROUTE
  return launch_status();
}

extern "C" int dash_train_route(const float* z, int64_t z_stride, int rows, int nblk_cols,
                                const int32_t* row_nblk, const uint8_t* cand, int64_t cand_stride,
                                float idx_scale, float floor_p, float sigma, int K, int Kout,
                                int32_t* idx, float* bias, uint8_t* valid, float* topv,
                                float* stat, void* stream) {
  using namespace dash;
  if (!z || !idx || !bias || !topv || !stat || rows < 0 || nblk_cols < 0) return kErrInvalid;
  if (z_stride < nblk_cols || (cand && cand_stride < nblk_cols)) return kErrInvalid;
  if (K < 1 || Kout < 1 || Kout < std::min(K, std::max(nblk_cols, 1))) return kErrInvalid;
  if (K > kTrMaxK || Kout > kTrMaxK) return kErrUnsupported;
  if (nblk_cols > 64 * 32) return kErrUnsupported;
  if (rows == 0) return kOk;
  if (nblk_cols == 0) return kErrInvalid;
  const float inv_sigma = (float)(1.0 / (double)sigma);
  dim3 grid((rows + kTrWaves - 1) / kTrWaves);
  hipStream_t st = (hipStream_t)stream;
  const int npl = (nblk_cols + 63) / 64;
#define DASH_TROUTE(N)                                                                           \
  hipLaunchKernelGGL(train_route_kernel<N>, grid, dim3(kTrWaves * kWave), 0, st, z, z_stride, rows, \
                     nblk_cols, row_nblk, cand, cand_stride, idx_scale, floor_p, inv_sigma, K, Kout, \
                     0, 0, idx, bias, valid, topv, (float2*)stat)
  if (npl <= 1) DASH_TROUTE(1);
  else if (npl <= 2) DASH_TROUTE(2);
  else if (npl <= 4) DASH_TROUTE(4);
  else if (npl <= 8) DASH_TROUTE(8);
  else if (npl <= 16) DASH_TROUTE(16);
  else DASH_TROUTE(32);
#undef DASH_TROUTE
  return launch_status();
}

extern "C" int dash_train_route_backward(const float* z, int64_t z_stride, int rows, int nblk_cols,
                                         const int32_t* row_nblk, const uint8_t* cand,
                                         int64_t cand_stride, float idx_scale, float floor_p,
                                         float sigma, int Kout, const int32_t* idx,
                                         const uint8_t* valid, const float* topv,
                                         const float* stat, const float* dbias, float* dz,
                                         int64_t dz_stride, void* stream) {
  using namespace dash;
  if (!z || !idx || !valid || !topv || !stat || !dbias || !dz || rows < 0 || nblk_cols < 0)
    return kErrInvalid;
  if (z_stride < nblk_cols || dz_stride < nblk_cols || (cand && cand_stride < nblk_cols))
    return kErrInvalid;
  if (Kout < 1 || Kout > kTrMaxK) return kErrUnsupported;
  if (nblk_cols > 64 * 32) return kErrUnsupported;
  if (rows == 0) return kOk;
  if (nblk_cols == 0) return kErrInvalid;
  const float inv_sigma = (float)(1.0 / (double)sigma);
  dim3 grid((rows + kTrWaves - 1) / kTrWaves);
  hipStream_t st = (hipStream_t)stream;
  const int npl = (nblk_cols + 63) / 64;
#define DASH_TRBWD(N)                                                                            \
  hipLaunchKernelGGL(train_route_bwd_kernel<N>, grid, dim3(kTrWaves * kWave), 0, st, z, z_stride,  \
                     rows, nblk_cols, row_nblk, cand, cand_stride, idx_scale, floor_p, inv_sigma,  \
                     Kout, idx, valid, topv, (const float2*)stat, dbias, dz, dz_stride)
  if (npl <= 1) DASH_TRBWD(1);
  else if (npl <= 2) DASH_TRBWD(2);
  else if (npl <= 4) DASH_TRBWD(4);
  else if (npl <= 8) DASH_TRBWD(8);
  else if (npl <= 16) DASH_TRBWD(16);
  else DASH_TRBWD(32);
#undef DASH_TRBWD
  return launch_status();
}

// ---------------------------------------------------------------------------
// Decode router: one query per sequence, one 1024-thread work-group per
// sequence.  Fuses the k_bar refresh of the tail block, the block scores and
// the routing; no cross-work-group communication.
// ---------------------------------------------------------------------------
namespace dash {

constexpr int kDrThreads = 1024;
constexpr int kDrMaxBlocks = 2048;

struct DecodeRouteArgs {
  const float* idx_q; int64_t iq_sb;
  const float* idx_k; SeqLayout lay_k;
  const int32_t* lens; const int32_t* q_pos; int S;
  const float* head_cls; int refresh_tail;
  int skip_tail;                     // the scores read no k_bar row past the last remote block
  float* kbar; int64_t kb_sb; int nblk_cap;
  // k_bar page pool: the row of block c of sequence b is kb_table[b * kb_ts + c]
  // (pages of one block each); null: row b * kb_sb / d + c
  const int32_t* kb_table; int64_t kb_ts;
  // window bounds [B, 2]: only blocks lo <= c < hi are scored (the others score as
  // not remote); null: every block
  const int32_t* bounds;
  const uint8_t* cand; int64_t cand_stride;
  int d, bs, local_blocks;
  float inv_sqrt_d, idx_scale, floor_p, inv_sigma;
  int K, topm, Kout;
  int32_t* idx; float* bias; uint8_t* valid;
  float* z; int64_t z_stride;
  // fused decode step: the slots as published words [B * Kout, 2] for the routed-slot
  // wavefronts of the same launch (null: none)
  uint64_t* pub;
};

__device__ __forceinline__ float* kbar_row(const DecodeRouteArgs& a, int b, int c) {
  return a.kb_table ? a.kbar + (int64_t)a.kb_table[(int64_t)b * a.kb_ts + c] * a.d
                    : a.kbar + (int64_t)b * a.kb_sb + (int64_t)c * a.d;
}

// 1.5-entmax of the sorted top M, the log-prior bias and the output slots of one
// decode row, by one wavefront with lane m holding entry m (each lane forms its own
// prefix sums serially), so the result is bit-for-bit the serial one.
__device__ __forceinline__ void decode_route_finish(const DecodeRouteArgs& a, int b, int lane, int M,
                                                    int Kp, const float* s_selv, const int* s_selk) {
#pragma clang fp contract(off)
  const float xv = lane < M ? s_selv[lane] : 0.f;
  const int kv = lane < M ? s_selk[lane] : 0x3fffffff;
  const float x0 = s_selv[0];
  const float X = __fdiv_rn(__fsub_rn(xv, x0), 2.0f);
  double cs = 0.0, cs2 = 0.0;
#pragma unroll
  for (int j = 0; j < kMaxM; ++j) {
    const float Xj = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(X), j));
    if (j <= lane) {
      cs += (double)Xj;
      cs2 += (double)__fmul_rn(Xj, Xj);
    }
  }
  float tau = 0.f;
  bool sup = false;
  if (lane < M) {
    const float rho = (float)(lane + 1);
    const float mean = __fdiv_rn((float)cs, rho);
    const float mean_sq = __fdiv_rn((float)cs2, rho);
    const float ss = __fmul_rn(rho, __fsub_rn(mean_sq, __fmul_rn(mean, mean)));
    const float delta = __fdiv_rn(__fsub_rn(1.0f, ss), rho);
    const float delta_nz = delta > 0.f ? delta : 0.f;
    tau = __fsub_rn(mean, __fsqrt_rn(delta_nz));
    sup = tau <= X;
  }
  const int support = max(__popcll(__ballot(sup)), 1);
  const float tau_star = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(tau), support - 1));
  const float tt = __fsub_rn(X, tau_star);
  const float cc = tt > 0.f ? tt : 0.f;
  const float prior = lane < M ? __fmul_rn(cc, cc) : 0.f;
  const float logp = logf(fmaxf(prior, a.floor_p));
  const bool va = (kv & (1 << 30)) != 0;
  // mean log-prior of the kept valid slots, summed in slot order
  float musum = 0.f;
  int cnt = 0;
  const uint64_t keep = __ballot(lane < Kp && va);
#pragma unroll
  for (int j = 0; j < kMaxM; ++j)
    if ((keep >> j) & 1ull) {
      musum += __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(logp), j));
      ++cnt;
    }
  const float mu = musum / (float)max(cnt, 1);
  for (int m = lane; m < a.Kout; m += kWave) {
    const bool kept = m < Kp;                   // m < Kp <= 16: lane m holds slot m
    const int c = kept ? (kv & 0x3fffffff) : -1;
    const float bv = kept && va ? (logp - mu) * a.inv_sigma : 0.f;
    a.idx[(int64_t)b * a.Kout + m] = c;
    a.bias[(int64_t)b * a.Kout + m] = bv;
    if (a.valid) a.valid[(int64_t)b * a.Kout + m] = kept && va ? 1 : 0;
    if (a.pub) publish_slot(a.pub, (int64_t)b * a.Kout + m, c, a.valid ? kept && va : true, bv);
  }
}

// Modes of decode_route_body.  The tail block holds the query, so with a window of
// at least one block (local_blocks >= 1) it is never a remote candidate: its summary
// is needed only by later steps, and its refresh can run in another work-group
// (kTailOnly) beside the routing, which then runs with refresh_tail = 0 and
// skip_tail = 1 (no read of the tail row).
constexpr int kRouteAll = 0;         // refresh (if refresh_tail), then route
constexpr int kTailOnly = 1;         // refresh only

template <int MODE = kRouteAll>
__device__ __forceinline__ void decode_route_body(const DecodeRouteArgs& a, int b) {
  constexpr int mode = MODE;
  __shared__ __attribute__((aligned(16))) float s_q[256];
  __shared__ __attribute__((aligned(16))) float s_tail[256];
  __shared__ float s_aw[256];
  __shared__ float s_red[2];
  __shared__ float s_part[8][128];
  __shared__ float s_x[kDrMaxBlocks];
  __shared__ int s_key[kDrMaxBlocks];
  __shared__ __attribute__((aligned(16))) float s_cx[kDrMaxBlocks + 4];
  __shared__ __attribute__((aligned(16))) int s_ck[kDrMaxBlocks + 4];
  __shared__ float s_cmax[kDrThreads / kWave][16];
  __shared__ float s_t0;
  __shared__ int s_ncand;
  __shared__ uint8_t s_flag[kDrMaxBlocks];
  __shared__ float s_selv[kMaxM];
  __shared__ int s_selk[kMaxM];
  __shared__ uint64_t s_wcand[kWave];
  __shared__ uint64_t s_wsel[kMaxM];

  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int len = a.lens ? min(max(a.lens[b], 0), a.S) : a.S;
  const int nblk = len > 0 ? (len + a.bs - 1) / a.bs : 0;     // <= nblk_cap (host check)
  // the query position, at most the last cached token (so the tail block is never remote)
  const int qp = a.q_pos ? min(a.q_pos[b], len - 1) : len - 1;
  const int lim = (qp >= 0 ? qp / a.bs : -1) - a.local_blocks;
  const int ct = nblk - 1;               // tail block
  constexpr bool own_refresh = mode == kRouteAll;   // and a.refresh_tail, at each use
  if (mode == kTailOnly && (!a.refresh_tail || nblk == 0)) return;
  if (nblk == 0) {
    for (int m = tid; m < a.Kout; m += kDrThreads) {
      a.idx[(int64_t)b * a.Kout + m] = -1;
      a.bias[(int64_t)b * a.Kout + m] = 0.f;
      if (a.valid) a.valid[(int64_t)b * a.Kout + m] = 0;
      if (a.pub) publish_slot(a.pub, (int64_t)b * a.Kout + m, -1, false, 0.f);
    }
    return;
  }
  if (mode != kTailOnly)
    for (int i = tid; i < a.d; i += kDrThreads) s_q[i] = a.idx_q[(int64_t)b * a.iq_sb + i];
  // The k_bar rows the scores read: every block, or (skip_tail) the remote ones only, so
  // that the tail row being rewritten elsewhere is never read (rows past the last
  // remote block read that block again, and a sequence with no remote block reads
  // head_cls, d floats, instead; those scores are masked).
  int c_clamp = a.skip_tail ? max(lim, 0) : nblk - 1;
  // window bounds: scores outside [blo, bhi) are not computed (their rows are not read)
  int blo = 0, bhi = nblk;
  if (a.bounds && mode != kTailOnly) {
    blo = min(max(a.bounds[2 * b], 0), nblk);
    bhi = min(max(a.bounds[2 * b + 1], blo), nblk);
  }
  const int c_lo = min(blo, c_clamp);
  c_clamp = max(min(c_clamp, bhi - 1), c_lo);
  // d = 128 and up to 512 blocks: every block's k_bar row is loaded now, 16 lanes
  // per row, so that the loads are in flight during the tail refresh
  const bool fast_scores = mode != kTailOnly && a.d == 128 && nblk <= 8 * (kDrThreads / 16);
  const int l16 = lane & 15, slot16 = tid >> 4;
  float4 kp[8][2];
  auto prefetch = [&](int r0, int r1) {
    if (!fast_scores) return;
#pragma unroll
    for (int r = r0; r < r1; ++r) {
      const int c = max(min(slot16 + r * (kDrThreads / 16), c_clamp), c_lo);
      const float* kr = (a.skip_tail && lim < 0) ? a.head_cls : kbar_row(a, b, c);
      kp[r][0] = *(const float4*)(kr + l16 * 4);
      kp[r][1] = *(const float4*)(kr + 64 + l16 * 4);
    }
  };
  prefetch(0, 4);
  if ((own_refresh && a.refresh_tail) || mode == kTailOnly) {
    const int t0 = ct * a.bs, n = len - t0;
    const float* hcp = a.head_cls;
    // logits of the tail tokens: 8 lanes per token, an eighth of the dims each
    // (the k_bar rows of the scores are already in flight)
    for (int j0 = 0; j0 < n; j0 += kDrThreads / 8) {
      const int j = j0 + tid / 8, part = tid % 8;
      float acc = 0.f;
      if (j < n) {
        const float* kr = a.idx_k + a.lay_k.row(b, t0 + j);
        const int q8 = a.d / 8;
        for (int i = part * q8; i < (part + 1) * q8; i += 4) {
          const float4 kv = *(const float4*)(kr + i);
          const float4 hv = *(const float4*)(hcp + i);
          acc += kv.x * hv.x + kv.y * hv.y + kv.z * hv.z + kv.w * hv.w;
        }
      }
      acc += __shfl_xor(acc, 1, kWave);
      acc += __shfl_xor(acc, 2, kWave);
      acc += __shfl_xor(acc, 4, kWave);
      if (j < n && part == 0) s_aw[j] = fminf(fmaxf(acc * a.inv_sqrt_d, -kActClamp), kActClamp);
    }
    prefetch(4, 8);
    __syncthreads();
    if (wv == 0) {
      float m = -INFINITY;
      for (int j = lane; j < n; j += kWave) m = fmaxf(m, s_aw[j]);
      m = wave_max(m);
      float sum = 0.f;
      for (int j = lane; j < n; j += kWave) sum += expf(s_aw[j] - m);
      sum = wave_sum(sum);
      if (lane == 0) { s_red[0] = m; s_red[1] = fmaxf(sum, 1e-6f); }
    }
    __syncthreads();
    for (int j = tid; j < n; j += kDrThreads) s_aw[j] = expf(s_aw[j] - s_red[0]) / s_red[1];
    __syncthreads();
    // weighted sum: 8 token groups x 128 dims, partials reduced through LDS
    const int jg = tid / 128, di = tid % 128;
    for (int i0 = 0; i0 < a.d; i0 += 128) {
      const int i = i0 + di;
      float acc = 0.f;
      if (i < a.d) {
#pragma unroll 8
        for (int j = jg; j < n; j += 8) acc += s_aw[j] * a.idx_k[a.lay_k.row(b, t0 + j) + i];
      }
      s_part[jg][di] = acc;
      __syncthreads();
      if (tid < 128 && i < a.d) {
        float t = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) t += s_part[g][tid];
        if (!(fabsf(t) <= 3.402823466e38f)) t = 0.f;
        s_tail[i] = t;
        kbar_row(a, b, ct)[i] = t;
      }
      __syncthreads();
    }
    if (mode == kTailOnly) return;
  }
  if (!(own_refresh && a.refresh_tail)) prefetch(4, 8);
  __syncthreads();
  // scores, the refreshed tail block from LDS
  if (fast_scores) {
    const float4 qa = *(const float4*)(s_q + l16 * 4), qb = *(const float4*)(s_q + 64 + l16 * 4);
    const float4 ta = *(const float4*)(s_tail + l16 * 4), tb = *(const float4*)(s_tail + 64 + l16 * 4);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int c = slot16 + r * (kDrThreads / 16);
      const bool tl = own_refresh && a.refresh_tail && c == ct;
      const float4 ka = tl ? ta : kp[r][0], kb = tl ? tb : kp[r][1];
      float v = qa.x * ka.x + qa.y * ka.y + qa.z * ka.z + qa.w * ka.w +
                qb.x * kb.x + qb.y * kb.y + qb.z * kb.z + qb.w * kb.w;
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
      if (l16 == 0 && c < nblk) {
        float zz = kScoreNeg;
        if (c <= lim && c >= blo && c < bhi) zz = fminf(fmaxf(v * a.inv_sqrt_d, -kActClamp), kActClamp);
        s_x[c] = zz;                     // stored to z after the barrier below
      }
    }
  } else {
    // 32 lanes per block (4 dims per lane per step), 32 blocks per pass, loads of
    // 8 passes issued before use
    const int l32 = lane & 31, row0 = tid / 32;
    for (int cb = 0; cb < nblk; cb += 8 * (kDrThreads / 32)) {
      float acc[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[r] = 0.f;
      for (int i = l32 * 4; i < a.d; i += 128) {
        float4 kv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int c = max(min(cb + row0 + r * (kDrThreads / 32), c_clamp), c_lo);
          kv[r] = *(const float4*)(((a.skip_tail && lim < 0) ? a.head_cls : kbar_row(a, b, c)) + i);
        }
        const float4 qv = *(const float4*)(s_q + i);
        const float4 tv = *(const float4*)(s_tail + i);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int c = cb + row0 + r * (kDrThreads / 32);
          const float4 k4 = (own_refresh && a.refresh_tail && c == ct) ? tv : kv[r];
          acc[r] += qv.x * k4.x + qv.y * k4.y + qv.z * k4.z + qv.w * k4.w;
        }
      }
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        float v = acc[r];
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
        const int c = cb + row0 + r * (kDrThreads / 32);
        if (l32 == 0 && c < nblk) {
          float zz = kScoreNeg;
          if (c <= lim && c >= blo && c < bhi) zz = fminf(fmaxf(v * a.inv_sqrt_d, -kActClamp), kActClamp);
          s_x[c] = zz;
          a.z[(int64_t)b * a.z_stride + c] = zz;
        }
      }
    }
  }
  __syncthreads();

  if (fast_scores) {
    // rows of up to 512 blocks: the selection and the entmax in wavefront 0 alone
    // (route_kernel's phase 1 and 2 on this row), no more work-group barriers; the
    // other wavefronts store the scores (after the barrier, so that it does not wait
    // for the stores)
    if (wv != 0) {
      for (int c = tid - kWave; c < nblk; c += kDrThreads - kWave) a.z[(int64_t)b * a.z_stride + c] = s_x[c];
      return;
    }
    uint8_t cb[8];
    float zv[8];
    bool any_cand = false;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = lane + kWave * i;
      zv[i] = c < nblk ? s_x[c] : kScoreNeg;
      cb[i] = (a.cand && c < nblk) ? a.cand[(int64_t)b * a.cand_stride + c] : 0;
      any_cand |= c < nblk && zv[i] > kScoreNeg * 0.5f && cb[i] != 0;
    }
    // rows without any candidate fall back to every remote block
    const bool use_cand = a.cand && __any(any_cand);
    uint32_t hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = lane + kWave * i;
      const bool remote = c < nblk && zv[i] > kScoreNeg * 0.5f;
      const bool cd = use_cand ? (remote && cb[i] != 0) : remote;
      float x = cd ? zv[i] * a.idx_scale : kEntmaxNeg;
      if (!(fabsf(x) <= 3.402823466e38f)) x = kEntmaxNeg;
      hi[i] = c < nblk ? ord_key(x) : 0u;
      cb[i] = cd ? 1 : 0;
    }
    const int Mw = a.topm > 0 ? max(1, min(a.topm, nblk)) : nblk;
    route_row_topm<8>(hi, cb, Mw, s_wcand, s_wsel);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool row_ok = lane < kMaxM;
    route_finish(s_wsel, row_ok ? Mw : 0, row_ok, b, a.floor_p, a.inv_sigma, a.K, a.Kout, a.idx,
                 a.bias, a.valid, a.pub);
    return;
  }

  // candidates, with the fall-back to every remote block
  bool any = false;
  for (int c = tid; c < nblk; c += kDrThreads) {
    const float z = s_x[c];
    const bool remote = z > kScoreNeg * 0.5f;
    bool cd = remote;
    if (a.cand) cd = cd && a.cand[(int64_t)b * a.cand_stride + c] != 0;
    s_x[c] = z;
    s_flag[c] = (remote ? 1 : 0) | (cd ? 2 : 0);
    any |= cd;
  }
  any = __syncthreads_or(any);
  for (int c = tid; c < nblk; c += kDrThreads) {
    const bool cd = any ? (s_flag[c] & 2) : (s_flag[c] & 1);
    float x = cd ? s_x[c] * a.idx_scale : kEntmaxNeg;
    if (!(fabsf(x) <= 3.402823466e38f)) x = kEntmaxNeg;
    s_x[c] = x;
    s_key[c] = c | (cd ? (1 << 30) : 0);
  }
  __syncthreads();
  const int M = a.topm > 0 ? max(1, min(a.topm, nblk)) : nblk;
  const int Kp = max(1, min(a.K, M));
  // Top-M prefilter: t0 = min over the 16 residue classes c mod 16 of the class
  // maximum.  At least 16 >= M entries reach t0, so the top M all do, and every
  // entry below t0 loses to every entry at or above it: ranking the entries
  // >= t0 among themselves gives their rank among all entries.
  {
    float cm = -INFINITY;
    for (int c = tid; c < nblk; c += kDrThreads) cm = fmaxf(cm, s_x[c]);
    cm = fmaxf(cm, __shfl_xor(cm, 16, kWave));   // tid % 16 == lane % 16 is the class
    cm = fmaxf(cm, __shfl_xor(cm, 32, kWave));
    if (lane < 16) s_cmax[wv][lane] = cm;
    if (tid == 0) s_ncand = 0;
  }
  __syncthreads();
  if (wv == 0) {
    float g = INFINITY;
    if (lane < 16) {
      g = -INFINITY;
#pragma unroll
      for (int w = 0; w < kDrThreads / kWave; ++w) g = fmaxf(g, s_cmax[w][lane]);
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) g = fminf(g, __shfl_xor(g, m, kWave));
    if (lane == 0) s_t0 = g;
  }
  __syncthreads();
  {
    const float t0v = s_t0;
    for (int c = tid; c < nblk; c += kDrThreads) {
      const float x = s_x[c];
      if (x >= t0v) {
        const int slot = atomicAdd(&s_ncand, 1);
        s_cx[slot] = x;
        s_ck[slot] = s_key[c];
      }
    }
  }
  __syncthreads();
  const int nc = s_ncand;
  // pad the candidates to a multiple of 4 with entries that lose every comparison
  if (tid < ((nc + 3) & ~3) - nc) {
    s_cx[nc + tid] = -INFINITY;
    s_ck[nc + tid] = 0x3fffffff;
  }
  __syncthreads();
  // exact rank among the candidates: branch-free, four entries per LDS read
  for (int i = tid; i < nc; i += kDrThreads) {
    const float x = s_cx[i];
    const int key = s_ck[i], ki = key & 0x3fffffff;
    int rank = 0;
    for (int j0 = 0; j0 < nc; j0 += 4) {
      const float4 xv = *reinterpret_cast<const float4*>(&s_cx[j0]);
      const int4 kv = *reinterpret_cast<const int4*>(&s_ck[j0]);
      rank += (int)(xv.x > x) | ((int)(xv.x == x) & (int)((kv.x & 0x3fffffff) < ki));
      rank += (int)(xv.y > x) | ((int)(xv.y == x) & (int)((kv.y & 0x3fffffff) < ki));
      rank += (int)(xv.z > x) | ((int)(xv.z == x) & (int)((kv.z & 0x3fffffff) < ki));
      rank += (int)(xv.w > x) | ((int)(xv.w == x) & (int)((kv.w & 0x3fffffff) < ki));
    }
    if (rank < M) { s_selv[rank] = x; s_selk[rank] = key; }
  }
  __syncthreads();
  if (wv != 0) return;
  decode_route_finish(a, b, lane, M, Kp, s_selv, s_selk);
}

// Work-groups 0 .. B-1 route one sequence each; with nrw = 2, a routes without the
// tail refresh (refresh_tail 0, skip_tail 1) and B .. 2B-1 refresh with rt.
__global__ __launch_bounds__(kDrThreads) void decode_route_kernel(DecodeRouteArgs a,
                                                                  DecodeRouteArgs rt, int B) {
  if ((int)blockIdx.x < B)
    decode_route_body<kRouteAll>(a, blockIdx.x);
  else
    decode_route_body<kTailOnly>(rt, (int)blockIdx.x - B);
}

// ---------------------------------------------------------------------------
// Fused decode step.  The window part of the attention does not depend on the
// routing, so it runs in the router's launch: work-groups 0 .. B-1 route one
// sequence each (as decode_route_kernel), B .. 2B-1 refresh the tail block's
// summary of one sequence each (beside its routing, which does not read it once
// the window spans a block), the rest are 16 wavefronts of window
// pieces, one piece of the window of one (sequence, head) per wavefront (32 or
// 64 keys, see ds_piece_keys; 32 keys per round trip keep a wavefront within the
// 128 registers a 1024-thread work-group allows), each writing an (o, m, l)
// partial.  The same wavefronts then take the routed slots of the (sequence, head)
// pairs (one slot each) once the routers have published them (ds_routed_slot), so
// the routed blocks load while other routers and pieces still run; a second launch
// merges.
// ---------------------------------------------------------------------------
constexpr int kDsPieceMin = 32;           // keys per window piece: 32, or 64 (see ds_piece_keys)
constexpr int64_t kDsWideTasks = 4096;

// Keys per window piece: 64 (two round trips per wavefront) while the window part
// is small enough that the router work-groups bound the first launch (fewer
// partials then shorten the merge: 8 sequences x 10 heads at a 1,024-token window,
// 43.2 -> 40.4 us per step), else 32 (more wavefronts; 32 sequences x 10 heads:
// 1,666 us per 12-layer step against 1,716 with 64).
inline int ds_piece_keys(int64_t B, int H, int local_window, int block_size) {
  const int64_t tasks = B * H * ((local_window + block_size - 1 + kDsPieceMin - 1) / kDsPieceMin);
  return tasks <= kDsWideTasks ? 2 * kDsPieceMin : kDsPieceMin;
}

__device__ __forceinline__ int ds_pieces(const DecodeArgs& da, const DcSpan& sp) {
  return sp.n_win > 0 ? (sp.qp + 1 - sp.w0 * da.bs + da.piece - 1) / da.piece : 0;
}

// With nrw = 2 (split), ra routes without the refresh (refresh_tail 0, skip_tail 1)
// and rt refreshes the tail blocks in work-groups B .. 2B-1.
constexpr int kDsCUs = 256;               // compute units of an MI355X

// Routed slot r of (b, h) in the fused step's first launch, once sequence b's router
// (a work-group of the same launch) has published its slots: the slots are waited
// for (bounded), filtered as dc_routed does (valid, remote, first occurrence, in slot
// order), and the r-th kept block is streamed into slot npw + r of the partials (an
// empty partial past the kept count).  The router work-groups have the lowest ids,
// so they are dispatched before any wavefront that waits for them.
constexpr int kPubSpinLimit = 1 << 16;    // polls (with a short sleep) before giving up

__device__ __forceinline__ void ds_routed_slot(const DecodeRouteArgs& ra, const DecodeArgs& da,
                                               int b, int h, int r, int npw, int lane) {
  const uint64_t* pw = ra.pub + 2 * ((int64_t)b * da.K + min(lane, da.K - 1));
  // every lane watches the last slot's bias word (one request per poll; the router's
  // wavefront stores all its slots together), then the slots are read
  const uint64_t* pl = ra.pub + 2 * ((int64_t)b * da.K + da.K - 1) + 1;
  for (int spin = 0; spin < kPubSpinLimit; ++spin) {
    if ((__hip_atomic_load(pl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kPubBit) != 0) break;
    __builtin_amdgcn_s_sleep(8);
  }
  uint64_t w0 = 0, w1 = 0;
  bool ok = lane >= da.K;
  for (int spin = 0;; ++spin) {
    if (!ok) {
      w0 = __hip_atomic_load(pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      w1 = __hip_atomic_load(pw + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ok = (w0 & kPubBit) != 0 && (w1 & kPubBit) != 0;
    }
    if (__all(ok) || spin >= kPubSpinLimit) break;
    __builtin_amdgcn_s_sleep(2);
  }
  const DcSpan sp = dc_span(da, b);
  int c = -1;
  float bl = 0.f;
  bool keep = false;
  if (lane < da.K && ok && sp.len > 0) {        // a slot never published counts as empty
    c = (int)(uint32_t)(w0 & 0xffffu) - 1;
    keep = ((w0 >> 16) & 1u) != 0 && c >= 0 && c < sp.nblk && c * da.bs < sp.ls;
    bl = __uint_as_float((uint32_t)w1) * 1.4426950408889634f;
  }
  // first occurrence: no earlier lane that passed the filter names the same block
  const int ck = keep ? c : -1;
  bool dup = false;
#pragma unroll
  for (int j = 0; j < kDcMaxK; ++j) {
    const int cj = __shfl(ck, j, kWave);
    dup |= j < lane && cj == c;
  }
  keep = keep && !dup;
  uint64_t mask = __ballot(keep);
  const int n_r = __popcll(mask);
  DcState st;
  dc_init(st, da, b, h, lane);
  if (r < n_r) {
    for (int i = 0; i < r; ++i) mask &= mask - 1ull;
    const int src = __builtin_ctzll(mask);
    const int cr = __builtin_amdgcn_readlane(c, src);
    const float br = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(bl), src));
    dc_block<32>(st, da, b, h, sp, cr, true, br);
  }
  dc_store_partial<128>(st, da.part + ((int64_t)(b * da.H + h) * (npw + da.K) + npw + r) * (128 + 2),
                        lane);
}

__global__ __launch_bounds__(kDrThreads) void decode_route_window_kernel(DecodeRouteArgs ra,
                                                                         DecodeRouteArgs rt,
                                                                         DecodeArgs da, int B,
                                                                         int nrw, int npw, int wpg,
                                                                         int ntask) {
  if ((int)blockIdx.x < B) {
    decode_route_body<kRouteAll>(ra, blockIdx.x);
    return;
  }
  if ((int)blockIdx.x < nrw * B) {
    decode_route_body<kTailOnly>(rt, (int)blockIdx.x - B);
    return;
  }
  // one task per wavefront, wpg wavefronts of each work-group (the others end at
  // once); the index is made uniform, so that its loads are scalar
  const int wv = (int)threadIdx.x / kWave;
  if (wv >= wpg) return;
  const int task = __builtin_amdgcn_readfirstlane(((int)blockIdx.x - nrw * B) * wpg + wv);
  if (task >= ntask) return;
  const int lane = wave_lane();
  if (task < B * da.H * npw) {
    const int piece = task % npw, bh = task / npw;
    const int h = bh % da.H, b = bh / da.H;
    const DcSpan sp = dc_span(da, b);
    DcState st;
    dc_init(st, da, b, h, lane);
    // pieces past the window write an empty partial, so that the merge reads every
    // slot without knowing the window's length
    if (piece < ds_pieces(da, sp)) {
      const int j0 = sp.w0 * da.bs + piece * da.piece;
      dc_keys<32>(st, da, b, h, sp, j0, min(j0 + da.piece, sp.len), false, 0.f);
    }
    dc_store_partial<128>(st, da.part + ((int64_t)bh * (npw + da.K) + piece) * (128 + 2), lane);
  }
  // then routed slot ntask - 1 - task: the wavefronts dispatched last take the
  // routed slots, so that their waits for the routers are the shortest
  const int rtask = ntask - 1 - task;
  if (ra.pub && rtask < B * da.H * da.K) {
    const int r = rtask % da.K, bh = rtask / da.K;
    ds_routed_slot(ra, da, bh / da.H, bh % da.H, r, npw, lane);
  }
}

// Routed blocks of the fused step in a launch of their own (grids of more than one
// round of work-groups, where the slots taken by the first launch's last wavefronts
// would lengthen its tail): one wavefront per routed slot of (b, h), 32 keys per
// round trip; slot npw + r of the partials (an empty partial past the routed count).
__global__ __launch_bounds__(64) void decode_routed_kernel(DecodeArgs da, int npw) {
  __shared__ int sTmp[kWave];
  __shared__ int sRC[kDcMaxK];
  __shared__ float sRB[kDcMaxK];
  const int r = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const DcSpan sp = dc_span(da, b);
  const int n_r = dc_routed(da, b, sp, lane, sTmp, sRC, sRB, [] { __syncthreads(); });
  DcState st;
  dc_init(st, da, b, h, lane);
  if (r < n_r) dc_block<32>(st, da, b, h, sp, sRC[r], true, sRB[r]);
  dc_store_partial<128>(st, da.part + ((int64_t)(b * da.H + h) * (npw + da.K) + npw + r) * (128 + 2),
                        lane);
}

// Merge of the fused step: the npw window-piece slots of (b, h) and its K routed
// slots (npw ..), one wavefront per (b, h).
__global__ __launch_bounds__(64) void decode_step_merge_kernel(DecodeArgs da, int npw,
                                                              uint64_t* pub) {
  __shared__ float sW[kWave];
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  // the step's last launch zeroes the slots sequence b's router published (every
  // reader of them ran in the first launch), so the next step starts from zero
  if (pub && h == 0 && lane < 2 * da.K) pub[2 * (int64_t)b * da.K + lane] = 0ull;
  // every slot holds a partial (empty ones past the window and the routed count),
  // so the loads need nothing but the launch arguments
  const int n = npw + da.K;
  const float* pb = da.part + (int64_t)(b * da.H + h) * (npw + da.K) * (128 + 2);
  auto part_at = [&](int s) -> const float* { return pb + s * (128 + 2); };
  float ms = -INFINITY, lsum = 0.f;
  if (lane < n) { ms = part_at(lane)[128]; lsum = part_at(lane)[129]; }
  dc_merge<128>(da, b, h, lane, n, ms, lsum, sW, part_at);
}

}  // namespace dash

namespace dash {
// Workspace of the fused decode step: the (o, m, l) partials of the smallest window
// pieces (the most of them) and the routed slots from its start; at its end, below
// its last whole-256-byte boundary, the published routing words [B, kDcMaxK, 2],
// which must be zero before the first step (each step zeroes them again).  Anchored
// at the end, the words of a smaller batch lie inside those of a larger one on the
// same buffer (as on the allocation-free entry's fixed array).
inline int64_t step_sync_offset(int B, int H, int D, int block_size, int local_window) {
  const int npw = (local_window + block_size - 1 + kDsPieceMin - 1) / kDsPieceMin;
  const int64_t part = (int64_t)B * H * (npw + kDcMaxK) * (D + 2) * (int64_t)sizeof(float);
  return (part + 255) / 256 * 256;
}
inline int64_t step_sync_bytes(int B) { return (int64_t)B * kDcMaxK * 2 * 8; }
inline int64_t step_pub_offset(int64_t workspace_bytes, int B) {
  return workspace_bytes / 256 * 256 - step_sync_bytes(B);
}

// Checks and packs the arguments of the decode router (shared by the router entry
// and the fused decode step).
static int decode_route_args(const float* idx_q, int64_t iq_sb, const float* idx_k,
                                 int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
                                 const int32_t* block_table, int64_t table_stride,
                                 int page_size, const int32_t* seq_lens, const int32_t* q_pos,
                                 int S, const float* head_cls, int refresh_tail, float* kbar,
                                 int64_t kb_sb, int nblk_cap, const int32_t* kb_table,
                                 int64_t kb_ts, const int32_t* bounds, const uint8_t* cand,
                                 int64_t cand_stride, int B, int d, int block_size,
                                 int local_blocks, float idx_scale, float floor_p, float sigma,
                                 int K, int topm, int Kout, int32_t* idx, float* bias,
                                 uint8_t* valid, float* z, int64_t z_stride, DecodeRouteArgs& a) {
  if (!idx_q || !idx_k || !head_cls || !kbar || !idx || !bias || !z) return kErrInvalid;
  if (B < 0 || d <= 0 || d > 256 || block_size <= 0 || block_size > 256) return kErrUnsupported;
  if (topm < 1 || topm > kMaxM) return kErrUnsupported;
  if (K < 1 || Kout < std::min(K, topm)) return kErrInvalid;
  if (nblk_cap <= 0 || nblk_cap > kDrMaxBlocks) return kErrUnsupported;
  if (block_table && page_size <= 0) return kErrInvalid;
  // S bounds every sequence's length (the kernels clamp lens to it), so the k_bar
  // cache and the score rows must hold ceil(S / block_size) blocks
  if (S < 0 || ((int64_t)S + block_size - 1) / block_size > nblk_cap) return kErrInvalid;
  if (d % 16 != 0 || kb_sb % 4 != 0 || (uintptr_t)kbar % 16 != 0) return kErrUnsupported;
  if (kb_table && kb_ts < nblk_cap) return kErrInvalid;
  if (ik_st % 4 != 0 || ik_sp % 4 != 0 || ik_sb % 4 != 0 || (uintptr_t)idx_k % 16 != 0 ||
      (uintptr_t)head_cls % 16 != 0)
    return kErrUnsupported;
  a.idx_q = idx_q; a.iq_sb = iq_sb;
  a.idx_k = idx_k;
  a.lay_k = SeqLayout{nullptr, block_table, table_stride, ik_sb, ik_sp, ik_st, page_size};
  a.lens = seq_lens; a.q_pos = q_pos; a.S = S;
  a.head_cls = head_cls; a.refresh_tail = refresh_tail; a.skip_tail = 0;
  a.kbar = kbar; a.kb_sb = kb_sb; a.nblk_cap = nblk_cap;
  a.kb_table = kb_table; a.kb_ts = kb_ts; a.bounds = bounds;
  a.cand = cand; a.cand_stride = cand_stride;
  a.d = d; a.bs = block_size; a.local_blocks = local_blocks;
  a.inv_sqrt_d = (float)(1.0 / sqrt((double)d));
  a.idx_scale = idx_scale; a.floor_p = floor_p; a.inv_sigma = (float)(1.0 / (double)sigma);
  a.K = K; a.topm = topm; a.Kout = Kout;
  a.idx = idx; a.bias = bias; a.valid = valid;
  a.z = z; a.z_stride = z_stride;
  a.pub = nullptr;
  return kOk;
}
}  // namespace dash

extern "C" int dash_decode_route(const float* idx_q, int64_t iq_sb, const float* idx_k,
                                 int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
                                 const int32_t* block_table, int64_t table_stride,
                                 int page_size, const int32_t* seq_lens, const int32_t* q_pos,
                                 int S, const float* head_cls, int refresh_tail, float* kbar,
                                 int64_t kb_sb, int nblk_cap, const int32_t* kb_table,
                                 int64_t kb_ts, const int32_t* bounds, const uint8_t* cand,
                                 int64_t cand_stride, int B, int d, int block_size,
                                 int local_blocks, float idx_scale, float floor_p, float sigma,
                                 int K, int topm, int Kout, int32_t* idx, float* bias,
                                 uint8_t* valid, float* z, int64_t z_stride, void* stream) {
  using namespace dash;
  DecodeRouteArgs a;
  const int st = decode_route_args(idx_q, iq_sb, idx_k, ik_sb, ik_st, ik_sp, block_table, table_stride,
                                   page_size, seq_lens, q_pos, S, head_cls, refresh_tail, kbar, kb_sb,
                                   nblk_cap, kb_table, kb_ts, bounds, cand, cand_stride, B, d,
                                   block_size, local_blocks,
                                   idx_scale, floor_p, sigma, K, topm, Kout, idx, bias, valid, z,
                                   z_stride, a);
  if (st != kOk || B == 0) return st;
  // the tail refresh beside the routing when the tail block cannot be remote
  const int nrw = (refresh_tail && local_blocks >= 1) ? 2 : 1;
  const DecodeRouteArgs rt = a;
  if (nrw == 2) { a.refresh_tail = 0; a.skip_tail = 1; }
  hipLaunchKernelGGL(decode_route_kernel, dim3(nrw * B), dim3(kDrThreads), 0, (hipStream_t)stream,
                     a, rt, B);
  return launch_status();
}

extern "C" int dash_decode_step_workspace_size(int B, int H, int D, int block_size,
                                               int local_window, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || H < 0 || D <= 0 || block_size <= 0 || local_window < 1) return kErrInvalid;
  *bytes = step_sync_offset(B, H, D, block_size, local_window) + step_sync_bytes(B);
  return kOk;
}

extern "C" int dash_decode_step(
    const float* idx_q, int64_t iq_sb, const float* idx_k, int64_t ik_sb, int64_t ik_st,
    int64_t ik_sp, const int32_t* block_table, int64_t table_stride, int page_size,
    const int32_t* seq_lens, const int32_t* q_pos, int S, const float* head_cls,
    int refresh_tail, float* kbar,
    int64_t kb_sb, int nblk_cap, const int32_t* kb_table, int64_t kb_ts, const int32_t* bounds,
    const uint8_t* cand, int64_t cand_stride, int d,
    int local_blocks, float idx_scale, float floor_p, float sigma, int K, int topm, int Kout,
    int32_t* idx, float* bias, uint8_t* valid, float* z, int64_t z_stride,
    const void* q, int64_t q_sb, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t k_sp,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t v_sp,
    void* out, int out_bf16, int64_t o_sb, int64_t o_sh, float* lse, int64_t lse_sb,
    int64_t lse_sh, int B, int H, int D, int block_size, int local_window, float scale,
    void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace dash;
  DecodeRouteArgs ra;
  const int rs = decode_route_args(idx_q, iq_sb, idx_k, ik_sb, ik_st, ik_sp, block_table,
                                   table_stride, page_size, seq_lens, q_pos, S, head_cls, refresh_tail,
                                   kbar, kb_sb, nblk_cap, kb_table, kb_ts, bounds, cand,
                                   cand_stride, B, d, block_size,
                                   local_blocks, idx_scale, floor_p, sigma, K, topm, Kout, idx, bias,
                                   valid, z, z_stride, ra);
  if (rs != kOk) return rs;
  if (!q || !k || !v || !out || H <= 0) return kErrInvalid;
  if (D != 128) return kErrUnsupported;
  if (Kout > kDcMaxK) return kErrUnsupported;
  if (block_size % 64 != 0 && block_size != 32) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if (block_table && page_size % block_size != 0) return kErrUnsupported;
  const int piece = ds_piece_keys(B, H, local_window, block_size);
  const int npw = (local_window + block_size - 1 + piece - 1) / piece;
  if (npw + Kout > kWave) return kErrUnsupported;     // partials of one merge wavefront
  if (B == 0) return kOk;
  const int64_t strides[] = {q_sb, q_sh, k_sb, k_sh, k_st, k_sp, v_sb, v_sh, v_st, v_sp};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  const void* ptrs[] = {q, k, v};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return kErrUnsupported;
  int64_t need = 0;
  dash_decode_step_workspace_size(B, H, D, block_size, local_window, &need);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0) return kErrWorkspace;
  DecodeArgs a;
  a.q = (const bf16*)q; a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st; a.k_sp = k_sp;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st; a.v_sp = v_sp;
  a.table = block_table; a.table_stride = table_stride; a.page = page_size;
  a.lens = seq_lens; a.q_pos = q_pos;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = Kout;
  a.out = out; a.out_bf16 = out_bf16; a.o_sb = o_sb; a.o_sh = o_sh;
  a.lse = lse; a.lse_sb = lse_sb; a.lse_sh = lse_sh;
  a.part = (float*)workspace;
  a.S = S; a.H = H; a.bs = block_size; a.lw = local_window; a.nsplit = npw; a.piece = piece;
  a.scale_log2e = scale * 1.4426950408889634f;
  // the tail refresh beside the routing when the tail block cannot be remote
  const int nrw = (refresh_tail && local_blocks >= 1) ? 2 : 1;
  // One wavefront per window piece; when the whole grid fits on the CUs at once
  // (one round of work-groups), the same wavefronts then take the routed slots
  // (extra wavefronts when there are more slots than pieces), else a second launch
  // does.  The window-only grid is sized first, as the routed slots add no
  // work-groups unless there are more slots than pieces.
  const int64_t wtasks = (int64_t)B * H * npw;
  // tasks per work-group: at most one per wavefront, and as few as give each CU
  // beside the routers' at most one work-group (a CU streams its pieces' rows at a
  // bounded rate, so few pieces go faster spread over more CUs)
  const int64_t free_cus = kDsCUs - nrw * (int64_t)B;
  auto wpg_for = [&](int64_t t) {
    return free_cus <= 0 ? kDrThreads / kWave
                         : (int)std::min<int64_t>(kDrThreads / kWave,
                                                  std::max<int64_t>(1, (t + free_cus - 1) / free_cus));
  };
  const int64_t stasks = (int64_t)B * H * std::max(npw, Kout);
  const int swpg = wpg_for(stasks);
  const bool in_launch = Kout > 0 && nrw * (int64_t)B + (stasks + swpg - 1) / swpg <= kDsCUs;
  const int64_t tasks = in_launch ? stasks : wtasks;
  if (tasks > 0x7fffffff) return kErrUnsupported;
  const DecodeRouteArgs rt = ra;
  if (nrw == 2) { ra.refresh_tail = 0; ra.skip_tail = 1; }
  // the partials end at most at step_sync_offset, the words start at or above it
  ra.pub = in_launch ? (uint64_t*)((char*)workspace + step_pub_offset(workspace_bytes, B)) : nullptr;
  const int wpg = wpg_for(tasks);
  const int64_t wgs = nrw * (int64_t)B + (tasks + wpg - 1) / wpg;
  if (wgs > 0x7fffffff) return kErrUnsupported;
  hipLaunchKernelGGL(decode_route_window_kernel, dim3((unsigned)wgs), dim3(kDrThreads), 0,
                     (hipStream_t)stream, ra, rt, a, B, nrw, npw, wpg, (int)tasks);
  if (Kout > 0 && !in_launch)
    hipLaunchKernelGGL(decode_routed_kernel, dim3(Kout, H, B), dim3(64), 0, (hipStream_t)stream, a,
                       npw);
  hipLaunchKernelGGL(decode_step_merge_kernel, dim3(H, B), dim3(64), 0, (hipStream_t)stream, a,
                     npw, ra.pub);
  return launch_status();
}

// ---------------------------------------------------------------------------
// Allocation-free decode step: the window and routed-block partials live in a
// fixed device array of this library instead of a caller workspace.  Each GPU
// holds its own copy; its address is looked up once per device (with that device
// current) on the first call there.  The partial slots a step reads are all
// written by the same step, so nothing needs clearing between calls; calls that
// overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
namespace dash {
constexpr int64_t kStepScratchBytes = 64ll << 20;
static __device__ __align__(256) float scratch[kStepScratchBytes / sizeof(float)];
constexpr int kMaxScratchDevices = 64;
static std::atomic<float*> g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

// The array's device address on the current device (hipGetSymbolAddress the first
// time); returns a status.
static int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxScratchDevices) return kErrUnsupported;
  float* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!addr) return kErrInvalid;
      p = (float*)addr;
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return kOk;
}
}  // namespace dash

extern "C" int64_t dash_decode_step_scratch_bytes(void) { return dash::kStepScratchBytes; }

extern "C" int dash_decode_step_noalloc(
    const float* idx_q, int64_t iq_sb, const float* idx_k, int64_t ik_sb, int64_t ik_st,
    int64_t ik_sp, const int32_t* block_table, int64_t table_stride, int page_size,
    const int32_t* seq_lens, const int32_t* q_pos, int S, const float* head_cls,
    int refresh_tail, float* kbar, int64_t kb_sb, int nblk_cap, const int32_t* kb_table,
    int64_t kb_ts, const int32_t* bounds, const uint8_t* cand,
    int64_t cand_stride, int d, int local_blocks, float idx_scale, float floor_p, float sigma,
    int K, int topm, int Kout, int32_t* idx, float* bias, uint8_t* valid, float* z,
    int64_t z_stride,
    const void* q, int64_t q_sb, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t k_sp,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t v_sp,
    void* out, int out_bf16, int64_t o_sb, int64_t o_sh, float* lse, int64_t lse_sb,
    int64_t lse_sh, int B, int H, int D, int block_size, int local_window, float scale,
    void* stream) {
  using namespace dash;
  int64_t need = 0;
  const int ws = dash_decode_step_workspace_size(B, H, D, block_size, local_window, &need);
  if (ws != kOk) return ws;
  if (need > kStepScratchBytes) return kErrScratch;
  float* ptr = nullptr;
  const int sst = scratch_on_current_device(&ptr);
  if (sst != kOk) return sst;
  return dash_decode_step(idx_q, iq_sb, idx_k, ik_sb, ik_st, ik_sp, block_table, table_stride,
                          page_size, seq_lens, q_pos, S, head_cls, refresh_tail, kbar, kb_sb,
                          nblk_cap, kb_table, kb_ts, bounds, cand, cand_stride, d, local_blocks,
                          idx_scale, floor_p, sigma,
                          K, topm, Kout, idx, bias, valid, z, z_stride, q, q_sb, q_sh, k, k_sb,
                          k_sh, k_st, k_sp, v, v_sb, v_sh, v_st, v_sp, out, out_bf16, o_sb, o_sh,
                          lse, lse_sb, lse_sh, B, H, D, block_size, local_window, scale, ptr,
                          kStepScratchBytes, stream);
}

// ---------------------------------------------------------------------------
// Router front end: the index projections' Gemma RMSNorm, optional RoPE and the
// finiteness guards (dash_attention.py:680-700 and the q/k path of
// modeling_deepseekv2.py:336-348), one wavefront per (row, q or k), two dims per
// lane.  The projection of both sides comes from one GEMM, [rows, 2d] (q then k).
// Every elementwise step is one correctly rounded operation as in the unfused
// sequence; in bf16 (bf16 projection and bf16 cos/sin) each RoPE product and the
// sum are rounded to bf16 as separate tensor ops round them.
// ---------------------------------------------------------------------------
namespace dash {

struct RouterQkArgs {
  const void* proj; int proj_bf16; int64_t proj_row; int64_t rows; int S;
  const float* wq; const float* wk; float eps;
  const void* cos; const void* sin; int cs_bf16; int64_t cs_sb, cs_st;
  float* iq; float* ik;
};

__device__ __forceinline__ float rb16(float x) { return (float)(bf16)x; }
__device__ __forceinline__ float finite_or_zero(float x) {
  return (fabsf(x) <= 3.402823466e38f) ? x : 0.f;
}

__global__ __launch_bounds__(256) void router_qk_kernel(RouterQkArgs a) {
#pragma clang fp contract(off)
  const int64_t task = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
  if (task >= a.rows * 2) return;
  const int64_t row = task >> 1;
  const int side = (int)(task & 1);            // 0: q, 1: k
  const int lane = wave_lane(), i0 = 2 * lane;
  constexpr int d = 128;
  float x0, x1;
  if (a.proj_bf16) {
    const bf16x2 v = *(const bf16x2*)((const bf16*)a.proj + row * a.proj_row + side * d + i0);
    x0 = (float)v[0]; x1 = (float)v[1];
  } else {
    const float2 v = *(const float2*)((const float*)a.proj + row * a.proj_row + side * d + i0);
    x0 = v.x; x1 = v.y;
  }
  x0 = finite_or_zero(x0);
  x1 = finite_or_zero(x1);
  const float ss = wave_sum(__fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1)));
  const float r = rsqrtf(__fadd_rn(__fmul_rn(ss, 1.0f / d), a.eps));
  const float* w = side ? a.wk : a.wq;
  const float2 wv = *(const float2*)(w + i0);
  float y0 = fminf(fmaxf(__fmul_rn(x0, r), -kActClamp), kActClamp);
  float y1 = fminf(fmaxf(__fmul_rn(x1, r), -kActClamp), kActClamp);
  y0 = fminf(fmaxf(__fmul_rn(y0, __fadd_rn(1.0f, wv.x)), -kActClamp), kActClamp);
  y1 = fminf(fmaxf(__fmul_rn(y1, __fadd_rn(1.0f, wv.y)), -kActClamp), kActClamp);
  if (a.proj_bf16) { y0 = rb16(y0); y1 = rb16(y1); }
  if (a.cos) {
    const int64_t b = row / a.S, t = row % a.S;
    const int64_t co = b * a.cs_sb + t * a.cs_st + i0;
    float c0, c1, s0, s1;
    if (a.cs_bf16) {
      const bf16x2 cv = *(const bf16x2*)((const bf16*)a.cos + co);
      const bf16x2 sv = *(const bf16x2*)((const bf16*)a.sin + co);
      c0 = (float)cv[0]; c1 = (float)cv[1]; s0 = (float)sv[0]; s1 = (float)sv[1];
    } else {
      const float2 cv = *(const float2*)((const float*)a.cos + co);
      const float2 sv = *(const float2*)((const float*)a.sin + co);
      c0 = cv.x; c1 = cv.y; s0 = sv.x; s1 = sv.y;
    }
    // rotate_half: dim i < d/2 takes -y[i + d/2], dim i >= d/2 takes y[i - d/2]
    const float p0 = __shfl_xor(y0, 32, kWave), p1 = __shfl_xor(y1, 32, kWave);
    const float h0 = lane < 32 ? -p0 : p0, h1 = lane < 32 ? -p1 : p1;
    const bool bf = a.proj_bf16 && a.cs_bf16;
    float t0 = __fmul_rn(y0, c0), t1 = __fmul_rn(y1, c1);
    float u0 = __fmul_rn(h0, s0), u1 = __fmul_rn(h1, s1);
    if (bf) { t0 = rb16(t0); t1 = rb16(t1); u0 = rb16(u0); u1 = rb16(u1); }
    y0 = __fadd_rn(t0, u0);
    y1 = __fadd_rn(t1, u1);
    if (bf) { y0 = rb16(y0); y1 = rb16(y1); }
  }
  float* out = (side ? a.ik : a.iq) + row * d + i0;
  *(float2*)out = make_float2(finite_or_zero(y0), finite_or_zero(y1));
}

}  // namespace dash

extern "C" int dash_router_qk_norm(const void* proj, int proj_bf16, int64_t proj_row,
                                   int64_t rows, int S, int d, const float* wq,
                                   const float* wk, float eps, const void* cos,
                                   const void* sin, int cs_bf16, int64_t cs_sb, int64_t cs_st,
                                   float* idx_q, float* idx_k, void* stream) {
  using namespace dash;
  if (!proj || !wq || !wk || !idx_q || !idx_k || rows < 0 || S <= 0) return kErrInvalid;
  if (d != 128) return kErrUnsupported;
  if ((cos == nullptr) != (sin == nullptr)) return kErrInvalid;
  const int es = proj_bf16 ? 2 : 4, cs = cs_bf16 ? 2 : 4;
  if (proj_row % 2 != 0 || (uintptr_t)proj % (2 * es) != 0) return kErrUnsupported;
  if ((uintptr_t)wq % 8 != 0 || (uintptr_t)wk % 8 != 0 || (uintptr_t)idx_q % 8 != 0 ||
      (uintptr_t)idx_k % 8 != 0)
    return kErrUnsupported;
  if (cos && ((uintptr_t)cos % (2 * cs) != 0 || (uintptr_t)sin % (2 * cs) != 0 ||
              cs_sb % 2 != 0 || cs_st % 2 != 0))
    return kErrUnsupported;
  if (rows == 0) return kOk;
  RouterQkArgs a;
  a.proj = proj; a.proj_bf16 = proj_bf16; a.proj_row = proj_row; a.rows = rows; a.S = S;
  a.wq = wq; a.wk = wk; a.eps = eps;
  a.cos = cos; a.sin = sin; a.cs_bf16 = cs_bf16; a.cs_sb = cs_sb; a.cs_st = cs_st;
  a.iq = idx_q; a.ik = idx_k;
  const int64_t grid = (rows * 2 + 3) / 4;
  if (grid > 0x7fffffff) return kErrUnsupported;
  hipLaunchKernelGGL(router_qk_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a);
  return launch_status();
}
