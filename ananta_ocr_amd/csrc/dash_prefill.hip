// DASH prefill attention on gfx950: block-sparse attention over the token
// window (t-LW, t] plus the routed remote blocks of each query, with the
// routed block's log-prior bias on its keys.
//
// Semantics follow the fused kernel sparse_gather_e2e_triton.py:34-115 (and the
// segment start of sparse_gather_triton.py:42,63,73):
//   window keys  j in [max(t-LW+1, kmin(t)), t]             bias 0
//   routed keys  j in routed block c, kmin(t) <= j < t-LW+1  bias b(t,c)
// (duplicated routed blocks count once, first slot wins; rows with no key give 0).
//
// Work decomposition: one work-group of 4 wavefronts per (128-query tile, head,
// sequence); each wavefront owns 32 queries.  Keys are staged in LDS 32 at a
// time.  For every key tile the wavefront computes S^T = K Q^T (32 keys x 32
// queries) with v_mfma_f32_32x32x16_bf16, applies masks/bias and the online
// softmax, and accumulates O^T = V^T P^T (128 dims x 32 queries), so each lane
// owns one query's softmax state and no cross-lane rescale is needed.
// The routed blocks of a tile are processed as the union over its queries,
// each query masking the blocks it did not select.

#include "dash_common.h"

namespace dash {

constexpr int kPfTQ = 128;        // queries per work-group
constexpr int kPfKT = 32;         // keys per LDS tile
constexpr int kPfMaxK = 16;       // routed slots per query
constexpr int kPfMaxBlocks = 2048;

struct PrefillArgs {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  bf16* o; int64_t o_sb, o_sh, o_st;
  float* lse; int64_t lse_sh;          // lse[token_row * lse_row + h * lse_sh]
  int64_t lse_row;
  const int32_t* idx; const uint8_t* valid; const float* bias; int K;   // [rows, K]
  const int32_t* cu;                   // varlen: [B+1]
  const int32_t* kmin;                 // per token row, or null
  int S, H, bs, lw;
  float scale_log2e;
};

__device__ __forceinline__ const bf16* seq_ptr(const bf16* base, const int32_t* cu, int b,
                                               int64_t sb, int64_t st) {
  return cu ? base + (int64_t)cu[b] * st : base + (int64_t)b * sb;
}

template <int D>
__global__ __launch_bounds__(256) void prefill_union_kernel(PrefillArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ __attribute__((aligned(16))) bf16 sK[kPfKT][D + 8];
  __shared__ __attribute__((aligned(16))) bf16 sVt[D][kPfKT + 4];
  __shared__ int32_t sIdx[kPfTQ][kPfMaxK];
  __shared__ float sBias[kPfTQ][kPfMaxK];
  __shared__ int32_t sCnt[kPfTQ];
  __shared__ uint32_t sBits[kPfMaxBlocks / 32];
  __shared__ int32_t sUnion[kPfMaxBlocks];
  __shared__ int32_t sNU;

  const int b = blockIdx.z, h = blockIdx.y;
  const int len = a.cu ? a.cu[b + 1] - a.cu[b] : a.S;
  const int t0 = blockIdx.x * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5;         // half of the wave: 0/1
  const int n = lane & 31;          // query column within the wave

  for (int i = tid; i < kPfMaxBlocks / 32; i += 256) sBits[i] = 0u;
  __syncthreads();

  // ---- routed blocks of every query row: filter, dedup, sort ascending ----
  if (tid < kPfTQ) {
    const int t = t0 + tid;
    int cnt = 0;
    if (t < len) {
      const int64_t row = token_row(a.cu, b, t, a.S);
      const int ls = t - a.lw + 1;
      const int km = a.kmin ? a.kmin[row] : 0;
      for (int s = 0; s < a.K; ++s) {
        const int c = a.idx[row * a.K + s];
        if (c < 0 || c >= nblk) continue;
        if (a.valid && !a.valid[row * a.K + s]) continue;
        // a routed block contributes only keys below the window start
        if (c * a.bs >= ls || (c + 1) * a.bs <= km) continue;
        bool dup = false;
        for (int u = 0; u < cnt; ++u) dup |= (sIdx[tid][u] == c);
        if (dup) continue;
        const float bv = a.bias[row * a.K + s];
        int u = cnt;
        while (u > 0 && sIdx[tid][u - 1] > c) {
          sIdx[tid][u] = sIdx[tid][u - 1];
          sBias[tid][u] = sBias[tid][u - 1];
          --u;
        }
        sIdx[tid][u] = c;
        sBias[tid][u] = bv;
        ++cnt;
        atomicOr(&sBits[c >> 5], 1u << (c & 31));
      }
    }
    sCnt[tid] = cnt;
  }
  __syncthreads();
  // ---- compact the union bitmap into an ascending block list ----
  if (wv == 0) {
    int base = 0;
    for (int w0 = 0; w0 < (nblk + 31) / 32; w0 += kWave) {
      const int w = w0 + lane;
      const uint32_t bits = (w < (nblk + 31) / 32) ? sBits[w] : 0u;
      const int c = __popc(bits);
      int incl = c;
#pragma unroll
      for (int s = 1; s < kWave; s <<= 1) {
        const int o = __shfl_up(incl, s, kWave);
        if (lane >= s) incl += o;
      }
      int off = base + incl - c;
      uint32_t bb = bits;
      while (bb) {
        const int bit = __ffs(bb) - 1;
        sUnion[off++] = w * 32 + bit;
        bb &= bb - 1;
      }
      base += __shfl(incl, kWave - 1, kWave);
    }
    if (lane == 0) sNU = base;
  }

  // ---- this lane's query and its Q^T operand (8 k-steps of 16 dims) ----
  const int tq = t0 + wv * 32 + n;
  const int tqc = min(tq, len - 1);
  const int64_t qrow = token_row(a.cu, b, tqc, a.S);
  const bf16* qb = seq_ptr(a.q, a.cu, b, a.q_sb, a.q_st) + (int64_t)h * a.q_sh;
  bf16x8 qop[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qop[kk] = *(const bf16x8*)(qb + (int64_t)tqc * a.q_st + kk * 16 + hl * 8);
  const int q_ls = tq - a.lw + 1;
  const int q_km = a.kmin ? a.kmin[qrow] : 0;
  const int q_lo = max(max(q_ls, q_km), 0);       // first window key

  floatx16 acc_o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  __syncthreads();
  const int nu = sNU;
  const int t_last = min(t0 + kPfTQ - 1, len - 1);
  const int jw0 = (max(t0 - a.lw + 1, 0) / kPfKT) * kPfKT;
  const int n_win = (t_last - jw0) / kPfKT + 1;
  const int subs = a.bs / kPfKT;
  const int n_items = n_win + nu * subs;

  const bf16* kb = seq_ptr(a.k, a.cu, b, a.k_sb, a.k_st) + (int64_t)h * a.k_sh;
  const bf16* vb = seq_ptr(a.v, a.cu, b, a.v_sb, a.v_st) + (int64_t)h * a.v_sh;
  const int myrow = wv * 32 + n;           // row within the tile
  int ptr = 0;                             // next routed block of this query
  bool cur_sel = false;
  float cur_bias = 0.f;
  const float log2e = 1.4426950408889634f;

  for (int it = 0; it < n_items; ++it) {
    const bool routed = it >= n_win;
    int j0, c = -1, sub = 0;
    if (!routed) {
      j0 = jw0 + it * kPfKT;
    } else {
      const int r = it - n_win;
      c = sUnion[r / subs];
      sub = r % subs;
      j0 = c * a.bs + sub * kPfKT;
    }
    // ---- stage K (row major) and V (transposed) for keys j0..j0+31 ----
    __syncthreads();
#pragma unroll
    for (int rep = 0; rep < 2; ++rep) {
      const int chunk = tid + rep * 256;           // 32 rows x 16 chunks of 8 dims
      const int kr = chunk >> 4, c8 = (chunk & 15) * 8;
      const int j = j0 + kr;
      bf16x8 kv8, vv8;
      if (j < len) {
        kv8 = *(const bf16x8*)(kb + (int64_t)j * a.k_st + c8);
        vv8 = *(const bf16x8*)(vb + (int64_t)j * a.v_st + c8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) { kv8[e] = (bf16)0.f; vv8[e] = (bf16)0.f; }
      }
      *(bf16x8*)&sK[kr][c8] = kv8;
#pragma unroll
      for (int e = 0; e < 8; ++e) sVt[c8 + e][kr] = vv8[e];
    }
    __syncthreads();

    // ---- does any query of this wavefront use this key tile? ----
    bool use;
    float brow = 0.f;
    if (!routed) {
      use = (j0 <= tq) && (j0 + kPfKT - 1 >= q_lo) && (tq < len);
    } else {
      if (sub == 0) {
        cur_sel = false;
        if (ptr < sCnt[myrow] && sIdx[myrow][ptr] == c) {
          cur_sel = true;
          cur_bias = sBias[myrow][ptr];
          ++ptr;
        }
      }
      use = cur_sel && (tq < len);
      brow = cur_bias * log2e;
    }
    if (!__any(use)) continue;

    // ---- S^T = K Q^T ----
    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const bf16x8 kop = *(const bf16x8*)&sK[n][kk * 16 + hl * 8];
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[kk], s, 0, 0, 0);
    }
    // ---- mask, bias, online softmax (base 2) ----
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = j0 + 8 * (r >> 2) + 4 * hl + (r & 3);
      bool ok;
      if (!routed) ok = use && key >= q_lo && key <= tq;
      else ok = use && key < q_ls && key >= q_km && key < len;
      const float x = ok ? s[r] * a.scale_log2e + brow : -INFINITY;
      s[r] = x;
      mloc = fmaxf(mloc, x);
    }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    float psum = 0.f;
    bf16x8 pop[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = exp2f(s[r] - m_use);
      psum += p;
      pop[r >> 3][r & 7] = (bf16)p;
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
    // ---- O^T += V^T P^T ----
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt) {
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const bf16* vrow = &sVt[dt * 32 + n][sl * 16 + 4 * hl];
        const bf16x4 lo = *(const bf16x4*)vrow;
        const bf16x4 hi = *(const bf16x4*)(vrow + 8);
        bf16x8 vop;
#pragma unroll
        for (int e = 0; e < 4; ++e) { vop[e] = lo[e]; vop[e + 4] = hi[e]; }
        acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop[sl], acc_o[dt], 0, 0, 0);
      }
    }
  }

  // ---- epilogue: normalise and store ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (tq < len) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16* ob = (a.cu ? a.o + (int64_t)a.cu[b] * a.o_st : a.o + (int64_t)b * a.o_sb) +
               (int64_t)h * a.o_sh + (int64_t)tq * a.o_st;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (bf16)(acc_o[dt][g * 4 + e] * inv);
        *(bf16x4*)(ob + dt * 32 + 8 * g + 4 * hl) = w;
      }
    if (a.lse && hl == 0) {
      const float lse = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.6931471805599453f : -INFINITY;
      a.lse[token_row(a.cu, b, tq, a.S) * a.lse_row + (int64_t)h * a.lse_sh] = lse;
    }
  }
}

}  // namespace dash

// ---------------------------------------------------------------------------
// C entry point
// ---------------------------------------------------------------------------
extern "C" int dash_attn_prefill(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    float* lse, int64_t lse_row, int64_t lse_sh,
    const int32_t* idx, const uint8_t* valid, const float* bias, int K,
    const int32_t* cu_seqlens, const int32_t* kmin,
    int B, int H, int S, int D, int block_size, int local_window, float scale,
    void* stream) {
  using namespace dash;
  if (!q || !k || !v || !o || B < 0 || H <= 0 || S < 0) return kErrInvalid;
  if (K > 0 && (!idx || !bias)) return kErrInvalid;
  if (D != 128) return kErrUnsupported;
  if (block_size <= 0 || block_size % kPfKT != 0 || block_size > 256) return kErrUnsupported;
  if (K < 0 || K > kPfMaxK) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if (B == 0 || S == 0) return kOk;
  if ((S + block_size - 1) / block_size > kPfMaxBlocks) return kErrUnsupported;
  // 16-byte rows for the bf16x8 loads and stores
  const int64_t strides[] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  const void* ptrs[] = {q, k, v, o};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return kErrUnsupported;
  PrefillArgs a;
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.o = (bf16*)o; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = lse; a.lse_row = lse_row; a.lse_sh = lse_sh;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = K;
  a.cu = cu_seqlens; a.kmin = kmin;
  a.S = S; a.H = H; a.bs = block_size; a.lw = local_window;
  a.scale_log2e = scale * 1.4426950408889634f;
  dim3 grid((S + kPfTQ - 1) / kPfTQ, H, B);
  hipLaunchKernelGGL(prefill_union_kernel<128>, grid, dim3(256), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
