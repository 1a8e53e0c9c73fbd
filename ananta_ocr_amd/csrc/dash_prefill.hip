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
// Work decomposition (hybrid):
//   * tile kernel: one work-group of 4 wavefronts per (128-query tile, head,
//     sequence), 32 queries per wavefront.  Keys are staged in LDS 32 at a time;
//     S^T = K Q^T (32 keys x 32 queries, v_mfma_f32_32x32x16_bf16), masks, bias,
//     online softmax (base 2), O^T += V^T P^T, so each lane owns one query's
//     softmax state.  It covers the window band and the routed blocks that many
//     queries of the tile share ("dense" blocks: every query masks the blocks it
//     did not select), then merges the partials of the other routed blocks.
//   * sparse kernel: routed (query, block) pairs whose block few queries of the
//     tile selected are grouped by block (plan -> scan -> scatter kernels); one
//     work-group stages the block's K/V in LDS once and runs up to 128 gathered
//     queries through the same MFMA tiles, writing a normalised bf16 partial and
//     its base-2 log-sum-exp per (pair, head).
// With no plan (dense_threshold <= 0) the tile kernel processes every routed
// block of the tile as a dense block.

#include "dash_common.h"

namespace dash {

constexpr int kPfTQ = 128;        // queries per tile work-group
constexpr int kPfMaxK = 16;       // routed slots per query
constexpr int kPfMaxBlocks = 2048;
constexpr int kPfCH = 128;        // pairs per sparse chunk

struct PrefillArgs {
  const bf16* q; const bf16* k; const bf16* v;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  bf16* o; int64_t o_sb, o_sh, o_st;
  float* lse; int64_t lse_row, lse_sh;  // lse[token_row * lse_row + h * lse_sh]
  const int32_t* idx; const uint8_t* valid; const float* bias; int K;   // [rows, K]
  const int32_t* cu;                   // varlen: [B+1]
  const int32_t* kmin;                 // per token row, or null
  int S, H, bs, lw, nblk_cap;
  float scale_log2e;
  // hybrid plan (null kind: every routed block is processed by the tile kernel)
  uint8_t* kind;                       // [rows, K]: 0 skip, 1 tile (dense), 2 sparse
  int dense_threshold;
  int32_t* blk_count;                  // [B, nblk_cap]  zero between calls
  int32_t* tile_base;                  // [B, ntiles_cap, nblk_cap] offset of a tile's pairs
  int ntiles_cap;
  int32_t* blk_off;                    // [B, nblk_cap]
  int32_t* num_chunks;                 // [B]
  int4* chunk_tab;                     // [B, chunk_cap]: block, start, count
  int chunk_cap;
  int32_t* pairs;                      // [rows * K] grouped by block per sequence
  float* part_lse;                     // [rows * K, H]  base-2 log-sum-exp
  bf16* part_o;                        // [rows * K, H, D]  normalised partial output
};

__device__ __forceinline__ int seq_len(const PrefillArgs& a, int b) {
  return a.cu ? a.cu[b + 1] - a.cu[b] : a.S;
}
__device__ __forceinline__ int64_t row0(const PrefillArgs& a, int b) {
  return a.cu ? (int64_t)a.cu[b] : (int64_t)b * a.S;
}
__device__ __forceinline__ const bf16* seq_ptr(const bf16* base, const int32_t* cu, int b,
                                               int64_t sb, int64_t st) {
  return cu ? base + (int64_t)cu[b] * st : base + (int64_t)b * sb;
}

// Keep a routed slot?  The block must exist, be valid, and have keys below the
// window start and at or above the segment start.
__device__ __forceinline__ bool slot_usable(const PrefillArgs& a, int c, int64_t p, int t, int nblk,
                                            int km) {
  if (c < 0 || c >= nblk) return false;
  if (a.valid && !a.valid[p]) return false;
  const int ls = t - a.lw + 1;
  return c * a.bs < ls && (c + 1) * a.bs > km;
}

// ---------------------------------------------------------------------------
// MFMA building blocks (32 queries per wavefront, lane = query n, half hl)
// ---------------------------------------------------------------------------
template <int D, int LDK>
__device__ __forceinline__ floatx16 qk_tile(const bf16 (*sK)[LDK], int krow0, const bf16x8 (&qop)[D / 16],
                                            int n, int hl) {
  floatx16 s;
#pragma unroll
  for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const bf16x8 kop = *(const bf16x8*)&sK[krow0 + n][kk * 16 + hl * 8];
    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[kk], s, 0, 0, 0);
  }
  return s;
}

// acc_o[dt] += V^T P^T over keys kbase .. kbase+15 of a row-major LDS V tile.
// ds_read_tr16_b64 (gfx950): within each 16-lane group, result lane i element j
// is element (i % 4) of the 8 bytes read by lane 4j + i/4.  Lane l reads the 4
// dims 32dt + 16((l/16)%2) + 4(l%4) .. +3 of key row kbase + 4hl + (l%16)/4 (and
// +8), which gives every lane the 8 keys kbase + 8(e/4) + 4hl + e%4 of its dim
// row m = l % 32: the same key order as the P^T operand built from S^T.
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

template <int D, int LDV>
__device__ __forceinline__ void pv_slice_tr(const bf16 (*sV)[LDV], int kbase, const bf16x8& pop,
                                            floatx16 (&acc_o)[D / 32], int lane) {
  const int hl = lane >> 5;
  const int row = kbase + 4 * hl + ((lane & 15) >> 2);
  const int colq = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    const int col = dt * 32 + colq;
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)&sV[row][col]);
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)&sV[row + 8][col]);
    bf16x8 vop;
    const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
    const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
    for (int e = 0; e < 4; ++e) { vop[e] = l4[e]; vop[e + 4] = h4[e]; }
    acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, acc_o[dt], 0, 0, 0);
  }
}

// Stage rows j0 .. j0+nrows-1 of K and V (both row-major) into LDS; rows at or
// beyond len are zero.  nrows * D / 8 chunks of 16 bytes over 256 threads.
template <int D, int LDK, int LDV>
__device__ __forceinline__ void stage_kv(bf16 (*sK)[LDK], bf16 (*sV)[LDV], const bf16* kb,
                                         const bf16* vb, int64_t k_st, int64_t v_st, int j0,
                                         int nrows, int len, int tid) {
  const int nchunks = nrows * (D / 8);
  for (int chunk = tid; chunk < nchunks; chunk += 256) {
    const int kr = chunk / (D / 8), c8 = (chunk % (D / 8)) * 8;
    const int j = j0 + kr;
    bf16x8 kv8, vv8;
    if (j < len) {
      kv8 = *(const bf16x8*)(kb + (int64_t)j * k_st + c8);
      vv8 = *(const bf16x8*)(vb + (int64_t)j * v_st + c8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { kv8[e] = (bf16)0.f; vv8[e] = (bf16)0.f; }
    }
    *(bf16x8*)&sK[kr][c8] = kv8;
    *(bf16x8*)&sV[kr][c8] = vv8;
  }
}

// Load the K <= 16 routed slots of one row: ids, validity and bias, with
// vector loads where the row is 16-byte aligned.
__device__ __forceinline__ void load_row_slots(const PrefillArgs& a, int64_t row, int32_t (&c)[kPfMaxK],
                                               uint32_t& vmask) {
  const int64_t p0 = row * a.K;
  if (a.K == kPfMaxK) {
    const int4* ip = (const int4*)(a.idx + p0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4 v = ip[q];
      c[4 * q] = v.x; c[4 * q + 1] = v.y; c[4 * q + 2] = v.z; c[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) c[s] = s < a.K ? a.idx[p0 + s] : -1;
  }
  vmask = 0;
  if (a.valid) {
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s)
      if (s < a.K && a.valid[p0 + s]) vmask |= 1u << s;
  } else {
    vmask = (a.K >= 32) ? 0xffffffffu : ((1u << a.K) - 1u);
  }
}

__global__ __launch_bounds__(kPfTQ) void prefill_plan_kernel(PrefillArgs a) {
  __shared__ int32_t sCnt[kPfMaxBlocks];
  const int b = blockIdx.y, tid = threadIdx.x;
  const int len = seq_len(a, b);
  const int t0 = blockIdx.x * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  for (int i = tid; i < nblk; i += kPfTQ) sCnt[i] = 0;
  __syncthreads();
  const int t = t0 + tid;
  const int64_t row = row0(a, b) + t;
  int32_t c[kPfMaxK];
  uint32_t vmask = 0, keep_mask = 0;
  if (t < len) {
    load_row_slots(a, row, c, vmask);
    const int km = a.kmin ? a.kmin[row] : 0;
    const int ls = t - a.lw + 1;
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) {
      bool ok = s < a.K && ((vmask >> s) & 1u) && c[s] >= 0 && c[s] < nblk &&
                c[s] * a.bs < ls && (c[s] + 1) * a.bs > km;
#pragma unroll
      for (int u = 0; u < s; ++u) ok = ok && !(((keep_mask >> u) & 1u) && c[u] == c[s]);
      if (ok) {
        keep_mask |= 1u << s;
        atomicAdd(&sCnt[c[s]], 1);
      }
    }
  }
  __syncthreads();
  // one global atomic per sparse block of this tile: reserves the tile's range
  // in the block's pair list (its base is kept for the scatter kernel)
  int32_t* tb = a.tile_base + ((int64_t)b * a.ntiles_cap + blockIdx.x) * a.nblk_cap;
  for (int cc = tid; cc < nblk; cc += kPfTQ) {
    const int n = sCnt[cc];
    if (n > 0 && n < a.dense_threshold)
      tb[cc] = atomicAdd(&a.blk_count[(int64_t)b * a.nblk_cap + cc], n);
  }
  if (t < len) {
    uint8_t kd[kPfMaxK];
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) {
      kd[s] = 0;
      if ((keep_mask >> s) & 1u) kd[s] = sCnt[c[s]] >= a.dense_threshold ? 1 : 2;
    }
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s)
      if (s < a.K) a.kind[row * a.K + s] = kd[s];
  }
}

// ---------------------------------------------------------------------------
// Scan: per sequence, block offsets of the sparse pairs and the chunk table.
// Resets the block counters (they are zero between calls).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void prefill_scan_kernel(PrefillArgs a) {
  __shared__ int32_t sC[kPfMaxBlocks];
  __shared__ int32_t sOff[kPfMaxBlocks];
  __shared__ int32_t sCh[kPfMaxBlocks];
  __shared__ int32_t sWave[2][16];
  const int b = blockIdx.x, tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int len = seq_len(a, b);
  const int nblk = len > 0 ? (len + a.bs - 1) / a.bs : 0;
  int32_t* cnt = a.blk_count + (int64_t)b * a.nblk_cap;
  // two entries per thread
  int v0 = 0, v1 = 0;
  const int e0 = tid * 2, e1 = tid * 2 + 1;
  if (e0 < a.nblk_cap) { v0 = e0 < nblk ? cnt[e0] : 0; cnt[e0] = 0; }
  if (e1 < a.nblk_cap) { v1 = e1 < nblk ? cnt[e1] : 0; cnt[e1] = 0; }
  const int c0 = (v0 + kPfCH - 1) / kPfCH, c1 = (v1 + kPfCH - 1) / kPfCH;
  int sp = v0 + v1, sc = c0 + c1;
  int ip = sp, ic = sc;
#pragma unroll
  for (int s = 1; s < kWave; s <<= 1) {
    const int op = __shfl_up(ip, s, kWave), oc = __shfl_up(ic, s, kWave);
    if (lane >= s) { ip += op; ic += oc; }
  }
  if (lane == kWave - 1) { sWave[0][wv] = ip; sWave[1][wv] = ic; }
  __syncthreads();
  int bp = 0, bc = 0;
  for (int w = 0; w < wv; ++w) { bp += sWave[0][w]; bc += sWave[1][w]; }
  const int xp = bp + ip - sp, xc = bc + ic - sc;   // exclusive prefix of this thread
  if (e0 < kPfMaxBlocks) { sC[e0] = v0; sOff[e0] = xp; sCh[e0] = xc; }
  if (e1 < kPfMaxBlocks) { sC[e1] = v1; sOff[e1] = xp + v0; sCh[e1] = xc + c0; }
  if (tid == 1023) a.num_chunks[b] = bc + ic;
  __syncthreads();
  int4* tab = a.chunk_tab + (int64_t)b * a.chunk_cap;
  for (int c = tid; c < nblk; c += 1024) {
    a.blk_off[(int64_t)b * a.nblk_cap + c] = sOff[c];
    const int n = sC[c];
    for (int i = 0; i * kPfCH < n; ++i)
      tab[sCh[c] + i] = make_int4(c, sOff[c] + i * kPfCH, min(kPfCH, n - i * kPfCH), 0);
  }
}

// ---------------------------------------------------------------------------
// Scatter: sparse pairs into per-block lists (order within a block is free).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kPfTQ) void prefill_scatter_kernel(PrefillArgs a) {
  __shared__ int32_t sFill[kPfMaxBlocks];
  const int b = blockIdx.y, tid = threadIdx.x;
  const int len = seq_len(a, b);
  const int t0 = blockIdx.x * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  for (int i = tid; i < nblk; i += kPfTQ) sFill[i] = 0;
  __syncthreads();
  const int t = t0 + tid;
  if (t >= len) return;
  const int64_t row = row0(a, b) + t;
  const int64_t base = row0(a, b) * a.K;
  const int32_t* tb = a.tile_base + ((int64_t)b * a.ntiles_cap + blockIdx.x) * a.nblk_cap;
  const int32_t* off = a.blk_off + (int64_t)b * a.nblk_cap;
  int32_t c[kPfMaxK];
  uint32_t vmask;
  load_row_slots(a, row, c, vmask);
  int pos[kPfMaxK];
  bool sp[kPfMaxK];
#pragma unroll
  for (int s = 0; s < kPfMaxK; ++s) {
    sp[s] = s < a.K && a.kind[row * a.K + s] == 2;
    pos[s] = sp[s] ? atomicAdd(&sFill[c[s]], 1) : 0;
  }
#pragma unroll
  for (int s = 0; s < kPfMaxK; ++s)
    if (sp[s]) a.pairs[base + off[c[s]] + tb[c[s]] + pos[s]] = (int32_t)(row * a.K + s - base);
}

// ---------------------------------------------------------------------------
// Sparse kernel: one chunk of <= 128 pairs of one routed block, one head.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void prefill_sparse_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) bf16 sK[64][D + 8];
  __shared__ __attribute__((aligned(16))) bf16 sV[64][D + 32];
  const int b = blockIdx.z, h = blockIdx.y, ch = blockIdx.x;
  if (ch >= a.num_chunks[b]) return;
  const int4 e = a.chunk_tab[(int64_t)b * a.chunk_cap + ch];
  const int c = e.x, start = e.y, npairs = e.z;
  const int len = seq_len(a, b);
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5, n = lane & 31;
  const int64_t r0 = row0(a, b);
  const bf16* kb = seq_ptr(a.k, a.cu, b, a.k_sb, a.k_st) + (int64_t)h * a.k_sh;
  const bf16* vb = seq_ptr(a.v, a.cu, b, a.v_sb, a.v_st) + (int64_t)h * a.v_sh;
  stage_kv<D, D + 8, D + 32>(sK, sV, kb, vb, a.k_st, a.v_st, c * a.bs, a.bs, len, tid);

  const int pi = wv * 32 + n;
  const bool active = pi < npairs;
  const int32_t pl = a.pairs[r0 * a.K + start + min(pi, npairs - 1)];   // pair index in sequence
  const int64_t p = r0 * a.K + pl;
  const int t = pl / a.K;
  const int ls = t - a.lw + 1;
  const int km = a.kmin ? a.kmin[r0 + t] : 0;
  const float bias2 = a.bias[p] * 1.4426950408889634f;
  const bf16* qb = seq_ptr(a.q, a.cu, b, a.q_sb, a.q_st) + (int64_t)h * a.q_sh + (int64_t)t * a.q_st;
  bf16x8 qop[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) qop[kk] = *(const bf16x8*)(qb + kk * 16 + hl * 8);
  __syncthreads();
  if (!__any(active)) return;

  const int nsub = a.bs / 32;     // 1 or 2 key sub-tiles of 32
  floatx16 s[2];
  float mloc = -INFINITY;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub < nsub) {
      s[sub] = qk_tile<D, D + 8>(sK, sub * 32, qop, n, hl);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = c * a.bs + sub * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
        const bool ok = active && key < ls && key >= km && key < len;
        const float x = ok ? s[sub][r] * a.scale_log2e + bias2 : -INFINITY;
        s[sub][r] = x;
        mloc = fmaxf(mloc, x);
      }
    }
  }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
  const float mu = (mloc == -INFINITY) ? 0.f : mloc;
  floatx16 acc_o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.f;
  float psum = 0.f;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (sub < nsub) {
      bf16x8 pop[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(s[sub][r] - mu);
        psum += pr;
        pop[r >> 3][r & 7] = (bf16)pr;
      }
      pv_slice_tr<D, D + 32>(sV, sub * 32, pop[0], acc_o, lane);
      pv_slice_tr<D, D + 32>(sV, sub * 32 + 16, pop[1], acc_o, lane);
    }
  }
  const float l_tot = psum + __shfl_xor(psum, 32, kWave);
  if (!active) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  bf16* po = a.part_o + (p * a.H + h) * D;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 w;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) w[q4] = (bf16)(acc_o[dt][g * 4 + q4] * inv);
      *(bf16x4*)(po + dt * 32 + 8 * g + 4 * hl) = w;
    }
  if (hl == 0) a.part_lse[p * a.H + h] = l_tot > 0.f ? mloc + log2f(l_tot) : -INFINITY;
}

// ---------------------------------------------------------------------------
// Tile kernel: window band + dense routed blocks + merge of the sparse partials.
// ---------------------------------------------------------------------------
// Register-staged K/V rows for the software pipeline of the tile kernel:
// thread tid holds chunks tid + 256*i (i < 4) of a 64-key x 128-dim tile.
struct KVRegs {
  bf16x8 k[4], v[4];
};

template <int D>
__device__ __forceinline__ void kv_prefetch(KVRegs& r, const bf16* kb, const bf16* vb,
                                            int64_t k_st, int64_t v_st, int j0, int nkeys,
                                            int len, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int chunk = tid + 256 * i;
    const int kr = chunk / (D / 8), c8 = (chunk % (D / 8)) * 8;
    const int j = j0 + kr;
    if (kr < nkeys && j < len) {
      r.k[i] = *(const bf16x8*)(kb + (int64_t)j * k_st + c8);
      r.v[i] = *(const bf16x8*)(vb + (int64_t)j * v_st + c8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) { r.k[i][e] = (bf16)0.f; r.v[i][e] = (bf16)0.f; }
    }
  }
}

template <int D, int LDK, int LDV>
__device__ __forceinline__ void kv_commit(const KVRegs& r, bf16 (*sK)[LDK], bf16 (*sV)[LDV],
                                          int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int chunk = tid + 256 * i;
    const int kr = chunk / (D / 8), c8 = (chunk % (D / 8)) * 8;
    *(bf16x8*)&sK[kr][c8] = r.k[i];
    *(bf16x8*)&sV[kr][c8] = r.v[i];
  }
}

// ---------------------------------------------------------------------------
// Tile kernel: window band + dense routed blocks + merge of the sparse partials.
// Items of up to 64 keys: the window band in 64-key steps, then one item per
// dense routed block (per 64 keys of it).  The next item's K/V is loaded into
// registers while the current one computes.
// ---------------------------------------------------------------------------
constexpr int kPfIT = 64;         // keys per item in the tile kernel

template <int D>
__global__ __launch_bounds__(256, 2) void prefill_tile_kernel(PrefillArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ __attribute__((aligned(16))) bf16 sK[kPfIT][D + 8];
  __shared__ __attribute__((aligned(16))) bf16 sV[kPfIT][D + 32];
  __shared__ int32_t sIdx[kPfTQ][kPfMaxK];
  __shared__ float sBias[kPfTQ][kPfMaxK];
  __shared__ int32_t sCnt[kPfTQ];
  __shared__ uint32_t sBits[kPfMaxBlocks / 32];
  __shared__ int32_t sUnion[kPfMaxBlocks];
  __shared__ int32_t sNU;

  const int b = blockIdx.z, h = blockIdx.y;
  const int len = seq_len(a, b);
  const int t0 = blockIdx.x * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5;         // half of the wave: 0/1
  const int n = lane & 31;          // query column within the wave
  const int64_t r0 = row0(a, b);

  for (int i = tid; i < kPfMaxBlocks / 32; i += 256) sBits[i] = 0u;
  __syncthreads();

  // ---- dense routed blocks of every query row: filter, dedup, sort ascending ----
  if (tid < kPfTQ) {
    const int t = t0 + tid;
    int cnt = 0;
    if (t < len) {
      const int64_t row = r0 + t;
      const int km = a.kmin ? a.kmin[row] : 0;
      for (int s = 0; s < a.K; ++s) {
        const int64_t p = row * a.K + s;
        const int c = a.idx[p];
        if (a.kind) {
          if (a.kind[p] != 1) continue;
        } else {
          if (!slot_usable(a, c, p, t, nblk, km)) continue;
          bool dup = false;
          for (int u = 0; u < cnt; ++u) dup |= (sIdx[tid][u] == c);
          if (dup) continue;
        }
        const float bv = a.bias[p];
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
  const int64_t qrow = r0 + tqc;
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
  const int jw0 = (max(t0 - a.lw + 1, 0) / kPfIT) * kPfIT;
  const int n_win = (t_last - jw0) / kPfIT + 1;
  const int ipb = (a.bs + kPfIT - 1) / kPfIT;      // items per routed block
  const int keys_rt = min(a.bs, kPfIT);            // keys per routed item
  const int n_items = n_win + nu * ipb;

  const bf16* kb = seq_ptr(a.k, a.cu, b, a.k_sb, a.k_st) + (int64_t)h * a.k_sh;
  const bf16* vb = seq_ptr(a.v, a.cu, b, a.v_sb, a.v_st) + (int64_t)h * a.v_sh;
  const int myrow = wv * 32 + n;           // row within the tile
  const int tw = t0 + wv * 32;             // first query of this wavefront
  int ptr = 0;                             // next dense block of this query
  bool cur_sel = false;
  float cur_bias = 0.f;
  const float log2e = 1.4426950408889634f;

  auto item_start = [&](int it, int& nkeys) -> int {
    if (it < n_win) { nkeys = kPfIT; return jw0 + it * kPfIT; }
    const int r = it - n_win;
    nkeys = keys_rt;
    return sUnion[r / ipb] * a.bs + (r % ipb) * kPfIT;
  };

  KVRegs pre;
  if (n_items > 0) {
    int nk0;
    const int j00 = item_start(0, nk0);
    kv_prefetch<D>(pre, kb, vb, a.k_st, a.v_st, j00, nk0, len, tid);
  }
  for (int it = 0; it < n_items; ++it) {
    const bool routed = it >= n_win;
    int nkeys;
    const int j0 = item_start(it, nkeys);
    int c = -1, sub_item = 0;
    if (routed) {
      const int r = it - n_win;
      c = sUnion[r / ipb];
      sub_item = r % ipb;
    }
    __syncthreads();                       // the previous item is done with LDS
    kv_commit<D, D + 8, D + 32>(pre, sK, sV, tid);
    __syncthreads();
    if (it + 1 < n_items) {
      int nk1;
      const int j1 = item_start(it + 1, nk1);
      kv_prefetch<D>(pre, kb, vb, a.k_st, a.v_st, j1, nk1, len, tid);
    }

    // ---- does any query of this wavefront use this item? ----
    bool use;
    float brow = 0.f;
    if (!routed) {
      use = (j0 <= tq) && (j0 + nkeys - 1 >= q_lo) && (tq < len);
    } else {
      if (sub_item == 0) {
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

    // ---- per 32-key sub-tile: S^T, masks, bias, online softmax, O^T += V^T P^T ----
    // A sub-tile is skipped when no key of it is visible to any query of the
    // wavefront, and needs no per-element mask when every key is visible to every
    // query (unselected routed queries carry a -inf bias instead).
    const int nsub = nkeys / 32;
    const float bsel = use ? brow : -INFINITY;
    for (int sb = 0; sb < nsub; ++sb) {
      const int k0 = j0 + sb * 32;
      bool full;
      if (!routed) {
        if (k0 > tw + 31 || k0 + 31 < max(tw - a.lw + 1, 0)) continue;
        full = !a.kmin && k0 + 31 <= tw && k0 >= tw + 31 - a.lw + 1 && tw + 31 < len;
      } else {
        full = !a.kmin && k0 + 31 < tw - a.lw + 1 && k0 + 31 < len;
      }
      floatx16 s = qk_tile<D, D + 8>(sK, sb * 32, qop, n, hl);
      float mloc = -INFINITY;
      if (full) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[r] = fmaf(s[r], a.scale_log2e, bsel);
          mloc = fmaxf(mloc, s[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * hl + (r & 3);
          bool ok;
          if (!routed) ok = use && key >= q_lo && key <= tq;
          else ok = use && key < q_ls && key >= q_km && key < len;
          const float x = ok ? fmaf(s[r], a.scale_log2e, brow) : -INFINITY;
          s[r] = x;
          mloc = fmaxf(mloc, x);
        }
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
      // Lazy rescale: the exponent reference m_run only moves when some query's
      // maximum exceeds it by more than 8 (probabilities stay <= 2^8).
      if (__any(mloc > m_run + 8.f)) {
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
        m_run = m_new;
      }
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
      bf16x8 pop[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(s[r] - m_use);
        l_run += pr;
        pop[r >> 3][r & 7] = (bf16)pr;
      }
      pv_slice_tr<D, D + 32>(sV, sb * 32, pop[0], acc_o, lane);
      pv_slice_tr<D, D + 32>(sV, sb * 32 + 16, pop[1], acc_o, lane);
    }
  }

  // ---- merge the sparse partials of this query ----
  if (a.kind && tq < len) {
    const int64_t row = r0 + tq;
    for (int s = 0; s < a.K; ++s) {
      const int64_t p = row * a.K + s;
      if (a.kind[p] != 2) continue;
      const float lse2 = a.part_lse[p * a.H + h];
      if (lse2 == -INFINITY) continue;
      const float m_new = fmaxf(m_run, lse2);
      const float alpha = fast_exp2(m_run - m_new);
      const float w = fast_exp2(lse2 - m_new);
      l_run = l_run * alpha + (hl == 0 ? w : 0.f);
      m_run = m_new;
      const bf16* po = a.part_o + (p * a.H + h) * D;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const bf16x4 ov = *(const bf16x4*)(po + dt * 32 + 8 * g + 4 * hl);
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            acc_o[dt][g * 4 + q4] = acc_o[dt][g * 4 + q4] * alpha + w * bf2f(ov[q4]);
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
      a.lse[(r0 + tq) * a.lse_row + (int64_t)h * a.lse_sh] = lse;
    }
  }
}

// Workspace layout of the hybrid plan (byte offsets, 256-byte aligned pieces).
struct PlanLayout {
  int64_t count, tbase, off, nchunks, tab, pairs, kind, plse, po, total;
  int chunk_cap, ntiles_cap;
};

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

inline PlanLayout plan_layout(int B, int H, int S_max, int64_t rows, int K, int D,
                              int nblk_cap) {
  PlanLayout L;
  L.chunk_cap = (int)((int64_t)S_max * K / kPfCH) + nblk_cap + 1;
  L.ntiles_cap = (S_max + kPfTQ - 1) / kPfTQ;
  const int64_t nbc = (int64_t)B * nblk_cap;
  int64_t o = 0;
  L.count = o; o = align256(o + nbc * 4);
  L.tbase = o; o = align256(o + nbc * L.ntiles_cap * 4);
  L.off = o; o = align256(o + nbc * 4);
  L.nchunks = o; o = align256(o + (int64_t)B * 4);
  L.tab = o; o = align256(o + (int64_t)B * L.chunk_cap * 16);
  L.pairs = o; o = align256(o + rows * K * 4);
  L.kind = o; o = align256(o + rows * K);
  L.plse = o; o = align256(o + rows * K * H * 4);
  L.po = o; o = align256(o + rows * K * H * D * 2);
  L.total = o;
  return L;
}

}  // namespace dash

// ---------------------------------------------------------------------------
// C entry points
// ---------------------------------------------------------------------------
extern "C" int dash_attn_prefill_workspace_size(int B, int H, int S_max, int64_t total_rows,
                                                int K, int D, int block_size, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || H <= 0 || S_max < 0 || total_rows < 0 || K < 0 || block_size <= 0)
    return kErrInvalid;
  const int nblk_cap = (S_max + block_size - 1) / block_size;
  *bytes = plan_layout(B, H, S_max, total_rows, K, D, nblk_cap).total;
  return kOk;
}

extern "C" int dash_attn_prefill(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    float* lse, int64_t lse_row, int64_t lse_sh,
    const int32_t* idx, const uint8_t* valid, const float* bias, int K,
    const int32_t* cu_seqlens, const int32_t* kmin,
    int B, int H, int S, int D, int block_size, int local_window, float scale,
    int dense_threshold, int64_t total_rows, void* workspace, int64_t workspace_bytes,
    void* stream) {
  using namespace dash;
  if (!q || !k || !v || !o || B < 0 || H <= 0 || S < 0) return kErrInvalid;
  if (K > 0 && (!idx || !bias)) return kErrInvalid;
  if (D != 128) return kErrUnsupported;
  if (block_size <= 0 || block_size % 32 != 0 || block_size > 256) return kErrUnsupported;
  if (K < 0 || K > kPfMaxK) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if (B == 0 || S == 0) return kOk;
  const int nblk_cap = (S + block_size - 1) / block_size;
  if (nblk_cap > kPfMaxBlocks) return kErrUnsupported;
  // 16-byte rows for the bf16x8 loads and stores
  const int64_t strides[] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  const void* ptrs[] = {q, k, v, o};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return kErrUnsupported;
  PrefillArgs a = {};
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.o = (bf16*)o; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = lse; a.lse_row = lse_row; a.lse_sh = lse_sh;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = K;
  a.cu = cu_seqlens; a.kmin = kmin;
  a.S = S; a.H = H; a.bs = block_size; a.lw = local_window; a.nblk_cap = nblk_cap;
  a.scale_log2e = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const int ntiles = (S + kPfTQ - 1) / kPfTQ;
  const bool hybrid = dense_threshold > 0 && K > 0 && block_size <= 64;
  if (hybrid) {
    if (total_rows <= 0) return kErrInvalid;
    const PlanLayout L = plan_layout(B, H, S, total_rows, K, D, nblk_cap);
    if (!workspace || workspace_bytes < L.total || (uintptr_t)workspace % 256 != 0)
      return kErrWorkspace;
    char* w = (char*)workspace;
    a.kind = (uint8_t*)(w + L.kind);
    a.dense_threshold = dense_threshold;
    a.blk_count = (int32_t*)(w + L.count);
    a.tile_base = (int32_t*)(w + L.tbase);
    a.ntiles_cap = L.ntiles_cap;
    a.blk_off = (int32_t*)(w + L.off);
    a.num_chunks = (int32_t*)(w + L.nchunks);
    a.chunk_tab = (int4*)(w + L.tab);
    a.chunk_cap = L.chunk_cap;
    a.pairs = (int32_t*)(w + L.pairs);
    a.part_lse = (float*)(w + L.plse);
    a.part_o = (bf16*)(w + L.po);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(ntiles, B), dim3(kPfTQ), 0, st, a);
    hipLaunchKernelGGL(prefill_scan_kernel, dim3(B), dim3(1024), 0, st, a);
    hipLaunchKernelGGL(prefill_scatter_kernel, dim3(ntiles, B), dim3(kPfTQ), 0, st, a);
    hipLaunchKernelGGL(prefill_sparse_kernel<128>, dim3(L.chunk_cap, H, B), dim3(256), 0, st, a);
  }
  hipLaunchKernelGGL(prefill_tile_kernel<128>, dim3(ntiles, H, B), dim3(256), 0, st, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
