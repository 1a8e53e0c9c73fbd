// Backward of the DASH prefill attention on gfx950: dQ, dK, dV and the gradient
// of every routed slot's bias, for the forward of dash_prefill.hip (window keys
// [max(t-LW+1, kmin(t)), t] with bias 0, keys of the routed blocks in
// [kmin(t), t-LW] with the block's bias; duplicated blocks count once).
// Counterpart of the Triton backward kernels of sparse_gather_e2e_triton.py:
// 118-262 (dq / d_bias) and :265-330 (dk / dv), with the same mathematics:
//   P = exp(scale q.k + b - lse),  dP = dO.v,  dS = P (dP - delta),
//   delta = sum_d O dO,  dV = sum_t P dO,  dK = scale sum_t dS q,
//   dQ = scale sum_j dS k,  d_bias(t, slot) = sum_heads sum_{j in the block} dS.
//
// Work decomposition (this file is included by dash_prefill.hip):
//   * delta kernel: delta = sum_d O dO per (row, head), 16 lanes per row;
//   * the forward's plan with every routed pair block-major (no dense blocks):
//     each routed block's (query, slot) pairs in chunk records;
//   * key-major kernel, one work-group per (64-key stage, head, sequence): the
//     stage's K and V stay in LDS while 64 queries at a time stream through it --
//     first the window band (every query whose window reaches the stage), then
//     the routed pairs of the stage's blocks, gathered.  Per 32-query chunk and
//     32-key half (one wavefront): S = Q K^T and dP = dO V^T on the matrix cores
//     (lane = key), P and dS in registers, dV^T += dO^T P and dK^T += Q^T dS with
//     the transposed operands read by ds_read_tr16_b64 from the staged rows.  dK
//     and dV are complete when the work-group ends (no atomics).  For routed
//     pairs it also writes dQ^T = K^T dS^T (dS transposed through LDS) and the
//     row sums of dS as fp32 partials per (head, pair);
//   * query-major kernel, one work-group per (128-query tile, head, sequence),
//     lane = query: dQ^T += K^T dS^T over the window band (S^T, dP^T recomputed),
//     plus the query's routed partials, times the scale;
//   * a small kernel sums the bias gradient partials over the heads per slot.

#pragma once

namespace dash {

struct BwdArgs {
  PrefillArgs p;                          // q, k, v, routing, varlen, plan workspace
  const bf16* o; int64_t o_sb, o_sh, o_st;
  const bf16* dout; int64_t do_sb, do_sh, do_st;
  const float* lse; int64_t lse_row, lse_sh;   // natural log, per (token row, head)
  float* delta;                           // [rows, H]
  bf16* dq; int64_t dq_sb, dq_sh, dq_st;
  bf16* dk; int64_t dk_sb, dk_sh, dk_st;
  bf16* dv; int64_t dv_sb, dv_sh, dv_st;
  float* dbias;                           // [rows, K] (null: not wanted)
  float* part_dq;                         // [H, ppos, nsub, 128] fp32, dims in MFMA lane order
  float* part_db;                         // [H, ppos, nsub] fp32
  float scale;                            // natural softmax scale
  int nstage;                             // 64-key stages per sequence (of nblk_cap blocks)
  int nsub;                               // 64-key stages per block (1 for blocks <= 64 keys)
};

template <typename T>
__device__ __forceinline__ T* seq_base(T* base, const int32_t* cu, int b, int64_t sb, int64_t st) {
  return cu ? base + (int64_t)cu[b] * st : base + (int64_t)b * sb;
}

// delta[row, h] = sum_d O[row, h, d] dO[row, h, d] in fp32; 16 lanes per (row, head).
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdArgs a, int64_t rows) {
  const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 16;
  const int sub = threadIdx.x & 15;
  const int H = a.p.H;
  const bool live = item < rows * H;
  float acc = 0.f;
  if (live) {
    const int64_t row = item / H;
    const int h = (int)(item % H);
    int64_t bo, bd;
    if (a.p.cu) {
      bo = row * a.o_st;
      bd = row * a.do_st;
    } else {
      const int64_t b = row / a.p.S, t = row % a.p.S;
      bo = b * a.o_sb + t * a.o_st;
      bd = b * a.do_sb + t * a.do_st;
    }
    const bf16x8 ov = *(const bf16x8*)(a.o + bo + (int64_t)h * a.o_sh + sub * 8);
    const bf16x8 dv = *(const bf16x8*)(a.dout + bd + (int64_t)h * a.do_sh + sub * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += bf2f(ov[e]) * bf2f(dv[e]);
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, kWave);
  if (live && sub == 0) a.delta[item] = acc;
}

// A operand of X^T (rows = dims 32 dt + lane % 32, k = 8 rows of a k_slot-swizzled
// 128-dim stage in the order kbase + 8 (e / 4) + 4 (lane / 32) + e % 4), by two
// transposing reads: the row order of the B operands built from accumulators.
__device__ __forceinline__ bf16x8 tr_frag_k(const bf16* sX, int kbase, int dt, int lane) {
  const int hl = lane >> 5;
  const int row = kbase + 4 * hl + ((lane & 15) >> 2);
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int within = 4 * (lane & 1);
  const int c = dt * 4 + cq;
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(sX + row * 128 + k_slot(row, c) * 8 + within));
  const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(sX + (row + 8) * 128 + k_slot(row + 8, c) * 8 + within));
  bf16x8 r;
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
  for (int e = 0; e < 4; ++e) { r[e] = l4[e]; r[e + 4] = h4[e]; }
  return r;
}

// B operand (k-step s of 16 rows) from a 32 x 32 accumulator: the lane's rows
// 16 s + 4 (lane / 32) + j and 16 s + 8 + 4 (lane / 32) + j, j < 4, as bf16.
__device__ __forceinline__ bf16x8 acc_bop(const floatx16& x, int s) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[j] = (bf16)x[8 * s + j];
    r[j + 4] = (bf16)x[8 * s + 4 + j];
  }
  return r;
}

// Loads rows of a 64-row, k_slot-swizzled stage from global memory: wavefront wv,
// lane l fills slot l % 16 of rows 16 u + 4 wv + l / 16 (u < 4) from the row
// pointer rowp(r) (chunk (l % 16) ^ (r % 16) of it).
template <typename RowPtr>
__device__ __forceinline__ void stage_rows(bf16* sX, int wv, int lane, RowPtr rowp) {
  const int r0 = 4 * wv + (lane >> 4), slot = lane & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 16 * u + r0;
    const bf16* src = rowp(r) + (slot ^ (r0 & 15)) * 8;
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(sX + (4 * u + wv) * 4 * 128),
                                     16, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Key-major kernel.
// ---------------------------------------------------------------------------
constexpr int kBwIT = 64;                 // keys of a stage, queries per step

__global__ __launch_bounds__(256, 1) void bwd_kv_kernel(BwdArgs a) {
  constexpr int D = 128;
  // K, V, Q and dO stages in one array: the end of the kernel reuses all four to
  // add the two query groups' dK and dV
  __shared__ __attribute__((aligned(16))) bf16 sBuf[4 * kBwIT * D];
  bf16* const sK = sBuf;
  bf16* const sV = sBuf + kBwIT * D;
  bf16* const sQ = sBuf + 2 * kBwIT * D;
  bf16* const sO = sBuf + 3 * kBwIT * D;                              // dO rows
  __shared__ __attribute__((aligned(16))) bf16 sDS[2][32][kBwIT + 8];  // dS [query][key]
  __shared__ float sL2[kBwIT], sDel[kBwIT], sB2[kBwIT];
  __shared__ int sLo[kBwIT], sHi[kBwIT], sRow[kBwIT], sPos[kBwIT];
  __shared__ float sDb[2][kBwIT];

  const PrefillArgs& p = a.p;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int stage = lid % a.nstage, bh = lid / a.nstage;
  const int h = bh % p.H, b = bh / p.H;
  const int len = seq_len(p, b);
  const int j0 = stage * kBwIT;
  // stages past the sequence exit, except those of a block that starts inside it
  // (blocks of more than 64 keys): they write that block's zero partials
  if (j0 / p.bs * p.bs >= len) return;
  const int sub = (j0 % p.bs) / kBwIT;     // this stage within its block (0 for blocks <= 64)
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int kh = wv & 1, qc = wv >> 1, hl = lane >> 5, n = lane & 31;
  const int64_t r0 = row0(p, b);
  const float c2 = a.scale * 1.4426950408889634f;
  const float log2e = 1.4426950408889634f;

  const bf16* kb = seq_base(p.k, p.cu, b, p.k_sb, p.k_st) + (int64_t)h * p.k_sh;
  const bf16* vb = seq_base(p.v, p.cu, b, p.v_sb, p.v_st) + (int64_t)h * p.v_sh;
  const bf16* qb = seq_base(p.q, p.cu, b, p.q_sb, p.q_st) + (int64_t)h * p.q_sh;
  const bf16* ob = seq_base(a.dout, p.cu, b, a.do_sb, a.do_st) + (int64_t)h * a.do_sh;
  stage_rows(sK, wv, lane, [&](int r) { return kb + (int64_t)min(j0 + r, len - 1) * p.k_st; });
  stage_rows(sV, wv, lane, [&](int r) { return vb + (int64_t)min(j0 + r, len - 1) * p.v_st; });

  floatx16 acc_dk[4], acc_dv[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc_dk[dt][r] = 0.f; acc_dv[dt][r] = 0.f; }

  const int key = j0 + 32 * kh + n;        // this lane's key
  const int kst = 32 * kh;                 // this wavefront's keys in the stage
  const int qst = 32 * qc;                 // this wavefront's queries in the step

  // One step over the 64 staged queries (rows of sQ / sO with per-query lse2,
  // delta, bias2 and visible key range [lo, hi] in LDS).  routed: also the dQ and
  // bias gradient partials.
  auto step = [&](bool routed) {
    floatx16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(sQ, qst + n, kk, hl),
                                                  k_frag(sK, kst + n, kk, hl), s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(sO, qst + n, kk, hl),
                                                   k_frag(sV, kst + n, kk, hl), dp, 0, 0, 0);
    }
    // P and dS, lane = key, rows = queries 8 g + 4 hl + j of this wavefront's chunk
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int q0 = qst + 8 * g + 4 * hl;
      const float4 l2 = *(const float4*)&sL2[q0];
      const float4 de = *(const float4*)&sDel[q0];
      const float4 b2 = *(const float4*)&sB2[q0];
      const int4 lo = *(const int4*)&sLo[q0];
      const int4 hi = *(const int4*)&sHi[q0];
      const float l2a[4] = {l2.x, l2.y, l2.z, l2.w};
      const float dea[4] = {de.x, de.y, de.z, de.w};
      const float b2a[4] = {b2.x, b2.y, b2.z, b2.w};
      const int loa[4] = {lo.x, lo.y, lo.z, lo.w};
      const int hia[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * g + j;
        const bool vis = key >= loa[j] && key <= hia[j];
        const float pr = vis ? fast_exp2(fmaf(s[r], c2, b2a[j] - l2a[j])) : 0.f;
        s[r] = pr;                                   // s now holds P
        dp[r] = pr * (dp[r] - dea[j]);               // dp now holds dS
      }
    }
    // dV^T += dO^T P and dK^T += Q^T dS over this wavefront's 32 queries
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pb = acc_bop(s, ks);
      const bf16x8 db = acc_bop(dp, ks);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        acc_dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_k(sO, qst + 16 * ks, dt, lane), pb,
                                                             acc_dv[dt], 0, 0, 0);
        acc_dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_k(sQ, qst + 16 * ks, dt, lane), db,
                                                             acc_dk[dt], 0, 0, 0);
      }
    }
    if (!routed) return;
    // dS transposed through LDS: sDS[qc][query][key of the stage]
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int j = 0; j < 4; ++j) sDS[qc][8 * g + 4 * hl + j][kst + n] = (bf16)dp[4 * g + j];
    // row sums of dS over this wavefront's 32 keys (fp32), one per query row
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = dp[r];
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
      dp[r] = v;
    }
    if (n == 0) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j) sDb[kh][qst + 8 * g + 4 * hl + j] = dp[4 * g + j];
    }
    __syncthreads();
    // dQ^T = K^T dS^T over the 64 keys: wavefront kh takes dims 64 kh .. 64 kh + 63
    floatx16 acc_q[2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_q[u][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16* row = &sDS[qc][n][16 * ks];
      const bf16x4 lo = *(const bf16x4*)(row + 4 * hl);
      const bf16x4 hi = *(const bf16x4*)(row + 8 + 4 * hl);
      bf16x8 dsb;
#pragma unroll
      for (int e = 0; e < 4; ++e) { dsb[e] = lo[e]; dsb[e + 4] = hi[e]; }
#pragma unroll
      for (int u = 0; u < 2; ++u)
        acc_q[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_k(sK, 16 * ks, 2 * kh + u, lane), dsb,
                                                           acc_q[u], 0, 0, 0);
    }
    // partials of the pair of query column n: dims 32 dt + 8 g + 4 hl + j
    const int pos = sPos[qst + n];
    if (pos >= 0) {
      const int64_t pi = ((int64_t)h * p.ppos + pos) * a.nsub + sub;
      float* pd = a.part_dq + pi * D;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(float4*)(pd + 32 * (2 * kh + u) + 8 * g + 4 * hl) =
              make_float4(acc_q[u][4 * g], acc_q[u][4 * g + 1], acc_q[u][4 * g + 2], acc_q[u][4 * g + 3]);
      if (kh == 0 && hl == 0) a.part_db[pi] = sDb[0][qst + n] + sDb[1][qst + n];
    }
  };

  const int LW = p.lw;
  // ---- window band: queries t in [j0, j0 + 63 + LW - 1] ----
  const int t_end = min(j0 + kBwIT - 1 + LW - 1, len - 1);
  for (int t0 = j0; t0 <= t_end; t0 += kBwIT) {
    __syncthreads();                        // the previous step is done with the stages
    stage_rows(sQ, wv, lane, [&](int r) { return qb + (int64_t)min(t0 + r, len - 1) * p.q_st; });
    stage_rows(sO, wv, lane, [&](int r) { return ob + (int64_t)min(t0 + r, len - 1) * a.do_st; });
    if (tid < kBwIT) {
      const int t = t0 + tid;
      const bool ok = t < len;
      const int64_t row = r0 + min(t, len - 1);
      const int km = p.kmin ? p.kmin[row] : 0;
      sL2[tid] = a.lse[row * a.lse_row + (int64_t)h * a.lse_sh] * log2e;
      sDel[tid] = a.delta[row * p.H + h];
      sB2[tid] = 0.f;
      sLo[tid] = ok ? max(max(t - LW + 1, km), 0) : 1;
      sHi[tid] = ok ? t : 0;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    step(false);
  }

  // ---- routed pairs of the stage's blocks ----
  const int bs = p.bs;
  const int c_first = j0 / bs, c_last = p.blk_count ? min(j0 + kBwIT - 1, len - 1) / bs : -1;
  for (int c = c_first; c <= c_last; ++c) {
    const int npairs = p.blk_count[(int64_t)b * p.nblk_cap + c];
    const int ch0 = p.blk_chunk[(int64_t)b * p.nblk_cap + c];
    for (int i0 = 0; i0 < npairs; i0 += kBwIT) {
      __syncthreads();
      if (tid < kBwIT) {
        const int i = i0 + tid;
        int t = 0, pos = -1, lo = 1, hi = 0;
        float bias2 = 0.f;
        if (i < npairs) {
          const int chunk = ch0 + i / kPfCH;
          if (chunk < p.chunk_cap) {
            const int pid = p.chunk_rec[((int64_t)b * p.chunk_cap + chunk) * kRec + kRecHead + i % kPfCH];
            t = min(max(pid / p.K, 0), len - 1);
            const int64_t row = r0 + t;
            pos = p.spos[row * p.K + pid % p.K];
            const int km = p.kmin ? p.kmin[row] : 0;
            lo = max(km, c * bs);
            hi = min(min(t - LW, (c + 1) * bs - 1), len - 1);
            bias2 = p.bias[row * p.K + pid % p.K] * log2e;
          }
        }
        const int64_t row = r0 + t;
        sRow[tid] = t;
        sPos[tid] = pos;
        sL2[tid] = a.lse[row * a.lse_row + (int64_t)h * a.lse_sh] * log2e;
        sDel[tid] = a.delta[row * p.H + h];
        sB2[tid] = bias2;
        sLo[tid] = lo;
        sHi[tid] = pos >= 0 ? hi : lo - 1;
      }
      __syncthreads();
      stage_rows(sQ, wv, lane, [&](int r) { return qb + (int64_t)sRow[r] * p.q_st; });
      stage_rows(sO, wv, lane, [&](int r) { return ob + (int64_t)sRow[r] * a.do_st; });
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      step(true);
    }
  }

  // ---- dK and dV: the two query groups' sums, written by wavefronts 0 and 1 ----
  __syncthreads();
  float* red = (float*)sBuf;                // 64 KB of stages, no longer read
  if (qc == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[((kh * 8 + dt) * 16 + r) * kWave + lane] = acc_dk[dt][r];
        red[((kh * 8 + 4 + dt) * 16 + r) * kWave + lane] = acc_dv[dt][r];
      }
  }
  __syncthreads();
  if (qc == 0 && key < len) {
    bf16* dkp = seq_base(a.dk, p.cu, b, a.dk_sb, a.dk_st) + (int64_t)h * a.dk_sh + (int64_t)key * a.dk_st;
    bf16* dvp = seq_base(a.dv, p.cu, b, a.dv_sb, a.dv_st) + (int64_t)h * a.dv_sh + (int64_t)key * a.dv_st;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 wk, wvv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * g + j;
          wk[j] = (bf16)((acc_dk[dt][r] + red[((kh * 8 + dt) * 16 + r) * kWave + lane]) * a.scale);
          wvv[j] = (bf16)(acc_dv[dt][r] + red[((kh * 8 + 4 + dt) * 16 + r) * kWave + lane]);
        }
        *(bf16x4*)(dkp + 32 * dt + 8 * g + 4 * hl) = wk;
        *(bf16x4*)(dvp + 32 * dt + 8 * g + 4 * hl) = wvv;
      }
  }
}

// ---------------------------------------------------------------------------
// Query-major kernel: dQ over the window band plus the routed partials.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void bwd_q_kernel(BwdArgs a) {
  constexpr int D = 128;
  __shared__ __attribute__((aligned(16))) bf16 sK[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV[kBwIT * D];
  const PrefillArgs& p = a.p;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int tile = lid % p.ntiles, bh = lid / p.ntiles;
  const int h = bh % p.H, b = bh / p.H;
  const int len = seq_len(p, b);
  const int t0 = tile * kPfTQ;
  if (t0 >= len) return;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5, n = lane & 31;
  const int64_t r0 = row0(p, b);
  const float c2 = a.scale * 1.4426950408889634f;
  const int tq = t0 + wv * 32 + n;
  const bool qvalid = tq < len;
  const int tqc = min(tq, len - 1);
  const int64_t qrow = r0 + tqc;
  const bf16* kb = seq_base(p.k, p.cu, b, p.k_sb, p.k_st) + (int64_t)h * p.k_sh;
  const bf16* vb = seq_base(p.v, p.cu, b, p.v_sb, p.v_st) + (int64_t)h * p.v_sh;
  const bf16* qb = seq_base(p.q, p.cu, b, p.q_sb, p.q_st) + (int64_t)h * p.q_sh;
  const bf16* ob = seq_base(a.dout, p.cu, b, a.do_sb, a.do_st) + (int64_t)h * a.do_sh;
  bf16x8 qop[D / 16], oop[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    qop[kk] = *(const bf16x8*)(qb + (int64_t)tqc * p.q_st + kk * 16 + hl * 8);
    oop[kk] = *(const bf16x8*)(ob + (int64_t)tqc * a.do_st + kk * 16 + hl * 8);
  }
  const float l2 = a.lse[qrow * a.lse_row + (int64_t)h * a.lse_sh] * 1.4426950408889634f;
  const float del = a.delta[qrow * p.H + h];
  const int km = p.kmin ? p.kmin[qrow] : 0;
  const int lo = qvalid ? max(max(tq - p.lw + 1, km), 0) : 1;
  const int hi = qvalid ? tq : 0;
  floatx16 acc_q[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_q[dt][r] = 0.f;

  // window keys of the tile: [max(t0 - LW + 1, 0), min(t0 + 127, len - 1)] in 64-key items
  const int k_lo = max(t0 - p.lw + 1, 0) / kBwIT * kBwIT;
  const int k_hi = min(t0 + kPfTQ - 1, len - 1);
  for (int j0 = k_lo; j0 <= k_hi; j0 += kBwIT) {
    __syncthreads();
    stage_rows(sK, wv, lane, [&](int r) { return kb + (int64_t)min(j0 + r, len - 1) * p.k_st; });
    stage_rows(sV, wv, lane, [&](int r) { return vb + (int64_t)min(j0 + r, len - 1) * p.v_st; });
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const bool need = __any(qvalid && lo <= j0 + kBwIT - 1 && hi >= j0);
    if (!need) continue;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      floatx16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(sK, 32 * hf + n, kk, hl), qop[kk], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(sV, 32 * hf + n, kk, hl), oop[kk], dp, 0, 0, 0);
      }
      // lane = query, rows = keys j0 + 32 hf + 8 g + 4 hl + j
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = j0 + 32 * hf + 8 * (r >> 2) + 4 * hl + (r & 3);
        const bool vis = key >= lo && key <= hi;
        const float pr = vis ? fast_exp2(fmaf(s[r], c2, -l2)) : 0.f;
        dp[r] = pr * (dp[r] - del);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 db = acc_bop(dp, ks);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
          acc_q[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_k(sK, 32 * hf + 16 * ks, dt, lane), db,
                                                              acc_q[dt], 0, 0, 0);
      }
    }
  }
  if (!qvalid) return;
  // the routed partials of this query (every kept routed slot is block-major)
  for (int s = 0; s < (p.kind ? p.K : 0); ++s) {
    if (p.kind[qrow * p.K + s] != 2) continue;
    const int pos = p.spos[qrow * p.K + s];
    if (pos < 0) continue;
    for (int u = 0; u < a.nsub; ++u) {
      const float* pd = a.part_dq + (((int64_t)h * p.ppos + pos) * a.nsub + u) * D;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 v4 = *(const float4*)(pd + 32 * dt + 8 * g + 4 * hl);
          acc_q[dt][4 * g] += v4.x; acc_q[dt][4 * g + 1] += v4.y;
          acc_q[dt][4 * g + 2] += v4.z; acc_q[dt][4 * g + 3] += v4.w;
        }
    }
  }
  bf16* dqp = seq_base(a.dq, p.cu, b, a.dq_sb, a.dq_st) + (int64_t)h * a.dq_sh + (int64_t)tq * a.dq_st;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 w;
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (bf16)(acc_q[dt][4 * g + j] * a.scale);
      *(bf16x4*)(dqp + 32 * dt + 8 * g + 4 * hl) = w;
    }
}

// d_bias[row, slot] = sum over heads of the slot's pair partial (0 for slots that
// are not kept routed pairs).
__global__ __launch_bounds__(256) void bwd_dbias_kernel(BwdArgs a, int64_t nslots) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nslots) return;
  float s = 0.f;
  if (a.p.kind[i] == 2) {
    const int pos = a.p.spos[i];
    if (pos >= 0)
      for (int h = 0; h < a.p.H; ++h)
        for (int u = 0; u < a.nsub; ++u) s += a.part_db[((int64_t)h * a.p.ppos + pos) * a.nsub + u];
  }
  a.dbias[i] = s;
}

}  // namespace dash
