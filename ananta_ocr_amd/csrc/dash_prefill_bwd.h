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
//     32-key half, two wavefronts (one per half of the head dims), each computing
//     S = Q K^T and dP = dO V^T on the matrix cores (lane = key), P and dS in
//     registers, and its dims of dV^T += dO^T P and dK^T += Q^T dS, the transposed
//     operands read by ds_read_tr16_b64.  dK
//     and dV are complete when the work-group ends (no atomics).  For routed
//     pairs it also writes dQ^T = K^T dS^T (dS through LDS, read transposed) and
//     the row sums of dS as fp32 partials per (head, pair).  The steps are
//     software-pipelined: a step's query rows load into the other of two LDS
//     buffers while the previous step computes, their row numbers and per-query
//     values one step earlier still, and a routed step's partials are stored
//     whole rows at a time at the start of the next step;
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
  // dQ partials of the routed pairs: [H, ppos, nsub, 128] fp16, the 64 dims a lane of the
  // query-major kernel adds contiguous (dim 32 dt + 8 g + 4 h + j at 64 h + 16 dt + 4 g + j);
  // each 32-dim piece is stored as its values times 2^-e, e the binary exponent of the
  // piece's largest magnitude (so every stored value lies in (-1, 1) and its rounding
  // error is at most 2^-11 of that magnitude), and part_dqs [H, ppos, nsub, 4] holds
  // the pieces' scales 2^e
  _Float16* part_dq;
  float* part_dqs;
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

// Row swizzle of the backward kernels' stages: 16-byte chunk c of row r sits in
// slot c ^ bw_swz(r % 16), bw_swz(r) = (r % 4) << 2 | (r / 4) % 4.  A bijection of
// the 16 rows, so that the row reads (16 consecutive rows, one chunk each) fall on
// 16 distinct slots, and with (r % 4) in the top two bits, so that the transposing
// reads (4 consecutive rows, 4 chunks of one 64-byte group each) fall on the 4
// different 64-byte groups: every read covers all 64 banks once.  (Chunk c ^ (r %
// 16) puts the transposing reads of 4 rows on one 64-byte group: 4-way conflicts.)
__device__ __forceinline__ int bw_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// A operand of X^T (rows = dims 32 dt + lane % 32, k = 8 rows of a bw_swz-swizzled
// 128-dim stage in the order kbase + 8 (e / 4) + 4 (lane / 32) + e % 4), by two
// transposing reads: the row order of the B operands built from accumulators.
__device__ __forceinline__ bf16x8 tr_frag_k(const bf16* sX, int kbase, int dt, int lane) {
  const int hl = lane >> 5;
  const int row = kbase + 4 * hl + ((lane & 15) >> 2);
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int within = 4 * (lane & 1);
  const int c = dt * 4 + cq;
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(sX + row * 128 + (c ^ bw_swz(row & 15)) * 8 + within));
  const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(sX + (row + 8) * 128 + (c ^ bw_swz((row + 8) & 15)) * 8 +
                                                             within));
  bf16x8 r;
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
  for (int e = 0; e < 4; ++e) { r[e] = l4[e]; r[e + 4] = h4[e]; }
  return r;
}

// Barrier for LDS data written by ds_write: the wavefront's LDS accesses
// complete (lgkmcnt 0) and nothing else is waited for, so that its outstanding
// global loads, among them the next step's direct-to-LDS row loads, stay in
// flight (a workgroup fence would wait for those too).  The empty asm keeps the
// compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xc07f);     // lgkmcnt(0); vmcnt and expcnt not waited for
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
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

// Loads rows of a 64-row, bw_swz-swizzled stage from global memory: wavefront wv,
// lane l fills slot l % 16 of rows 16 u + 4 wv + l / 16 (u < 4) from the row
// pointer rowp(r) (chunk (l % 16) ^ bw_swz(r % 16) of it).
template <typename RowPtr>
__device__ __forceinline__ void stage_rows(bf16* sX, int wv, int lane, RowPtr rowp) {
  const int r0 = 4 * wv + (lane >> 4), slot = lane & 15;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 16 * u + r0;
    const bf16* src = rowp(r) + (slot ^ bw_swz(r0 & 15)) * 8;
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(sX + (4 * u + wv) * 4 * 128),
                                     16, 0, 0);
  }
}

// Lane byte offsets of the transposing reads of a stage (see bw_tr_lane_off): the
// reads of k-step ks (rows qbase + 16 ks ..), dim tile dt are at 4096 ks + (lo ^ 64 dt)
// and 4096 ks + (hi ^ 64 dt) of the stage (the row's swizzle is the same for every
// k-step, and the dim tile only flips address bits 6-7).
struct TrOff {
  uint32_t lo, hi;
};
__device__ __forceinline__ bf16x8 tr_frag_at(const bf16* sX, const TrOff& t, int ks, int dt) {
  const char* p = (const char*)sX + 4096 * ks;
  const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(p + (t.lo ^ (uint32_t)(dt << 6))));
  const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_short4*)(__attribute__((address_space(3))) void*)(p + (t.hi ^ (uint32_t)(dt << 6))));
  bf16x8 r;
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
  const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
  for (int e = 0; e < 4; ++e) { r[e] = l4[e]; r[e + 4] = h4[e]; }
  return r;
}

// ---------------------------------------------------------------------------
// Key-major kernel.
// ---------------------------------------------------------------------------
constexpr int kBwIT = 64;                 // keys of a stage, queries per step

// Per-query values of one step of the key-major kernel: base-2 log-sum-exp,
// delta, base-2 bias, the visible key range [lo, hi] and the pair position
// (routed steps; -1 for none).
struct KvMeta {
  float l2[kBwIT], del[kBwIT], b2[kBwIT];
  int lo[kBwIT], hi[kBwIT], pos[kBwIT];
};

// What one query slot of a step loads for its KvMeta: the row and its values,
// loaded one step before they are stored (see bwd_kv_kernel).
struct KvMetaLoad {
  int t, pos;
  bool ok;
  float lse, del, bias;
  int km;
};

// Row read of a bw_swz stage: keys krow (lane % 32 of a 32-row half), dims
// 16 kk + 8 (lane / 32) .. +7.
__device__ __forceinline__ bf16x8 bw_k_frag(const bf16* sX, int krow, int kk, int hl) {
  return *(const bf16x8*)(sX + krow * 128 + ((2 * kk + hl) ^ bw_swz(krow & 15)) * 8);
}

// Lane part of the row reads (k_frag_at) of a bw_swz stage: row n, chunk
// (2 kk + hl) ^ bw_swz(n % 16).
__device__ __forceinline__ uint32_t bw_k_lane_off(int n, int hl) {
  return (uint32_t)(n * 256) | (uint32_t)((hl << 4) ^ (bw_swz(n & 15) << 4));
}

// Lane offsets of the transposing reads (tr_frag_at) of a bw_swz stage for row base
// qbase (a multiple of 16): row qbase + 4 hl + rr (and + 8), chunk 4 dt + cq, whose
// slot is (4 dt + cq) ^ bw_swz(4 hl + rr) = 4 (dt ^ rr) + (cq ^ hl) (rows + 8:
// cq ^ (hl | 2)); the dim tile dt only flips address bits 6-7.
__device__ __forceinline__ TrOff bw_tr_lane_off(int qbase, int lane) {
  const int hl = lane >> 5, rr = (lane & 15) >> 2;
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const uint32_t in = (uint32_t)(64 * rr + 8 * (lane & 1));
  const uint32_t lo = (uint32_t)((qbase + 4 * hl + rr) * 256 + 16 * (cq ^ hl)) + in;
  const uint32_t hi = (uint32_t)((qbase + 4 * hl + rr + 8) * 256 + 16 * (cq ^ (hl | 2))) + in;
  return {lo, hi};
}

// Loads rows of a 64-row, bw_swz-swizzled stage by 8 wavefronts: wavefront wv,
// lane l fills slot l % 16 of rows 32 u + r0 (r0 = 4 wv + l / 16, u < 2) from the
// row pointer rowp(r).
template <typename RowPtr>
__device__ __forceinline__ void stage_rows8(bf16* sX, int wv, int lane, RowPtr rowp) {
  const int r0 = 4 * wv + (lane >> 4), slot = lane & 15;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int r = 32 * u + r0;
    __builtin_amdgcn_global_load_lds((const void*)(rowp(r) + (slot ^ bw_swz(r0 & 15)) * 8),
                                     (__attribute__((address_space(3))) void*)(sX + (32 * u + 4 * wv) * 128),
                                     16, 0, 0);
  }
}
// The same with the lane's two row numbers given (rw.x: row r0, rw.y: row 32 + r0);
// row numbers are >= 0 and the row stride is below 2^32 elements.
__device__ __forceinline__ void stage_rows8r(bf16* sX, int wv, int lane, const bf16* xb, int64_t x_st,
                                             int2 rw) {
  const int r0 = 4 * wv + (lane >> 4), slot = lane & 15;
  const int rr[2] = {rw.x, rw.y};
#pragma unroll
  for (int u = 0; u < 2; ++u)
    __builtin_amdgcn_global_load_lds((const void*)(xb + (uint64_t)(uint32_t)rr[u] * (uint32_t)x_st +
                                                   (slot ^ bw_swz(r0 & 15)) * 8),
                                     (__attribute__((address_space(3))) void*)(sX + (32 * u + 4 * wv) * 128),
                                     16, 0, 0);
}

// Key-major kernel, eight wavefronts: wavefront (kh, qc, dh) = (wv % 2, wv / 2 % 2,
// wv / 4) owns keys 32 kh .. + 31 of the stage, queries 32 qc .. + 31 of a step and
// head dims 64 dh .. + 63 of dK and dV, so that two wavefronts fit on a SIMD.  Per
// step both wavefronts of a (kh, qc) pair compute S, P, dP and dS (the products are
// cheap here; an exchange through LDS cost a barrier), and each adds its dims'
// share of dV^T += dO^T P and dK^T += Q^T dS.  Routed steps: dQ^T = K^T dS^T
// for the step's 64 queries x 128 dims, one 32 x 32 tile per wavefront (dims
// 32 (2 dh + kh) ..), and the bias-gradient row sums.
// Software pipeline over the steps: step s computes on the query rows in buffer
// s % 2 with the per-query values in sM[s % 2]; meanwhile the rows of step s + 1
// load into the other buffer (row numbers from sRow[(s + 1) % 2]), and wavefront 0
// loads the values of step s + 1 and the pair ids of step s + 2, which it stores
// after the products (sM[(s + 1) % 2], sRow[s % 2]).  A routed step's dQ^T partials
// wait in LDS and are stored at the start of the next step, so that the wait that
// ends a step does not wait for stores just issued.  One wait and one barrier end
// each step.
__global__ __launch_bounds__(512, 1) void bwd_kv_kernel(BwdArgs a) {
  constexpr int D = 128;
  __shared__ __attribute__((aligned(16))) bf16 sK[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sQ0[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sQ1[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sO0[kBwIT * D];   // dO rows
  __shared__ __attribute__((aligned(16))) bf16 sO1[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sDS[2][kBwIT][36];  // dS [qc][key][query]
  __shared__ __attribute__((aligned(16))) KvMeta sM[2];
  // row numbers of a step for the loads: query slot q at [q % 32][q / 32]
  __shared__ __attribute__((aligned(16))) int sRow[2][32][2];
  __shared__ float sDb[2][kBwIT];
  // per wavefront 4 KB: the dQ^T staging of a routed step until the start of the next
  __shared__ __attribute__((aligned(16))) float sX[8][1024];

  const PrefillArgs& p = a.p;
  // Stages in order per (sequence, head) stream, each stream's stages on one XCD
  // (stream_stage_item): an early stage takes the routed pairs of every later query
  // (block 0 of 27,300 tokens ~6,000 of them, the last blocks almost none), so the
  // heavy stages start first and the light ones fill the end (numbered per (head,
  // stage) and contiguous per XCD instead, the heavy stages of some heads started
  // last: 2.61 -> 2.04 ms), while neighbouring stages, whose window bands overlap,
  // share one L2.
  int bh, stage;
  if (!stream_stage_item((int)blockIdx.x, p.B * p.H, a.nstage, bh, stage)) return;
  const int h = bh % p.H, b = bh / p.H;
  const int len = seq_len(p, b);
  const int j0 = stage * kBwIT;
  if (j0 / p.bs * p.bs >= len) return;
  const int sub = (j0 % p.bs) / kBwIT;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int kh = wv & 1, qc = (wv >> 1) & 1, dh = wv >> 2, hl = lane >> 5, n = lane & 31;
  const int64_t r0 = row0(p, b);
  const float c2 = a.scale * 1.4426950408889634f;
  const float log2e = 1.4426950408889634f;

  const bf16* kb = seq_base(p.k, p.cu, b, p.k_sb, p.k_st) + (int64_t)h * p.k_sh;
  const bf16* vb = seq_base(p.v, p.cu, b, p.v_sb, p.v_st) + (int64_t)h * p.v_sh;
  const bf16* qb = seq_base(p.q, p.cu, b, p.q_sb, p.q_st) + (int64_t)h * p.q_sh;
  const bf16* ob = seq_base(a.dout, p.cu, b, a.do_sb, a.do_st) + (int64_t)h * a.do_sh;
  stage_rows8(sK, wv, lane, [&](int r) { return kb + (int64_t)min(j0 + r, len - 1) * p.k_st; });
  stage_rows8(sV, wv, lane, [&](int r) { return vb + (int64_t)min(j0 + r, len - 1) * p.v_st; });

  const int LW = p.lw, bs = p.bs;
  const int t_end = min(j0 + kBwIT - 1 + LW - 1, len - 1);
  const int n_win = t_end >= j0 ? (t_end - j0) / kBwIT + 1 : 0;
  const int c_first = j0 / bs;
  const int c_last = p.blk_count ? min(j0 + kBwIT - 1, len - 1) / bs : c_first - 1;  // <= c_first + 1
  int np0 = 0, np1 = 0, ch00 = 0, ch01 = 0;
  if (c_last >= c_first) {
    np0 = p.blk_count[(int64_t)b * p.nblk_cap + c_first];
    ch00 = p.blk_chunk[(int64_t)b * p.nblk_cap + c_first];
  }
  if (c_last > c_first) {
    np1 = p.blk_count[(int64_t)b * p.nblk_cap + c_first + 1];
    ch01 = p.blk_chunk[(int64_t)b * p.nblk_cap + c_first + 1];
  }
  const int rs0 = (np0 + kBwIT - 1) / kBwIT;
  const int n_steps = n_win + rs0 + (np1 + kBwIT - 1) / kBwIT;

  auto pair_of = [&](int u) -> int {
    const int v = u - n_win;
    const bool second = v >= rs0;
    const int np = second ? np1 : np0, ch0 = second ? ch01 : ch00;
    const int i = (second ? v - rs0 : v) * kBwIT + tid;
    if (i >= np) return -1;
    const int chunk = ch0 + i / kPfCH;
    if (chunk >= p.chunk_cap) return -1;
    return p.chunk_rec[((int64_t)b * p.chunk_cap + chunk) * kRec + kRecHead + i % kPfCH];
  };
  auto row_of = [&](int u, int pid) -> int {
    if (u < n_win) return min(j0 + u * kBwIT + tid, len - 1);
    return pid >= 0 ? min(pid / p.K, len - 1) : 0;
  };
  auto meta_load = [&](int u, int pid) -> KvMetaLoad {
    KvMetaLoad m;
    m.t = u < n_win ? j0 + u * kBwIT + tid : row_of(u, pid);
    m.ok = u < n_win ? m.t < len : pid >= 0;
    const int64_t row = r0 + min(m.t, len - 1);
    m.km = p.kmin ? p.kmin[row] : 0;
    m.lse = a.lse[row * a.lse_row + (int64_t)h * a.lse_sh];
    m.del = a.delta[row * p.H + h];
    m.pos = -1;
    m.bias = 0.f;
    if (u >= n_win && pid >= 0) {
      m.pos = p.spos[row * p.K + pid % p.K];
      m.bias = p.bias[row * p.K + pid % p.K];
    }
    return m;
  };
  auto meta_store = [&](int u, const KvMetaLoad& m, KvMeta& M) {
    int lo, hi;
    if (u < n_win) {
      lo = m.ok ? max(max(m.t - LW + 1, m.km), 0) : 1;
      hi = m.ok ? m.t : 0;
    } else {
      const int c = u - n_win < rs0 ? c_first : c_first + 1;
      lo = m.ok ? max(m.km, c * bs) : 1;
      hi = m.ok && m.pos >= 0 ? min(min(m.t - LW, (c + 1) * bs - 1), len - 1) : lo - 1;
    }
    M.l2[tid] = m.lse * log2e;
    M.del[tid] = m.del;
    M.b2[tid] = m.bias * log2e;
    M.lo[tid] = lo;
    M.hi[tid] = hi;
    M.pos[tid] = m.ok ? m.pos : -1;
  };

  floatx16 acc_dk[2], acc_dv[2];           // dims 64 dh + 32 t ..
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc_dk[t][r] = 0.f; acc_dv[t][r] = 0.f; }

  const uint32_t kl0 = bw_k_lane_off(n, hl);
  const TrOff tq0 = bw_tr_lane_off(32 * qc, lane), tk0 = bw_tr_lane_off(0, lane);
  const int key = j0 + 32 * kh + n;
  const int kst = 32 * kh, qst = 32 * qc;
  const int dtq = 2 * dh + kh;             // this wavefront's dQ dim tile
  float* const xs = sX[wv];                // own staging area

  int pid_next = -1;
  if (n_steps > 0) {
    if (wv == 0) {
      const int pid0 = n_win > 0 ? -1 : pair_of(0);
      pid_next = n_steps > 1 && n_win <= 1 ? pair_of(1) : -1;
      meta_store(0, meta_load(0, pid0), sM[0]);
      sRow[0][tid & 31][tid >> 5] = row_of(0, pid0);
      if (n_steps > 1) sRow[1][tid & 31][tid >> 5] = row_of(1, pid_next);
    }
    __syncthreads();
    const int2 rw = *(const int2*)&sRow[0][4 * wv + (lane >> 4)][0];
    stage_rows8r(sQ0, wv, lane, qb, p.q_st, rw);
    stage_rows8r(sO0, wv, lane, ob, a.do_st, rw);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // dQ^T partials of a routed step wait in the wavefront's area (query row r at 32
  // halves, 8-byte chunk c in slot c ^ (r % 8), the row's scale at float 512 + r) and
  // are stored at the start of the next step, 8 lanes per 64-byte row piece.
  bool pend = false;
  int64_t pend_pi = -1;
  float pend_db = 0.f;
  auto store_pending = [&](int par) {
    if (pend) {
      const int c = lane & 7;
      const _Float16* const xh = (const _Float16*)xs;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + (lane >> 3);
        const int pos = sM[par].pos[qst + r];
        const f16x4 v = *(const f16x4*)(xh + r * 32 + ((c ^ (r & 7)) << 2));
        if (pos >= 0) {
          const int64_t pi = ((int64_t)h * p.ppos + pos) * a.nsub + sub;
          *(f16x4*)(a.part_dq + pi * D + (c & 1) * 64 + 16 * dtq + 4 * (c >> 1)) = v;
          if (c == 0) a.part_dqs[pi * 4 + dtq] = xs[512 + r];
        }
      }
      if (kh == 0 && dh == 0 && hl == 0 && pend_pi >= 0) a.part_db[pend_pi] = pend_db;
    }
    pend = false;
  };

  auto step = [&](int s, auto par_tag) {
    constexpr int P = decltype(par_tag)::value;
    const bf16* const sQ = P == 0 ? sQ0 : sQ1;
    const bf16* const sO = P == 0 ? sO0 : sO1;
    bf16* const sQn = P == 0 ? sQ1 : sQ0;
    bf16* const sOn = P == 0 ? sO1 : sO0;
    const KvMeta& M = sM[P];
    const bool routed = s >= n_win;
    store_pending(P ^ 1);
    if (s + 1 < n_steps) {
      const int2 rw = *(const int2*)&sRow[P ^ 1][4 * wv + (lane >> 4)][0];
      stage_rows8r(sQn, wv, lane, qb, p.q_st, rw);
      stage_rows8r(sOn, wv, lane, ob, a.do_st, rw);
    }
    uint32_t kl = kl0;
    TrOff tq = tq0, tk = tk0;
    asm volatile("" : "+v"(kl), "+v"(tq.lo), "+v"(tq.hi), "+v"(tk.lo), "+v"(tk.hi));
    KvMetaLoad ml = {};
    int pid2 = -1;
    if (wv == 0) {
      if (s + 1 < n_steps) ml = meta_load(s + 1, pid_next);
      if (s + 2 < n_steps && s + 2 >= n_win) pid2 = pair_of(s + 2);
    }

    // S and dP of the (kh, qc) tile, lane = key, rows = queries 8 g + 4 hl + j of the
    // chunk.  Both wavefronts of a dim pair compute both (the matrix cores have room;
    // no exchange and no barrier between them).  The next k-step's four operand reads
    // are issued before the current k-step's two products, fenced by scheduling
    // barriers (left to itself the scheduler reads just before each product).
    floatx16 xs_, xd_;
#pragma unroll
    for (int r = 0; r < 16; ++r) { xs_[r] = 0.f; xd_[r] = 0.f; }
    {
      auto rd = [&](int kk, bf16x8 (&f)[4]) {
        f[0] = k_frag_at(sQ, kl, qc, kk);
        f[1] = k_frag_at(sK, kl, kh, kk);
        f[2] = k_frag_at(sO, kl, qc, kk);
        f[3] = k_frag_at(sV, kl, kh, kk);
      };
      bf16x8 f0[4], f1[4];
      rd(0, f0);
#pragma unroll
      for (int kk = 0; kk < D / 16; kk += 2) {
        rd(kk + 1, f1);
        __builtin_amdgcn_sched_barrier(0);
        xs_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f0[0], f0[1], xs_, 0, 0, 0);
        xd_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f0[2], f0[3], xd_, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        if (kk + 2 < D / 16) rd(kk + 2, f0);
        __builtin_amdgcn_sched_barrier(0);
        xs_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f1[0], f1[1], xs_, 0, 0, 0);
        xd_ = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f1[2], f1[3], xd_, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    float pr[16], ds[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int q0 = qst + 8 * g + 4 * hl;
      const float4 l2 = *(const float4*)&M.l2[q0];
      const float4 b2 = *(const float4*)&M.b2[q0];
      const float4 de = *(const float4*)&M.del[q0];
      const int4 lo = *(const int4*)&M.lo[q0];
      const int4 hi = *(const int4*)&M.hi[q0];
      const float l2a[4] = {l2.x, l2.y, l2.z, l2.w};
      const float b2a[4] = {b2.x, b2.y, b2.z, b2.w};
      const float dea[4] = {de.x, de.y, de.z, de.w};
      const int loa[4] = {lo.x, lo.y, lo.z, lo.w};
      const int hia[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * g + j;
        const float e = fast_exp2(fmaf(xs_[r], c2, b2a[j] - l2a[j]));
        const bool vis = (key >= loa[j]) & (key <= hia[j]);
        pr[r] = vis ? e : 0.f;
        ds[r] = pr[r] * (xd_[r] - dea[j]);
      }
    }
    // this wavefront's dims of dV^T += dO^T P and dK^T += Q^T dS (operand reads
    // issued together, as above)
    floatx16 pf, df;
#pragma unroll
    for (int r = 0; r < 16; ++r) { pf[r] = pr[r]; df[r] = ds[r]; }
    {
      bf16x8 fo[2][2], fq[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          fo[ks][t] = tr_frag_at(sO, tq, ks, 2 * dh + t);
          fq[ks][t] = tr_frag_at(sQ, tq, ks, 2 * dh + t);
        }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8 pb = acc_bop(pf, ks);
        const bf16x8 db = acc_bop(df, ks);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          acc_dv[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fo[ks][t], pb, acc_dv[t], 0, 0, 0);
          acc_dk[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fq[ks][t], db, acc_dk[t], 0, 0, 0);
        }
      }
    }
    if (routed) {
      if (dh == 0) {
        // dS through LDS (sDS[qc][key][query]) and its row sums over this
        // wavefront's 32 keys
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 w;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[j] = (bf16)ds[4 * g + j];
          *(bf16x4*)&sDS[qc][kst + n][8 * g + 4 * hl] = w;
        }
        // the row sums in fp32: ds through the wavefront's staging area (free between the
        // previous step's partial stores and this step's staging) as [key][query], in the
        // staging's swizzle, then lanes q and q + 32 add 16 keys each (16 shuffle-sums of
        // 32 lanes cost more)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(float4*)(xs + n * 32 + (((2 * g + hl) ^ (n & 7)) << 2)) =
              make_float4(ds[4 * g], ds[4 * g + 1], ds[4 * g + 2], ds[4 * g + 3]);
        wave_lds_sync();
        {
          const int q = lane & 31;
          float sum = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = 16 * hl + i;
            sum += xs[key * 32 + (((q >> 2) ^ (key & 7)) << 2) + (q & 3)];
          }
          sum += __shfl_xor(sum, 32, kWave);
          if (hl == 0) sDb[kh][qst + q] = sum;
        }
        wave_lds_sync();
      }
      lds_barrier();
      // dQ^T tile dtq = K^T dS^T over the stage's 64 keys for the chunk's 32 queries
      floatx16 acc_q;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_q[r] = 0.f;
      const int tg = lane >> 4;
      const uint32_t dsa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) bf16*)
          &sDS[qc][4 * (tg >> 1) + ((lane & 15) >> 2)][16 * (tg & 1) + 4 * (lane & 3)];
      bf16x4 dst[8];
      asm volatile(
          "ds_read_b64_tr_b16 %0, %8\n"
          "ds_read_b64_tr_b16 %1, %8 offset:576\n"
          "ds_read_b64_tr_b16 %2, %8 offset:1152\n"
          "ds_read_b64_tr_b16 %3, %8 offset:1728\n"
          "ds_read_b64_tr_b16 %4, %8 offset:2304\n"
          "ds_read_b64_tr_b16 %5, %8 offset:2880\n"
          "ds_read_b64_tr_b16 %6, %8 offset:3456\n"
          "ds_read_b64_tr_b16 %7, %8 offset:4032\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(dst[0]), "=&v"(dst[1]), "=&v"(dst[2]), "=&v"(dst[3]), "=&v"(dst[4]), "=&v"(dst[5]),
            "=&v"(dst[6]), "=&v"(dst[7])
          : "v"(dsa)
          : "memory");
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8 dsb;
#pragma unroll
        for (int e = 0; e < 4; ++e) { dsb[e] = dst[2 * ks][e]; dsb[e + 4] = dst[2 * ks + 1][e]; }
        acc_q = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_at(sK, tk, ks, dtq), dsb, acc_q, 0, 0, 0);
      }
      // staged for the next step: dims 32 dtq + 8 g + 4 hl + j of query n, in fp16 after
      // scaling by 2^-e (lanes n and n + 32 hold the two halves of the piece); the
      // scale 2^e at xs[512 + n]
      float mx = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fabsf(acc_q[r]));
      mx = xor32_max(mx);
      const int ex = min(__builtin_amdgcn_frexp_expf(mx), 127);
      _Float16* const xh = (_Float16*)xs;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 hv;
#pragma unroll
        for (int j = 0; j < 4; ++j) hv[j] = (_Float16)ldexpf(acc_q[4 * g + j], -ex);
        *(f16x4*)(xh + n * 32 + (((2 * g + hl) ^ (n & 7)) << 2)) = hv;
      }
      if (hl == 0) xs[512 + n] = ldexpf(1.f, ex);
      const int pos = M.pos[qst + n];
      pend_pi = pos >= 0 ? ((int64_t)h * p.ppos + pos) * a.nsub + sub : -1;
      pend_db = sDb[0][qst + n] + sDb[1][qst + n];
      pend = true;
    }

    if (wv == 0) {
      if (s + 1 < n_steps) meta_store(s + 1, ml, sM[P ^ 1]);
      if (s + 2 < n_steps) sRow[P][tid & 31][tid >> 5] = row_of(s + 2, pid2);
      pid_next = pid2;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  int s = 0;
  for (; s + 1 < n_steps; s += 2) {
    step(s, std::integral_constant<int, 0>{});
    step(s + 1, std::integral_constant<int, 1>{});
  }
  if (s < n_steps) step(s, std::integral_constant<int, 0>{});
  store_pending((n_steps - 1) & 1);

  // ---- dK and dV: the two query chunks' sums (16 KB per (kh, dh) pair) ----
  const int ri = kh + 2 * dh;
  float* const red = (float*)(ri == 0 ? sQ0 : ri == 1 ? sQ1 : ri == 2 ? sO0 : sO1);
  if (qc == 1) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        red[(t * 16 + r) * kWave + lane] = acc_dk[t][r];
        red[((2 + t) * 16 + r) * kWave + lane] = acc_dv[t][r];
      }
  }
  __syncthreads();
  if (qc == 0 && key < len) {
    bf16* dkp = seq_base(a.dk, p.cu, b, a.dk_sb, a.dk_st) + (int64_t)h * a.dk_sh + (int64_t)key * a.dk_st;
    bf16* dvp = seq_base(a.dv, p.cu, b, a.dv_sb, a.dv_st) + (int64_t)h * a.dv_sh + (int64_t)key * a.dv_st;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 wk, wvv;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * g + j;
          wk[j] = (bf16)((acc_dk[t][r] + red[(t * 16 + r) * kWave + lane]) * a.scale);
          wvv[j] = (bf16)(acc_dv[t][r] + red[((2 + t) * 16 + r) * kWave + lane]);
        }
        *(bf16x4*)(dkp + 64 * dh + 32 * t + 8 * g + 4 * hl) = wk;
        *(bf16x4*)(dvp + 64 * dh + 32 * t + 8 * g + 4 * hl) = wvv;
      }
  }
}

// ---------------------------------------------------------------------------
// Query-major kernel: dQ over the window band plus the routed partials.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void bwd_q_kernel(BwdArgs a) {
  constexpr int D = 128;
  // double-buffered window stages (distinct arrays, so that reads of one never wait
  // for the loads into the other)
  __shared__ __attribute__((aligned(16))) bf16 sK0[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV0[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sK1[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV1[kBwIT * D];
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

  // window keys of the tile: [max(t0 - LW + 1, 0), min(t0 + 127, len - 1)] in 64-key
  // items; item i + 1 loads into the other stage while item i computes
  const int k_lo = max(t0 - p.lw + 1, 0) / kBwIT * kBwIT;
  const int k_hi = min(t0 + kPfTQ - 1, len - 1);
  const int nit = k_hi >= k_lo ? (k_hi - k_lo) / kBwIT + 1 : 0;
  auto stage = [&](bf16* sKx, bf16* sVx, int j0) {
    stage_rows(sKx, wv, lane, [&](int r) { return kb + (int64_t)min(j0 + r, len - 1) * p.k_st; });
    stage_rows(sVx, wv, lane, [&](int r) { return vb + (int64_t)min(j0 + r, len - 1) * p.v_st; });
  };
  if (nit > 0) stage(sK0, sV0, k_lo);
  auto item = [&](int it, auto par_tag) {
    constexpr int P = decltype(par_tag)::value;
    const bf16* const sK = P == 0 ? sK0 : sK1;
    const bf16* const sV = P == 0 ? sV0 : sV1;
    const int j0 = k_lo + it * kBwIT;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();                       // item it landed; item it - 1 is done
    if (it + 1 < nit) stage(P == 0 ? sK1 : sK0, P == 0 ? sV1 : sV0, j0 + kBwIT);
    const bool need = __any(qvalid && lo <= j0 + kBwIT - 1 && hi >= j0);
    if (!need) return;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      floatx16 s, dp;
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw_k_frag(sK, 32 * hf + n, kk, hl), qop[kk], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw_k_frag(sV, 32 * hf + n, kk, hl), oop[kk], dp, 0, 0, 0);
      }
      // lane = query, rows = keys j0 + 32 hf + 8 g + 4 hl + j; the visibility test
      // only where some query of the wavefront does not see all 32 keys
      const int k0 = j0 + 32 * hf;
      if (__all(!qvalid || (lo <= k0 && hi >= k0 + 31))) {
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] = fast_exp2(fmaf(s[r], c2, -l2)) * (dp[r] - del);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + 8 * (r >> 2) + 4 * hl + (r & 3);
          const bool vis = key >= lo && key <= hi;
          const float pr = vis ? fast_exp2(fmaf(s[r], c2, -l2)) : 0.f;
          dp[r] = pr * (dp[r] - del);
        }
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
  };
  for (int it = 0; it < nit; it += 2) {
    item(it, std::integral_constant<int, 0>{});
    if (it + 1 < nit) item(it + 1, std::integral_constant<int, 1>{});
  }
  if (!qvalid) return;
  // The routed partials of this query (every kept routed slot is block-major), in
  // slot order and, within a slot, sub-block order.  Slots in groups of 16: the
  // group's kinds and pair positions are loaded before any is used, then the
  // partial rows two at a time (both rows' loads in flight before either is added).
  for (int g0 = 0; p.kind && g0 < p.K; g0 += kPfMaxK) {
    const int ng = min(kPfMaxK, p.K - g0);
    const int64_t q0 = qrow * p.K + g0;
    int32_t pos[kPfMaxK];
    uint32_t live = 0;
    if (p.slots_vec) {                     // ng is a multiple of 4
      uint32_t kw[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bool in = 4 * q < ng;
        kw[q] = in ? *(const uint32_t*)(p.kind + q0 + 4 * q) : 0u;
        const int4 pv = in ? *(const int4*)(p.spos + q0 + 4 * q) : make_int4(-1, -1, -1, -1);
        pos[4 * q] = pv.x; pos[4 * q + 1] = pv.y; pos[4 * q + 2] = pv.z; pos[4 * q + 3] = pv.w;
      }
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s)
        if (((kw[s >> 2] >> (8 * (s & 3))) & 0xffu) == 2 && pos[s] >= 0) live |= 1u << s;
    } else {
      uint8_t kd[kPfMaxK];
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s) {
        kd[s] = s < ng ? p.kind[q0 + s] : 0;
        pos[s] = s < ng ? p.spos[q0 + s] : -1;
      }
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s)
        if (kd[s] == 2 && pos[s] >= 0) live |= 1u << s;
    }
    if (!__any(live != 0u)) continue;
    const int ne = ng * a.nsub;            // (slot, sub-block) rows of the group
    for (int e0 = 0; e0 < ne; e0 += 2) {
      f16x4 buf[2][16];
      float4 sc[2];                        // the scales of the row's four 32-dim pieces
      bool in[2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int e = e0 + q, s = e / a.nsub, u = e - s * a.nsub;
        in[q] = e < ne && ((live >> s) & 1u);
        if (in[q]) {
          const int64_t pr = ((int64_t)h * p.ppos + pos[s]) * a.nsub + u;
          const _Float16* pd = a.part_dq + pr * D + 64 * hl;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const f16x8 w = *(const f16x8*)(pd + 8 * k);
            buf[q][2 * k] = f16x4{w[0], w[1], w[2], w[3]};
            buf[q][2 * k + 1] = f16x4{w[4], w[5], w[6], w[7]};
          }
          sc[q] = *(const float4*)(a.part_dqs + pr * 4);
        }
      }
#pragma unroll
      for (int q = 0; q < 2; ++q)
        if (in[q]) {
          const float sca[4] = {sc[q].x, sc[q].y, sc[q].z, sc[q].w};
#pragma unroll
          for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f16x4 v4 = buf[q][4 * dt + g];
#pragma unroll
              for (int j = 0; j < 4; ++j) acc_q[dt][4 * g + j] = fmaf((float)v4[j], sca[dt], acc_q[dt][4 * g + j]);
            }
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
