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

// Sum over the 32 lanes of a half-wavefront (lanes 0-31 and 32-63 separately),
// every lane of the half gets it: rotations by 8 and 4 and the quad exchanges
// within each 16-lane row (DPP), then the other row of the half (permlane16 swap).
__device__ __forceinline__ float half32_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4e, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xb1, 0xf, 0xf, false));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
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

// Loads the query rows of a 64-row step into a k_slot-swizzled stage: wavefront
// wv, lane l fills slot l % 16 of rows 16 u + r0 (r0 = 4 wv + l / 16, u < 4) from
// the row numbers rw (component u for row 16 u + r0) -- stage_rows with the four row
// numbers of a lane read at once.  Row numbers are >= 0 and the row stride is below
// 2^32 elements (one 32 x 32 -> 64-bit multiply per row).
__device__ __forceinline__ void stage_rows4(bf16* sX, int wv, int lane, const bf16* xb, int64_t x_st,
                                            int4 rw) {
  const int r0 = 4 * wv + (lane >> 4), slot = lane & 15;
  const int rr[4] = {rw.x, rw.y, rw.z, rw.w};
#pragma unroll
  for (int u = 0; u < 4; ++u)
    __builtin_amdgcn_global_load_lds((const void*)(xb + (uint64_t)(uint32_t)rr[u] * (uint32_t)x_st +
                                                   (slot ^ (r0 & 15)) * 8),
                                     (__attribute__((address_space(3))) void*)(sX + (4 * u + wv) * 4 * 128),
                                     16, 0, 0);
}

// Lane byte offsets of tr_frag_k's reads for row base qbase (a multiple of 16): the
// reads of k-step ks (rows qbase + 16 ks ..), dim tile dt are at 4096 ks + (lo ^ 64 dt)
// and 4096 ks + (hi ^ 64 dt) of the stage (the row's swizzle is the same for every
// k-step, and the dim tile only flips address bits 6-7).
struct TrOff {
  uint32_t lo, hi;
};
__device__ __forceinline__ TrOff tr_lane_off(int qbase, int lane) {
  const int hl = lane >> 5, rr = (lane & 15) >> 2;
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const uint32_t lo = (uint32_t)((qbase + 4 * hl + rr) * 256 + 64 * hl + 16 * (cq ^ rr) + 8 * (lane & 1));
  return {lo, (lo ^ 128u) + 2048u};
}
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

__global__ __launch_bounds__(256, 1) void bwd_kv_kernel(BwdArgs a) {
  constexpr int D = 128;
  // The stage's K and V, and two buffers of query rows (Q and dO), each a
  // separately named array so that the reads of one never wait for the loads into
  // another; the end of the kernel reuses the four query-row buffers to add the
  // two query groups' dK and dV.
  __shared__ __attribute__((aligned(16))) bf16 sK[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sQ0[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sQ1[kBwIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sO0[kBwIT * D];   // dO rows
  __shared__ __attribute__((aligned(16))) bf16 sO1[kBwIT * D];
  // dS [key][query] per query group, rows of 32 queries padded to 72 bytes
  __shared__ __attribute__((aligned(16))) bf16 sDS[2][kBwIT][36];
  __shared__ __attribute__((aligned(16))) KvMeta sM[2];
  // row numbers of a step for the loads: query slot q at [q % 16][q / 16], so that
  // a lane reads the four rows it loads at once
  __shared__ __attribute__((aligned(16))) int sRow[2][16][4];
  __shared__ float sDb[2][kBwIT];
  __shared__ __attribute__((aligned(16))) float sSt[4][32 * 64];   // dQ^T staging per wavefront

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

  // The steps: the window band (queries j0 + 64 w .. + 63 up to t_end, every
  // query whose window reaches the stage), then the routed pairs of the stage's
  // blocks (one, or two for 32-key blocks), 64 at a time.
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

  // Query slot tid (< 64) of step u.  Routed steps: the pair id from the chunk
  // records (-1: no pair), loaded first; then the row's values.
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

  floatx16 acc_dk[4], acc_dv[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc_dk[dt][r] = 0.f; acc_dv[dt][r] = 0.f; }

  const uint32_t kl0 = k_lane_off(n, hl);  // k_frag_at offsets (rows 32 qc + n, 32 kh + n)
  const TrOff tq0 = tr_lane_off(32 * qc, lane), tk0 = tr_lane_off(0, lane);
  const int key = j0 + 32 * kh + n;        // this lane's key
  const int kst = 32 * kh;                 // this wavefront's keys in the stage
  const int qst = 32 * qc;                 // this wavefront's queries in the step

  // Software pipeline over the steps.  Step s computes on the query rows in
  // buffer s % 2 with the values in sM[s % 2]; meanwhile it loads the rows of step
  // s + 1 into the other buffer (their row numbers are in sRow[(s + 1) % 2]), and
  // wavefront 0 loads the values of step s + 1 and the pair ids of step s + 2,
  // which it stores after the products (sM[(s + 1) % 2], sRow[s % 2]).  One wait
  // and one barrier end each step.
  int pid_next = -1;                       // pair id of step s + 1 (query slot tid)
  if (n_steps > 0) {
    if (wv == 0) {
      const int pid0 = n_win > 0 ? -1 : pair_of(0);
      pid_next = n_steps > 1 && n_win <= 1 ? pair_of(1) : -1;
      meta_store(0, meta_load(0, pid0), sM[0]);
      sRow[0][tid & 15][tid >> 4] = row_of(0, pid0);
      if (n_steps > 1) sRow[1][tid & 15][tid >> 4] = row_of(1, pid_next);
    }
    __syncthreads();
    const int4 rw = *(const int4*)&sRow[0][4 * wv + (lane >> 4)][0];
    stage_rows4(sQ0, wv, lane, qb, p.q_st, rw);
    stage_rows4(sO0, wv, lane, ob, a.do_st, rw);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // dQ^T and bias-gradient partials of a routed step, stored at the start of the
  // next step, so that the wait that ends a step does not wait for stores just
  // issued.  The wavefront's dQ^T tiles (its 32 queries x dims 64 kh .. + 63) wait
  // in its LDS staging area, query row r at 64 floats with 16-byte chunk c in slot
  // c ^ (r % 16); the store writes each pair's 256 bytes whole (16 lanes per row).
  bool pend = false;
  int64_t pend_pi = -1;                    // bias-gradient partial of query column n
  float pend_db = 0.f;
  auto store_pending = [&](int par) {
    if (pend) {
      const int rb = 8 * (lane >> 4), c = lane & 15;   // rows rb .. rb + 7, chunk c
      const int4 pa = *(const int4*)&sM[par].pos[qst + rb];
      const int4 pb = *(const int4*)&sM[par].pos[qst + rb + 4];
      const int pos8[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
      const float* st = sSt[wv];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = rb + i;
        const float4 v = *(const float4*)(st + r * 64 + ((c ^ (r & 15)) << 2));
        if (pos8[i] >= 0) {
          const int64_t pi = ((int64_t)h * p.ppos + pos8[i]) * a.nsub + sub;
          *(float4*)(a.part_dq + pi * D + 64 * kh + 4 * c) = v;
        }
      }
      if (kh == 0 && hl == 0 && pend_pi >= 0) a.part_db[pend_pi] = pend_db;
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
      const int4 rw = *(const int4*)&sRow[P ^ 1][4 * wv + (lane >> 4)][0];
      stage_rows4(sQn, wv, lane, qb, p.q_st, rw);
      stage_rows4(sOn, wv, lane, ob, a.do_st, rw);
    }
    // Lane offsets pass through an empty asm each step, so that the compiler
    // derives the per-read LDS addresses here instead of keeping them all live.
    uint32_t kl = kl0;
    TrOff tq = tq0, tk = tk0;
    asm volatile("" : "+v"(kl), "+v"(tq.lo), "+v"(tq.hi), "+v"(tk.lo), "+v"(tk.hi));
    KvMetaLoad ml = {};
    int pid2 = -1;
    if (wv == 0) {
      if (s + 1 < n_steps) ml = meta_load(s + 1, pid_next);
      if (s + 2 < n_steps && s + 2 >= n_win) pid2 = pair_of(s + 2);
    }

    floatx16 sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { sc[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag_at(sQ, kl, qc, kk), k_frag_at(sK, kl, kh, kk),
                                                   sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag_at(sO, kl, qc, kk), k_frag_at(sV, kl, kh, kk),
                                                   dp, 0, 0, 0);
    }
    // operand reads two k-steps ahead of the products
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int kk = 0; kk < D / 16 - 2; ++kk) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    // P and dS, lane = key, rows = queries 8 g + 4 hl + j of this wavefront's chunk
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int q0 = qst + 8 * g + 4 * hl;
      const float4 l2 = *(const float4*)&M.l2[q0];
      const float4 de = *(const float4*)&M.del[q0];
      const float4 b2 = *(const float4*)&M.b2[q0];
      const int4 lo = *(const int4*)&M.lo[q0];
      const int4 hi = *(const int4*)&M.hi[q0];
      const float l2a[4] = {l2.x, l2.y, l2.z, l2.w};
      const float dea[4] = {de.x, de.y, de.z, de.w};
      const float b2a[4] = {b2.x, b2.y, b2.z, b2.w};
      const int loa[4] = {lo.x, lo.y, lo.z, lo.w};
      const int hia[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * g + j;
        // branch-free, so that the products and the softmax stay one scheduling region
        const float e = fast_exp2(fmaf(sc[r], c2, b2a[j] - l2a[j]));
        const bool vis = (key >= loa[j]) & (key <= hia[j]);
        const float pr = vis ? e : 0.f;
        sc[r] = pr;                                  // sc now holds P
        dp[r] = pr * (dp[r] - dea[j]);               // dp now holds dS
      }
    }
    // dV^T += dO^T P and dK^T += Q^T dS over this wavefront's 32 queries
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pb = acc_bop(sc, ks);
      const bf16x8 db = acc_bop(dp, ks);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        acc_dv[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_at(sO, tq, ks, dt), pb, acc_dv[dt],
                                                             0, 0, 0);
        acc_dk[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_at(sQ, tq, ks, dt), db, acc_dk[dt],
                                                             0, 0, 0);
      }
    }
    // operand reads four products ahead
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    if (routed) {
      // dS through LDS: sDS[qc][key of the stage][query], the lane's 4 queries
      // 8 g + 4 hl .. + 3 of its key in one 8-byte write
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = (bf16)dp[4 * g + j];
        *(bf16x4*)&sDS[qc][kst + n][8 * g + 4 * hl] = w;
      }
      // row sums of dS over this wavefront's 32 keys (fp32), one per query row
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] = half32_sum(dp[r]);
      if (n == 0) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int j = 0; j < 4; ++j) sDb[kh][qst + 8 * g + 4 * hl + j] = dp[4 * g + j];
      }
      lds_barrier();
      // dQ^T = K^T dS^T over the 64 keys: wavefront kh takes dims 64 kh .. 64 kh + 63
      floatx16 acc_q[2];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_q[u][r] = 0.f;
      // B operand of dS^T (query n, keys 16 ks + 4 hl + e and + 8) by transposing
      // reads: in each 16-lane group (queries 16 (g % 2) .., half g / 2) lane 4 j + m
      // reads keys row kb + j, queries 4 m .. + 3 of the group.  The reads are one asm
      // block with its own LDS wait: issued by the builtin they would also wait for
      // the next step's row loads (vmcnt), which are in flight.
      const int tg = lane >> 4;
      const uint32_t dsa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) bf16*)
          &sDS[qc][4 * (tg >> 1) + ((lane & 15) >> 2)][16 * (tg & 1) + 4 * (lane & 3)];
      bf16x4 dst[8];                       // [2 ks + half]: keys 16 ks + 8 half + 4 hl ..
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
#pragma unroll
        for (int u = 0; u < 2; ++u)
          acc_q[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag_at(sK, tk, ks, 2 * kh + u), dsb,
                                                             acc_q[u], 0, 0, 0);
      }
      // the partials of the pair of query column n, stored at the start of the next
      // step (see store_pending): dims 64 kh + 32 u + 8 g + 4 hl + j
      float* st = sSt[wv];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          *(float4*)(st + n * 64 + (((8 * u + 2 * g + hl) ^ (n & 15)) << 2)) =
              make_float4(acc_q[u][4 * g], acc_q[u][4 * g + 1], acc_q[u][4 * g + 2], acc_q[u][4 * g + 3]);
      const int pos = M.pos[qst + n];
      pend_pi = pos >= 0 ? ((int64_t)h * p.ppos + pos) * a.nsub + sub : -1;
      pend_db = sDb[0][qst + n] + sDb[1][qst + n];
      pend = true;
    }

    if (wv == 0) {
      if (s + 1 < n_steps) meta_store(s + 1, ml, sM[P ^ 1]);
      if (s + 2 < n_steps) sRow[P][tid & 15][tid >> 4] = row_of(s + 2, pid2);
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

  // ---- dK and dV: the two query groups' sums, written by wavefronts 0 and 1 ----
  float* const redk = (float*)(kh ? sQ1 : sQ0);     // 16 KB each, no longer read
  float* const redv = (float*)(kh ? sO1 : sO0);
  if (qc == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        redk[(dt * 16 + r) * kWave + lane] = acc_dk[dt][r];
        redv[(dt * 16 + r) * kWave + lane] = acc_dv[dt][r];
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
          wk[j] = (bf16)((acc_dk[dt][r] + redk[(dt * 16 + r) * kWave + lane]) * a.scale);
          wvv[j] = (bf16)(acc_dv[dt][r] + redv[(dt * 16 + r) * kWave + lane]);
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
