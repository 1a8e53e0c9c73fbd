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
//   * plan -> scan -> scatter kernels: per 128-query tile, a routed block is
//     "dense" if at least dense_threshold of the tile's queries selected it;
//     the other (query, block) pairs are "sparse" and are grouped by block.
//   * sparse kernel: one work-group per chunk of up to 256 sparse pairs of one
//     block and head stages the block's K/V in LDS once and runs the gathered
//     queries through the MFMA tiles, writing a normalised bf16 partial and its
//     base-2 log-sum-exp per (pair, head).
//   * tile kernel: one work-group of 4 wavefronts per (128-query tile, head,
//     sequence), 32 queries per wavefront.  64-key items (the window band, then
//     the tile's dense blocks) stream through double-buffered LDS stages filled
//     by direct global->LDS loads; S^T = K Q^T with v_mfma_f32_32x32x16_bf16 so
//     that each lane owns one query's softmax state; base-2 online softmax;
//     O^T += V^T P^T; finally the query's sparse partials are merged in.
// With no plan (dense_threshold <= 0) the tile kernel processes every routed
// block of the tile as a dense block; when its grid alone cannot fill the chip,
// the items of each tile are divided among work-groups (more for the tiles with
// more remote blocks), each writing a normalised bf16 partial per row, and a merge
// kernel combines them.

#include "dash_common.h"

#include <type_traits>

namespace dash {

constexpr int kPfTQ = 128;        // queries per tile work-group
constexpr int kPfMaxK = 16;       // routed slots per query processed as one group
constexpr int kPfMaxSlots = 64;   // routed slots per query (groups of kPfMaxK; above
                                  // kPfMaxK every routed pair goes block-major)
constexpr int kPfMaxBlocks = 2048;
// Keys per tile-kernel item (a double-buffered LDS stage) and the work-groups per
// CU that the stage size and the register budget allow.
constexpr int kTileIT = 64;
constexpr int kTileOcc = 2;
constexpr int kSplitMax = 8;      // work-groups (parts) per split tile
constexpr int kPfCH = 256;        // pairs per sparse chunk (work-group)
// A chunk record: block id, pair count, 2 unused words, then up to kPfCH pair ids
// (token * K + slot within the sequence), so that a work-group reads its chunk's
// header and pair ids in one round trip.
constexpr int kRecHead = 4;
constexpr int kRec = kRecHead + kPfCH;
// Largest K/V token stride (elements) whose 64-row byte offsets within a stage fit 32 bits:
// 64 rows x 2 B x stride + 256 B of chunk offset < 2^32.
constexpr int64_t kMaxKeyRowStride = (int64_t(1) << 25) - 64;

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
  // K % 4 == 0 with 16-byte aligned ids and biases and 4-byte aligned validity: the
  // slots of a row are read and written four at a time
  int slots_vec;
  int S, H, bs, lw, nblk_cap;
  int ntiles;                          // 128-query tiles per sequence (of S)
  float scale_log2e;
  // hybrid plan (null kind: every routed block is processed by the tile kernel)
  uint8_t* kind;                       // [rows, K]: 0 skip, 1 tile (dense), 2 sparse
  int dense_threshold;
  int32_t* blk_count;                  // [B, nblk_cap], cleared at the start of a call
  int32_t* tile_base;                  // [B, ntiles_cap, nblk_cap] offset of a tile's pairs
  int ntiles_cap;
  int32_t* blk_chunk;                  // [B, nblk_cap] first chunk of each block
  int32_t* num_chunks;                 // [B]
  int32_t* chunk_pref;                 // [B+1] prefix sums of num_chunks
  int32_t* done;                       // arrival counter of the scan (follows blk_count)
  int32_t* err;                        // nonzero: a plan count exceeded its capacity (follows done)
  int B;
  // packed documents (cu): the tile grid runs over the documents' real tiles in one
  // order, head-major, so that the XCDs get equal shares (the scan kernel writes these):
  // tile_pref [B+1] the first tile of each document, tile_doc [ntv] the document of
  // each tile; ntv bounds the number of tiles
  int32_t* tile_pref;
  int32_t* tile_doc;
  int ntv;
  int32_t* chunk_rec;                  // [B, chunk_cap, kRec] chunk records
  int chunk_cap;
  // sparse partials, one per (head, pair position) (see part_row): a pair's
  // position is its place in the chunk records, chunk-major over all sequences
  int32_t* spos;                       // [rows, K] position of each sparse pair
  int64_t ppos;                        // positions per head
  // the normalised partial output of a pair as bytes, dims in MFMA lane order (see
  // part_index): dim value = (byte - 128) * scale, scale = (the row's largest
  // magnitude) / 127, so that a stored value is off by at most half a step, 1/254
  // of that magnitude
  float2* part_ls;                     // [H, ppos]  (base-2 log-sum-exp, scale)
  uint8_t* part_q;                     // [H, ppos, D]
  // split tiles (no plan; split_items > 0): tile t of every sequence is cut into
  // tile_parts(t) parts of split_items items (the last part takes the rest); part p
  // of tile tl (the logical (sequence, head, tile) id) writes its rows' normalised
  // output and base-2 log-sum-exp to slot tl * kSplitMax + p
  int split_items;
  int split_parts;                     // parts per (sequence, head): the sum over tiles
  bf16* split_o;                       // [tiles, kSplitMax, kPfTQ, D] bf16, dims in order
  float* split_lse;                    // [tiles, kSplitMax, kPfTQ]
};

// Upper bound of the items of tile t (no plan) of a sequence of S tokens: its
// window items, and the items of every block a routed slot of its rows may name
// (blocks with a key before the window of its last row; at most K per row).
__host__ __device__ inline int tile_item_bound(int t, int S, int lw, int bs, int K) {
  const int t0 = t * kPfTQ;
  const int t_last = (t0 + kPfTQ - 1 < S - 1) ? t0 + kPfTQ - 1 : S - 1;
  const int jw0 = (t0 - lw + 1 > 0 ? t0 - lw + 1 : 0) / kTileIT * kTileIT;
  const int n_win = (t_last - jw0) / kTileIT + 1;
  const int ipb = (bs + kTileIT - 1) / kTileIT;
  const int far = t_last - lw;
  const int n_rem = far >= 0 ? far / bs + 1 : 0;
  return n_win + ipb * (n_rem < kPfTQ * K ? n_rem : kPfTQ * K);
}
// Parts of tile t at `items` items per part (1 .. kSplitMax).
__host__ __device__ inline int tile_parts(int t, int S, int lw, int bs, int K, int items) {
  const int n = (tile_item_bound(t, S, lw, bs, K) + items - 1) / items;
  return n < 1 ? 1 : (n > kSplitMax ? kSplitMax : n);
}

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

// Position of dim 32 dt + 8 g + 4 hl + q of a partial row: the 64 dims a lane
// half hl owns in the MFMA accumulator layout are contiguous, in (dt, g, q) order.
__device__ __forceinline__ int part_index(int hl, int dt, int g, int q) {
  return hl * 64 + dt * 16 + g * 4 + q;
}

// Index of the sparse partial of (pair position, head): head, then position, so
// that the partials a sparse wavefront writes (32 consecutive pairs of a chunk)
// are neighbours in memory.
template <typename Args>
__device__ __forceinline__ int64_t part_row(const Args& a, int64_t pos, int h) {
  return (int64_t)h * a.ppos + pos;
}

// Where the scatter kernel stores the q-th sparse pair of a block whose chunks start
// at chunk bch of its sequence: the index of its chunk record (within the
// sequence's chunk_cap records) and its partial position (pair positions of the
// sequence start at pos0).  False if either falls outside the workspace, which
// consistent plan counts never produce.
__host__ __device__ inline bool scatter_target(int64_t chunk_cap, int64_t ppos, int64_t pos0,
                                               int64_t bch, int64_t q, int64_t* rec_chunk,
                                               int64_t* pair_pos) {
  *rec_chunk = bch + q / kPfCH;
  *pair_pos = pos0 + bch * kPfCH + q;
  return bch >= 0 && q >= 0 && *rec_chunk < chunk_cap && *pair_pos < ppos;
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

// ds_read_tr16_b64 (gfx950) operands: 4 x 16-bit values read from LDS.
typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

// Load the routed slots g0 .. g0+15 of one row (K <= 64): ids and validity, four
// slots per load where slots_vec allows (ng is then a multiple of 4); slots past K get
// id -1.
__device__ __forceinline__ void load_row_slots(const PrefillArgs& a, int64_t row, int g0,
                                               int32_t (&c)[kPfMaxK], uint32_t& vmask) {
  const int64_t p0 = row * a.K + g0;
  const int ng = min(kPfMaxK, a.K - g0);
  if (a.slots_vec) {
    const int4* ip = (const int4*)(a.idx + p0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4 v = 4 * q < ng ? ip[q] : make_int4(-1, -1, -1, -1);
      c[4 * q] = v.x; c[4 * q + 1] = v.y; c[4 * q + 2] = v.z; c[4 * q + 3] = v.w;
    }
    vmask = 0;
    if (a.valid) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w = 4 * q < ng ? *(const uint32_t*)(a.valid + p0 + 4 * q) : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((w >> (8 * e)) & 0xffu) vmask |= 1u << (4 * q + e);
      }
    } else {
      vmask = (1u << ng) - 1u;
    }
    return;
  }
#pragma unroll
  for (int s = 0; s < kPfMaxK; ++s) c[s] = s < ng ? a.idx[p0 + s] : -1;
  vmask = 0;
  if (a.valid) {
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s)
      if (s < ng && a.valid[p0 + s]) vmask |= 1u << s;
  } else {
    vmask = (1u << ng) - 1u;
  }
}

// Plan: per 128-query tile, the queries selecting each routed block; a block
// chosen by at least dense_threshold of them is "dense" (kind 1, processed by the
// tile kernel), otherwise its pairs are "sparse" (kind 2) and reserve a range of
// the block's pair list.  Duplicate and unusable slots get kind 0 (first slot of a
// block wins).  Slots are handled in groups of 16 in registers; every slot's id
// (0 where not kept) goes to LDS for the dedup of later groups and the kinds.
__global__ __launch_bounds__(kPfTQ) void prefill_plan_kernel(PrefillArgs a) {
  __shared__ int32_t sCnt[kPfMaxBlocks];
  __shared__ int16_t sId[kPfMaxSlots][kPfTQ];      // every slot's block id, per row
  const int b = blockIdx.y, tid = threadIdx.x;
  const int len = seq_len(a, b);
  const int t0 = blockIdx.x * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  for (int i = tid; i < nblk; i += kPfTQ) sCnt[i] = 0;
  __syncthreads();
  const int t = t0 + tid;
  const int64_t row = row0(a, b) + t;
  uint64_t keep_all = 0;
  if (t < len) {
    const int km = a.kmin ? a.kmin[row] : 0;
    const int ls = t - a.lw + 1;
    for (int g0 = 0; g0 < a.K; g0 += kPfMaxK) {
      int32_t c[kPfMaxK];
      uint32_t vmask, keep_mask = 0;
      load_row_slots(a, row, g0, c, vmask);
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s) {
        bool ok = ((vmask >> s) & 1u) && c[s] >= 0 && c[s] < nblk && c[s] * a.bs < ls &&
                  (c[s] + 1) * a.bs > km;
#pragma unroll
        for (int u = 0; u < s; ++u) ok = ok && !(((keep_mask >> u) & 1u) && c[u] == c[s]);
        for (int u = 0; ok && u < g0; ++u)
          ok = !(((keep_all >> u) & 1ull) && sId[u][tid] == c[s]);
        if (ok) {
          keep_mask |= 1u << s;
          atomicAdd(&sCnt[c[s]], 1);
        }
        if (g0 + s < kPfMaxSlots) sId[g0 + s][tid] = (int16_t)(ok ? c[s] : 0);
      }
      keep_all |= (uint64_t)keep_mask << g0;
    }
  }
  __syncthreads();
  // one global atomic per sparse block of this tile: reserves the tile's range
  // in the block's pair list (its base is kept for the scatter kernel).  A thread's
  // atomics are all issued before any base is stored: stored one by one, each
  // atomic waited for the store before it (the counters and the bases may alias
  // for all the compiler knows), one round trip per block.
  int32_t* tb = a.tile_base + ((int64_t)b * a.ntiles_cap + blockIdx.x) * a.nblk_cap;
  {
    constexpr int kPer = kPfMaxBlocks / kPfTQ;   // blocks per thread at most
    int base[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int cc = tid + k * kPfTQ;
      const int n = cc < nblk ? sCnt[cc] : 0;
      base[k] = (n > 0 && n < a.dense_threshold)
                    ? atomicAdd(&a.blk_count[(int64_t)b * a.nblk_cap + cc], n) : -1;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (base[k] >= 0) tb[tid + k * kPfTQ] = base[k];
  }
  if (t < len) {
    auto kind_of = [&](int s) -> uint32_t {
      if (!((keep_all >> s) & 1ull)) return 0u;
      return sCnt[sId[s][tid]] >= a.dense_threshold ? 1u : 2u;
    };
    if (a.K % kPfMaxK == 0) {               // 16 kinds per 16-byte store
      for (int g0 = 0; g0 < a.K; g0 += kPfMaxK) {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int s = 0; s < kPfMaxK; ++s) w[s >> 2] |= kind_of(g0 + s) << (8 * (s & 3));
        *(uint4*)(a.kind + row * a.K + g0) = make_uint4(w[0], w[1], w[2], w[3]);
      }
    } else if (a.K % 4 == 0) {              // 4 kinds per 4-byte store
      for (int s0 = 0; s0 < a.K; s0 += 4) {
        uint32_t w = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) w |= kind_of(s0 + e) << (8 * e);
        *(uint32_t*)(a.kind + row * a.K + s0) = w;
      }
    } else {
      for (int s = 0; s < a.K; ++s) a.kind[row * a.K + s] = (uint8_t)kind_of(s);
    }
  }
}

// ---------------------------------------------------------------------------
// The block counters and the arrival counter are cleared at the start of every
// call: a workspace reused by calls of other shapes holds other data there.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_clear_kernel(int32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ---------------------------------------------------------------------------
// Scan: per sequence, the first chunk of every block and the chunk record
// headers.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void prefill_scan_kernel(PrefillArgs a) {
  __shared__ int32_t sC[kPfMaxBlocks];
  __shared__ int32_t sCh[kPfMaxBlocks];
  __shared__ int32_t sWave[2][16];
  const int b = blockIdx.x, tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int len = seq_len(a, b);
  const int nblk = len > 0 ? (len + a.bs - 1) / a.bs : 0;
  int32_t* cnt = a.blk_count + (int64_t)b * a.nblk_cap;
  // two entries per thread
  int v0 = 0, v1 = 0;
  const int e0 = tid * 2, e1 = tid * 2 + 1;
  if (e0 < nblk) v0 = cnt[e0];
  if (e1 < nblk) v1 = cnt[e1];
  const int c0 = (v0 + kPfCH - 1) / kPfCH, c1 = (v1 + kPfCH - 1) / kPfCH;
  const int sc = c0 + c1;
  int ic = sc;
#pragma unroll
  for (int s = 1; s < kWave; s <<= 1) {
    const int oc = __shfl_up(ic, s, kWave);
    if (lane >= s) ic += oc;
  }
  if (lane == kWave - 1) sWave[1][wv] = ic;
  __syncthreads();
  int bc = 0;
  for (int w = 0; w < wv; ++w) bc += sWave[1][w];
  const int xc = bc + ic - sc;                       // exclusive prefix of this thread
  if (e0 < kPfMaxBlocks) { sC[e0] = v0; sCh[e0] = xc; }
  if (e1 < kPfMaxBlocks) { sC[e1] = v1; sCh[e1] = xc + c0; }
  if (a.tile_doc) {
    // this sequence's first tile in the one order of all sequences' tiles
    int pre = 0;
    for (int bb = tid; bb < b; bb += 1024) pre += (seq_len(a, bb) + kPfTQ - 1) / kPfTQ;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) pre += __shfl_xor(pre, m, kWave);
    __syncthreads();
    if (lane == 0) sWave[0][wv] = pre;
    __syncthreads();
    int first = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) first += sWave[0][w];
    const int nt = (len + kPfTQ - 1) / kPfTQ;
    if (tid == 0) {
      a.tile_pref[b] = first;
      if (b == (int)gridDim.x - 1) a.tile_pref[b + 1] = first + nt;
    }
    for (int i = tid; i < nt; i += 1024)
      if (first + i < a.ntv) a.tile_doc[first + i] = b;
    __syncthreads();
  }
  __shared__ int sLast;
  if (tid == 1023) {
    // the sparse grid covers no chunk past the sequence's records
    a.num_chunks[b] = min(bc + ic, a.chunk_cap);
    if (gridDim.x == 1) {                  // one sequence: its count is the prefix
      a.chunk_pref[0] = 0;
      a.chunk_pref[1] = min(bc + ic, a.chunk_cap);
      sLast = 0;
    } else {
      __threadfence();
      sLast = atomicAdd(a.done, 1) == (int)gridDim.x - 1;
    }
  }
  __syncthreads();
  int32_t* rec = a.chunk_rec + (int64_t)b * a.chunk_cap * kRec;
  for (int c = tid; c < nblk; c += 1024) {
    a.blk_chunk[(int64_t)b * a.nblk_cap + c] = sCh[c];
    const int n = sC[c];
    for (int i = 0; i * kPfCH < n; ++i) {
      if (sCh[c] + i >= a.chunk_cap) {       // never with consistent counts
        atomicOr(a.err, 1);
        break;
      }
      *(int2*)(rec + (int64_t)(sCh[c] + i) * kRec) = make_int2(c, min(kPfCH, n - i * kPfCH));
    }
  }
  // The sequence that finishes last writes the prefix sums of the chunk counts
  // (the sparse kernel maps its grid onto the real chunks with them).
  if (sLast) {
    __threadfence();
    const int nseq = (int)gridDim.x;
    int carry = 0;
    for (int base = 0; base < nseq; base += 1024) {
      const int i = base + tid;
      const int v = i < nseq ? __hip_atomic_load(&a.num_chunks[i], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT) : 0;
      int x = v;
#pragma unroll
      for (int s2 = 1; s2 < kWave; s2 <<= 1) {
        const int y = __shfl_up(x, s2, kWave);
        if (lane >= s2) x += y;
      }
      __syncthreads();
      if (lane == kWave - 1) sWave[0][wv] = x;
      __syncthreads();
      int wb = 0, tot = 0;
      for (int w = 0; w < 16; ++w) {
        if (w < wv) wb += sWave[0][w];
        tot += sWave[0][w];
      }
      if (i < nseq) a.chunk_pref[i + 1] = carry + wb + x;
      carry += tot;
    }
    if (tid == 0) a.chunk_pref[0] = 0;
  }
}

// ---------------------------------------------------------------------------
// Scatter: sparse pairs into the chunk records of their block (order within a
// block is free).
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
  const int32_t* bch = a.blk_chunk + (int64_t)b * a.nblk_cap;
  int32_t* rec = a.chunk_rec + (int64_t)b * a.chunk_cap * kRec;
  const int64_t pos0 = (int64_t)a.chunk_pref[b] * kPfCH;   // first pair position of the sequence
  for (int g0 = 0; g0 < a.K; g0 += kPfMaxK) {
    int32_t c[kPfMaxK];
    uint32_t vmask;
    load_row_slots(a, row, g0, c, vmask);
    const int ng = min(kPfMaxK, a.K - g0);
    int pos[kPfMaxK];
    bool sp[kPfMaxK];
    if (a.slots_vec) {
      uint32_t kw[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        kw[q] = 4 * q < ng ? *(const uint32_t*)(a.kind + row * a.K + g0 + 4 * q) : 0u;
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s) sp[s] = ((kw[s >> 2] >> (8 * (s & 3))) & 0xffu) == 2;
    } else {
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s) sp[s] = s < ng && a.kind[row * a.K + g0 + s] == 2;
    }
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) pos[s] = sp[s] ? atomicAdd(&sFill[c[s]], 1) : 0;
    // the slots' tile bases and first chunks are all loaded before the first record is
    // stored (the records may alias them for all the compiler knows, which made every
    // slot wait for the stores of the slot before it)
    int qs[kPfMaxK], ch[kPfMaxK];
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) {
      qs[s] = sp[s] ? tb[c[s]] + pos[s] : 0;        // position in the block's pair list
      ch[s] = sp[s] ? bch[c[s]] : 0;
    }
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s)
      if (sp[s]) {
        const int64_t slot = row * a.K + g0 + s;
        const int q = qs[s];
        int64_t rc, pp;
        if (scatter_target(a.chunk_cap, a.ppos, pos0, ch[s], q, &rc, &pp)) {
          rec[rc * kRec + kRecHead + q % kPfCH] = (int32_t)(slot - base);
          a.spos[slot] = (int32_t)pp;
        } else {                                       // never with consistent counts
          atomicOr(a.err, 2);
          a.spos[slot] = -1;                           // the tile kernel skips the slot
        }
      }
  }
}


// ---------------------------------------------------------------------------
// Tile kernel: window band + dense routed blocks + merge of the sparse partials.
//
// Items of up to 64 keys: the window band in 64-key steps, then the dense routed
// blocks of the tile in ascending order (64 keys per item).  K and V of an item
// are 64 x 128 bf16 tiles in LDS, double-buffered: the next item's tiles are
// fetched straight into LDS (16-byte global_load_lds per lane) while the current
// one computes, one barrier per item.  Rows are stored as 16 chunks of 16 bytes
// with the chunk slot XOR-swizzled by the row, so that the K operand reads
// (ds_read_b128: 16 lanes a clock read 16 rows at one chunk) and the
// transposing V reads (ds_read_b64_tr_b16: 32 lanes a clock read 4 rows at 4
// adjacent chunks) hit distinct banks of gfx950's 256-byte-per-clock LDS
// (measured conflict-free with SQ_LDS_BANK_CONFLICT).
// Per item and wavefront (32 queries): S^T for both 32-key halves, the
// visible-key mask as a per-query key range (no
// mask when the whole half is visible to every query), base-2 online softmax
// with a lazy rescale, O^T += V^T P^T.
// ---------------------------------------------------------------------------
constexpr int kPfIT = 64;         // keys of a sparse-kernel stage (one routed block)

__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((r & 3) << 2); }

// Per-lane element offsets of the direct loads of a stage of ROWS keys by 4
// wavefronts: wavefront wv issues the 4-row groups wv, wv+4, ...; lane l of a
// group fills slot l % 16 of row 4 grp + l / 16 with chunk slot ^ swizzle(row).
template <int ROWS>
struct FetchOffsets {
  static constexpr int kN = ROWS / 16;     // 4-row groups per wavefront
  uint32_t k[kN], v[kN];
  int r[kN];
};

template <int ROWS>
__device__ __forceinline__ FetchOffsets<ROWS> fetch_offsets(int64_t k_st, int64_t v_st, int wv,
                                                            int lane) {
  FetchOffsets<ROWS> f;
#pragma unroll
  for (int u = 0; u < FetchOffsets<ROWS>::kN; ++u) {
    const int grp = u * 4 + wv;
    const int r = grp * 4 + (lane >> 4), slot = lane & 15;
    f.r[u] = r;
    f.k[u] = (uint32_t)(r * k_st + k_slot(r, slot) * 8);
    f.v[u] = (uint32_t)(r * v_st + v_slot(r, slot) * 8);
  }
  return f;
}

// Issue the loads of K and V rows j0 .. j0+ROWS-1 of one head into a swizzled
// stage; rows at or beyond len repeat row len-1 (their keys are masked).
template <int D, int ROWS>
__device__ __forceinline__ void tile_fetch(bf16* sKs, bf16* sVs, const bf16* kb, const bf16* vb,
                                           int64_t k_st, int64_t v_st, int j0, int len, int wv,
                                           int lane, const FetchOffsets<ROWS>& f) {
  static_assert(D == 128, "16 chunks per row");
  const bf16* kb0 = kb + (int64_t)j0 * k_st;
  const bf16* vb0 = vb + (int64_t)j0 * v_st;
  const bool inside = j0 + ROWS <= len;
#pragma unroll
  for (int u = 0; u < FetchOffsets<ROWS>::kN; ++u) {
    const int grp = u * 4 + wv;
    const bf16* kp;
    const bf16* vp;
    if (inside) {
      kp = kb0 + f.k[u];
      vp = vb0 + f.v[u];
    } else {
      const int64_t dj = min(j0 + f.r[u], len - 1) - (j0 + f.r[u]);   // <= 0
      kp = kb0 + f.k[u] + dj * k_st;
      vp = vb0 + f.v[u] + dj * v_st;
    }
    __builtin_amdgcn_global_load_lds((const void*)kp,
                                     (__attribute__((address_space(3))) void*)(sKs + grp * 4 * D),
                                     16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)vp,
                                     (__attribute__((address_space(3))) void*)(sVs + grp * 4 * D),
                                     16, 0, 0);
  }
}

// Issue the loads of rows j0 .. j0+ROWS-1 of one matrix (K or V) into a
// swizzled stage by 4 wavefronts; rows at or beyond len repeat row len-1.
// Wavefront wv fills rows 16u + r0 (r0 = 4 wv + lane/16), chunk slot lane % 16,
// for u = 0 .. ROWS/16-1.  The swizzles of both matrices depend on the row only
// through row % 16 = r0, so the lane's swizzled chunk is one byte offset cb for
// every u; lane_off = 2 r0 x_st + cb.
template <int D, int ROWS>
__device__ __forceinline__ void rows_fetch(bf16* sX, const bf16* xb, int64_t x_st, uint32_t lane_off,
                                           uint32_t cb, int r0, int j0, int len, int wv) {
  static_assert(D == 128, "16 chunks per row");
  const char* xb0 = (const char*)(xb + (int64_t)j0 * x_st);
  const uint32_t row_b = (uint32_t)x_st * 2u;
  if (j0 + ROWS <= len) {
#pragma unroll
    for (int u = 0; u < ROWS / 16; ++u)
      __builtin_amdgcn_global_load_lds((const void*)(xb0 + (lane_off + (uint32_t)(16 * u) * row_b)),
                                       (__attribute__((address_space(3))) void*)(sX + (4 * u + wv) * 4 * D),
                                       16, 0, 0);
  } else {
    // rows past the end read the last row; the item may start at or past the end (the
    // second 64-key item of a routed block of more than 64 keys that the sequence ends
    // inside), so the row is addressed from the sequence base with 64-bit arithmetic
    // rather than as an unsigned offset from j0, which such a start would wrap
#pragma unroll
    for (int u = 0; u < ROWS / 16; ++u) {
      const int row = min(j0 + 16 * u + r0, len - 1);
      __builtin_amdgcn_global_load_lds((const void*)((const char*)(xb + (int64_t)row * x_st) + cb),
                                       (__attribute__((address_space(3))) void*)(sX + (4 * u + wv) * 4 * D),
                                       16, 0, 0);
    }
  }
}

// Lane part of the byte offset of the K operand reads (see k_frag): row n of a
// stage and, for k-step kk, chunk ((2 kk + hl) ^ (n % 16)), whose byte offset
// 16 ((2 kk + hl) ^ (n % 16)) = 32 kk ^ (16 hl ^ 16 (n % 16)).  So the read of
// half hf, k-step kk is at 8192 hf + (kl ^ 32 kk): one XOR per k-step.
__device__ __forceinline__ uint32_t k_lane_off(int n, int hl) {
  return (uint32_t)(n * 256) | (uint32_t)((hl << 4) ^ ((n & 15) << 4));
}
__device__ __forceinline__ bf16x8 k_frag_at(const bf16* sKs, uint32_t kl, int hf, int kk) {
  return *(const bf16x8*)((const char*)sKs + hf * 8192 + (kl ^ (uint32_t)(kk << 5)));
}

// Lane part of the byte offset of the transposing V reads (see pv_tr_swz): row
// 4 hl + rr (rr = (lane % 16) / 4, which is also the row's swizzle row % 4),
// bytes 8 (lane % 2) within chunk 4 dt + cq, whose swizzled slot gives byte
// offset 16 cq + 64 (dt ^ rr).  The read of tile dt is at (vl ^ 64 dt), plus
// 256 kbase (and 2048 for the rows 8 further).
__device__ __forceinline__ uint32_t v_lane_off(int lane) {
  const int hl = lane >> 5;
  const int rr = (lane & 15) >> 2;
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  return (uint32_t)((4 * hl + rr) * 256 + 8 * (lane & 1) + 16 * cq + 64 * rr);
}
__device__ __forceinline__ void pv_at(const bf16* sVs, uint32_t vl, int kbase, const bf16x8& pop,
                                      floatx16 (&acc_o)[4]) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const char* p = (const char*)sVs + kbase * 256 + (vl ^ (uint32_t)(dt << 6));
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)p);
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)(p + 2048));
    bf16x8 vop;
    const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
    const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
    for (int e = 0; e < 4; ++e) { vop[e] = l4[e]; vop[e + 4] = h4[e]; }
    acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, acc_o[dt], 0, 0, 0);
  }
}

// K operand of keys krow0 + (lane % 32), dims 16 kk + 8 (lane / 32) .. +7.
__device__ __forceinline__ bf16x8 k_frag(const bf16* sKs, int krow, int kk, int hl) {
  return *(const bf16x8*)(sKs + krow * 128 + k_slot(krow, 2 * kk + hl) * 8);
}

// acc_o[dt] += V^T P^T over keys kbase .. kbase+15 of a swizzled V stage.
// ds_read_tr16_b64 (gfx950): within each 16-lane group, result lane i element j
// is element (i % 4) of the 8 bytes read by lane 4j + i/4.  Lane l reads the 4
// dims 32dt + 16((l/16)%2) + 4(l%4) .. +3 of key row kbase + 4hl + (l%16)/4 (and
// +8), which gives every lane the 8 keys kbase + 8(e/4) + 4hl + e%4 of its dim
// row m = l % 32: the same key order as the P^T operand built from S^T.
__device__ __forceinline__ void pv_tr_swz(const bf16* sVs, int kbase, const bf16x8& pop,
                                          floatx16 (&acc_o)[4], int lane) {
  const int hl = lane >> 5;
  const int row = kbase + 4 * hl + ((lane & 15) >> 2);
  const int cq = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int within = 4 * (lane & 1);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int c = dt * 4 + cq;
    const short4v lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)(sVs + row * 128 + v_slot(row, c) * 8 + within));
    const short4v hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_short4*)(__attribute__((address_space(3))) void*)(sVs + (row + 8) * 128 + v_slot(row + 8, c) * 8 + within));
    bf16x8 vop;
    const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo);
    const bf16x4 h4 = __builtin_bit_cast(bf16x4, hi);
#pragma unroll
    for (int e = 0; e < 4; ++e) { vop[e] = l4[e]; vop[e + 4] = h4[e]; }
    acc_o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, acc_o[dt], 0, 0, 0);
  }
}

// Orders a wavefront's LDS writes before its later LDS reads of other lanes'
// data (and reads before later writes): the compiler otherwise treats each lane's
// LDS accesses as independent of the other lanes'.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Maximum over lanes l and l^32, every lane gets it (v_permlane32_swap).
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// First dense block > c of the tile's bitmap (nwords 32-bit words), or -1.
__device__ __forceinline__ int next_union(const uint32_t* sBits, int nwords, int c, int lane) {
  const int b0 = c + 1;
  const int w = (b0 >> 5) + lane;
  uint32_t bits = 0;
  if (w < nwords) {
    bits = sBits[w];
    if (lane == 0) bits &= ~0u << (b0 & 31);
  }
  const uint64_t nz = __ballot(bits != 0);
  if (nz == 0) return -1;
  const int f = __builtin_ctzll(nz);
  const uint32_t fb = __builtin_amdgcn_readlane(bits, f);
  return __builtin_amdgcn_readfirstlane((((b0 >> 5) + f) << 5) + (int)__builtin_ctz(fb));
}

// The j-th (from 0) dense block of the tile's bitmap (nwords <= 64 words, one per
// lane); j is below the number of set bits.
__device__ __forceinline__ int nth_union(const uint32_t* sBits, int nwords, int j, int lane) {
  const uint32_t bits = lane < nwords ? sBits[lane] : 0u;
  const int cnt = __popc(bits);
  int x = cnt;                             // inclusive prefix of the counts over lanes
#pragma unroll
  for (int s = 1; s < kWave; s <<= 1) {
    const int y = __shfl_up(x, s, kWave);
    if (lane >= s) x += y;
  }
  const int f = __builtin_ctzll(__ballot(x > j));   // the word holding it
  const int before = __builtin_amdgcn_readlane(x - cnt, f);
  uint32_t w = __builtin_amdgcn_readlane(bits, f);
  for (int i = before; i < j; ++i) w &= w - 1u;      // drop the lower set bits
  return __builtin_amdgcn_readfirstlane((f << 5) + (int)__builtin_ctz(w));
}

template <int D, int IT, int OCC>
__global__ __launch_bounds__(256, OCC) void prefill_tile_kernel(PrefillArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ __attribute__((aligned(16))) bf16 sK0[IT * D];
  __shared__ __attribute__((aligned(16))) bf16 sK1[IT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV0[IT * D];
  __shared__ __attribute__((aligned(16))) bf16 sV1[IT * D];
  __shared__ __attribute__((aligned(16))) int16_t sIdx[kPfTQ][kPfMaxK];
  __shared__ __attribute__((aligned(16))) float sBias[kPfTQ][kPfMaxK];
  __shared__ uint32_t sBits[kPfMaxBlocks / 32];

  // logical order (sequence, head, tile), tile fastest, contiguous per XCD; packed
  // documents in the order (head, tile of all documents), so that every logical id
  // below the tile count is a real tile and the XCDs get equal shares
  // (split tiles: (sequence, head, part of all tiles), the parts of a tile
  // consecutive)
  int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  int part = 0, nparts = 1;
  if (a.split_items > 0) {
    const int j = lid % a.split_parts;
    const int bh = lid / a.split_parts;
    int t = 0, pre = 0;
    for (; t < a.ntiles; ++t) {
      nparts = tile_parts(t, a.S, a.lw, a.bs, a.K, a.split_items);
      if (j < pre + nparts) break;
      pre += nparts;
    }
    if (t >= a.ntiles) return;             // never: the grid holds split_parts per (b, h)
    part = j - pre;
    lid = bh * a.ntiles + t;
  }
  // partial slot of a split tile
  const int split_slot = lid * kSplitMax + part;
  int tile, h, b;
  if (a.tile_doc) {
    const int g = lid % a.ntv;
    h = lid / a.ntv;
    if (g >= a.tile_pref[a.B]) return;
    b = a.tile_doc[g];
    tile = g - a.tile_pref[b];
  } else {
    tile = lid % a.ntiles;
    const int bh = lid / a.ntiles;
    h = bh % a.H;
    b = bh / a.H;
  }
  const int len = seq_len(a, b);
  const int t0 = tile * kPfTQ;
  if (t0 >= len) return;
  const int nblk = (len + a.bs - 1) / a.bs;
  const int nwords = (nblk + 31) / 32;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5;         // half of the wave: 0/1
  const int n = lane & 31;          // query column within the wave
  const int64_t r0 = row0(a, b);

  // ---- this lane's query and its Q^T operand (8 k-steps of 16 dims), loaded
  // first so that the loads overlap the routed slots' loads below ----
  const int tq = t0 + wv * 32 + n;
  const bool qvalid = tq < len;
  const int tqc = min(tq, len - 1);
  const int64_t qrow = r0 + tqc;
  const bf16* qb = seq_ptr(a.q, a.cu, b, a.q_sb, a.q_st) + (int64_t)h * a.q_sh;
  bf16x8 qop[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qop[kk] = *(const bf16x8*)(qb + (int64_t)tqc * a.q_st + kk * 16 + hl * 8);

  for (int i = tid; i < kPfMaxBlocks / 32; i += 256) sBits[i] = 0u;
  __syncthreads();

  // ---- dense routed blocks of every query row: filter, dedup, sort ascending ----
  if (tid < kPfTQ) {
    const int t = t0 + tid;
    int cnt = 0;
    auto insert = [&](int c, float bv) {
      if (cnt >= kPfMaxK) return;        // dense lists hold 16 blocks (K > 16 plans none)
      int u = cnt;
      while (u > 0 && sIdx[tid][u - 1] > c) {
        sIdx[tid][u] = sIdx[tid][u - 1];
        sBias[tid][u] = sBias[tid][u - 1];
        --u;
      }
      sIdx[tid][u] = (int16_t)c;
      sBias[tid][u] = bv;
      ++cnt;
      atomicOr(&sBits[c >> 5], 1u << (c & 31));
    };
    if (t < len && a.K <= kPfMaxK && (!a.kind || a.slots_vec)) {
      // Rows of up to 16 slots, every load issued before any is used (four slots per
      // load where slots_vec allows).  Dense slots: with a plan, its kind-1 slots
      // (the plan has already dropped duplicate and unusable slots); without one,
      // every usable slot whose block no earlier usable slot names.  They are sorted
      // by block id with a bitonic network on the keys id << 5 | slot in registers
      // (ids < 2048; other slots, and slots past K, take id 2048 and sort last); the
      // biases, stored in slot order, are then gathered by slot.
      const int64_t p0 = (r0 + t) * a.K;
      int32_t cs[kPfMaxK];
      float bs4[kPfMaxK];
      uint32_t dmask = 0;                  // slots whose block goes with the tile
      if (a.slots_vec) {
        uint32_t kw[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const bool in = 4 * q < a.K;
          kw[q] = (in && a.kind) ? *(const uint32_t*)(a.kind + p0 + 4 * q) : 0u;
          const int4 iv = in ? ((const int4*)(a.idx + p0))[q] : make_int4(-1, -1, -1, -1);
          const float4 bv = in ? ((const float4*)(a.bias + p0))[q] : make_float4(0.f, 0.f, 0.f, 0.f);
          cs[4 * q] = iv.x; cs[4 * q + 1] = iv.y; cs[4 * q + 2] = iv.z; cs[4 * q + 3] = iv.w;
          bs4[4 * q] = bv.x; bs4[4 * q + 1] = bv.y; bs4[4 * q + 2] = bv.z; bs4[4 * q + 3] = bv.w;
        }
        if (a.kind) {
#pragma unroll
          for (int s = 0; s < kPfMaxK; ++s)
            if (((kw[s >> 2] >> (8 * (s & 3))) & 0xffu) == 1) dmask |= 1u << s;
        }
      } else {
#pragma unroll
        for (int s = 0; s < kPfMaxK; ++s) {
          cs[s] = s < a.K ? a.idx[p0 + s] : -1;
          bs4[s] = s < a.K ? a.bias[p0 + s] : 0.f;
        }
      }
      if (!a.kind) {
        uint32_t vmask;
        if (a.slots_vec && a.valid) {
          vmask = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t w = 4 * q < a.K ? *(const uint32_t*)(a.valid + p0 + 4 * q) : 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if ((w >> (8 * e)) & 0xffu) vmask |= 1u << (4 * q + e);
          }
        } else if (a.valid) {
          vmask = 0;
#pragma unroll
          for (int s = 0; s < kPfMaxK; ++s)
            if (s < a.K && a.valid[p0 + s]) vmask |= 1u << s;
        } else {
          vmask = a.K >= 32 ? ~0u : (1u << a.K) - 1u;
        }
        const int km = a.kmin ? a.kmin[r0 + t] : 0;
        const int ls = t - a.lw + 1;
#pragma unroll
        for (int s = 0; s < kPfMaxK; ++s) {
          const int c = cs[s];
          bool keep = ((vmask >> s) & 1u) && c >= 0 && c < nblk && c * a.bs < ls && (c + 1) * a.bs > km;
#pragma unroll
          for (int u = 0; u < s; ++u) keep = keep && !(((dmask >> u) & 1u) && cs[u] == c);
          if (keep) dmask |= 1u << s;
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ((float4*)&sBias[tid][0])[q] = make_float4(bs4[4 * q], bs4[4 * q + 1], bs4[4 * q + 2], bs4[4 * q + 3]);
      uint32_t key[kPfMaxK];
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s)
        key[s] = ((((dmask >> s) & 1u) ? (uint32_t)cs[s] : (uint32_t)kPfMaxBlocks) << 5) | (uint32_t)s;
#pragma unroll
      for (int k = 2; k <= kPfMaxK; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1)
#pragma unroll
          for (int i = 0; i < kPfMaxK; ++i) {
            const int l = i ^ j;
            if (l > i) {
              const uint32_t x = key[i], y = key[l];
              const bool asc = (i & k) == 0;
              key[i] = asc ? min(x, y) : max(x, y);
              key[l] = asc ? max(x, y) : min(x, y);
            }
          }
      float sb[kPfMaxK];
#pragma unroll
      for (int p = 0; p < kPfMaxK; ++p) sb[p] = sBias[tid][key[p] & 31u];
      int16_t ids[kPfMaxK];
#pragma unroll
      for (int p = 0; p < kPfMaxK; ++p) {
        const int c = (int)(key[p] >> 5);
        ids[p] = (int16_t)c;
        if (c < kPfMaxBlocks) {
          ++cnt;
          atomicOr(&sBits[c >> 5], 1u << (c & 31));
        }
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        int4 w;
        w.x = (uint16_t)ids[8 * q + 0] | ((uint32_t)(uint16_t)ids[8 * q + 1] << 16);
        w.y = (uint16_t)ids[8 * q + 2] | ((uint32_t)(uint16_t)ids[8 * q + 3] << 16);
        w.z = (uint16_t)ids[8 * q + 4] | ((uint32_t)(uint16_t)ids[8 * q + 5] << 16);
        w.w = (uint16_t)ids[8 * q + 6] | ((uint32_t)(uint16_t)ids[8 * q + 7] << 16);
        ((int4*)&sIdx[tid][0])[q] = w;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ((float4*)&sBias[tid][0])[q] = make_float4(sb[4 * q], sb[4 * q + 1], sb[4 * q + 2], sb[4 * q + 3]);
    } else if (t < len) {
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
        insert(c, a.bias[p]);
      }
    }
    // id 2048 (no block) ends every list
    for (int u = cnt; u < kPfMaxK; ++u) sIdx[tid][u] = (int16_t)kPfMaxBlocks;
  }

  const int q_ls = tq - a.lw + 1;
  const int q_km = a.kmin ? a.kmin[qrow] : 0;
  const int q_lo = max(max(q_ls, q_km), 0);       // first window key
  const int r_hi = min(q_ls, len) - 1;            // last key a routed block may give

  floatx16 acc_o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const bf16* kb = seq_ptr(a.k, a.cu, b, a.k_sb, a.k_st) + (int64_t)h * a.k_sh;
  const bf16* vb = seq_ptr(a.v, a.cu, b, a.v_sb, a.v_st) + (int64_t)h * a.v_sh;
  const int t_last = min(t0 + kPfTQ - 1, len - 1);
  const int jw0 = (max(t0 - a.lw + 1, 0) / IT) * IT;
  const int n_win = (t_last - jw0) / IT + 1;
  const int ipb = (a.bs + IT - 1) / IT;            // items per routed block
  __syncthreads();
  int nu = 0;
  {
    const uint32_t wbits = lane < nwords ? sBits[lane] : 0u;
    nu = __popc(wbits);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) nu += __shfl_xor(nu, m, kWave);
    nu = __builtin_amdgcn_readfirstlane(nu);
  }
  const int n_items = n_win + nu * ipb;
  // this work-group's items [i0, i1): all of them, or with split tiles the part's
  // split_items (the last part: the rest), cut at routed-block boundaries
  int i0 = 0, i1 = n_items;
  if (a.split_items > 0) {
    auto cut = [&](int x) {
      x = min(x, n_items);
      return x <= n_win ? x : n_win + (x - n_win) / ipb * ipb;
    };
    i0 = cut(part * a.split_items);
    i1 = part == nparts - 1 ? n_items : cut((part + 1) * a.split_items);
  }
  // first dense block of the share (0 when it starts in the window band)
  const int c_first = (i0 > n_win && i0 < i1) ? nth_union(sBits, nwords, (i0 - n_win) / ipb, lane) : 0;
  // fetch byte offsets: row r0 of a 16-row group and its swizzled chunk
  const int fr0 = wv * 4 + (lane >> 4);
  const uint32_t fkc = (uint32_t)(k_slot(fr0, lane & 15) * 16), fvc = (uint32_t)(v_slot(fr0, lane & 15) * 16);
  const uint32_t fk0 = (uint32_t)(fr0 * a.k_st * 2) + fkc, fv0 = (uint32_t)(fr0 * a.v_st * 2) + fvc;
  const uint32_t kl0 = k_lane_off(n, hl), vl0 = v_lane_off(lane);
  const int myrow = wv * 32 + n;
  const float log2e = 1.4426950408889634f;
  const float csc = a.scale_log2e;

  // Fetch iterator: block and sub-item of the last item whose K rows were fetched.
  int pf_c = c_first - 1, pf_sub = ipb - 1;
  int jk = 0, ck = -1, subk = 0;           // that item's first key, block, sub-item
  auto advance = [&](int it) {
    if (it >= n_win && ++pf_sub >= ipb) { pf_sub = 0; pf_c = next_union(sBits, nwords, pf_c, lane); }
    jk = it < n_win ? jw0 + it * IT : pf_c * a.bs + pf_sub * IT;
    ck = pf_c;
    subk = pf_sub;
  };
  if (i1 > i0) {
    advance(i0);
    rows_fetch<D, IT>(sK0, kb, a.k_st, fk0, fkc, fr0, jk, len, wv);
  }
  // Cursor into this query's ascending dense-block list (ended by id 2048): the
  // next candidate block is read one match ahead.
  int ptr = 0;
  while (c_first > 0 && ptr < kPfMaxK && sIdx[myrow][ptr] < c_first) ++ptr;
  int cand_c = ptr < kPfMaxK ? sIdx[myrow][ptr] : kPfMaxBlocks;
  float cur_b = -INFINITY;                 // bias (base 2) of the current routed block

  // Software pipeline over the items: step i computes S^T of item i, its row
  // maximum and its probabilities P, and O^T += V^T P^T of item i-1 (whose P the
  // previous step left in registers), so that the VALU work on item i runs while
  // the matrix core multiplies item i-1.  K of item i sits in stage sK[i % 2], V in
  // sV[i % 2]; step i fetches K(i+1) and V(i).  A lazy rescale (the reference
  // m_run only moves when some query's maximum exceeds it by more than 8, so
  // probabilities stay <= 2^8) applies its factor to O at the start of the next
  // step, after O^T(i-1) is complete.
  // Per item: the visible-key range of the query as (kq, span) (key j is visible
  // when j - lo, as unsigned, is <= span) and its bias; whether some query of the
  // wavefront sees a key of the item (need) and whether every query with a finite
  // bias sees all of them (full).  An item nobody needs gets S = -inf, so P = 0;
  // the V stage read before item 0 is zero-filled, so that every step runs the
  // same straight-line O^T update.
  bf16x8 pP[2][2][2];                      // [parity][half][16-key group]
#pragma unroll
  for (int hf = 0; hf < 2; ++hf)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int q = 0; q < 8; ++q) pP[1][hf][j][q] = (bf16)0.f;
  for (int i = tid; i < IT * D / 8; i += 256) ((uint4*)sV1)[i] = make_uint4(0u, 0u, 0u, 0u);
  float alpha_o = 1.f;                     // pending factor of acc_o
  bool o_pending = false;
  const bf16x2 ones = {(bf16)1.f, (bf16)1.f};

  auto step = [&](int it, auto par_tag) {
    constexpr int P = decltype(par_tag)::value;
    // parity P is a compile-time constant, so that every LDS array is named
    // statically and the reads of one stage do not wait for the loads into another
    bf16* const sKc = P == 0 ? sK0 : sK1;     // K(it)
    bf16* const sKn = P == 0 ? sK1 : sK0;     // K(it+1) is fetched here
    bf16* const sVc = P == 0 ? sV0 : sV1;     // V(it) is fetched here
    const bf16* const sVp = P == 0 ? sV1 : sV0;  // V(it-1)
    // Lane offsets pass through an empty asm each step, so that the compiler
    // derives the per-read addresses here instead of keeping them all live.
    uint32_t kl = kl0, vl = vl0, fk = fk0, fv = fv0;
    asm volatile("" : "+v"(kl), "+v"(vl), "+v"(fk), "+v"(fv));
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();                       // K(it), V(it-1) landed; step it-1 is done
    // S^T of item it first, so that its reads and MFMAs overlap the fetches and
    // the bookkeeping below (an item nobody needs, or the drain step, computes a
    // discarded S^T from whatever the stage holds)
    // raised wave priority over the compute of the step (two wavefronts of other
    // work-groups share each SIMD: the one in its MFMA stretch is preferred)
    __builtin_amdgcn_s_setprio(1);
    floatx16 sc[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sc[hf][r] = 0.f;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        sc[hf] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag_at(sKc, kl, hf, kk), qop[kk], sc[hf],
                                                         0, 0, 0);
    }
    bool need = false, full = false;
    float bl = -INFINITY;
    int kq = 0;
    uint32_t span = 0;
    if (it < i1) {
      rows_fetch<D, IT>(sVc, vb, a.v_st, fv, fvc, fr0, jk, len, wv);
      // item it: visible keys and bias of this query
      int lo, hi;
      if (it < n_win) {
        lo = q_lo; hi = tq;
        bl = qvalid ? 0.f : -INFINITY;
      } else {
        if (subk == 0) {
          cur_b = -INFINITY;
          if (cand_c == ck) {
            cur_b = sBias[myrow][ptr] * log2e;
            ++ptr;
            cand_c = ptr < kPfMaxK ? sIdx[myrow][ptr] : kPfMaxBlocks;
          }
        }
        lo = q_km; hi = min(r_hi, ck * a.bs + a.bs - 1);
        bl = qvalid ? cur_b : -INFINITY;
      }
      const int j0 = jk;
      const bool live = bl != -INFINITY && lo <= hi;
      need = __any(live && lo <= j0 + IT - 1 && hi >= j0);
      full = __all(!live || (lo <= j0 && j0 + IT - 1 <= hi));
      span = lo <= hi ? (uint32_t)(hi - lo) : 0u;
      kq = j0 + 4 * hl - (lo <= hi ? lo : 0x40000000);
      if (it + 1 < i1) {
        advance(it + 1);
        rows_fetch<D, IT>(sKn, kb, a.k_st, fk, fkc, fr0, jk, len, wv);
      }
    }
    if (o_pending) {                       // O^T(it-2) is complete
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha_o;
      alpha_o = 1.f;
      o_pending = false;
    }
    if (!need) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[hf][r] = -INFINITY;
    } else if (!full) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t d = (uint32_t)(kq + 32 * hf + 8 * (r >> 2) + (r & 3));
          sc[hf][r] = d <= span ? sc[hf][r] : -INFINITY;
        }
    }
    // O^T += V^T P^T of item it-1
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      pv_at(sVp, vl, 32 * hf, pP[P ^ 1][hf][0], acc_o);
      pv_at(sVp, vl, 32 * hf + 16, pP[P ^ 1][hf][1], acc_o);
    }
    // row maximum in base 2 (the scale is positive: max(fma(s, c, b)) =
    // fma(max s, c, b)), the rescale decision, p = 2^(s c + b - m) in bf16 and
    // the row sum of the bf16 p
    float mraw = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 16; ++r) mraw = fmaxf(mraw, sc[hf][r]);
    const float mloc = xor32_max(fmaf(mraw, a.scale_log2e, bl));
    const bool up = mloc > m_run + 8.f;
    const float alpha = up ? fast_exp2(m_run - mloc) : 1.f;   // 0 when m_run = -inf
    l_run *= alpha;
    alpha_o *= alpha;
    o_pending = o_pending || __any(up);
    m_run = up ? mloc : m_run;
    const float off = bl - ((m_run == -INFINITY) ? 0.f : m_run);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        pP[P][hf][r >> 3][r & 7] = (bf16)fast_exp2(fmaf(sc[hf][r], a.scale_log2e, off));
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 8; q += 2) {
          const bf16x2 pp = {pP[P][hf][j][q], pP[P][hf][j][q + 1]};
          l_run = __builtin_amdgcn_fdot2_f32_bf16(pp, ones, l_run, false);
        }
    __builtin_amdgcn_s_setprio(0);
  };
  for (int it = i0; it <= i1; it += 2) {
    step(it, std::integral_constant<int, 0>{});
    if (it + 1 <= i1) step(it + 1, std::integral_constant<int, 1>{});
  }

  // Arguments used only from here on are read again through an opaque copy of
  // the kernel-argument pointer, so that they occupy no scalar registers during
  // the item loop.
  const __attribute__((address_space(4))) char* kap =
      (const __attribute__((address_space(4))) char*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(kap));
  const __attribute__((address_space(4))) PrefillArgs& pa =
      *(const __attribute__((address_space(4))) PrefillArgs*)kap;

  // ---- merge the sparse partials of this query ----
  // All kinds, pair positions and log-sum-exps are loaded first and the
  // reference moves once to their maximum; partial rows are lane-contiguous and
  // read with 16-byte loads.
  // Slots are merged in groups of 16.
  float qbias = 0.f;                       // -128 x the bytes' weights, added to every dim
  for (int g0 = 0; pa.kind && g0 < pa.K; g0 += kPfMaxK) {
    const int64_t p0 = (r0 + tqc) * pa.K + g0;
    const int ng = min(kPfMaxK, pa.K - g0);
    float l2[kPfMaxK];
    int32_t sp[kPfMaxK];                   // positions (read for sparse slots only)
    uint32_t smask = 0;
    if (pa.slots_vec) {                    // ng is a multiple of 4
      uint32_t kw[4];
#pragma unroll
      for (int g = 0; g < kPfMaxK / 4; ++g) {
        const bool in = 4 * g < ng;
        kw[g] = in ? *(const uint32_t*)(pa.kind + p0 + 4 * g) : 0u;
        const int4 pv = in ? *(const int4*)(pa.spos + p0 + 4 * g) : make_int4(0, 0, 0, 0);
        sp[4 * g] = pv.x; sp[4 * g + 1] = pv.y; sp[4 * g + 2] = pv.z; sp[4 * g + 3] = pv.w;
      }
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s)
        if (qvalid && ((kw[s >> 2] >> (8 * (s & 3))) & 0xffu) == 2) smask |= 1u << s;
    } else {
#pragma unroll
      for (int s = 0; s < kPfMaxK; ++s) sp[s] = 0;
      for (int s = 0; s < ng; ++s)
        if (qvalid && pa.kind[p0 + s] == 2) {
          smask |= 1u << s;
          sp[s] = pa.spos[p0 + s];
        }
    }
    float qs[kPfMaxK];                     // the partial rows' byte scales
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) {
      const float2 ls = (((smask >> s) & 1u) && sp[s] >= 0) ? pa.part_ls[part_row(pa, sp[s], h)]
                                                           : make_float2(-INFINITY, 0.f);
      l2[s] = ls.x;
      qs[s] = ls.y;
    }
    float mx = m_run;
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s) mx = fmaxf(mx, l2[s]);
    if (mx > m_run) {
      const float alpha = fast_exp2(m_run - mx);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc_o[dt][r] *= alpha;
      qbias *= alpha;
      m_run = mx;
    }
    // Slots in 4 batches of 4: a batch's loads (the lanes' live slots only) are
    // all in flight before any is accumulated, so the merge waits on memory at
    // most four times.
    uint32_t live = 0;
#pragma unroll
    for (int s = 0; s < kPfMaxK; ++s)
      if (l2[s] != -INFINITY) live |= 1u << s;
    const uint8_t* po = pa.part_q + part_row(pa, 0, h) * D + part_index(hl, 0, 0, 0);
#pragma unroll
    for (int sb = 0; sb < kPfMaxK; sb += 4) {
      const uint32_t gm = (live >> sb) & 15u;
      if (!__any(gm != 0u)) continue;
      uint4 buf[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if ((gm >> u) & 1u) {
#pragma unroll
          for (int q = 0; q < 4; ++q) buf[u][q] = *(const uint4*)(po + (int64_t)sp[sb + u] * D + q * 16);
        }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if ((gm >> u) & 1u) {
          const float w = fast_exp2(l2[sb + u] - m_run);
          if (hl == 0) l_run += w;
          // value = (byte - 128) * scale: the bytes times w * scale here, the -128 in qbias
          const float c = w * qs[sb + u];
          qbias = fmaf(-128.f, c, qbias);
#pragma unroll
          for (int dt = 0; dt < D / 32; ++dt) {
            const uint32_t wd[4] = {buf[u][dt].x, buf[u][dt].y, buf[u][dt].z, buf[u][dt].w};
#pragma unroll
            for (int r = 0; r < 16; ++r)
              acc_o[dt][r] = fmaf(c, (float)((wd[r >> 2] >> (8 * (r & 3))) & 0xffu), acc_o[dt][r]);
          }
        }
    }
  }
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_o[dt][r] += qbias;

  // ---- epilogue: normalise and store ----
  const float l_tot = xor32_sum(l_run);
  if (pa.split_items > 0) {
    const int64_t slot = split_slot;
    if (qvalid) {
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      bf16* so = pa.split_o + (slot * kPfTQ + myrow) * D;
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = (bf16)(acc_o[dt][g * 4 + e] * inv);
          *(bf16x4*)(so + dt * 32 + 8 * g + 4 * hl) = w;
        }
      if (hl == 0) pa.split_lse[slot * kPfTQ + myrow] = l_tot > 0.f ? m_run + log2f(l_tot) : -INFINITY;
    }
    return;
  }
  if (qvalid) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    bf16* ob = (pa.cu ? pa.o + (int64_t)pa.cu[b] * pa.o_st : pa.o + (int64_t)b * pa.o_sb) +
               (int64_t)h * pa.o_sh + (int64_t)tq * pa.o_st;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = (bf16)(acc_o[dt][g * 4 + e] * inv);
        *(bf16x4*)(ob + dt * 32 + 8 * g + 4 * hl) = w;
      }
    if (pa.lse && hl == 0) {
      const float lse = l_tot > 0.f ? (m_run + log2f(l_tot)) * 0.6931471805599453f : -INFINITY;
      pa.lse[(r0 + tq) * pa.lse_row + (int64_t)h * pa.lse_sh] = lse;
    }
  }
}

// ---------------------------------------------------------------------------
// Merge of split tiles: each (row, head) row's partials, weighted by
// 2^(lse_p - max) in fp32; 16 lanes of 8 dims per row, 16 rows per work-group.
// Rows no share saw a key of give 0 (log-sum-exp -inf), as an unsplit tile does.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_split_merge_kernel(PrefillArgs a) {
  constexpr int D = 128;
  const int64_t item = (int64_t)blockIdx.x * 16 + threadIdx.x / 16;   // (tile id, row)
  const int sub = threadIdx.x & 15;
  if (item >= (int64_t)a.ntiles * a.H * a.B * kPfTQ) return;
  const int64_t tl = item / kPfTQ;
  const int r = (int)(item % kPfTQ);
  const int tile = (int)(tl % a.ntiles);
  const int bh = (int)(tl / a.ntiles);
  const int h = bh % a.H, b = bh / a.H;
  const int t = tile * kPfTQ + r;
  if (t >= seq_len(a, b)) return;
  const int P = tile_parts(tile, a.S, a.lw, a.bs, a.K, a.split_items);
  const float* ls = a.split_lse + tl * kSplitMax * kPfTQ + r;
  // every part's log-sum-exp and row piece loaded before any is used (one round trip)
  float l[kSplitMax];
  bf16x8 x[kSplitMax];
#pragma unroll
  for (int p = 0; p < kSplitMax; ++p) {
    l[p] = p < P ? ls[p * kPfTQ] : -INFINITY;
    if (p < P) x[p] = *(const bf16x8*)(a.split_o + ((tl * kSplitMax + p) * kPfTQ + r) * D + sub * 8);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int p = 0; p < kSplitMax; ++p) mx = fmaxf(mx, l[p]);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (mx != -INFINITY) {
#pragma unroll
    for (int p = 0; p < kSplitMax; ++p) {
      if (l[p] == -INFINITY) continue;
      const float w = exp2f(l[p] - mx);
      wsum += w;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += w * bf2f(x[p][e]);
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  bf16x8 y;
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = (bf16)(acc[e] * inv);
  bf16* ob = (a.cu ? a.o + (int64_t)a.cu[b] * a.o_st : a.o + (int64_t)b * a.o_sb) +
             (int64_t)h * a.o_sh + (int64_t)t * a.o_st;
  *(bf16x8*)(ob + sub * 8) = y;
  if (a.lse && sub == 0)
    a.lse[(row0(a, b) + t) * a.lse_row + (int64_t)h * a.lse_sh] =
        wsum > 0.f ? (mx + log2f(wsum)) * 0.6931471805599453f : -INFINITY;
}

// ---------------------------------------------------------------------------
// Sparse kernel: one chunk of up to 256 (query, block) pairs of one routed
// block, one head.  The block's K and V rows are staged in LDS once (swizzled
// like the tile kernel's stages); then each wavefront runs rounds of 32 gathered
// queries (pairs 32 wv + 128 j + lane of the chunk): S^T = K Q^T, the query's
// visible keys of the block with its routed bias, softmax, O^T = V^T P^T, and
// writes the normalised bf16 partial (lane order, see part_index) and its
// base-2 log-sum-exp per (pair, head).  No barrier after the staging.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256, 3) void prefill_sparse_kernel(PrefillArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ __attribute__((aligned(16))) bf16 sKs[kPfIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sVs[kPfIT * D];
  __shared__ __attribute__((aligned(16))) bf16 sTr[4 * 16 * D];   // per wavefront: 16 partial rows
  // The first H * (total chunks) work-groups of the grid take the real chunks
  // (the hardware deals consecutive work-groups to the 8 XCDs in turn, so every
  // XCD gets an equal share); the rest exit.  Logical order (sequence, head,
  // chunk), chunk fastest, contiguous per XCD.
  const int nreal = a.H * a.chunk_pref[a.B];
  if ((int)blockIdx.x >= nreal) return;
  const int lid = xcd_logical_id(blockIdx.x, nreal);
  int b = 0;
  {
    int hi = a.B;                          // the last sequence b with H * pref[b] <= lid
    while (hi - b > 1) {
      const int mid = (b + hi) >> 1;
      if (a.H * a.chunk_pref[mid] <= lid) b = mid; else hi = mid;
    }
  }
  const int pb = a.chunk_pref[b], nc = a.chunk_pref[b + 1] - pb;
  const int hc = lid - a.H * pb;
  const int h = hc / nc, ch = hc % nc;
  if ((int64_t)(pb + ch + 1) * kPfCH > a.ppos) return;     // never with consistent counts
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int hl = lane >> 5, n = lane & 31;
  // header and pair ids in one round trip: lanes past the count take the first id
  const int32_t* rec = a.chunk_rec + ((int64_t)b * a.chunk_cap + ch) * kRec;
  const int c = rec[0], npairs = rec[1];
  const int pid_first = rec[kRecHead];
  int pid_raw[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) pid_raw[j] = rec[kRecHead + wv * 32 + 128 * j + n];
  const int len = seq_len(a, b);
  const int64_t r0 = row0(a, b);
  const bf16* kb = seq_ptr(a.k, a.cu, b, a.k_sb, a.k_st) + (int64_t)h * a.k_sh;
  const bf16* vb = seq_ptr(a.v, a.cu, b, a.v_sb, a.v_st) + (int64_t)h * a.v_sh;
  const FetchOffsets<kPfIT> fo = fetch_offsets<kPfIT>(a.k_st, a.v_st, wv, lane);
  tile_fetch<D, kPfIT>(sKs, sVs, kb, vb, a.k_st, a.v_st, c * a.bs, len, wv, lane, fo);

  const bf16* qb = seq_ptr(a.q, a.cu, b, a.q_sb, a.q_st) + (int64_t)h * a.q_sh;
  const int nkeys = min(a.bs, kPfIT);
  const int kfirst = c * a.bs;
  const int nrounds = npairs > wv * 32 ? (npairs - wv * 32 + 127) / 128 : 0;
  auto pair_id = [&](int j) {
    return wv * 32 + 128 * j + n < npairs ? pid_raw[j] : pid_first;
  };
  // a round's per-query inputs: Q rows, routed bias, segment start.  The Q rows
  // of the wavefront's 32 pairs are loaded row-contiguously, 16 lanes per row and
  // 4 rows per load (q[kk] of lane l: 16 bytes l % 16 of the row of pair 4 kk +
  // l / 16), and rearranged into the MFMA operand layout through LDS per round.
  struct RoundIn {
    bf16x8 q[D / 16];
    float bias;
    int km;
  };
  auto load_round = [&](int pid, RoundIn& in) {
    const int t = pid / a.K;                   // pid is in [0, len * K): see pids below
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const int tk = __shfl(t, 4 * kk + (lane >> 4), kWave);
      in.q[kk] = *(const bf16x8*)(qb + (int64_t)tk * a.q_st + (lane & 15) * 8);
    }
    in.bias = a.bias[r0 * a.K + pid];
    in.km = a.kmin ? a.kmin[r0 + t] : 0;
  };
  // Both rounds' inputs (pair ids, Q rows, biases) are loaded before the first
  // partial store: loads and stores share one counter on gfx9 and may complete
  // out of order, so a load issued before a store cannot be waited for alone.
  constexpr int kMaxRounds = kPfCH / 128;
  static_assert(kMaxRounds == 2, "two rounds of 128 pairs per chunk");
  int pids[kMaxRounds];
#pragma unroll
  for (int j = 0; j < kMaxRounds; ++j)
    pids[j] = j < nrounds ? min(max(pair_id(j), 0), len * a.K - 1) : 0;
  RoundIn inA, inB;
  if (nrounds > 0) load_round(pids[0], inA);
  if (nrounds > 1) load_round(pids[1], inB);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const bf16x2 ones = {(bf16)1.f, (bf16)1.f};

  bf16* const st = sTr + wv * 16 * D;
  auto round = [&](int j, const RoundIn& cur) {
    // Q^T operand of this lane's pair: rows pass through the wavefront's 16-row LDS
    // scratch in two pieces, 16-byte chunk c of row r at slot c ^ (r % 16)
    bf16x8 qop[D / 16];
#pragma unroll
    for (int piece = 0; piece < 2; ++piece) {
#pragma unroll
      for (int kk = 4 * piece; kk < 4 * piece + 4; ++kk) {
        const int rr = 4 * (kk - 4 * piece) + (lane >> 4);
        *(bf16x8*)(st + (rr * 16 + ((lane & 15) ^ rr)) * 8) = cur.q[kk];
      }
      wave_lds_sync();
      if ((n >> 4) == piece) {
        const int rr = n & 15;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk)
          qop[kk] = *(const bf16x8*)(st + (rr * 16 + ((2 * kk + hl) ^ rr)) * 8);
      }
      wave_lds_sync();
    }
    const int pid_cur = pids[j];
    const bool active = wv * 32 + 128 * j + n < npairs;
    const int t = pid_cur / a.K;
    const int q_ls = t - a.lw + 1;
    const int lo = cur.km;
    const int hi = min(q_ls, len) - 1;
    const uint32_t span = (active && hi >= lo) ? (uint32_t)(hi - lo) : 0u;
    const int lo_eff = (active && hi >= lo) ? lo : 0x40000000;
    const float bl = cur.bias * 1.4426950408889634f;
    floatx16 s[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[hf][r] = 0.f;
      if (32 * hf >= nkeys) continue;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        s[hf] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_frag(sKs, 32 * hf + n, kk, hl), qop[kk],
                                                        s[hf], 0, 0, 0);
    }
    float mraw = -INFINITY;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      if (32 * hf >= nkeys) continue;
      const int kq = kfirst + 32 * hf + 4 * hl - lo_eff;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t d = (uint32_t)(kq + 8 * (r >> 2) + (r & 3));
        mraw = fmaxf(mraw, d <= span ? s[hf][r] : -INFINITY);
      }
    }
    const float mloc = xor32_max(mraw == -INFINITY ? -INFINITY : fmaf(mraw, a.scale_log2e, bl));
    const float off = bl - (mloc == -INFINITY ? 0.f : mloc);
    floatx16 acc_o[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc_o[dt][r] = 0.f;
    float psum = 0.f;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      if (32 * hf >= nkeys) continue;
      const int kq = kfirst + 32 * hf + 4 * hl - lo_eff;
      bf16x8 pop[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t d = (uint32_t)(kq + 8 * (r >> 2) + (r & 3));
        const float pr = fast_exp2(fmaf(s[hf][r], a.scale_log2e, off));
        pop[r >> 3][r & 7] = (bf16)(d <= span ? pr : 0.f);
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int e2 = 0; e2 < 8; e2 += 2) {
          const bf16x2 pp = {pop[jj][e2], pop[jj][e2 + 1]};
          psum = __builtin_amdgcn_fdot2_f32_bf16(pp, ones, psum, false);
        }
      pv_tr_swz(sVs, 32 * hf, pop[0], acc_o, lane);
      pv_tr_swz(sVs, 32 * hf + 16, pop[1], acc_o, lane);
    }
    const float l_tot = xor32_sum(psum);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    // The row as bytes: the normalised values times 127 / (their largest magnitude),
    // rounded, plus 128 (lanes n and n + 32 hold the two halves of row n).
    float amax = 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) amax = fmaxf(amax, fabsf(acc_o[dt][r]));
    amax = xor32_max(amax) * inv;
    const float qk = amax > 0.f ? inv * (127.f / amax) : 0.f;
    const float qscale = amax * (1.f / 127.f);
    // The wavefront's 32 partial rows (consecutive positions) leave through LDS in
    // two pieces of 16 rows, so that every store instruction writes 1 KB
    // contiguously (whole 128-byte lines) instead of 16 bytes of 64 different
    // rows.  Rows of lanes past the chunk's pair count are written too: their
    // positions belong to this chunk and are never read.  In LDS, 16-byte chunk c
    // of row r sits at slot c ^ (r % 8): the rows a write instruction covers then
    // fall on distinct banks.
    const int64_t pw = part_row(a, (int64_t)(pb + ch) * kPfCH + wv * 32 + 128 * j, h);
    uint8_t* const stq = (uint8_t*)st;
#pragma unroll
    for (int piece = 0; piece < 2; ++piece) {
      if ((n >> 4) == piece) {
        const int rr = n & 15;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt) {
          uint32_t w4[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            uint32_t w = 0u;
#pragma unroll
            for (int e = 0; e < 4; ++e)
              w |= (uint32_t)fmaf(acc_o[dt][4 * q + e], qk, 128.5f) << (8 * e);
            w4[q] = w;
          }
          const int cidx = part_index(hl, dt, 0, 0) / 16;
          *(uint4*)(stq + rr * D + ((cidx ^ (rr & 7)) * 16)) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
      }
      wave_lds_sync();                     // other lanes' rows are read below
      char* const dst = (char*)(a.part_q + (pw + 16 * piece) * D);
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int rr = 8 * k + (lane >> 3), cidx = lane & 7;
        *(uint4*)(dst + k * 1024 + lane * 16) = *(const uint4*)(stq + rr * D + ((cidx ^ (rr & 7)) * 16));
      }
      wave_lds_sync();                     // and overwritten by the next piece
    }
    if (active && hl == 0)
      a.part_ls[pw + n] = make_float2(l_tot > 0.f ? mloc + log2f(l_tot) : -INFINITY, qscale);
  };
  if (nrounds > 0) round(0, inA);
  if (nrounds > 1) round(1, inB);
}

// Workspace layout of the hybrid plan (byte offsets, 256-byte aligned pieces).
// Slots of a row read and written four at a time: K a multiple of 4, ids and biases
// 16-byte aligned, validity 4-byte aligned (a row starts at row * K).
inline int slots_vectorizable(int K, const int32_t* idx, const uint8_t* valid,
                              const float* bias) {
  if (K <= 0 || K % 4 != 0) return 0;
  if ((uintptr_t)idx % 16 != 0 || (uintptr_t)bias % 16 != 0) return 0;
  if (valid && (uintptr_t)valid % 4 != 0) return 0;
  return 1;
}

struct PlanLayout {
  int64_t count, done, err, tbase, bch, nchunks, cpref, rec, kind, spos, plse, po, tpref,
      tdoc, total;
  int64_t ppos;
  int chunk_cap, ntiles_cap, ntv;
};

inline int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// Split tiles (no plan) when the grid of tiles (tiles per sequence x heads x
// sequences) is below kSplitSlots, one round of two work-groups on each of the 256
// CUs: the items per part are the fewest (from kSplitMinItems) whose parts over all
// tiles fit that round, so that the tiles with many remote blocks get more parts.
// Each part repeats the tile's prologue (its rows' routed lists, ~6 us), so parts
// stay above a few items.  A work-group finds its tile by walking the parts of the
// sequence's tiles (two divisions each), so sequences of more than kSplitMaxTiles
// tiles are not split.
constexpr int64_t kSplitSlots = 512;
constexpr int kSplitMinItems = 6;
constexpr int kSplitMaxTiles = 64;
inline int64_t seq_split_parts(int ntiles, int S, int lw, int bs, int K, int items) {
  int64_t n = 0;
  for (int t = 0; t < ntiles; ++t) n += tile_parts(t, S, lw, bs, K, items);
  return n;
}
// Items per part (0: no split) and the parts per (sequence, head).
inline int split_items_for(int ntiles, int64_t seqheads, int S, int lw, int bs, int K,
                           int64_t* parts) {
  *parts = ntiles;
  if (ntiles <= 0 || ntiles > kSplitMaxTiles || (int64_t)ntiles * seqheads >= kSplitSlots) return 0;
  int hi = 1;
  for (int t = 0; t < ntiles; ++t) hi = std::max(hi, tile_item_bound(t, S, lw, bs, K));
  if (hi <= kSplitMinItems) return 0;
  // parts decrease as the items per part grow: the smallest items in
  // [kSplitMinItems, hi] whose parts fit, else hi (kSplitMax parts at most per tile)
  int lo = kSplitMinItems, up = hi;
  while (lo < up) {
    const int mid = (lo + up) / 2;
    if (seq_split_parts(ntiles, S, lw, bs, K, mid) * seqheads <= kSplitSlots) up = mid; else lo = mid + 1;
  }
  const int64_t n = seq_split_parts(ntiles, S, lw, bs, K, lo);
  if (n <= ntiles) return 0;                 // one part per tile: no split
  *parts = n;
  return lo;
}
// Workspace of the split partials: bf16 rows, then the base-2 log-sum-exps, kSplitMax
// slots per tile.
inline int64_t split_o_bytes(int64_t tiles, int D) {
  return align256(tiles * kSplitMax * kPfTQ * D * 2);
}
inline int64_t split_bytes(int64_t tiles, int ntiles, int D) {
  return tiles < kSplitSlots && ntiles <= kSplitMaxTiles
             ? split_o_bytes(tiles, D) + align256(tiles * kSplitMax * kPfTQ * 4) : 0;
}

inline PlanLayout plan_layout(int B, int H, int S_max, int64_t rows, int K, int D,
                              int nblk_cap, int bs) {
  PlanLayout L;
  L.chunk_cap = (int)((int64_t)S_max * K / kPfCH) + nblk_cap + 1;
  L.ntiles_cap = (S_max + kPfTQ - 1) / kPfTQ;
  const int64_t nbc = (int64_t)B * nblk_cap;
  int64_t o = 0;
  L.count = o; o += nbc * 4;
  L.done = o;
  L.err = o + 4; o = align256(o + 8);
  L.tbase = o; o = align256(o + nbc * L.ntiles_cap * 4);
  L.bch = o; o = align256(o + nbc * 4);
  L.nchunks = o; o = align256(o + (int64_t)B * 4);
  L.cpref = o; o = align256(o + (int64_t)(B + 1) * 4);
  L.rec = o; o = align256(o + (int64_t)B * L.chunk_cap * kRec * 4);
  L.kind = o; o = align256(o + rows * K);
  L.spos = o; o = align256(o + rows * K * 4);
  // chunks over all sequences: at most (pairs / kPfCH) full ones plus one partly
  // filled chunk per block, and a sequence of len rows has ceil(len / bs) blocks
  L.ppos = (rows * K / kPfCH + rows / bs + B + 2) * kPfCH;
  L.plse = o; o = align256(o + L.ppos * H * 8);
  L.po = o; o = align256(o + L.ppos * H * D);
  // tiles of all sequences in one order: sum ceil(len / kPfTQ) <= (rows + (kPfTQ - 1) B) / kPfTQ
  L.ntv = (int)((rows + (int64_t)(kPfTQ - 1) * B) / kPfTQ) + 1;
  L.tpref = o; o = align256(o + (int64_t)(B + 1) * 4);
  L.tdoc = o; o = align256(o + (int64_t)L.ntv * 4);
  L.total = o;
  return L;
}

}  // namespace dash

#include "dash_prefill_bwd.h"

namespace dash {
// Workspace of the backward: the plan (as the forward's, every routed pair
// block-major), per (head, pair position) the fp32 bias-gradient partials and the
// scaled fp16 dQ partials with their scales (four 32-dim pieces a row), delta.
struct BwdLayout {
  PlanLayout P;
  int64_t pdb, pdq, pdqs, delta, total;
};

inline BwdLayout bwd_layout(int B, int H, int S_max, int64_t rows, int K, int D, int nblk_cap,
                            int bs) {
  BwdLayout L;
  L.P = plan_layout(B, H, S_max, rows, K, D, nblk_cap, bs);
  int64_t o = L.P.plse;                    // the forward's partials are not needed
  const int64_t nsub = (bs + 63) / 64;     // 64-key stages per block
  L.pdb = o; o = align256(o + L.P.ppos * H * nsub * 4);
  L.pdq = o; o = align256(o + L.P.ppos * H * nsub * (int64_t)D * 2);
  L.pdqs = o; o = align256(o + L.P.ppos * H * nsub * 4 * 4);
  L.delta = o; o = align256(o + rows * H * 4);
  L.total = o;
  return L;
}
}  // namespace dash

// ---------------------------------------------------------------------------
// C entry points
// ---------------------------------------------------------------------------
extern "C" int dash_attn_prefill_error_offset(int B, int H, int S_max, int64_t total_rows,
                                              int K, int D, int block_size, int64_t* offset) {
  using namespace dash;
  if (!offset || B < 0 || H <= 0 || S_max < 0 || total_rows < 0 || K < 0 || block_size <= 0)
    return kErrInvalid;
  const int nblk_cap = (S_max + block_size - 1) / block_size;
  *offset = plan_layout(B, H, S_max, total_rows, K, D, nblk_cap, block_size).err;
  return kOk;
}

extern "C" int dash_prefill_plan_target(int64_t chunk_cap, int64_t ppos, int64_t pos0,
                                        int64_t block_chunk, int64_t q, int64_t* rec_chunk,
                                        int64_t* pair_pos) {
  using namespace dash;
  if (!rec_chunk || !pair_pos) return kErrInvalid;
  return scatter_target(chunk_cap, ppos, pos0, block_chunk, q, rec_chunk, pair_pos) ? kOk
                                                                                    : kErrInvalid;
}

extern "C" int dash_attn_prefill_workspace_size(int B, int H, int S_max, int64_t total_rows,
                                                int K, int D, int block_size, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || H <= 0 || S_max < 0 || total_rows < 0 || K < 0 || block_size <= 0)
    return kErrInvalid;
  const int nblk_cap = (S_max + block_size - 1) / block_size;
  const int ntiles = (S_max + kPfTQ - 1) / kPfTQ;
  const int64_t tiles = (int64_t)ntiles * H * B;
  *bytes = std::max(plan_layout(B, H, S_max, total_rows, K, D, nblk_cap, block_size).total,
                    split_bytes(tiles, ntiles, D));
  return kOk;
}

extern "C" int dash_attn_prefill_split_workspace_size(int B, int H, int S_max, int D,
                                                      int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || H <= 0 || S_max < 0 || D <= 0) return kErrInvalid;
  const int ntiles = (S_max + kPfTQ - 1) / kPfTQ;
  const int64_t tiles = (int64_t)ntiles * H * B;
  *bytes = split_bytes(tiles, ntiles, D);
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
  if (K < 0 || K > kPfMaxSlots) return kErrUnsupported;
  // above 16 slots every routed pair goes through the block-major sparse kernel
  if (K > kPfMaxK) {
    if (block_size > kPfIT) return kErrUnsupported;
    if (dense_threshold <= 0) return kErrWorkspace;
    dense_threshold = kPfTQ + 1;
  }
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
  // the K/V stage loads form a row's byte offset inside a 64-key item in 32 bits
  if (k_st > kMaxKeyRowStride || v_st > kMaxKeyRowStride) return kErrUnsupported;
  PrefillArgs a = {};
  a.q = (const bf16*)q; a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.q_sb = q_sb; a.q_sh = q_sh; a.q_st = q_st;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st;
  a.o = (bf16*)o; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.lse = lse; a.lse_row = lse_row; a.lse_sh = lse_sh;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = K;
  a.cu = cu_seqlens; a.kmin = kmin;
  a.slots_vec = slots_vectorizable(K, idx, valid, bias);
  a.S = S; a.H = H; a.bs = block_size; a.lw = local_window; a.nblk_cap = nblk_cap;
  a.B = B;
  a.scale_log2e = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const int ntiles = (S + kPfTQ - 1) / kPfTQ;
  a.ntiles = ntiles;
  const bool hybrid = dense_threshold > 0 && K > 0 && block_size <= 64;
  if (hybrid) {
    if (total_rows <= 0) return kErrInvalid;
    // the plan's arrays hold total_rows rows: B * S without cu_seqlens (with them,
    // cu_seqlens[B], which the host does not read, is the caller's to pass)
    if (!cu_seqlens && total_rows != (int64_t)B * S) return kErrInvalid;
    const PlanLayout L = plan_layout(B, H, S, total_rows, K, D, nblk_cap, block_size);
    if (!workspace || workspace_bytes < L.total || (uintptr_t)workspace % 256 != 0)
      return kErrWorkspace;
    char* w = (char*)workspace;
    a.kind = (uint8_t*)(w + L.kind);
    a.dense_threshold = dense_threshold;
    a.blk_count = (int32_t*)(w + L.count);
    a.tile_base = (int32_t*)(w + L.tbase);
    a.ntiles_cap = L.ntiles_cap;
    a.blk_chunk = (int32_t*)(w + L.bch);
    a.num_chunks = (int32_t*)(w + L.nchunks);
    a.chunk_pref = (int32_t*)(w + L.cpref);
    a.done = (int32_t*)(w + L.done);
    a.err = (int32_t*)(w + L.err);
    a.chunk_rec = (int32_t*)(w + L.rec);
    a.chunk_cap = L.chunk_cap;
    a.spos = (int32_t*)(w + L.spos);
    a.ppos = L.ppos;
    a.part_ls = (float2*)(w + L.plse);
    a.part_q = (uint8_t*)(w + L.po);
    if (cu_seqlens) {
      a.tile_pref = (int32_t*)(w + L.tpref);
      a.tile_doc = (int32_t*)(w + L.tdoc);
      a.ntv = L.ntv;
    }
    const int ncount = (int)((L.err - L.count) / 4) + 1;  // block counters, arrival, error
    hipLaunchKernelGGL(prefill_clear_kernel, dim3((ncount + 255) / 256), dim3(256), 0, st,
                       a.blk_count, ncount);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(ntiles, B), dim3(kPfTQ), 0, st, a);
    hipLaunchKernelGGL(prefill_scan_kernel, dim3(B), dim3(1024), 0, st, a);
    hipLaunchKernelGGL(prefill_scatter_kernel, dim3(ntiles, B), dim3(kPfTQ), 0, st, a);
    hipLaunchKernelGGL(prefill_sparse_kernel<128>, dim3(L.chunk_cap * H * B), dim3(256), 0, st, a);
  }
  const int64_t tiles = (int64_t)ntiles * H * B;
  int64_t tile_grid = a.tile_doc ? (int64_t)a.ntv * H : tiles;
  if (!hybrid && K <= kPfMaxK && workspace && (uintptr_t)workspace % 256 == 0 &&
      workspace_bytes >= split_bytes(tiles, ntiles, D)) {
    // no plan: split the tiles of a grid too small to fill the chip (with a
    // workspace to hold the partials; without one every tile is one work-group)
    int64_t parts = 0;
    const int items = split_items_for(ntiles, (int64_t)H * B, S, local_window, block_size, K, &parts);
    if (items > 0) {
      a.split_items = items;
      a.split_parts = (int)parts;
      a.split_o = (bf16*)workspace;
      a.split_lse = (float*)((char*)workspace + split_o_bytes(tiles, D));
      tile_grid = parts * H * B;
    }
  }
  if (tile_grid > INT32_MAX) return kErrUnsupported;
  hipLaunchKernelGGL((prefill_tile_kernel<128, kTileIT, kTileOcc>), dim3((unsigned)tile_grid), dim3(256),
                     0, st, a);
  if (a.split_items > 0)
    hipLaunchKernelGGL(prefill_split_merge_kernel, dim3((unsigned)((tiles * kPfTQ + 15) / 16)), dim3(256),
                       0, st, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}

extern "C" int dash_attn_prefill_backward_workspace_size(int B, int H, int S_max,
                                                         int64_t total_rows, int K, int D,
                                                         int block_size, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || H <= 0 || S_max < 0 || total_rows < 0 || K < 0 || block_size <= 0)
    return kErrInvalid;
  const int nblk_cap = (S_max + block_size - 1) / block_size;
  *bytes = bwd_layout(B, H, S_max, total_rows, K, D, nblk_cap, block_size).total;
  return kOk;
}

extern "C" int dash_attn_prefill_backward(
    const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
    const void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
    const void* dout, int64_t do_sb, int64_t do_sh, int64_t do_st,
    const float* lse, int64_t lse_row, int64_t lse_sh,
    const int32_t* idx, const uint8_t* valid, const float* bias, int K,
    const int32_t* cu_seqlens, const int32_t* kmin,
    int B, int H, int S, int D, int block_size, int local_window, float scale,
    void* dq, int64_t dq_sb, int64_t dq_sh, int64_t dq_st,
    void* dk, int64_t dk_sb, int64_t dk_sh, int64_t dk_st,
    void* dv, int64_t dv_sb, int64_t dv_sh, int64_t dv_st,
    float* dbias, int64_t total_rows, void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace dash;
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv) return kErrInvalid;
  if (B < 0 || H <= 0 || S < 0 || total_rows < 0) return kErrInvalid;
  if (K > 0 && (!idx || !bias)) return kErrInvalid;
  if (D != 128) return kErrUnsupported;
  if (block_size <= 0 || block_size % 32 != 0 || block_size > 256) return kErrUnsupported;
  if (K < 0 || K > kPfMaxSlots) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if (B == 0 || S == 0) return kOk;
  // delta and the pair arrays hold total_rows rows: B * S without cu_seqlens (with them,
  // cu_seqlens[B], which the host does not read, is the caller's to pass)
  if (!cu_seqlens && total_rows != (int64_t)B * S) return kErrInvalid;
  const int nblk_cap = (S + block_size - 1) / block_size;
  if (nblk_cap > kPfMaxBlocks) return kErrUnsupported;
  const int64_t strides[] = {q_sb, q_sh, q_st, k_sb, k_sh, k_st, v_sb, v_sh, v_st, o_sb, o_sh, o_st,
                             do_sb, do_sh, do_st, dq_sb, dq_sh, dq_st, dk_sb, dk_sh, dk_st,
                             dv_sb, dv_sh, dv_st};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  // the key-major kernel forms the row offsets of Q and dO as 32 x 32-bit products
  if (q_st < 0 || q_st > INT32_MAX || do_st < 0 || do_st > INT32_MAX) return kErrUnsupported;
  // K/V stage loads as in the forward
  if (k_st > kMaxKeyRowStride || v_st > kMaxKeyRowStride) return kErrUnsupported;
  const void* ptrs[] = {q, k, v, o, dout, dq, dk, dv};
  for (const void* ptr : ptrs)
    if ((uintptr_t)ptr % 16 != 0) return kErrUnsupported;
  const BwdLayout L = bwd_layout(B, H, S, total_rows, K, D, nblk_cap, block_size);
  if (!workspace || workspace_bytes < L.total || (uintptr_t)workspace % 256 != 0)
    return kErrWorkspace;
  char* w = (char*)workspace;
  BwdArgs a = {};
  PrefillArgs& p = a.p;
  p.q = (const bf16*)q; p.k = (const bf16*)k; p.v = (const bf16*)v;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_st = q_st;
  p.k_sb = k_sb; p.k_sh = k_sh; p.k_st = k_st;
  p.v_sb = v_sb; p.v_sh = v_sh; p.v_st = v_st;
  p.idx = idx; p.valid = valid; p.bias = bias; p.K = K;
  p.cu = cu_seqlens; p.kmin = kmin;
  p.slots_vec = slots_vectorizable(K, idx, valid, bias);
  p.S = S; p.H = H; p.bs = block_size; p.lw = local_window; p.nblk_cap = nblk_cap;
  p.scale_log2e = scale * 1.4426950408889634f;
  p.ntiles = (S + kPfTQ - 1) / kPfTQ;
  p.B = B;
  a.o = (const bf16*)o; a.o_sb = o_sb; a.o_sh = o_sh; a.o_st = o_st;
  a.dout = (const bf16*)dout; a.do_sb = do_sb; a.do_sh = do_sh; a.do_st = do_st;
  a.lse = lse; a.lse_row = lse_row; a.lse_sh = lse_sh;
  a.dq = (bf16*)dq; a.dq_sb = dq_sb; a.dq_sh = dq_sh; a.dq_st = dq_st;
  a.dk = (bf16*)dk; a.dk_sb = dk_sb; a.dk_sh = dk_sh; a.dk_st = dk_st;
  a.dv = (bf16*)dv; a.dv_sb = dv_sb; a.dv_sh = dv_sh; a.dv_st = dv_st;
  a.dbias = dbias;
  a.scale = scale;
  a.nsub = (block_size + kBwIT - 1) / kBwIT;
  a.nstage = (int)(((int64_t)nblk_cap * block_size + kBwIT - 1) / kBwIT);
  a.delta = (float*)(w + L.delta);
  a.part_db = (float*)(w + L.pdb);
  a.part_dq = (_Float16*)(w + L.pdq);
  a.part_dqs = (float*)(w + L.pdqs);
  hipStream_t st = (hipStream_t)stream;
  const int64_t nitems = total_rows * H;
  if (nitems > 0)
    hipLaunchKernelGGL(bwd_delta_kernel, dim3((unsigned)((nitems * 16 + 255) / 256)), dim3(256), 0, st,
                       a, total_rows);
  if (K > 0) {
    p.kind = (uint8_t*)(w + L.P.kind);
    p.dense_threshold = kPfTQ + 1;         // no dense blocks: every routed pair block-major
    p.blk_count = (int32_t*)(w + L.P.count);
    p.tile_base = (int32_t*)(w + L.P.tbase);
    p.ntiles_cap = L.P.ntiles_cap;
    p.blk_chunk = (int32_t*)(w + L.P.bch);
    p.num_chunks = (int32_t*)(w + L.P.nchunks);
    p.chunk_pref = (int32_t*)(w + L.P.cpref);
    p.done = (int32_t*)(w + L.P.done);
    p.err = (int32_t*)(w + L.P.err);
    p.chunk_rec = (int32_t*)(w + L.P.rec);
    p.chunk_cap = L.P.chunk_cap;
    p.spos = (int32_t*)(w + L.P.spos);
    p.ppos = L.P.ppos;
    const int ncount = (int)((L.P.err - L.P.count) / 4) + 1;
    hipLaunchKernelGGL(prefill_clear_kernel, dim3((ncount + 255) / 256), dim3(256), 0, st,
                       p.blk_count, ncount);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(p.ntiles, B), dim3(kPfTQ), 0, st, p);
    hipLaunchKernelGGL(prefill_scan_kernel, dim3(B), dim3(1024), 0, st, p);
    hipLaunchKernelGGL(prefill_scatter_kernel, dim3(p.ntiles, B), dim3(kPfTQ), 0, st, p);
  }
  hipLaunchKernelGGL(bwd_kv_kernel, dim3(stream_stage_grid(B * H, a.nstage)), dim3(512), 0, st, a);
  hipLaunchKernelGGL(bwd_q_kernel, dim3(p.ntiles * H * B), dim3(256), 0, st, a);
  if (dbias && K > 0 && total_rows > 0)
    hipLaunchKernelGGL(bwd_dbias_kernel, dim3((unsigned)((total_rows * K + 255) / 256)), dim3(256), 0,
                       st, a, total_rows * K);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
