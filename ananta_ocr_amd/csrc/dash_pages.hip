// Page-aware routing candidates on gfx950: which key blocks a query may route to,
// from the token ids of an OCR prompt (image tokens grouped into pages by <PAGE>
// markers or by a fixed image-token count per page).
//
// Semantics follow the reference's candidate domain:
//   page ids       _build_page_aware_ids  (_sparse_base_impl.py:2189-2259)
//   prefill mask   _build_kl_candidate_mask / _build_page_aware_image_block_mask
//                  (_sparse_base_impl.py:2436-2484), as _dash_block_cand calls it
//                  (modeling_deepseekv2.py:96-110)
//   decode allow   _uocr_dash_decode_allow (modeling_anantaocr.py:450-496)
//
// Work decomposition: one 1024-thread work-group per prompt row scans the token ids
// (block-wide prefix sums of the marker and image counts, chunk by chunk); one
// wavefront per key block summarises the image pages it holds; one wavefront per
// query row writes its candidate row, four blocks per lane per store.  All of it is
// integer work on a few MB, bounded by latency rather than by HBM.

#include "dash_common.h"

namespace dash {

constexpr int kPgThreads = 1024;

// Inclusive prefix sum over the work-group of a packed pair of counts (high and low
// 32 bits; neither exceeds 2^31).  sWave holds one entry per wavefront.
__device__ __forceinline__ uint64_t block_incl_scan(uint64_t v, uint64_t* sWave, uint64_t& total) {
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
#pragma unroll
  for (int s = 1; s < kWave; s <<= 1) {
    const uint64_t o = __shfl_up(v, s, kWave);
    if (lane >= s) v += o;
  }
  if (lane == kWave - 1) sWave[wv] = v;
  __syncthreads();
  uint64_t base = 0, tot = 0;
  for (int w = 0; w < kPgThreads / kWave; ++w) {
    if (w < wv) base += sWave[w];
    tot += sWave[w];
  }
  __syncthreads();
  total = tot;
  return base + v;
}

__device__ __forceinline__ int block_max_int(int v, int* sRed) {
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, kWave));
  if (lane == 0) sRed[wv] = v;
  __syncthreads();
  int r = sRed[0];
  for (int w = 1; w < kPgThreads / kWave; ++w) r = max(r, sRed[w]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ int block_sum_int(int v, int* sRed) {
  const int lane = wave_lane(), wv = threadIdx.x / kWave;
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  if (lane == 0) sRed[wv] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < kPgThreads / kWave; ++w) r += sRed[w];
  __syncthreads();
  return r;
}

// Token rows are cut into chunks of up to kPgThreads tokens (a multiple of the block
// size, so that a chunk holds whole key blocks) and scanned in two launches: the
// summary kernel counts each chunk's markers and image tokens in parallel, then
// every chunk's work-group takes its prefix from the summaries of the chunks before
// it and finishes its tokens.  Summary of chunk k of row b, int32 x 4:
//   markers, image tokens, last image position in the row (-1: none),
//   markers at or before that last image position.
constexpr int kSumWords = 4;

__device__ __forceinline__ int chunk_tokens(int bs) {
  return bs <= kPgThreads ? (kPgThreads / bs) * bs : kPgThreads;
}

__global__ __launch_bounds__(kPgThreads) void page_summary_kernel(
    const int64_t* __restrict__ ids, int64_t ids_sb, int L, int64_t img_id, int64_t page_id,
    int chunk, int nchunks, int32_t* __restrict__ summ, int32_t* __restrict__ enabled) {
  __shared__ int sRed[kPgThreads / kWave];
  const int k = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  if (enabled && k == 0 && tid == 0) enabled[2 * b + 1] = 0;    // set by page_ids_kernel
  const int t = k * chunk + tid;
  const bool live = tid < chunk && t < L;
  const int64_t id = live ? ids[(int64_t)b * ids_sb + t] : -1;
  const bool im = live && id == img_id, mk = live && id == page_id;
  const int nmk = block_sum_int(mk ? 1 : 0, sRed);
  const int nim = block_sum_int(im ? 1 : 0, sRed);
  const int last = block_max_int(im ? t : -1, sRed);
  const int mk_upto = block_sum_int((mk && t <= last) ? 1 : 0, sRed);
  if (tid == 0) {
    int32_t* o = summ + ((int64_t)b * nchunks + k) * kSumWords;
    o[0] = nmk; o[1] = nim; o[2] = last; o[3] = mk_upto;
  }
}

// Prefix of chunk k from the summaries, by wavefront 0: markers and image tokens
// before the chunk, the row's image-token count, last image position and prompt
// page count (markers at or before the last image token).
struct ChunkPrefix {
  int mk, im, nimg, last, prompt_pages;
};

__device__ __forceinline__ ChunkPrefix chunk_prefix(const int32_t* summ, int b, int k,
                                                    int nchunks, ChunkPrefix* sOut) {
  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    const int32_t* row = summ + (int64_t)b * nchunks * kSumWords;
    int mk = 0, im = 0, nimg = 0, last = -1, kl = -1;
    for (int j = lane; j < nchunks; j += kWave) {
      const int4 v = *(const int4*)(row + j * kSumWords);
      if (j < k) { mk += v.x; im += v.y; }
      nimg += v.y;
      if (v.z > last) { last = v.z; kl = j; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      mk += __shfl_xor(mk, m, kWave);
      im += __shfl_xor(im, m, kWave);
      nimg += __shfl_xor(nimg, m, kWave);
      const int ol = __shfl_xor(last, m, kWave), ok = __shfl_xor(kl, m, kWave);
      if (ol > last) { last = ol; kl = ok; }
    }
    // markers before the chunk of the last image token, plus its markers up to it
    int pre = 0;
    for (int j = lane; j < kl; j += kWave) pre += row[j * kSumWords];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) pre += __shfl_xor(pre, m, kWave);
    if (lane == 0)
      *sOut = ChunkPrefix{mk, im, nimg, last, kl >= 0 ? pre + row[kl * kSumWords + 3] : 0};
  }
  __syncthreads();
  return *sOut;
}

// Page ids of one chunk of a prompt row (_sparse_base_impl.py:2189-2225):
//   cum_pages[t]  = number of <PAGE> markers at positions <= t
//   last_img      = last image-token position (-1: none)
//   prompt_pages  = cum_pages[last_img] (0 without an image token)
//   marker mode   = prompt_pages > 0
//   image page    = marker mode ? cum_pages - 1 : (image tokens before t) / per_page, -1 off images
//   query page    = t <= last_img ? cum_pages - 1 : cum_pages - 1 - (marker mode ? prompt_pages : 0),
//                   -1 inside the prompt unless page_scope_prefill, -1 when negative
// enabled[b] = (row has an image token, row has a query page): chunk 0 writes the first;
// the summary kernel clears the second and any chunk with a query page sets it.
__global__ __launch_bounds__(kPgThreads) void page_ids_kernel(
    const int64_t* __restrict__ ids, int64_t ids_sb, int L, int64_t img_id, int64_t page_id,
    int per_page, int page_scope_prefill, int chunk, int nchunks,
    const int32_t* __restrict__ summ, uint8_t* __restrict__ img_mask,
    int32_t* __restrict__ img_page, int32_t* __restrict__ q_page, int32_t* __restrict__ enabled) {
  __shared__ uint64_t sWave[kPgThreads / kWave];
  __shared__ int sRed[kPgThreads / kWave];
  __shared__ ChunkPrefix sPre;
  const int k = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const ChunkPrefix pre = chunk_prefix(summ, b, k, nchunks, &sPre);
  const bool marker_mode = pre.prompt_pages > 0;
  const int t = k * chunk + tid;
  const bool live = tid < chunk && t < L;
  const int64_t id = live ? ids[(int64_t)b * ids_sb + t] : -1;
  const bool im = live && id == img_id, mk = live && id == page_id;
  uint64_t tot;
  const uint64_t inc = block_incl_scan(((uint64_t)mk << 32) | (uint64_t)im, sWave, tot);
  const int cum = pre.mk + (int)(inc >> 32), run = pre.im + (int)(inc & 0xffffffffu);
  int qp = -1;
  if (live) {
    int ip = -1;
    if (im) ip = marker_mode ? cum - 1 : (run - 1) / per_page;
    const int raw = cum - 1;
    const bool in_pre = t <= pre.last;
    qp = in_pre ? raw : raw - (marker_mode ? pre.prompt_pages : 0);
    if (in_pre && !page_scope_prefill) qp = -1;
    if (qp < 0) qp = -1;
    const int64_t o = (int64_t)b * L + t;
    img_mask[o] = im ? 1 : 0;
    img_page[o] = ip;
    q_page[o] = qp;
  }
  const int anyq = block_sum_int(qp >= 0 ? 1 : 0, sRed);
  if (tid == 0 && enabled) {
    if (k == 0) enabled[2 * b] = pre.nimg > 0 ? 1 : 0;
    if (anyq > 0) enabled[2 * b + 1] = 1;
  }
}

// The image pages of key block c of row b: smallest and largest page id (-1, -1 with no
// image token) and a bit per page bmin .. bmin + 63 present in the block.
__global__ __launch_bounds__(kWave) void block_pages_kernel(
    const int32_t* __restrict__ img_page, int64_t ip_sb, int L, int bs, int nblk,
    int32_t* __restrict__ bmin, int32_t* __restrict__ bmax, uint64_t* __restrict__ bits) {
  const int c = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int32_t* row = img_page + (int64_t)b * ip_sb;
  const int j0 = c * bs, j1 = min(j0 + bs, L);
  int mn = 0x7fffffff, mx = -1;
  for (int j = j0 + lane; j < j1; j += kWave) {
    const int p = row[j];
    if (p >= 0) { mn = min(mn, p); mx = max(mx, p); }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    mn = min(mn, __shfl_xor(mn, m, kWave));
    mx = max(mx, __shfl_xor(mx, m, kWave));
  }
  uint64_t bt = 0;
  if (mx >= 0)
    for (int j = j0 + lane; j < j1; j += kWave) {
      const int p = row[j];
      if (p >= 0 && p - mn < 64) bt |= 1ull << (p - mn);
    }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)bt, m, kWave);
    const uint32_t hi = __shfl_xor((uint32_t)(bt >> 32), m, kWave);
    bt |= ((uint64_t)hi << 32) | lo;
  }
  if (lane == 0) {
    const int64_t o = (int64_t)b * nblk + c;
    bmin[o] = mx >= 0 ? mn : -1;
    bmax[o] = mx;
    bits[o] = bt;
  }
}

// Does key block c hold an image token of page qp?  Pages within bmin + 63 are in the
// bits; wider blocks (more than 64 page ids apart) are scanned.
__device__ __forceinline__ bool block_has_page(int qp, int mn, int mx, uint64_t bt,
                                               const int32_t* ip_row, int j0, int j1) {
  if (qp < 0 || mx < 0 || qp < mn || qp > mx) return false;
  if (qp - mn < 64) return ((bt >> (qp - mn)) & 1ull) != 0;
  for (int j = j0; j < j1; ++j)
    if (ip_row[j] == qp) return true;
  return false;
}

// Candidate row of each query: one work-group per 32 query rows of one sequence,
// the sequence's block summaries staged in LDS, one wavefront per row at a time.  A
// wavefront loads the positions and pages of its 8 rows up front (lane r for row r);
// for a row, lane l tests blocks l, l + 64, ... (neighbouring LDS entries) into a
// per-wavefront LDS copy of the row, shifted by the row's misalignment so that it
// then leaves in aligned 4-byte words (byte stores only for the words the row
// shares with its neighbours):
//   mode 0  blocks holding an image token of the query's page (query page = q_page[pos])
//   mode 1  blocks holding any image token (every query the same)
//   mode 2  every block
// and a row with no candidate opens to every block (the reference's per-query fallback).
constexpr int kCandRows = 32;
constexpr int kCandMaxBlocks = 2048;

__global__ __launch_bounds__(256) void block_cand_kernel(
    const int32_t* __restrict__ q_page, int64_t qp_sb, int Lqp, const int32_t* __restrict__ pos,
    int64_t pos_sb, int Lq, const int32_t* __restrict__ img_page, int64_t ip_sb, int Lk,
    const int32_t* __restrict__ bmin, const int32_t* __restrict__ bmax,
    const uint64_t* __restrict__ bits, int nblk, int mode, int bs, uint8_t* __restrict__ cand,
    int64_t cand_sb, int64_t cand_st) {
  constexpr int kWaves = 256 / kWave, kPerWave = kCandRows / kWaves;
  __shared__ int4 sBlk[kCandMaxBlocks];            // bmin, bmax, bits (lo, hi)
  __shared__ __attribute__((aligned(16))) uint8_t sRow[kWaves][kCandMaxBlocks + 8];
  const int lane = wave_lane(), wv = threadIdx.x / kWave, b = blockIdx.y;
  const int64_t bo = (int64_t)b * nblk;
  if (mode != 2)
    for (int c = threadIdx.x; c < nblk; c += 256) {
      const uint64_t bt = mode == 0 ? bits[bo + c] : 0ull;
      sBlk[c] = make_int4(mode == 0 ? bmin[bo + c] : 0, bmax[bo + c], (int)(uint32_t)bt,
                          (int)(uint32_t)(bt >> 32));
    }
  // this wavefront's rows and their query pages, loaded together
  const int t0 = blockIdx.x * kCandRows + wv * kPerWave;
  int my_qp = -1;
  if (mode == 0 && lane < kPerWave && t0 + lane < Lq) {
    const int p = pos ? pos[(int64_t)b * pos_sb + t0 + lane] : t0 + lane;
    my_qp = q_page[(int64_t)b * qp_sb + min(max(p, 0), Lqp - 1)];
  }
  __syncthreads();
  const int32_t* ipr = img_page ? img_page + (int64_t)b * ip_sb : nullptr;
  uint8_t* srow = sRow[wv];
  for (int r = 0; r < kPerWave; ++r) {
    const int t = t0 + r;
    if (t >= Lq) break;
    const int qp = __shfl(my_qp, r, kWave);
    uint8_t* row = cand + (int64_t)b * cand_sb + (int64_t)t * cand_st;
    const int m = (int)((uintptr_t)row & 3);
    uint8_t* base = row - m;                        // 4-byte aligned
    bool a = false;
    for (int c = lane; c < nblk; c += kWave) {
      bool v = true;
      if (mode != 2) {
        const int4 e = sBlk[c];
        if (mode == 1) {
          v = e.y >= 0;
        } else {
          const uint64_t bt = ((uint64_t)(uint32_t)e.w << 32) | (uint32_t)e.z;
          v = block_has_page(qp, e.x, e.y, bt, ipr, c * bs, min(c * bs + bs, Lk));
        }
      }
      a |= v;
      srow[m + c] = v ? 1 : 0;
    }
    const bool any = __any(a);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int nwords = (m + nblk + 3) / 4;
    for (int i = lane; i < nwords; i += kWave) {
      const int c0 = 4 * i - m;
      const uint32_t word = any ? *(const uint32_t*)(srow + 4 * i) : 0x01010101u;
      if (c0 >= 0 && c0 + 3 < nblk) {
        *(uint32_t*)(base + 4 * i) = word;
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (c0 + u >= 0 && c0 + u < nblk) base[4 * i + u] = (uint8_t)((word >> (8 * u)) & 1u);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Decode page state of a chunk of a prompt row (modeling_anantaocr.py:465-479): per
// token the page cum - 1 once a marker has been seen, else (image tokens before it) /
// per_page, -1 off images; per key block of the chunk the smallest and largest of
// those (-1, -1 with none).  Chunk 0 writes the row's prompt page count (markers up
// to the last image token) and marker count; blocks past the row are cleared.
__global__ __launch_bounds__(kPgThreads) void decode_page_state_kernel(
    const int64_t* __restrict__ ids, int64_t ids_sb, int L, int64_t img_id, int64_t page_id,
    int per_page, int bs, int nblk, int chunk, int nchunks, const int32_t* __restrict__ summ,
    int32_t* __restrict__ bmin, int32_t* __restrict__ bmax, int32_t* __restrict__ prompt_pages,
    int32_t* __restrict__ markers) {
  __shared__ uint64_t sWave[kPgThreads / kWave];
  __shared__ int sMin[kPgThreads], sMax[kPgThreads];
  __shared__ ChunkPrefix sPre;
  const int k = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int64_t bo = (int64_t)b * nblk;
  const ChunkPrefix pre = chunk_prefix(summ, b, k, nchunks, &sPre);
  const int t = k * chunk + tid;
  const bool live = tid < chunk && t < L;
  const int64_t id = live ? ids[(int64_t)b * ids_sb + t] : -1;
  const bool im = live && id == img_id, mk = live && id == page_id;
  uint64_t tot;
  const uint64_t inc = block_incl_scan(((uint64_t)mk << 32) | (uint64_t)im, sWave, tot);
  const int cum = pre.mk + (int)(inc >> 32), run = pre.im + (int)(inc & 0xffffffffu);
  int page = -1;
  if (im) page = cum > 0 ? cum - 1 : (run - 1) / per_page;
  sMin[tid] = page >= 0 ? page : 0x7fffffff;
  sMax[tid] = page;
  __syncthreads();
  const int nb = chunk / bs;                 // whole blocks per chunk (bs <= kPgThreads)
  if (tid < nb) {
    const int c = k * nb + tid;
    if (c < nblk && c * bs < L) {
      int mn = 0x7fffffff, mx = -1;
      for (int j = tid * bs; j < tid * bs + bs; ++j) { mn = min(mn, sMin[j]); mx = max(mx, sMax[j]); }
      bmin[bo + c] = mx >= 0 ? mn : -1;
      bmax[bo + c] = mx;
    }
  }
  if (k == 0) {
    for (int c = (L + bs - 1) / bs + tid; c < nblk; c += kPgThreads) { bmin[bo + c] = -1; bmax[bo + c] = -1; }
    if (tid == 0) {
      prompt_pages[b] = pre.prompt_pages;
      int tot_mk = 0;
      for (int j = 0; j < nchunks; ++j) tot_mk += summ[((int64_t)b * nchunks + j) * kSumWords];
      markers[b] = tot_mk;
    }
  }
}

// Decode allow row (modeling_anantaocr.py:480-496): the new token's marker updates the
// count; the query page is markers - 1 - prompt_pages (-1 when negative); a block is
// allowed if bmin <= page <= bmax; a row with no such block (or no page) allows all.
__global__ __launch_bounds__(256) void decode_allow_kernel(
    const int64_t* __restrict__ new_ids, int64_t new_stride, int64_t page_id,
    const int32_t* __restrict__ bmin, const int32_t* __restrict__ bmax, int nblk_state,
    const int32_t* __restrict__ prompt_pages, int32_t* __restrict__ markers, int nblk,
    uint8_t* __restrict__ allow, int64_t allow_sb) {
  __shared__ int sAny;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int m = markers[b] + (new_ids[(int64_t)b * new_stride] == page_id ? 1 : 0);
  int qp = m - 1 - prompt_pages[b];
  if (qp < 0) qp = -1;
  if (tid == 0) sAny = 0;
  __syncthreads();
  const int64_t bo = (int64_t)b * nblk_state;
  bool a = false;
  for (int c = tid; c < min(nblk, nblk_state); c += 256) {
    const int mn = bmin[bo + c], mx = bmax[bo + c];
    a |= qp >= 0 && mn >= 0 && mn <= qp && mx >= qp;
  }
  if (a) sAny = 1;
  __syncthreads();
  const bool open = qp < 0 || sAny == 0;
  for (int c = tid; c < nblk; c += 256) {
    bool s = false;
    if (c < nblk_state) {
      const int mn = bmin[bo + c], mx = bmax[bo + c];
      s = qp >= 0 && mn >= 0 && mn <= qp && mx >= qp;
    }
    allow[(int64_t)b * allow_sb + c] = (s || open) ? 1 : 0;
  }
  __syncthreads();
  if (tid == 0) markers[b] = m;
}


// ---------------------------------------------------------------------------
// Window bounds of decode rows (the serving router's _win_bounds_kernel,
// whl:sglang/srt/layers/attention/unlimited_dash_ops/route_triton.py:466-505, for
// one decode query per sequence): the span [lo, hi) of the blocks that are allowed
// and remote (c <= q_blk - local_blocks, c * bs < len); with none, the live remote
// width [0, ceil(len / bs)) (or [0, 0) when no block is remote); fit = the span is at
// most `tile` blocks wide.  One work-group of 256 threads per sequence.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void win_bounds_kernel(const uint8_t* __restrict__ allow,
                                                         int64_t allow_sb, int allow_w,
                                                         const int32_t* __restrict__ lens,
                                                         const int32_t* __restrict__ q_pos, int S,
                                                         int nblk_cap, int bs, int local_blocks,
                                                         int tile, int32_t* __restrict__ bounds,
                                                         uint8_t* __restrict__ fit) {
  __shared__ int s_lo[256 / kWave], s_hi[256 / kWave];
  const int b = blockIdx.x, tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int len = lens ? min(max(lens[b], 0), S) : S;
  const int qp = q_pos ? min(q_pos[b], len - 1) : len - 1;
  const int q_blk = qp >= 0 ? qp / bs : -1;
  const int lim = q_blk - local_blocks;
  const int w = min(nblk_cap, allow_w);
  int lo = nblk_cap, hi = -1;
  for (int c = tid; c < w; c += 256) {
    const bool keep = allow[(int64_t)b * allow_sb + c] != 0 && c <= lim && (int64_t)c * bs < len;
    if (keep) { lo = min(lo, c); hi = max(hi, c); }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    lo = min(lo, __shfl_xor(lo, m, kWave));
    hi = max(hi, __shfl_xor(hi, m, kWave));
  }
  if (lane == 0) { s_lo[wv] = lo; s_hi[wv] = hi; }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < 256 / kWave; ++i) { lo = min(lo, s_lo[i]); hi = max(hi, s_hi[i]); }
    lo = min(lo, s_lo[0]); hi = max(hi, s_hi[0]);
    const bool any_r = hi >= 0;
    const int n_blk = (len + bs - 1) / bs;
    const int w_seq = min(nblk_cap, max(n_blk, 1));
    const bool no_remote = len <= 0 || lim < 0;
    const int lo_v = any_r ? lo : 0;
    const int hi_v = any_r ? hi + 1 : (no_remote ? 0 : w_seq);
    bounds[2 * b] = lo_v;
    bounds[2 * b + 1] = hi_v;
    if (fit) fit[b] = (hi_v - lo_v) <= tile ? 1 : 0;
  }
}


// ---------------------------------------------------------------------------------
// Page2D RoPE coordinates (_build_page_rope_pos / _page_rope_offsets,
// _sparse_base_impl.py:2269-2362).  Per prompt row, with cum[t] = <PAGE> markers at
// positions <= t, last = the last image-token position and n = cum[last] (the prompt's
// pages):
//   page[t] = t <= last ? cum[t] : cum[t] - n       (page 0 = the text before the first
//                                                    marker and after the last image)
//   tok[t]  = (tokens at positions <= t with the same page) - 1
// Up to `last` the page never decreases and page p spans [m_p, m_{p+1}) (m_p = the p-th
// marker, m_0 = 0); after `last` page p spans the p-th to (p+1)-th marker after it (from
// last + 1 for page 0), and its count continues from the prefill count
//   pf[p] = min(m_{p+1}, last + 1) - m_p   (p <= n; 0 for later pages).
// So a token's count is its distance from the start of its run plus, after `last`, pf of
// its page, which needs only the marker positions: the page kernel writes page ids and
// every marker's position (mpos[cum - 1] = t), the count kernel the counts, pf and the
// optional span scaling, the meta kernel the batch's page count and whether every row
// has a marker at or before its last image token (else the reference falls back to 1-D).

__device__ __forceinline__ int64_t rope_pf(const int32_t* mpos, int n, int last, int64_t p) {
  if (p < 0 || p > n) return 0;
  const int64_t end = p < n ? (int64_t)mpos[p] : (int64_t)last + 1;
  const int64_t start = p == 0 ? 0 : (int64_t)mpos[p - 1];
  return end - start;
}

__global__ __launch_bounds__(kPgThreads) void rope_page_kernel(
    const int64_t* __restrict__ ids, int64_t ids_sb, int L, int64_t img_id, int64_t page_id,
    int chunk, int nchunks, const int32_t* __restrict__ summ, int64_t* __restrict__ page,
    int32_t* __restrict__ mpos) {
  __shared__ uint64_t sWave[kPgThreads / kWave];
  __shared__ ChunkPrefix sPre;
  const int k = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const ChunkPrefix pre = chunk_prefix(summ, b, k, nchunks, &sPre);
  const int t = k * chunk + tid;
  const bool live = tid < chunk && t < L;
  const int64_t id = live ? ids[(int64_t)b * ids_sb + t] : -1;
  const bool mk = live && id == page_id;
  uint64_t tot;
  const uint64_t inc = block_incl_scan((uint64_t)mk, sWave, tot);
  const int cum = pre.mk + (int)inc;
  if (live) {
    const int n = pre.last >= 0 ? pre.prompt_pages : 0;
    page[(int64_t)b * L + t] = t <= pre.last ? cum : cum - n;
    if (mk) mpos[(int64_t)b * L + cum - 1] = t;
  }
}

__global__ __launch_bounds__(kPgThreads) void rope_tok_kernel(
    int L, int chunk, int nchunks, const int32_t* __restrict__ summ,
    const int64_t* __restrict__ page, const int32_t* __restrict__ mpos, int span,
    int64_t* __restrict__ tok, int64_t* __restrict__ pf_cnt, int64_t pf_stride) {
  __shared__ ChunkPrefix sPre;
  const int k = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const ChunkPrefix pre = chunk_prefix(summ, b, k, nchunks, &sPre);
  const int last = pre.last;
  const int n = last >= 0 ? pre.prompt_pages : 0;
  const int32_t* mp = mpos + (int64_t)b * L;
  const int t = k * chunk + tid;
  if (tid < chunk && t < L) {
    const int64_t pg = page[(int64_t)b * L + t];
    const bool in_pre = t <= last;
    const int64_t cum = in_pre ? pg : pg + n;
    const int lastmk = cum > 0 ? mp[cum - 1] : -1;
    const int seg0 = in_pre ? max(lastmk, 0) : max(lastmk, last + 1);
    const int64_t run = (int64_t)(t - seg0);
    const int64_t pfk = rope_pf(mp, n, last, pg);
    int64_t tk = in_pre ? run : pfk + run;
    if (span > 0 && pg > 0) {
      if (in_pre) {
        // round(tok * span / max(pf, 1)) in fp32, half to even, as torch.round
        const float x = __fdiv_rn(__fmul_rn((float)tk, (float)span), (float)max(pfk, (int64_t)1));
        tk = (int64_t)rintf(x);
      } else {
        tk = (int64_t)span + (tk - pfk);
      }
    }
    tok[(int64_t)b * L + t] = tk;
  }
  // the prefill count of every page id 0 .. L (the row's pages are at most L + 1)
  for (int64_t p = (int64_t)k * chunk + tid; p <= L; p += (int64_t)chunk * nchunks)
    if (tid < chunk) pf_cnt[(int64_t)b * pf_stride + p] = rope_pf(mp, n, last, p);
}

// meta[0] = 1 + the largest page id of any row; meta[1] = 1 if every row has a marker at
// or before its last image token (then it also has an image token and a marker).
__global__ __launch_bounds__(kWave) void rope_meta_kernel(int B, int nchunks,
                                                          const int32_t* __restrict__ summ,
                                                          int64_t* __restrict__ meta) {
  const int lane = threadIdx.x;
  int maxpg = 0, ok = 1;
  for (int b = 0; b < B; ++b) {
    const int32_t* row = summ + (int64_t)b * nchunks * kSumWords;
    int total = 0, last = -1, kl = -1;
    for (int j = lane; j < nchunks; j += kWave) {
      total += row[j * kSumWords];
      const int lj = row[j * kSumWords + 2];
      if (lj > last) { last = lj; kl = j; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      total += __shfl_xor(total, m, kWave);
      const int ol = __shfl_xor(last, m, kWave), ok2 = __shfl_xor(kl, m, kWave);
      if (ol > last) { last = ol; kl = ok2; }
    }
    int pre = 0;
    for (int j = lane; j < kl; j += kWave) pre += row[j * kSumWords];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) pre += __shfl_xor(pre, m, kWave);
    const int n = kl >= 0 ? pre + row[kl * kSumWords + 3] : 0;
    maxpg = max(maxpg, max(n, total - n));
    if (n <= 0) ok = 0;
  }
  if (lane == 0) {
    meta[0] = (int64_t)maxpg + 1;
    meta[1] = ok;
  }
}

// cos / sin of the two-axis RoPE (DeepseekV2IndexerRotary2D.forward,
// _sparse_base_impl.py:1876-1891): frequency pair j < n_tok turns with the token
// coordinate, pair n_tok + i with the page coordinate (mod page_mod when > 0); both
// halves of the row repeat the pairs (cat(ang, ang)).  Angles and cos/sin in fp32, then
// the output dtype.  One thread per (token, pair).
__global__ __launch_bounds__(256) void rope2d_cos_sin_kernel(
    const int64_t* __restrict__ tok, const int64_t* __restrict__ page, int64_t pos_sb, int S,
    int64_t rows, const float* __restrict__ inv_tok, int n_tok, const float* __restrict__ inv_page,
    int half, int page_mod, void* __restrict__ cos_out, void* __restrict__ sin_out, int out_bf16,
    int64_t cs_sb, int64_t cs_st) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * half) return;
  const int64_t r = i / half;
  const int j = (int)(i - r * half);
  const int64_t b = r / S, t = r - b * S;
  float ang;
  if (j < n_tok) {
    ang = __fmul_rn((float)tok[b * pos_sb + t], inv_tok[j]);
  } else {
    int64_t p = page[b * pos_sb + t];
    if (page_mod > 0) {
      p %= page_mod;
      if (p < 0) p += page_mod;
    }
    ang = __fmul_rn((float)p, inv_page[j - n_tok]);
  }
  float sv, cv;
  sincosf(ang, &sv, &cv);
  const int64_t o = b * cs_sb + t * cs_st;
  if (out_bf16) {
    bf16* c = (bf16*)cos_out + o;
    bf16* s = (bf16*)sin_out + o;
    c[j] = (bf16)cv; c[j + half] = (bf16)cv;
    s[j] = (bf16)sv; s[j + half] = (bf16)sv;
  } else {
    float* c = (float*)cos_out + o;
    float* s = (float*)sin_out + o;
    c[j] = cv; c[j + half] = cv;
    s[j] = sv; s[j + half] = sv;
  }
}

// One decode token per row advances the page coordinates (_main_rope_coords decode branch,
// _sparse_base_impl.py:1384-1390): a <PAGE> token moves to the next page (at most the last
// page id of the prompt, meta[0] - 1) and restarts at that page's prefill count; any
// other token counts one further.  state page/tok [B] are updated; the new coordinates are
// also written to out_tok / out_page [B].
__global__ __launch_bounds__(256) void rope_advance_kernel(
    const int64_t* __restrict__ new_ids, int64_t new_stride, int B, int64_t page_id,
    int64_t* __restrict__ page, int64_t* __restrict__ tok, const int64_t* __restrict__ pf_cnt,
    int64_t pf_stride, const int64_t* __restrict__ meta, int64_t* __restrict__ out_tok,
    int64_t* __restrict__ out_page) {
  const int b = blockIdx.x * 256 + threadIdx.x;
  if (b >= B) return;
  const bool is_pg = new_ids[(int64_t)b * new_stride] == page_id;
  int64_t pg = page[b];
  int64_t tk = tok[b];
  if (is_pg) {
    pg = min(pg + 1, meta[0] - 1);
    tk = pf_cnt[(int64_t)b * pf_stride + max(pg, (int64_t)0)];
  } else {
    tk = tk + 1;
  }
  page[b] = pg;
  tok[b] = tk;
  if (out_tok) out_tok[b] = tk;
  if (out_page) out_page[b] = pg;
}

}  // namespace dash

namespace {
inline int pages_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? dash::kOk : (int)e;
}
}  // namespace

extern "C" int dash_pages_workspace_size(int B, int L, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || L < 0) return kErrInvalid;
  // chunks hold at least 513 tokens (or 512 with a block size up to 512)
  *bytes = (int64_t)B * ((L + 511) / 512 + 1) * kSumWords * (int64_t)sizeof(int32_t);
  return kOk;
}

namespace {
int page_summaries(const int64_t* ids, int64_t ids_sb, int B, int L, int64_t img_id,
                   int64_t page_id, int chunk, void* workspace, int64_t workspace_bytes,
                   int32_t* enabled, hipStream_t st, int* nchunks_out) {
  using namespace dash;
  const int nchunks = (L + chunk - 1) / chunk;
  int64_t need = 0;
  dash_pages_workspace_size(B, L, &need);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0) return kErrWorkspace;
  if (B > 65535) return kErrUnsupported;
  hipLaunchKernelGGL(page_summary_kernel, dim3(nchunks, B), dim3(kPgThreads), 0, st, ids, ids_sb,
                     L, img_id, page_id, chunk, nchunks, (int32_t*)workspace, enabled);
  *nchunks_out = nchunks;
  return kOk;
}
}  // namespace

extern "C" int dash_page_ids(const int64_t* ids, int64_t ids_sb, int B, int L,
                             int64_t image_token_id, int64_t page_token_id, int per_page_tokens,
                             int page_scope_prefill, uint8_t* image_mask, int32_t* image_page_ids,
                             int32_t* query_page_ids, int32_t* enabled, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  using namespace dash;
  if (B < 0 || L < 0 || per_page_tokens < 1) return kErrInvalid;
  if (B == 0 || L == 0) return kOk;
  if (!ids || !image_mask || !image_page_ids || !query_page_ids) return kErrInvalid;
  hipStream_t st = (hipStream_t)stream;
  int nchunks = 0;
  const int rs = page_summaries(ids, ids_sb, B, L, image_token_id, page_token_id, kPgThreads,
                                workspace, workspace_bytes, enabled, st, &nchunks);
  if (rs != kOk) return rs;
  hipLaunchKernelGGL(page_ids_kernel, dim3(nchunks, B), dim3(kPgThreads), 0, st, ids, ids_sb, L,
                     image_token_id, page_token_id, per_page_tokens, page_scope_prefill, kPgThreads,
                     nchunks, (const int32_t*)workspace, image_mask, image_page_ids, query_page_ids,
                     enabled);
  return pages_status();
}

extern "C" int dash_block_pages(const int32_t* image_page_ids, int64_t ipi_sb, int B, int L,
                                int block_size, int nblk, int32_t* bmin, int32_t* bmax,
                                uint64_t* bits, void* stream) {
  using namespace dash;
  if (B < 0 || L < 0 || nblk < 0 || block_size <= 0) return kErrInvalid;
  if (B == 0 || nblk == 0) return kOk;
  if (!image_page_ids || !bmin || !bmax || !bits) return kErrInvalid;
  hipLaunchKernelGGL(block_pages_kernel, dim3(nblk, B), dim3(kWave), 0, (hipStream_t)stream,
                     image_page_ids, ipi_sb, L, block_size, nblk, bmin, bmax, bits);
  return pages_status();
}

extern "C" int dash_block_cand(const int32_t* query_page_ids, int64_t qpi_sb, int Lqp,
                               const int32_t* pos, int64_t pos_sb, int Lq,
                               const int32_t* image_page_ids, int64_t ipi_sb, int Lk,
                               const int32_t* bmin, const int32_t* bmax, const uint64_t* bits,
                               int nblk, int mode, int B, int block_size, uint8_t* cand,
                               int64_t cand_sb, int64_t cand_st, void* stream) {
  using namespace dash;
  if (B < 0 || Lq < 0 || nblk < 0 || block_size <= 0 || mode < 0 || mode > 2) return kErrInvalid;
  if (B == 0 || Lq == 0 || nblk == 0) return kOk;
  if (!cand) return kErrInvalid;
  if (nblk > kCandMaxBlocks) return kErrUnsupported;
  if (mode == 0 && (!query_page_ids || Lqp <= 0 || !image_page_ids || !bmin || !bmax || !bits))
    return kErrInvalid;
  if (mode == 1 && !bmax) return kErrInvalid;
  if (B > 65535) return kErrUnsupported;
  hipLaunchKernelGGL(block_cand_kernel, dim3((Lq + kCandRows - 1) / kCandRows, B), dim3(256), 0,
                     (hipStream_t)stream,
                     query_page_ids, qpi_sb, Lqp, pos, pos_sb, Lq, image_page_ids, ipi_sb, Lk,
                     bmin, bmax, bits, nblk, mode, block_size, cand, cand_sb, cand_st);
  return pages_status();
}

extern "C" int dash_decode_page_state(const int64_t* ids, int64_t ids_sb, int B, int L,
                                      int64_t image_token_id, int64_t page_token_id,
                                      int per_page_tokens, int block_size, int nblk,
                                      int32_t* bmin, int32_t* bmax, int32_t* prompt_pages,
                                      int32_t* markers, void* workspace, int64_t workspace_bytes,
                                      void* stream) {
  using namespace dash;
  if (B < 0 || L < 0 || per_page_tokens < 1 || block_size <= 0 || nblk < 0) return kErrInvalid;
  if (block_size > kPgThreads) return kErrUnsupported;
  if ((int64_t)nblk * block_size < L) return kErrInvalid;
  if (B == 0) return kOk;
  if (!ids || !bmin || !bmax || !prompt_pages || !markers) return kErrInvalid;
  hipStream_t st = (hipStream_t)stream;
  if (L == 0) {
    hipLaunchKernelGGL(decode_page_state_kernel, dim3(1, B), dim3(kPgThreads), 0, st, ids, ids_sb, 0,
                       image_token_id, page_token_id, per_page_tokens, block_size, nblk,
                       (kPgThreads / block_size) * block_size, 0, (const int32_t*)workspace, bmin,
                       bmax, prompt_pages, markers);
    return pages_status();
  }
  const int chunk = (kPgThreads / block_size) * block_size;
  int nchunks = 0;
  const int rs = page_summaries(ids, ids_sb, B, L, image_token_id, page_token_id, chunk, workspace,
                                workspace_bytes, nullptr, st, &nchunks);
  if (rs != kOk) return rs;
  hipLaunchKernelGGL(decode_page_state_kernel, dim3(nchunks, B), dim3(kPgThreads), 0, st, ids,
                     ids_sb, L, image_token_id, page_token_id, per_page_tokens, block_size, nblk,
                     chunk, nchunks, (const int32_t*)workspace, bmin, bmax, prompt_pages, markers);
  return pages_status();
}

extern "C" int dash_decode_allow(const int64_t* new_ids, int64_t new_stride, int B,
                                 int64_t page_token_id, const int32_t* bmin, const int32_t* bmax,
                                 int nblk_state, const int32_t* prompt_pages, int32_t* markers,
                                 int nblk, uint8_t* allow, int64_t allow_sb, void* stream) {
  using namespace dash;
  if (B < 0 || nblk_state < 0 || nblk < 0) return kErrInvalid;
  if (B == 0) return kOk;
  if (!new_ids || !prompt_pages || !markers || !allow) return kErrInvalid;
  if (nblk_state > 0 && (!bmin || !bmax)) return kErrInvalid;
  hipLaunchKernelGGL(decode_allow_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, new_ids,
                     new_stride, page_token_id, bmin, bmax, nblk_state, prompt_pages, markers,
                     nblk, allow, allow_sb);
  return pages_status();
}

extern "C" int dash_decode_win_bounds(const uint8_t* allow, int64_t allow_sb, int allow_w,
                                      const int32_t* seq_lens, const int32_t* q_pos, int B, int S,
                                      int nblk_cap, int block_size, int local_blocks, int tile,
                                      int32_t* bounds, uint8_t* fit, void* stream) {
  using namespace dash;
  if (B < 0 || S < 0 || nblk_cap < 0 || allow_w < 0 || block_size <= 0 || local_blocks < 0)
    return kErrInvalid;
  if (B == 0) return kOk;
  if (!allow || !bounds) return kErrInvalid;
  if (allow_sb < allow_w) return kErrInvalid;
  hipLaunchKernelGGL(win_bounds_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, allow, allow_sb,
                     allow_w, seq_lens, q_pos, S, nblk_cap, block_size, local_blocks, tile, bounds,
                     fit);
  return pages_status();
}

extern "C" int dash_page_rope_workspace_size(int B, int L, int64_t* bytes) {
  using namespace dash;
  if (!bytes || B < 0 || L < 0) return kErrInvalid;
  int64_t summ = 0;
  dash_pages_workspace_size(B, L, &summ);
  *bytes = (summ + 255) / 256 * 256 + (int64_t)B * L * (int64_t)sizeof(int32_t);
  return kOk;
}

extern "C" int dash_page_rope_pos(const int64_t* ids, int64_t ids_sb, int B, int L,
                                  int64_t image_token_id, int64_t page_token_id, int page_span,
                                  int64_t* tok, int64_t* page, int64_t* pf_cnt, int64_t pf_stride,
                                  int64_t* meta, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  using namespace dash;
  if (B < 0 || L < 0 || page_span < 0) return kErrInvalid;
  if (!meta) return kErrInvalid;
  if (B == 0 || L == 0) {
    if (B == 0) return kOk;
    return kErrInvalid;
  }
  if (!ids || !tok || !page || !pf_cnt || pf_stride < (int64_t)L + 1) return kErrInvalid;
  int64_t need = 0;
  dash_page_rope_workspace_size(B, L, &need);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 256 != 0) return kErrWorkspace;
  int64_t summ = 0;
  dash_pages_workspace_size(B, L, &summ);
  int32_t* mpos = (int32_t*)((char*)workspace + (summ + 255) / 256 * 256);
  hipStream_t st = (hipStream_t)stream;
  int nchunks = 0;
  const int rs = page_summaries(ids, ids_sb, B, L, image_token_id, page_token_id, kPgThreads,
                                workspace, workspace_bytes, nullptr, st, &nchunks);
  if (rs != kOk) return rs;
  hipLaunchKernelGGL(rope_page_kernel, dim3(nchunks, B), dim3(kPgThreads), 0, st, ids, ids_sb, L,
                     image_token_id, page_token_id, kPgThreads, nchunks,
                     (const int32_t*)workspace, page, mpos);
  hipLaunchKernelGGL(rope_tok_kernel, dim3(nchunks, B), dim3(kPgThreads), 0, st, L, kPgThreads,
                     nchunks, (const int32_t*)workspace, (const int64_t*)page,
                     (const int32_t*)mpos, page_span, tok, pf_cnt, pf_stride);
  hipLaunchKernelGGL(rope_meta_kernel, dim3(1), dim3(kWave), 0, st, B, nchunks,
                     (const int32_t*)workspace, meta);
  return pages_status();
}

extern "C" int dash_rope2d_cos_sin(const int64_t* tok, const int64_t* page, int64_t pos_sb, int B,
                                   int S, const float* inv_tok, int n_tok, const float* inv_page,
                                   int page_pairs, int page_mod, void* cos_out, void* sin_out,
                                   int out_bf16, int64_t cs_sb, int64_t cs_st, void* stream) {
  using namespace dash;
  if (B < 0 || S < 0 || n_tok < 0 || page_pairs < 0 || page_mod < 0) return kErrInvalid;
  if (n_tok + page_pairs <= 0) return kErrInvalid;
  const int64_t rows = (int64_t)B * S;
  if (rows == 0) return kOk;
  if (!tok || !page || !cos_out || !sin_out || (n_tok > 0 && !inv_tok) ||
      (page_pairs > 0 && !inv_page))
    return kErrInvalid;
  const int half = n_tok + page_pairs;
  if (cs_st < 2 * half) return kErrInvalid;
  const int64_t n = rows * half;
  if ((n + 255) / 256 > INT32_MAX) return kErrUnsupported;
  hipLaunchKernelGGL(rope2d_cos_sin_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, tok, page, pos_sb, S, rows, inv_tok, n_tok, inv_page,
                     half, page_mod, cos_out, sin_out, out_bf16, cs_sb, cs_st);
  return pages_status();
}

extern "C" int dash_page_rope_advance(const int64_t* new_ids, int64_t new_stride, int B,
                                      int64_t page_token_id, int64_t* page, int64_t* tok,
                                      const int64_t* pf_cnt, int64_t pf_stride,
                                      const int64_t* meta, int64_t* out_tok, int64_t* out_page,
                                      void* stream) {
  using namespace dash;
  if (B < 0) return kErrInvalid;
  if (B == 0) return kOk;
  if (!new_ids || !page || !tok || !pf_cnt || !meta || pf_stride < 1) return kErrInvalid;
  hipLaunchKernelGGL(rope_advance_kernel, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     new_ids, new_stride, B, page_token_id, page, tok, pf_cnt, pf_stride, meta,
                     out_tok, out_page);
  return pages_status();
}
