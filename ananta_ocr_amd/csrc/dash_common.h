// Shared device helpers for the DASH HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace dash {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float floatx16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float floatx4;

// Sentinels of the reference router (dash_attention.py:600-604,
// modeling_deepseekv2.py:56).
constexpr float kScoreNeg = -1.0e9f;
constexpr float kEntmaxNeg = -1.0e4f;
constexpr float kActClamp = 1.0e4f;
constexpr float kGradClamp = 1.0e4f;   // gradient sanitizer bound (dash_attention.py:603)

constexpr int kWave = 64;

// Status codes returned by every C entry point.
enum Status : int {
  kOk = 0,
  kErrUnsupported = -2,   // a shape or parameter the library does not implement
  kErrInvalid = -3,       // inconsistent arguments (null pointer, negative size...)
  kErrWorkspace = -4,     // caller-provided workspace too small
  kErrScratch = -5,       // beyond the fixed scratch of the allocation-free entry point
};

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }

// 2^x with the bare v_exp_f32 (no denormal range fix-up): the attention softmax
// only feeds it x <= small positive values and needs no denormal results;
// -inf gives 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int wave_lane() { return threadIdx.x & (kWave - 1); }

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Work-groups of a 1-D grid are dispatched to the 8 XCDs round-robin by linear
// id, and each XCD has its own L2.  This maps linear id L of n to a logical id
// such that every XCD runs a contiguous range of logical ids (neighbouring tiles
// or chunks, which share K/V rows, then meet in the same L2).
__device__ __forceinline__ int xcd_logical_id(int L, int n) {
  constexpr int kXcd = 8;
  const int x = L % kXcd, k = L / kXcd;
  const int q = n / kXcd, r = n % kXcd;
  return x * q + min(x, r) + k;
}

// Stream-local stage order over the XCDs: ns streams (e.g. (sequence, head) pairs)
// of nst stages each, stage 0 the heaviest.  XCD x = L % 8 takes, stage by stage,
// the whole streams x, x + 8, ... (q = ns / 8 of them) and, of the r = ns % 8 other
// streams, stage s of stream 8 q + j whenever (s r + j) % 8 == x; its k-th work-group
// (k = L / 8) takes the k-th of these items.  Every XCD thus runs its streams'
// stages in order, neighbouring stages of one stream share its L2, and the heavy
// stages of every stream start first.  Returns false for the ids past an XCD's
// items (the grid is stream_stage_grid work-groups).
__host__ __device__ inline int stream_stage_before(int s, int x, int q, int r) {
  return q * s + (s * r - x + 7) / 8;    // items of XCD x at stages < s
}
__host__ __device__ inline bool stream_stage_item(int L, int ns, int nst, int& stream, int& stage) {
  const int x = L & 7, k = L >> 3;
  const int q = ns >> 3, r = ns & 7;
  int s = (int)((int64_t)k * 8 / (8 * q + r));
  if (s > nst) s = nst;
  while (s > 0 && stream_stage_before(s, x, q, r) > k) --s;
  while (s < nst && stream_stage_before(s + 1, x, q, r) <= k) ++s;
  if (s >= nst) return false;
  const int o = k - stream_stage_before(s, x, q, r);
  if (o < q) {
    stream = x + 8 * o;
  } else {
    const int j = (x - (s * r & 7)) & 7;
    if (o > q || j >= r) return false;
    stream = 8 * q + j;
  }
  stage = s;
  return true;
}
__host__ __device__ inline int stream_stage_grid(int ns, int nst) {
  return 8 * ((ns >> 3) * nst + (nst * (ns & 7) + 7) / 8);
}

// Where token t of sequence b lives, for the three layouts the path uses:
//   contiguous  row = b*stride_b + t*stride_t
//   varlen      row = (cu[b] + t)*stride_t          (packed documents)
//   paged       row = table[b][t / page]*stride_page + (t % page)*stride_t
struct SeqLayout {
  const int32_t* cu;          // [B+1] or null
  const int32_t* table;       // [B, table_stride] or null
  int64_t table_stride;
  int64_t stride_b;           // contiguous layout
  int64_t stride_page;        // paged layout
  int64_t stride_t;
  int page;                   // tokens per page (paged layout)

  __device__ __forceinline__ int64_t row(int b, int t) const {
    if (table) {
      const int p = table[(int64_t)b * table_stride + t / page];
      return (int64_t)p * stride_page + (int64_t)(t % page) * stride_t;
    }
    if (cu) return (int64_t)(cu[b] + t) * stride_t;
    return (int64_t)b * stride_b + (int64_t)t * stride_t;
  }
};

// Length of sequence b: cu_seqlens, explicit lengths, or the common length.
__device__ __forceinline__ int seq_length(const int32_t* cu, const int32_t* lens, int b, int S) {
  if (cu) return cu[b + 1] - cu[b];
  if (lens) return lens[b];
  return S;
}

// Flat row index of (sequence b, token t) for per-token outputs such as the
// block scores or the routed indices: varlen rows are packed, the others are b*S+t.
__device__ __forceinline__ int64_t token_row(const int32_t* cu, int b, int t, int S) {
  if (cu) return (int64_t)cu[b] + t;
  return (int64_t)b * S + t;
}

}  // namespace dash
