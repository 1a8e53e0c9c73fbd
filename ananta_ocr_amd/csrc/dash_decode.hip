// DASH decode attention on gfx950: one query per sequence against the cached
// keys, over the token window (q-LW, q] plus the keys below the window of the
// routed remote blocks (with the block bias), as modeling_deepseekv2.py:424-451
// defines it.  Cache layouts: contiguous [B,H,S,D] (any strides) or paged
// [pages, page, H, D] + block table.
//
// HBM-streaming split-K: the key set of every (sequence, head) is cut into units
// of one key block (window blocks first, then the routed blocks).  Work-group
// `split` (one wavefront) of (b, h) takes units split, split+nsplit, ...  A
// wavefront streams a unit with 16-byte loads, 16 lanes per key row (K and V
// loads of the unit are all issued before the first use), row sums by DPP,
// online softmax in base 2.  Every wavefront writes an (o, m, l) partial; a
// merge kernel (one wavefront per (b, h)) combines them with a log-sum-exp.

#include "dash_decode_unit.h"

namespace dash {

template <int D>
__global__ __launch_bounds__(64) void decode_attn_kernel(DecodeArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ int sTmp[kWave];
  __shared__ int sRC[kDcMaxSlots];
  __shared__ float sRB[kDcMaxSlots];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const DcSpan sp = dc_span(a, b);
  // ---- routed blocks (only wavefronts that own a routed unit need them) ----
  int n_r = 0;
  // first unit index >= n_win in this wavefront's sequence split, split + nsplit, ...
  const int u_first_routed =
      split >= sp.n_win ? split : split + a.nsplit * ((sp.n_win - split + a.nsplit - 1) / a.nsplit);
  if (u_first_routed < sp.n_win + a.K)
    n_r = dc_routed(a, b, sp, lane, sTmp, sRC, sRB, [] { __syncthreads(); });
  const int n_units = sp.n_win + n_r;

  DcState st;
  dc_init(st, a, b, h, lane);
  for (int u = split; u < n_units; u += a.nsplit) {
    const bool routed = u >= sp.n_win;
    const int cu = routed ? sRC[u - sp.n_win] : sp.w0 + u;
    const float blog = routed ? sRB[u - sp.n_win] : 0.f;
    dc_block<16>(st, a, b, h, sp, cu, routed, blog);
  }
  const int bh = b * a.H + h;
  dc_store_partial<D>(st, a.part + ((int64_t)bh * a.nsplit + split) * (D + 2), lane);
}

// Merge of the nsplit partials of every (b, h): one wavefront per (b, h).
template <int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
  __shared__ float sW[kDcMaxSplit];
  const int h = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int bh = b * a.H + h;
  const float* pb = a.part + (int64_t)bh * a.nsplit * (D + 2);
  float ms = -INFINITY, lsum = 0.f;
  if (lane < a.nsplit) { ms = pb[lane * (D + 2) + D]; lsum = pb[lane * (D + 2) + D + 1]; }
  dc_merge<D>(a, b, h, lane, a.nsplit, ms, lsum, sW,
              [&](int s) { return pb + s * (D + 2); });
}

}  // namespace dash

extern "C" int dash_attn_decode_workspace_size(int B, int H, int D, int nsplit, int64_t* bytes) {
  if (!bytes || B < 0 || H < 0 || nsplit <= 0) return dash::kErrInvalid;
  *bytes = (int64_t)B * H * nsplit * (D + 2) * (int64_t)sizeof(float);
  return dash::kOk;
}

extern "C" int dash_attn_decode(
    const void* q, int64_t q_sb, int64_t q_sh,
    const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t k_sp,
    const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t v_sp,
    const int32_t* block_table, int64_t table_stride, int page_size,
    const int32_t* seq_lens, const int32_t* q_pos,
    const int32_t* idx, const uint8_t* valid, const float* bias, int K,
    void* out, int out_bf16, int64_t o_sb, int64_t o_sh,
    float* lse, int64_t lse_sb, int64_t lse_sh,
    int B, int H, int S, int D, int block_size, int local_window, float scale, int nsplit,
    void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace dash;
  if (!q || !k || !v || !out || B < 0 || H <= 0) return kErrInvalid;
  if (K > 0 && (!idx || !bias)) return kErrInvalid;
  if (D != 128) return kErrUnsupported;
  if (K < 0 || K > kDcMaxSlots) return kErrUnsupported;
  if (block_size <= 0 || (block_size % 64 != 0 && block_size != 32)) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if (block_table && (page_size <= 0 || page_size % block_size != 0)) return kErrUnsupported;
  if (nsplit <= 0 || nsplit > kDcMaxSplit) return kErrUnsupported;
  if (B == 0) return kOk;
  const int64_t strides[] = {q_sb, q_sh, k_sb, k_sh, k_st, k_sp, v_sb, v_sh, v_st, v_sp};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  const void* ptrs[] = {q, k, v};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return kErrUnsupported;
  int64_t need = 0;
  dash_attn_decode_workspace_size(B, H, D, nsplit, &need);
  if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16 != 0) return kErrWorkspace;
  DecodeArgs a;
  a.q = (const bf16*)q; a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st; a.k_sp = k_sp;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st; a.v_sp = v_sp;
  a.table = block_table; a.table_stride = table_stride; a.page = page_size;
  a.lens = seq_lens; a.q_pos = q_pos;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = K;
  a.out = out; a.out_bf16 = out_bf16; a.o_sb = o_sb; a.o_sh = o_sh;
  a.lse = lse; a.lse_sb = lse_sb; a.lse_sh = lse_sh;
  a.part = (float*)workspace;
  a.S = S; a.H = H; a.bs = block_size; a.lw = local_window; a.nsplit = nsplit;
  a.scale_log2e = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(decode_attn_kernel<128>, dim3(nsplit, H, B), dim3(64), 0,
                     (hipStream_t)stream, a);
  hipLaunchKernelGGL(decode_merge_kernel<128>, dim3(H, B), dim3(64), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
