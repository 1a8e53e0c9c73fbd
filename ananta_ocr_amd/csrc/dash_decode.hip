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

#include "dash_common.h"

namespace dash {

constexpr int kDcMaxK = 16;
constexpr int kDcMaxSplit = 64;

struct DecodeArgs {
  const bf16* q; int64_t q_sb, q_sh;
  const bf16* k; const bf16* v;
  int64_t k_sb, k_sh, k_st, k_sp;
  int64_t v_sb, v_sh, v_st, v_sp;
  const int32_t* table; int64_t table_stride; int page;
  const int32_t* lens; const int32_t* q_pos;
  const int32_t* idx; const uint8_t* valid; const float* bias; int K;
  void* out; int out_bf16; int64_t o_sb, o_sh;
  float* lse; int64_t lse_sb, lse_sh;
  float* part;                   // [B*H*nsplit, D + 2]: o[D], m, l
  int S, H, bs, lw, nsplit;
  float scale_log2e;
};

__device__ __forceinline__ int64_t dc_row(const DecodeArgs& a, int b, int j, int64_t sb,
                                          int64_t st, int64_t sp) {
  if (a.table) {
    const int p = a.table[(int64_t)b * a.table_stride + j / a.page];
    return (int64_t)p * sp + (int64_t)(j % a.page) * st;
  }
  return (int64_t)b * sb + (int64_t)j * st;
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
  return v;
}

template <int D>
__global__ __launch_bounds__(64) void decode_attn_kernel(DecodeArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ int sTmp[kWave];
  __shared__ int sRC[kDcMaxK];
  __shared__ float sRB[kDcMaxK];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int len = a.lens ? a.lens[b] : a.S;
  const int qp = a.q_pos ? a.q_pos[b] : len - 1;
  const int ls = qp - a.lw + 1;
  const int lo = max(ls, 0);
  const int nblk = len > 0 ? (len + a.bs - 1) / a.bs : 0;
  const float log2e = 1.4426950408889634f;
  const int w0 = lo / a.bs;
  const int n_win = (len > 0 && qp >= 0) ? qp / a.bs - w0 + 1 : 0;
  // ---- routed blocks (only wavefronts that own a routed unit need them): lanes < K
  // load the slots; keep valid, remote, first occurrence, in slot order ----
  int n_r = 0;
  // first unit index >= n_win in this wavefront's sequence split, split + nsplit, ...
  const int u_first_routed =
      split >= n_win ? split : split + a.nsplit * ((n_win - split + a.nsplit - 1) / a.nsplit);
  if (u_first_routed < n_win + a.K) {
    int c = -1;
    float bl = 0.f;
    bool keep = false;
    if (lane < a.K && len > 0) {
      const int64_t o = (int64_t)b * a.K + lane;
      c = a.idx[o];
      keep = c >= 0 && c < nblk && c * a.bs < ls && (!a.valid || a.valid[o] != 0);
      bl = a.bias[o] * log2e;
    }
    sTmp[lane] = keep ? c : -1;
    __syncthreads();
    if (keep)
      for (int j = 0; j < lane; ++j) keep &= (sTmp[j] != c);
    const uint64_t mask = __ballot(keep);
    if (keep) {
      const int pos = __popcll(mask & ((1ull << lane) - 1ull));
      sRC[pos] = c;
      sRB[pos] = bl;
    }
    __syncthreads();
    n_r = __popcll(mask);
  }
  const int n_units = n_win + n_r;

  const int g = lane >> 4, dl = (lane & 15) * 8;
  const bf16x8 qv8 = *(const bf16x8*)(a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + dl);
  bf16x2 qp2[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) { qp2[e][0] = qv8[2 * e]; qp2[e][1] = qv8[2 * e + 1]; }

  float m_run = -INFINITY, l_run = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;

  const bf16* kh = a.k + (int64_t)h * a.k_sh;
  const bf16* vh = a.v + (int64_t)h * a.v_sh;
  for (int u = split; u < n_units; u += a.nsplit) {
    const bool routed = u >= n_win;
    const int cu = routed ? sRC[u - n_win] : w0 + u;
    const float blog = routed ? sRB[u - n_win] : 0.f;
    const int jend = min((cu + 1) * a.bs, len);
    for (int jb = cu * a.bs; jb < jend; jb += 64) {
      bf16x8 kr[16], vr[16];
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int j = min(jb + 4 * st + g, len - 1);
        kr[st] = *(const bf16x8*)(kh + dc_row(a, b, j, a.k_sb, a.k_st, a.k_sp) + dl);
      }
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int j = min(jb + 4 * st + g, len - 1);
        vr[st] = *(const bf16x8*)(vh + dc_row(a, b, j, a.v_sb, a.v_st, a.v_sp) + dl);
      }
      float s[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bf16x2 kk;
          kk[0] = kr[st][2 * e];
          kk[1] = kr[st][2 * e + 1];
          acc = __builtin_amdgcn_fdot2_f32_bf16(qp2[e], kk, acc, false);
        }
        acc = row16_sum(acc);
        const int key = jb + 4 * st + g;
        bool ok = key < jend;
        ok = ok && (routed ? (key < ls) : (key >= lo && key <= qp));
        s[st] = ok ? acc * a.scale_log2e + blog : -INFINITY;
        mloc = fmaxf(mloc, s[st]);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, kWave));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float p = fast_exp2(s[st] - m_use);
        l_run += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fmaf(p, bf2f(vr[st][e]), o[e]);
      }
      m_run = m_new;
    }
  }
  // ---- this wavefront's partial: sum the four lane groups (they share m_run) ----
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += __shfl_xor(o[e], 16, kWave);
    o[e] += __shfl_xor(o[e], 32, kWave);
  }
  const int bh = b * a.H + h;
  float* part = a.part + ((int64_t)bh * a.nsplit + split) * (D + 2);
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) part[dl + e] = o[e];
  }
  if (lane == 0) { part[D] = m_run; part[D + 1] = l_run; }

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
  const float M = wave_max(ms);
  const float Mu = (M == -INFINITY) ? 0.f : M;
  const float w = lane < a.nsplit ? fast_exp2(ms - Mu) : 0.f;
  const float L = wave_sum(lsum * w);
  sW[lane] = w;
  __syncthreads();
  const float inv = L > 0.f ? 1.f / L : 0.f;
  float acc0 = 0.f, acc1 = 0.f;
  for (int s = 0; s < a.nsplit; ++s) {
    const float2 ov = *(const float2*)(pb + s * (D + 2) + lane * 2);
    acc0 += ov.x * sW[s];
    acc1 += ov.y * sW[s];
  }
  const int64_t off = (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + lane * 2;
  if (a.out_bf16) {
    bf16x2 r;
    r[0] = (bf16)(acc0 * inv);
    r[1] = (bf16)(acc1 * inv);
    *(bf16x2*)((bf16*)a.out + off) = r;
  } else {
    *(float2*)((float*)a.out + off) = make_float2(acc0 * inv, acc1 * inv);
  }
  if (a.lse && lane == 0)
    a.lse[(int64_t)b * a.lse_sb + (int64_t)h * a.lse_sh] =
        L > 0.f ? (M + log2f(L)) * 0.6931471805599453f : -INFINITY;
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
  if (K < 0 || K > kDcMaxK) return kErrUnsupported;
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
