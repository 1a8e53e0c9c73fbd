// DASH decode attention on gfx950: one query per sequence against the cached
// keys, over the token window (q-LW, q] plus the routed remote blocks (with the
// block bias), as modeling_deepseekv2.py:424-451 defines it.  Cache layouts:
// contiguous [B,H,S,D] (any strides) or paged [pages, page, H, D] + block table.
//
// HBM-streaming split-K: the key set of every (sequence, head) is cut into
// units of one key block; work-group `split` of (b,h) takes units
// split, split+nsplit, ...; each wavefront streams a unit with 16-byte loads
// (16 lanes per key row), keeps an online softmax, and the work-group writes one
// (m, l, o) partial.  A merge kernel combines the partials with a log-sum-exp.

#include "dash_common.h"

namespace dash {

constexpr int kDcMaxK = 16;
constexpr int kDcMaxUnits = 64 + kDcMaxK;

struct DecodeArgs {
  const bf16* q; int64_t q_sb, q_sh;
  const bf16* k; const bf16* v;
  int64_t k_sb, k_sh, k_st, k_sp;
  int64_t v_sb, v_sh, v_st, v_sp;
  const int32_t* table; int64_t table_stride; int page;
  const int32_t* lens; const int32_t* q_pos;
  const int32_t* idx; const uint8_t* valid; const float* bias; int K;
  float* part;                   // [B*H*nsplit, D + 2]: o[D], m, l
  int S, H, D, bs, lw, nsplit;
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

template <int D>
__global__ __launch_bounds__(256) void decode_split_kernel(DecodeArgs a) {
  static_assert(D == 128, "head_dim 128");
  __shared__ int32_t sUnitC[kDcMaxUnits];     // block id of unit
  __shared__ float sUnitB[kDcMaxUnits];       // bias (log2 units) of unit
  __shared__ int32_t sUnitR[kDcMaxUnits];     // 1 = routed, 0 = window
  __shared__ int32_t sNU;
  __shared__ float sM[4], sL[4];
  __shared__ float sO[4][D];

  const int split = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = wave_lane(), wv = tid / kWave;
  const int len = a.lens ? a.lens[b] : a.S;
  const int qp = a.q_pos ? a.q_pos[b] : len - 1;
  const int ls = qp - a.lw + 1;
  const int lo = max(ls, 0);
  const float log2e = 1.4426950408889634f;

  if (tid == 0) {
    int nu = 0;
    if (len > 0 && qp >= 0) {
      for (int c = lo / a.bs; c <= qp / a.bs; ++c) {
        sUnitC[nu] = c; sUnitB[nu] = 0.f; sUnitR[nu] = 0; ++nu;
      }
      const int nblk = (len + a.bs - 1) / a.bs;
      const int nwin = nu;
      for (int s = 0; s < a.K; ++s) {
        const int c = a.idx[(int64_t)b * a.K + s];
        if (c < 0 || c >= nblk) continue;
        if (a.valid && !a.valid[(int64_t)b * a.K + s]) continue;
        if (c * a.bs >= ls) continue;
        bool dup = false;
        for (int u = nwin; u < nu; ++u) dup |= (sUnitC[u] == c);
        if (dup) continue;
        sUnitC[nu] = c; sUnitB[nu] = a.bias[(int64_t)b * a.K + s] * log2e; sUnitR[nu] = 1; ++nu;
      }
    }
    sNU = nu;
  }
  __syncthreads();
  const int nu = sNU;

  // this lane's slice of q: dims (lane%16)*8 .. +7
  const int g = lane >> 4, dl = (lane & 15) * 8;
  const bf16x8 qv8 = *(const bf16x8*)(a.q + (int64_t)b * a.q_sb + (int64_t)h * a.q_sh + dl);
  float qf[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) qf[e] = bf2f(qv8[e]);

  float m_run = -INFINITY, l_run = 0.f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.f;

  const bf16* kh = a.k + (int64_t)h * a.k_sh;
  const bf16* vh = a.v + (int64_t)h * a.v_sh;
  for (int u = split + a.nsplit * wv; u < nu; u += a.nsplit * 4) {
    const int c = sUnitC[u];
    const bool routed = sUnitR[u] != 0;
    const float bl = sUnitB[u];
    for (int j0 = c * a.bs; j0 < (c + 1) * a.bs; j0 += 64) {
      // 16 key rows per lane group: key = j0 + 4*st + g
      bf16x8 kr[16];
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int j = min(j0 + 4 * st + g, len - 1);
        kr[st] = *(const bf16x8*)(kh + dc_row(a, b, j, a.k_sb, a.k_st, a.k_sp) + dl);
      }
      float s[16];
      float mloc = -INFINITY;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(qf[e], bf2f(kr[st][e]), acc);
        acc += __shfl_xor(acc, 1, kWave);
        acc += __shfl_xor(acc, 2, kWave);
        acc += __shfl_xor(acc, 4, kWave);
        acc += __shfl_xor(acc, 8, kWave);
        const int key = j0 + 4 * st + g;
        bool ok = key < (c + 1) * a.bs && key < len;
        ok = ok && (routed ? (key < ls) : (key >= lo && key <= qp));
        s[st] = ok ? acc * a.scale_log2e + bl : -INFINITY;
        mloc = fmaxf(mloc, s[st]);
      }
      bf16x8 vr[16];
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int j = min(j0 + 4 * st + g, len - 1);
        vr[st] = *(const bf16x8*)(vh + dc_row(a, b, j, a.v_sb, a.v_st, a.v_sp) + dl);
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, kWave));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, kWave));
      const float m_new = fmaxf(m_run, mloc);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = exp2f(m_run - m_use);
      l_run *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float p = exp2f(s[st] - m_use);
        l_run += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fmaf(p, bf2f(vr[st][e]), o[e]);
      }
      m_run = m_new;
    }
  }
  // combine the four lane groups of the wavefront (they share m_run)
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    o[e] += __shfl_xor(o[e], 16, kWave);
    o[e] += __shfl_xor(o[e], 32, kWave);
  }
  if (lane == 0) { sM[wv] = m_run; sL[wv] = l_run; }
  if (lane < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sO[wv][dl + e] = o[e];
  }
  __syncthreads();
  // combine the four wavefronts and write the partial
  float M = fmaxf(fmaxf(sM[0], sM[1]), fmaxf(sM[2], sM[3]));
  const float Mu = (M == -INFINITY) ? 0.f : M;
  float* part = a.part + ((int64_t)(b * a.H + h) * a.nsplit + split) * (D + 2);
  if (tid < D) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) acc += sO[w][tid] * exp2f(sM[w] - Mu);
    part[tid] = acc;
  }
  if (tid == 0) {
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) L += sL[w] * exp2f(sM[w] - Mu);
    part[D] = M;
    part[D + 1] = L;
  }
}

template <int D>
__global__ __launch_bounds__(D) void decode_merge_kernel(const float* __restrict__ part,
                                                         int nsplit, int H, void* out,
                                                         int out_bf16, int64_t o_sb,
                                                         int64_t o_sh, float* lse,
                                                         int64_t lse_sb, int64_t lse_sh) {
  const int h = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const float* p = part + (int64_t)(b * H + h) * nsplit * (D + 2);
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p[s * (D + 2) + D]);
  const float Mu = (M == -INFINITY) ? 0.f : M;
  float L = 0.f, acc = 0.f;
  for (int s = 0; s < nsplit; ++s) {
    const float w = exp2f(p[s * (D + 2) + D] - Mu);
    L += p[s * (D + 2) + D + 1] * w;
    acc += p[s * (D + 2) + t] * w;
  }
  const float r = L > 0.f ? acc / L : 0.f;
  const int64_t off = (int64_t)b * o_sb + (int64_t)h * o_sh + t;
  if (out_bf16) ((bf16*)out)[off] = (bf16)r;
  else ((float*)out)[off] = r;
  if (lse && t == 0)
    lse[(int64_t)b * lse_sb + (int64_t)h * lse_sh] =
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
  if (block_size <= 0 || block_size % 64 != 0 && block_size != 32) return kErrUnsupported;
  if (local_window < 1) return kErrInvalid;
  if ((local_window + block_size - 1) / block_size + 1 > kDcMaxUnits - kDcMaxK) return kErrUnsupported;
  if (block_table && (page_size <= 0 || page_size % block_size != 0)) return kErrUnsupported;
  if (nsplit <= 0) return kErrInvalid;
  if (B == 0) return kOk;
  const int64_t strides[] = {q_sb, q_sh, k_sb, k_sh, k_st, k_sp, v_sb, v_sh, v_st, v_sp};
  for (int64_t s : strides)
    if (s % 8 != 0) return kErrUnsupported;
  const void* ptrs[] = {q, k, v};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return kErrUnsupported;
  int64_t need = 0;
  dash_attn_decode_workspace_size(B, H, D, nsplit, &need);
  if (!workspace || workspace_bytes < need) return kErrWorkspace;
  DecodeArgs a;
  a.q = (const bf16*)q; a.q_sb = q_sb; a.q_sh = q_sh;
  a.k = (const bf16*)k; a.v = (const bf16*)v;
  a.k_sb = k_sb; a.k_sh = k_sh; a.k_st = k_st; a.k_sp = k_sp;
  a.v_sb = v_sb; a.v_sh = v_sh; a.v_st = v_st; a.v_sp = v_sp;
  a.table = block_table; a.table_stride = table_stride; a.page = page_size;
  a.lens = seq_lens; a.q_pos = q_pos;
  a.idx = idx; a.valid = valid; a.bias = bias; a.K = K;
  a.part = (float*)workspace;
  a.S = S; a.H = H; a.D = D; a.bs = block_size; a.lw = local_window; a.nsplit = nsplit;
  a.scale_log2e = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(decode_split_kernel<128>, dim3(nsplit, H, B), dim3(256), 0, st, a);
  hipLaunchKernelGGL(decode_merge_kernel<128>, dim3(H, B), dim3(128), 0, st,
                     (const float*)workspace, nsplit, H, out, out_bf16, o_sb, o_sh, lse,
                     lse_sb, lse_sh);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
