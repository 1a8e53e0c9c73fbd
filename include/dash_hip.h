/*
 * dash_hip.h -- C ABI of the MI355X (gfx950) DASH attention library
 * (libdash_hip.so).  Plain pointers, sizes and strides; no framework types.
 *
 * Conventions shared by every entry point
 *   - Every pointer argument is a device pointer unless stated otherwise; the
 *     caller owns every buffer (outputs and workspace included).  The library
 *     allocates nothing.  It keeps no state between calls, except for the
 *     allocation-free decode entry point (dash_decode_step_noalloc): a fixed 64 MiB
 *     device array per GPU, held until the process ends, and that array's address per
 *     device, looked up on the first call on each device.  The decode step's workspace
 *     (caller-owned) keeps the zeros its routing words need from one call to the next.
 *   - Strides are in elements, not bytes.  The innermost (feature) axis must be
 *     contiguous; bf16 tensors need 16-byte aligned rows.
 *   - `stream` is a hipStream_t; all work is enqueued on it, nothing synchronises.
 *   - Return value: 0 ok, -2 unsupported shape/parameter (the Python layer raises
 *     NotImplementedError), -3 invalid argument, -4 workspace too small, -5 sizes beyond
 *     the fixed scratch of the allocation-free entry point, >0 a hipError_t.
 *   - Sequence layouts: contiguous ([B, S, ...] with a batch stride), varlen
 *     (`cu_seqlens` [B+1] prefix sums over a packed token axis; every sequence has
 *     its own block grid starting at its first token) or paged (`block_table`
 *     [B, table_stride] of physical page ids; token t of sequence b lives in page
 *     block_table[b][t / page_size] at row t % page_size).
 *
 * Reference interfaces replaced (paths are in the ANANTA_OCR repository).
 */
#ifndef DASH_HIP_H
#define DASH_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header (1). */
int dash_abi_version(void);

/* Human-readable text for a status code. Host pointer, static storage. */
const char* dash_status_string(int status);

/*
 * Stage-0 block summaries k_bar[b, c, :] = sum_j softmax_j(k_j.head_cls/sqrt(d)) k_j over
 * the real tokens of key block c (mean pooling when head_cls == 0).
 * Replaces the head_cls summary of DashAttention._block_scores_headcls
 * (dash_attention.py:851-888) and _block_scores_infer (modeling_deepseekv2.py:362-377).
 *   idx_k      fp32 index keys; token rows addressed by (ik_sb, ik_st) contiguous,
 *              cu_seqlens (varlen) or block_table/ik_sp/page_size (paged)
 *   seq_lens   [B] key lengths (contiguous/paged) or NULL for S
 *   tail_only  1: recompute only the last block of every sequence (decode refresh)
 *   kbar       [B, nblk_cap, d] fp32, batch stride kb_sb
 */
int dash_kbar(const float* idx_k, int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
              const int32_t* cu_seqlens, const int32_t* seq_lens,
              const int32_t* block_table, int64_t table_stride, int page_size,
              const float* head_cls, int B, int S, int d, int block_size, int tail_only,
              float* kbar, int64_t kb_sb, int nblk_cap, void* stream);

/*
 * Block scores z[row, c] = clamp(idx_q.k_bar_c/sqrt(d), +-1e4) for remote blocks
 * (c <= q_pos//block_size - local_blocks, c < nblk of the sequence), -1e9 otherwise.
 * Replaces the scoring loop of _block_scores_infer (modeling_deepseekv2.py:378-386) /
 * DashAttention._block_scores_headcls (dash_attention.py:890-904).
 *   idx_q   fp32 [B, Lq, d] (iq_sb, iq_st) or varlen via cu_q
 *   q_pos   per query row position (NULL: the row index within the sequence)
 *   cu_k/lens_k  key lengths per sequence (NULL/NULL: S)
 *   z       fp32 rows (b*Lq + t, or cu_q[b] + t) with row stride z_stride
 */
int dash_block_scores(const float* idx_q, int64_t iq_sb, int64_t iq_st,
                      const int32_t* cu_q, int Lq, const int32_t* q_pos,
                      const float* kbar, int64_t kb_sb, int nblk_cap,
                      const int32_t* cu_k, const int32_t* lens_k, int S, int B,
                      int d, int block_size, int local_blocks, float* z,
                      int64_t z_stride, void* stream);

/*
 * Indexer stage-0 scores: per key block, max over keys seg[t] <= j < max(pos[t]-LW+1,0),
 * j < Sk of q_t.k_j.  mode 0 = the torch form of modeling_deepseekv2.py:387-400 /
 * dash_attention.py:815-835 (clamp +-1e4, -1e9 for empty blocks, seg ignored when NULL);
 * mode 1 = triton_block_max_score (sparse_gather_triton.py:395-467; no clamp, -inf).
 *   q [B, C, d], k [B, Sk, d] fp32; pos/seg [B, C] int32 with batch stride ps_sb;
 *   out[b*o_sb + t*o_sc + c], nblk blocks.
 */
int dash_block_max_score(const float* q, int64_t q_sb, int64_t q_st, int C,
                         const int32_t* pos, const int32_t* seg, int64_t ps_sb,
                         const float* k, int64_t k_sb, int64_t k_st, int Sk, int B,
                         int d, int block_size, int local_window, int nblk, int mode,
                         float* out, int64_t o_sb, int64_t o_sc, void* stream);

/*
 * Router front end after the index projections: Gemma RMSNorm (scale 1 + w, eps,
 * activations clamped to +-1e4), optional RoPE (rotate-half, cos/sin rows of the
 * first d dims) and the finiteness guards of _router_qk (modeling_deepseekv2.py:336-348)
 * with GemmaRMSNorm (dash_attention.py:680-700).  proj [rows, proj_row] holds both
 * projections of a row, q at [0, d) and k at [d, 2d) (one GEMM with the two weights
 * stacked), bf16 or fp32; cos/sin (optional, both or neither) at b*cs_sb + t*cs_st for
 * row = b*S + t, bf16 or fp32.  Steps round as the unfused tensor ops do: fp32 math,
 * the normed rows rounded to the projection dtype, RoPE in bf16 when both the
 * projection and cos/sin are bf16, else fp32.  idx_q/idx_k fp32 [rows, d].  d == 128.
 */
int dash_router_qk_norm(const void* proj, int proj_bf16, int64_t proj_row, int64_t rows, int S,
                        int d, const float* wq, const float* wk, float eps, const void* cos,
                        const void* sin, int cs_bf16, int64_t cs_sb, int64_t cs_st,
                        float* idx_q, float* idx_k, void* stream);

/*
 * Fused router front end for bf16 hidden states, one launch: nan_to_num of the
 * hidden states, the index q/k projections (w_q / w_k bf16 [128, hidden], and the same
 * weights packed by dash_router_front_pack_weights into w_pack [256 * hidden]; fp32
 * accumulation, rounded to bf16 as the bf16 linear layer), Gemma RMSNorm with
 * (1 + weight), RoPE (cos/sin [.., S, >=128] bf16 or fp32, or none) and the finiteness
 * guards -- replaces _router_qk (modeling_deepseekv2.py:336-348) with _RMSNorm.forward
 * (dash_attention.py:680-700).  idx_q / idx_k fp32 [B, S, 128] (row stride 128, batch
 * strides iq_sb / ik_sb) are written when non-null.  With head_cls (stage 0
 * "head_cls", block_size 32 or 64) it also writes the block summaries kbar
 * [B, nblk_cap, 128] (the pooling of _block_scores_infer, modeling_deepseekv2.py:
 * 362-379) from the index keys still on chip.  hidden % 64 == 0; 16-byte aligned
 * hidden rows and weights.
 */
int dash_router_front(const void* hs, int64_t hs_sb, int64_t hs_st, int B, int S, int hidden,
                      const void* w_pack, const void* w_q, const void* w_k,
                      const float* wq_norm, const float* wk_norm, float eps, const void* cos,
                      const void* sin, int cs_bf16, int64_t cs_sb, int64_t cs_st,
                      const float* head_cls, int block_size, float inv_sqrt_d, float* idx_q,
                      int64_t iq_sb, float* idx_k, int64_t ik_sb, float* kbar, int64_t kb_sb,
                      int nblk_cap, void* stream);
/* The q_proj / k_proj weights (bf16 [128, hidden] each, row-major) in the operand order
 * of dash_router_front: w_pack bf16 [256 * hidden]; repack when the weights change. */
int dash_router_front_pack_weights(const void* w_q, const void* w_k, int hidden, void* w_pack,
                                   void* stream);

/*
 * Inference routing of every score row: candidates (remote, optionally AND cand,
 * falling back to remote), x = z*idx_scale, top-M by (value desc, block id asc),
 * 1.5-entmax prior over the M values, first K' = max(1,min(K,M)) slots, bias =
 * valid ? (log(max(prior,floor)) - mean_valid)/sigma : 0.
 * Replaces _infer_route_select (modeling_deepseekv2.py:309-333) with entmax15
 * (dash_attention.py:615-662).  nblk_cols <= 2048.  topm in 1..16: one kernel whose
 * entmax matches the serial sort-based computation bit for bit.  topm <= 0 (entmax
 * over the whole row, as modeling_deepseekv2.py:323 allows) or topm > 16: one row per
 * wavefront, the threshold by bisection in double then exact on the support; K <= 64.
 *   z         fp32 [rows, z_stride]; row_nblk optional per-row block count
 *   cand      optional uint8 [rows, cand_stride]
 *   idx/bias/valid  [rows, Kout]; slots >= K' get idx -1, bias 0, valid 0.
 *   idx holds the selected block id also where valid == 0 (as topk does).
 */
int dash_route(const float* z, int64_t z_stride, int rows, int nblk_cols,
               const int32_t* row_nblk, const uint8_t* cand, int64_t cand_stride,
               float idx_scale, float floor_p, float sigma, int K, int topm, int Kout,
               int32_t* idx, float* bias, uint8_t* valid, void* stream);

/*
 * Training routing of every score row (dash_attention.py:906-960, _route then
 * _select_and_bias): candidates as dash_route; x = cand ? z*idx_scale : -1e4
 * (non-finite -> -1e4); prior = 1.5-entmax(x) over the row's first nb columns
 * (nb = row_nblk[r] or nblk_cols); the K' = max(1, min(K, nb)) largest of
 * (cand ? prior : -1), ties to the lower block id; valid = candidate; bias =
 * valid ? clamp((log(max(prior,floor)) - mean_valid)/sigma, +-1e4) : 0.
 * K <= 64, Kout <= 64, Kout >= K', nblk_cols <= 2048.
 *   idx/bias/valid/topv [rows, Kout]: slots >= K' get idx -1, bias 0, valid 0, topv -1.
 *   topv is the masked prior of each slot (-1 for a non-candidate).
 *   stat fp32 [rows, 2]: the row maximum of x and the entmax threshold, which
 *   dash_train_route_backward uses to recompute the prior.
 */
int dash_train_route(const float* z, int64_t z_stride, int rows, int nblk_cols,
                     const int32_t* row_nblk, const uint8_t* cand, int64_t cand_stride,
                     float idx_scale, float floor_p, float sigma, int K, int Kout, int32_t* idx,
                     float* bias, uint8_t* valid, float* topv, float* stat, void* stream);

/*
 * Gradient of dash_train_route's bias with respect to z, as autograd differentiates
 * _route/_select_and_bias (dash_attention.py:906-960) through the clamp, the
 * centred log of the clamped prior and _Entmax15.backward (dash_attention.py:650-658).
 * Takes the same z/row_nblk/cand/scalars as the forward call and its idx, valid,
 * topv and stat outputs; dbias fp32 [rows, Kout]; writes dz fp32 [rows, dz_stride]
 * for every column < nblk_cols (0 outside the candidates).
 */
int dash_train_route_backward(const float* z, int64_t z_stride, int rows, int nblk_cols,
                              const int32_t* row_nblk, const uint8_t* cand, int64_t cand_stride,
                              float idx_scale, float floor_p, float sigma, int Kout,
                              const int32_t* idx, const uint8_t* valid, const float* topv,
                              const float* stat, const float* dbias, float* dz, int64_t dz_stride,
                              void* stream);

/*
 * Prefill block-sparse attention (q_len == k_len), bf16 in/out, fp32 accumulation:
 * window keys [max(t-LW+1, kmin[t]), t] with bias 0 and the keys kmin[t] <= j < t-LW+1
 * of the routed blocks idx[t, :] (skipped where idx < 0 or valid == 0) with bias[t, slot].
 * Replaces triton_gather_attention_e2e / _e2e_attn_fwd_kernel
 * (sparse_gather_e2e_triton.py:34-115, :342-391) and, with bias = 0 and kmin = the
 * packing segment start, triton_gather_attention (sparse_gather_triton.py:29-104,
 * :343-392).  q/k/v/o [B, H, S, D] by strides (or varlen via cu_seqlens, S = the longest
 * sequence); lse (optional) fp32 at lse[token_row*lse_row + h*lse_sh].  D == 128,
 * block_size in {32, 64, ..., 256}, K <= 64.  K > 16 needs block_size <= 64 and a
 * workspace (dense_threshold > 0): every routed pair then takes the sparse path.
 * dense_threshold > 0 (block_size <= 64): routed blocks selected by fewer than
 * dense_threshold of the 128 queries of a tile go through the block-major sparse path,
 * which needs `workspace` (dash_attn_prefill_workspace_size bytes, 256-byte aligned, any
 * contents: the call clears its counters first) and total_rows (B*S, or cu_seqlens[B]).
 * dense_threshold <= 0: every routed block of a tile is processed with the tile; when
 * the grid of tiles (ceil(S / 128) x H x B) is too small to fill the chip and a workspace
 * of dash_attn_prefill_split_workspace_size bytes is given, each tile's items are divided
 * among several work-groups whose partials a second launch merges (no workspace: one
 * work-group per tile).  Calls sharing a workspace must not overlap.
 */
int dash_attn_prefill(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                      const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                      const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                      void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                      float* lse, int64_t lse_row, int64_t lse_sh,
                      const int32_t* idx, const uint8_t* valid, const float* bias, int K,
                      const int32_t* cu_seqlens, const int32_t* kmin,
                      int B, int H, int S, int D, int block_size, int local_window,
                      float scale, int dense_threshold, int64_t total_rows,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of dash_attn_prefill (the sparse path's plan, or split tiles). */
int dash_attn_prefill_workspace_size(int B, int H, int S_max, int64_t total_rows, int K, int D,
                                     int block_size, int64_t* bytes);

/* Workspace bytes of dash_attn_prefill's split tiles (dense_threshold <= 0); 0 when the
 * grid of tiles needs no split (512 tiles or more, or sequences of more than 64 tiles).  No counterpart in the reference (whose Triton kernel
 * launches one program per query tile): a property of this library's decomposition. */
int dash_attn_prefill_split_workspace_size(int B, int H, int S_max, int D, int64_t* bytes);

/* Workspace bytes of dash_attn_prefill_backward. */
int dash_attn_prefill_backward_workspace_size(int B, int H, int S_max, int64_t total_rows, int K,
                                              int D, int block_size, int64_t* bytes);

/*
 * Backward of dash_attn_prefill: dq, dk, dv (bf16, the layouts and strides of q, k, v)
 * and dbias fp32 [total_rows, K] (the gradient of every routed slot's bias: summed over
 * heads and the block's visible keys for the first valid slot of a block, 0 for the other
 * slots; NULL: not computed).  Replaces the Triton backward of the fused gather attention
 * (_E2EGatherAttnFn.backward, sparse_gather_e2e_triton.py:311-339, with its dq/d_bias
 * kernel :118-190 and dk/dv kernel :193-262).  o and lse (natural log, lse[row * lse_row
 * + h * lse_sh]) are the forward's outputs; dout the gradient of o.  Same routing, varlen
 * and kmin arguments as the forward; block_size in {32, 64, ..., 256}, K <= 64, D == 128.
 * workspace: dash_attn_prefill_backward_workspace_size bytes, 256-byte aligned, any
 * contents.  Calls sharing a workspace must not overlap.
 */
int dash_attn_prefill_backward(const void* q, int64_t q_sb, int64_t q_sh, int64_t q_st,
                               const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                               const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                               const void* o, int64_t o_sb, int64_t o_sh, int64_t o_st,
                               const void* dout, int64_t do_sb, int64_t do_sh, int64_t do_st,
                               const float* lse, int64_t lse_row, int64_t lse_sh,
                               const int32_t* idx, const uint8_t* valid, const float* bias,
                               int K, const int32_t* cu_seqlens, const int32_t* kmin,
                               int B, int H, int S, int D, int block_size, int local_window,
                               float scale,
                               void* dq, int64_t dq_sb, int64_t dq_sh, int64_t dq_st,
                               void* dk, int64_t dk_sb, int64_t dk_sh, int64_t dk_st,
                               void* dv, int64_t dv_sb, int64_t dv_sh, int64_t dv_st,
                               float* dbias, int64_t total_rows, void* workspace,
                               int64_t workspace_bytes, void* stream);

/*
 * Byte offset, inside a dash_attn_prefill workspace of these sizes, of the plan's int32
 * error word: 0 after a call whose pair counts fit the workspace; nonzero if a chunk
 * record or partial position would have fallen outside it (such writes are skipped and
 * the affected pairs contribute nothing).  Cleared at the start of every call.  No
 * counterpart in the reference (its Triton kernels keep no plan).
 */
int dash_attn_prefill_error_offset(int B, int H, int S_max, int64_t total_rows, int K, int D,
                                   int block_size, int64_t* offset);

/*
 * Host-side form of the scatter kernel's bounds rule (the same function runs in the
 * kernel): the chunk record and partial position of the q-th sparse pair of a block whose
 * chunks start at block_chunk, for a sequence whose pair positions start at pos0.
 * Returns 0 if both fall inside (chunk_cap records, ppos positions), else -3.  Host code
 * only (no device pointers): for checks of the plan arithmetic without a GPU.
 */
int dash_prefill_plan_target(int64_t chunk_cap, int64_t ppos, int64_t pos0, int64_t block_chunk,
                             int64_t q, int64_t* rec_chunk, int64_t* pair_pos);

/*
 * Decode router, one query per sequence at q_pos[b] (NULL: the last cached token,
 * seq_lens[b]-1; a position past the last cached token is taken as that token):
 * refreshes k_bar of the tail block (refresh_tail = 1), scores every block of the
 * sequence (remote: c <= q_pos[b] / block_size - local_blocks) and routes the row exactly
 * as dash_route does.  Replaces the decode routing of
 * _dash_decode_forward (modeling_deepseekv2.py:481-496: _block_scores_infer over the whole
 * index-key cache + _infer_route_select), keeping the summaries of complete blocks cached.
 *   idx_q    fp32 [B, d] rows (iq_sb); idx_k index-key cache addressed like dash_kbar
 *   kbar     [B, nblk_cap, d] fp32 cache (updated in place at the tail block), or with
 *            kb_table a page pool [pages, d]: the row of block c of sequence b is
 *            kb_table[b * kb_ts + c] (one page per block; the serving path's KBarCache,
 *            whl:sglang/srt/layers/attention/unlimited_dash_ops/dash_stage0.py:106-148),
 *            kb_ts >= nblk_cap
 *   bounds   optional int32 [B, 2] (lo, hi) from dash_decode_win_bounds: only blocks
 *            lo <= c < hi are scored, the others score as not remote (their k_bar rows are
 *            not read).  With bounds computed from the same candidate rows the routing is
 *            identical to the unbounded one; z outside the span reads -1e9.
 *   z        [B, z_stride] fp32 scores (written, for inspection)
 *   One 1024-thread work-group per sequence; with refresh_tail and local_blocks >= 1 a
 *   second one per sequence refreshes the tail block beside the routing (the tail block
 *   holds the query, so it is never remote and the routing does not read its row).
 *   nblk_cap <= 2048, d <= 256.
 */
int dash_decode_route(const float* idx_q, int64_t iq_sb, const float* idx_k,
                      int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
                      const int32_t* block_table, int64_t table_stride, int page_size,
                      const int32_t* seq_lens, const int32_t* q_pos, int S,
                      const float* head_cls, int refresh_tail,
                      float* kbar, int64_t kb_sb, int nblk_cap, const int32_t* kb_table,
                      int64_t kb_ts, const int32_t* bounds, const uint8_t* cand,
                      int64_t cand_stride, int B, int d, int block_size, int local_blocks,
                      float idx_scale, float floor_p, float sigma, int K, int topm, int Kout,
                      int32_t* idx, float* bias, uint8_t* valid, float* z, int64_t z_stride,
                      void* stream);

/* Workspace bytes dash_attn_decode needs for (B, H, D, nsplit). */
int dash_attn_decode_workspace_size(int B, int H, int D, int nsplit, int64_t* bytes);

/*
 * Decode attention, one query per sequence at q_pos[b] (default seq_lens[b]-1):
 * window (q-LW, q] plus the keys < q-LW+1 of the routed blocks idx[b, :] with their bias.
 * Replaces _decode_attend (modeling_deepseekv2.py:424-451) as called by
 * _dash_decode_forward (:454-500).  Cache: contiguous [B, H, S, D] (k_sb, k_sh, k_st) or
 * paged [pages, page_size, H, D] (k_sp, k_st, k_sh + block_table).  Split-K over nsplit
 * (<= 64) wavefronts per (b, h), then a merge kernel.  out [B, H, D] fp32 (out_bf16 = 0)
 * or bf16, lse optional.  D == 128, block_size 32 or a multiple of 64, K <= 64.
 * workspace: dash_attn_decode_workspace_size bytes (the split partials), 16-byte aligned.
 */
int dash_attn_decode(const void* q, int64_t q_sb, int64_t q_sh,
                     const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t k_sp,
                     const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t v_sp,
                     const int32_t* block_table, int64_t table_stride, int page_size,
                     const int32_t* seq_lens, const int32_t* q_pos,
                     const int32_t* idx, const uint8_t* valid, const float* bias, int K,
                     void* out, int out_bf16, int64_t o_sb, int64_t o_sh,
                     float* lse, int64_t lse_sb, int64_t lse_sh,
                     int B, int H, int S, int D, int block_size, int local_window,
                     float scale, int nsplit, void* workspace, int64_t workspace_bytes,
                     void* stream);

/* Workspace bytes dash_decode_step needs (the window and routed partials and the
 * routing words the routers hand to the same launch). */
int dash_decode_step_workspace_size(int B, int H, int D, int block_size, int local_window,
                                    int64_t* bytes);

/*
 * One decode step: dash_decode_route followed by dash_attn_decode of its routing for
 * the query at q_pos[b] (NULL: seq_lens[b]-1), the way _dash_decode_forward (modeling_deepseekv2.py:
 * 454-500) chains _infer_route_select and _decode_attend.  The router arguments are
 * those of dash_decode_route (idx/bias/valid/z are its outputs, [B, Kout]); the
 * attention arguments those of dash_attn_decode with K = Kout.  The window part of the
 * attention runs in the router's launch (it does not depend on the routing).  When that
 * launch fits on the GPU's CUs at once, its window wavefronts then take the routed blocks
 * as each sequence's router publishes its slots; otherwise a second launch does.  The
 * last launch merges.  Kout <= 16; ceil((local_window + block_size - 1) / 32) + Kout <=
 * 64.  workspace: at least dash_decode_step_workspace_size bytes, 16-byte aligned.
 * Its last B * 256 bytes below its last whole-256-byte boundary hold the routing words
 * the routers hand to the same launch: they must be zero before the first call (a
 * zero-filled buffer), and every call leaves them zero.  Pass a buffer with the same
 * workspace_bytes on every call; a smaller batch may use a buffer sized for a larger
 * one.  Calls that share a workspace must not overlap.
 */
int dash_decode_step(const float* idx_q, int64_t iq_sb, const float* idx_k, int64_t ik_sb,
                     int64_t ik_st, int64_t ik_sp, const int32_t* block_table,
                     int64_t table_stride, int page_size, const int32_t* seq_lens,
                     const int32_t* q_pos, int S,
                     const float* head_cls, int refresh_tail, float* kbar, int64_t kb_sb,
                     int nblk_cap, const int32_t* kb_table, int64_t kb_ts, const int32_t* bounds,
                     const uint8_t* cand, int64_t cand_stride, int d,
                     int local_blocks, float idx_scale, float floor_p, float sigma, int K,
                     int topm, int Kout, int32_t* idx, float* bias, uint8_t* valid, float* z,
                     int64_t z_stride,
                     const void* q, int64_t q_sb, int64_t q_sh,
                     const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st, int64_t k_sp,
                     const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st, int64_t v_sp,
                     void* out, int out_bf16, int64_t o_sb, int64_t o_sh,
                     float* lse, int64_t lse_sb, int64_t lse_sh,
                     int B, int H, int D, int block_size, int local_window, float scale,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Page ids of prompt rows: replaces _build_page_aware_ids (_sparse_base_impl.py:2189-2259).
 *   ids          int64 token ids [B, L] (row stride ids_sb)
 *   image_mask   u8 [B, L]: token == image_token_id
 *   image_page_ids int32 [B, L]: page of each image token (-1 elsewhere): <PAGE> markers
 *                seen so far - 1 when the prompt has a marker before its last image token,
 *                else (image tokens before it) / per_page_tokens
 *   query_page_ids int32 [B, L]: the page a query at that position belongs to (-1: none;
 *                inside the prompt only with page_scope_prefill)
 *   enabled      int32 [B, 2] or NULL: (row has an image token, row has a query page)
 *   workspace    dash_pages_workspace_size(B, L) bytes, 16-byte aligned (chunk summaries)
 * Two launches: per-chunk marker and image counts, then every chunk from its prefix.
 */
int dash_page_ids(const int64_t* ids, int64_t ids_sb, int B, int L, int64_t image_token_id,
                  int64_t page_token_id, int per_page_tokens, int page_scope_prefill,
                  uint8_t* image_mask, int32_t* image_page_ids, int32_t* query_page_ids,
                  int32_t* enabled, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of dash_page_ids and dash_decode_page_state for B rows of L tokens. */
int dash_pages_workspace_size(int B, int L, int64_t* bytes);

/*
 * Image pages of every key block: bmin/bmax int32 [B, nblk] (-1 with no image token) and
 * bits u64 [B, nblk] (bit k: page bmin + k has an image token in the block), from
 * image_page_ids [B, L] (row stride ipi_sb).  Feeds dash_block_cand.
 */
int dash_block_pages(const int32_t* image_page_ids, int64_t ipi_sb, int B, int L,
                     int block_size, int nblk, int32_t* bmin, int32_t* bmax, uint64_t* bits,
                     void* stream);

/*
 * Per-query routing candidates [B, Lq, nblk] u8 (strides cand_sb, cand_st): replaces
 * _build_kl_candidate_mask (_sparse_base_impl.py:2457-2484) as _dash_block_cand calls it
 * (modeling_deepseekv2.py:96-110).  mode 0: blocks holding an image token of the query's
 * page (query_page_ids [B, Lqp] at pos [B, Lq], clamped; pos NULL: 0..Lq-1); mode 1:
 * blocks holding any image token; mode 2: every block.  A row with no candidate allows
 * every block (the reference's per-query fallback).  nblk <= 2048.
 */
int dash_block_cand(const int32_t* query_page_ids, int64_t qpi_sb, int Lqp, const int32_t* pos,
                    int64_t pos_sb, int Lq, const int32_t* image_page_ids, int64_t ipi_sb,
                    int Lk, const int32_t* bmin, const int32_t* bmax, const uint64_t* bits,
                    int nblk, int mode, int B, int block_size, uint8_t* cand, int64_t cand_sb,
                    int64_t cand_st, void* stream);

/*
 * Decode page state of prompt rows: the prefill branch of _uocr_dash_decode_allow
 * (modeling_anantaocr.py:465-479).  bmin/bmax int32 [B, nblk] (the smallest/largest image
 * page of each block, -1 with none; nblk * block_size >= L), prompt_pages int32 [B]
 * (markers up to the last image token), markers int32 [B] (markers in the row).
 * block_size <= 1024; workspace: dash_pages_workspace_size(B, L) bytes, 16-byte aligned.
 */
int dash_decode_page_state(const int64_t* ids, int64_t ids_sb, int B, int L,
                           int64_t image_token_id, int64_t page_token_id, int per_page_tokens,
                           int block_size, int nblk, int32_t* bmin, int32_t* bmax,
                           int32_t* prompt_pages, int32_t* markers, void* workspace,
                           int64_t workspace_bytes, void* stream);

/*
 * Decode allow row: the decode branch of _uocr_dash_decode_allow (modeling_anantaocr.py:
 * 480-496).  new_ids int64 [B] (stride new_stride) is the step's token; markers is
 * updated in place.  allow u8 [B, nblk] (row stride allow_sb): blocks with
 * bmin <= page <= bmax for the query's page, or every block when it has none.
 */
int dash_decode_allow(const int64_t* new_ids, int64_t new_stride, int B, int64_t page_token_id,
                      const int32_t* bmin, const int32_t* bmax, int nblk_state,
                      const int32_t* prompt_pages, int32_t* markers, int nblk, uint8_t* allow,
                      int64_t allow_sb, void* stream);

/*
 * Window bounds of decode rows, as the serving router computes them
 * (_win_bounds_kernel, whl:sglang/srt/layers/attention/unlimited_dash_ops/
 * route_triton.py:466-505, one decode query per sequence): for the query at q_pos[b]
 * (NULL: len - 1), the span [lo, hi) of blocks c < min(nblk_cap, allow_w) with
 * allow[b, c] != 0, c <= q_pos / block_size - local_blocks and c * block_size < len;
 * with none, [0, min(nblk_cap, max(ceil(len / block_size), 1))), or [0, 0) when no
 * block is remote.  bounds int32 [B, 2]; fit (optional) u8 [B] = (hi - lo <= tile).
 * Replaces win_bounds_decode (route_triton.py:508-526).
 */
int dash_decode_win_bounds(const uint8_t* allow, int64_t allow_sb, int allow_w,
                           const int32_t* seq_lens, const int32_t* q_pos, int B, int S,
                           int nblk_cap, int block_size, int local_blocks, int tile,
                           int32_t* bounds, uint8_t* fit, void* stream);

/*
 * Page2D RoPE coordinates of prompt rows: tok[b, t] (running count of tokens of the same
 * page up to t, minus 1, optionally scaled by page_span) and page[b, t] (<PAGE> markers up
 * to t; after the last image token, minus the prompt's pages), int64 [B, L] row stride L;
 * pf_cnt[b, p] (tokens of page p up to the last image token) for p = 0 .. L, int64 with row
 * stride pf_stride >= L + 1; meta int64 [2] = (1 + the largest page id of the batch, 1 if
 * every row has a <PAGE> marker at or before its last image token, else 0: then the
 * reference falls back to 1-D RoPE).  Replaces _build_page_rope_pos and _page_rope_offsets
 * (_sparse_base_impl.py:2269-2362) without host synchronisation (ids pre-padded / cut to L
 * as the reference does).  workspace: dash_page_rope_workspace_size bytes, 256-byte aligned.
 */
int dash_page_rope_workspace_size(int B, int L, int64_t* bytes);
int dash_page_rope_pos(const int64_t* ids, int64_t ids_sb, int B, int L, int64_t image_token_id,
                       int64_t page_token_id, int page_span, int64_t* tok, int64_t* page,
                       int64_t* pf_cnt, int64_t pf_stride, int64_t* meta, void* workspace,
                       int64_t workspace_bytes, void* stream);

/*
 * cos / sin [B, S, 2 * (n_tok + page_pairs)] (bf16 or fp32, batch/token strides cs_sb,
 * cs_st) of the two-axis RoPE at coordinates tok / page (int64, batch stride pos_sb):
 * pair j < n_tok turns by tok * inv_tok[j], pair n_tok + i by (page mod page_mod, when
 * page_mod > 0) * inv_page[i], and the second half of the row repeats the first.
 * Replaces DeepseekV2IndexerRotary2D.forward (_sparse_base_impl.py:1876-1891).
 */
int dash_rope2d_cos_sin(const int64_t* tok, const int64_t* page, int64_t pos_sb, int B, int S,
                        const float* inv_tok, int n_tok, const float* inv_page, int page_pairs,
                        int page_mod, void* cos, void* sin, int out_bf16, int64_t cs_sb,
                        int64_t cs_st, void* stream);

/*
 * One decode token per row advances the page coordinates in place: page[b] / tok[b] (int64
 * [B]); a <PAGE> token moves to min(page + 1, meta[0] - 1) and restarts at pf_cnt[b, page],
 * any other token increments tok.  The new (tok, page) are also written to out_tok /
 * out_page when non-null.  Replaces the decode branch of _main_rope_coords
 * (_sparse_base_impl.py:1384-1390); pf_cnt and meta as dash_page_rope_pos writes them.
 */
int dash_page_rope_advance(const int64_t* new_ids, int64_t new_stride, int B,
                           int64_t page_token_id, int64_t* page, int64_t* tok,
                           const int64_t* pf_cnt, int64_t pf_stride, const int64_t* meta,
                           int64_t* out_tok, int64_t* out_page, void* stream);

/*
 * Allocation-free decode step.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops).
 * Same arguments and results as dash_decode_step without the workspace: the window and
 * routed-block partials live in a fixed 64 MiB device array of this library
 * (dash_decode_step_scratch_bytes()), one per GPU, held until the process ends.  Sizes
 * whose dash_decode_step_workspace_size exceeds it return -5.  Calls that overlap on one
 * GPU share that array and race; nothing in it needs clearing between calls.
 */
int dash_decode_step_noalloc(const float* idx_q, int64_t iq_sb, const float* idx_k,
                             int64_t ik_sb, int64_t ik_st, int64_t ik_sp,
                             const int32_t* block_table, int64_t table_stride, int page_size,
                             const int32_t* seq_lens, const int32_t* q_pos, int S,
                             const float* head_cls, int refresh_tail, float* kbar,
                             int64_t kb_sb, int nblk_cap, const int32_t* kb_table,
                             int64_t kb_ts, const int32_t* bounds, const uint8_t* cand,
                             int64_t cand_stride, int d, int local_blocks, float idx_scale,
                             float floor_p, float sigma, int K, int topm, int Kout,
                             int32_t* idx, float* bias, uint8_t* valid, float* z,
                             int64_t z_stride,
                             const void* q, int64_t q_sb, int64_t q_sh,
                             const void* k, int64_t k_sb, int64_t k_sh, int64_t k_st,
                             int64_t k_sp,
                             const void* v, int64_t v_sb, int64_t v_sh, int64_t v_st,
                             int64_t v_sp,
                             void* out, int out_bf16, int64_t o_sb, int64_t o_sh,
                             float* lse, int64_t lse_sb, int64_t lse_sh,
                             int B, int H, int D, int block_size, int local_window, float scale,
                             void* stream);

/* Bytes of the fixed scratch array dash_decode_step_noalloc uses (per GPU). */
int64_t dash_decode_step_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* DASH_HIP_H */
