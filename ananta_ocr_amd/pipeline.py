"""DASH prefill and decode passes built from the HIP ops.

``prefill`` is the inference prefill of modeling_deepseekv2.py:403-421 (k_bar ->
block scores -> route -> fused attention) and ``decode_step`` the decode step of
modeling_deepseekv2.py:481-498, except that the k_bar cache is refreshed only at
the tail block instead of being rebuilt from the whole index-key cache every step
(the summaries of complete blocks never change).
"""

import math

import torch

from . import ops


def prefill(q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale, floor,
            sigma, K, topm, scale=None, cu_seqlens=None, max_seqlen=None, block_cand=None,
            return_routing=False):
    """q/k/v bf16 [B,H,S,D] (or [1,H,T,D] + cu_seqlens), idx_q/idx_k fp32 [B,S,d].
    With cu_seqlens, max_seqlen (the longest document) keeps the pass free of host
    synchronisations, so that it can be captured in a HIP graph."""
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    kb = ops.kbar(idx_k, head_cls, block_size, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    z = ops.block_scores(idx_q, kb, block_size, local_blocks, cu_seqlens=cu_seqlens,
                         max_seqlen=max_seqlen)
    if cu_seqlens is not None:
        lens = (cu_seqlens[1:] - cu_seqlens[:-1]).to(torch.int32)
        nblk_doc = (lens + block_size - 1) // block_size
        row_nblk = torch.repeat_interleave(nblk_doc, lens.long(), output_size=z.shape[0])
        width = max(1, min(int(K), int(topm))) if int(topm) > 0 else max(1, int(K))
        idx, bias, valid = ops.route(z, block_cand, idx_scale, floor, sigma, K, topm,
                                     row_nblk=row_nblk, width=width)
    else:
        idx, bias, valid = ops.route(z, block_cand, idx_scale, floor, sigma, K, topm)
    out = ops.attn_prefill(q, k, v, idx, bias, valid, block_size, local_blocks * block_size,
                           scale, cu_seqlens=cu_seqlens, max_seqlen=max_seqlen)
    if return_routing:
        return out, (idx, bias, valid.bool())
    return out


class DecodeState:
    """Per-layer decode state: the k_bar cache [B, nblk_cap, d] of the index keys."""

    paged = False

    def __init__(self, kbar):
        self.kbar = kbar


class KBarPageCache:
    """Per-layer k_bar page pool: one fp32 summary per physical KV page [num_pages, d]
    (one page is one routing block), the serving path's KBarCache
    (whl:sglang/srt/layers/attention/unlimited_dash_ops/dash_stage0.py:106-148).  The
    summaries stay with their pages, so sequences can join, leave or be reordered in the
    batch without moving them; the decode router reads the pool through the block table
    and rewrites the tail page's row in place."""

    paged = True

    def __init__(self, num_pages, dim, device):
        # one spare row past the pool takes the writes of table entries that are not
        # refreshed (refresh_from), so that every write of a step is one index_copy_
        self._buf = torch.zeros(num_pages + 1, dim, dtype=torch.float32, device=device)
        self.kbar = self._buf[:num_pages]

    def put(self, pages, k_bar):
        """Write the summaries k_bar [n, d] of the given physical pages [n]."""
        self.kbar[pages.reshape(-1).long()] = k_bar.reshape(-1, self.kbar.shape[1]).float()

    def put_sequences(self, idx_k, head_cls, block_size, block_table, seq_lens):
        """Summaries of every page the sequences use (after their prefill): idx_k is the
        paged index-key cache [pages, block_size, d], block_table [B, P], seq_lens [B]."""
        nblk = block_table.shape[1]
        kb = ops.kbar(idx_k, head_cls, block_size, seq_lens=seq_lens, nblk_cap=nblk,
                      block_table=block_table, page_size=block_size)
        nb = (seq_lens.to(torch.int64) + block_size - 1) // block_size
        used = torch.arange(nblk, device=kb.device)[None, :] < nb[:, None]
        self.kbar[block_table.to(torch.int64)[used]] = kb[used]

    def refresh_tail(self, idx_k, head_cls, block_size, block_table, seq_lens, tail_pages=1):
        """Recompute the last tail_pages summaries of every sequence
        (dash_stage0.py:121-148) -- the decode router already refreshes the last one."""
        nblk = block_table.shape[1]
        kb = ops.kbar(idx_k, head_cls, block_size, seq_lens=seq_lens, nblk_cap=nblk,
                      block_table=block_table, page_size=block_size,
                      tail_only=tail_pages == 1)
        nb = (seq_lens.to(torch.int64) + block_size - 1) // block_size
        c = torch.arange(nblk, device=kb.device)[None, :]
        sel = (c < nb[:, None]) & (c >= nb[:, None] - int(tail_pages))
        self.kbar[block_table.to(torch.int64)[sel]] = kb[sel]


    def refresh_from(self, idx_k, head_cls, block_size, block_table, seq_lens, first_block):
        """Recompute the summaries of blocks first_block[b] .. of every sequence (an extend
        step's boundary page and new pages, kbar_all_plan of route_triton.py:576-601),
        without a host synchronisation."""
        nblk = block_table.shape[1]
        kb = ops.kbar(idx_k, head_cls, block_size, seq_lens=seq_lens, nblk_cap=nblk,
                      block_table=block_table, page_size=block_size)
        nb = (seq_lens.to(torch.int64) + block_size - 1) // block_size
        c = torch.arange(nblk, device=kb.device)[None, :]
        sel = (c < nb[:, None]) & (c >= first_block.to(torch.int64)[:, None])
        dump = self._buf.shape[0] - 1
        tgt = torch.where(sel, block_table.to(torch.int64), torch.full_like(c, dump))
        self._buf.index_copy_(0, tgt.reshape(-1), kb.reshape(-1, kb.shape[-1]))


def extend_prefill(state, q, k_cache, v_cache, idx_q, idx_k, head_cls, block_size,
                   local_blocks, idx_scale, floor, sigma, K, topm, block_table, seq_lens,
                   context_lens, cu_seqlens_q, max_query_len=None, scale=None,
                   block_cand=None, out_dtype=torch.bfloat16, return_routing=False):
    """Extend (chunked or prefix-cached) prefill over a paged cache: the query rows of
    request b are the tokens at positions context_lens[b] .. seq_lens[b] - 1 (rows
    cu_seqlens_q[b] .. cu_seqlens_q[b + 1] - 1 of q), attending the request's whole
    cached sequence, as the serving backend's extend path does
    (whl:sglang/srt/layers/attention/unlimited_ocr_v2_backend.py:1302-1335, :1454-1463;
    route_prefill_triton, route_triton.py:529-678) with the routing of
    _infer_route_select (modeling_deepseekv2.py:309-333) per request:

    * the k_bar page pool (state, a KBarPageCache) is refreshed from each request's
      boundary page (context_lens // block_size) on;
    * block scores of each query row at q_pos = context_len + row against the request's
      summaries (remote: c <= q_pos // block_size - local_blocks, c < its block count);
    * routing (top-M, 1.5-entmax, first K, centred log-prior bias) per row;
    * attention of each row over the window (q_pos - LW, q_pos] and its routed blocks.

    q [T,H,D] bf16, k_cache / v_cache [pages, block_size, H, D] bf16 (the new tokens
    already written), idx_q [T,d] fp32, idx_k the paged index keys [pages, block_size, d]
    (new ones written), block_table [B,P] int32 (pages of block_size tokens), seq_lens /
    context_lens [B], cu_seqlens_q [B+1].  max_query_len (the longest request chunk) keeps
    the pass free of host synchronisations.  Returns out [T,H,D] (out_dtype)."""
    if not getattr(state, "paged", False):
        raise NotImplementedError("extend_prefill takes a k_bar page pool (KBarPageCache)")
    T, H, D = q.shape
    B = block_table.shape[0]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    dev = q.device
    seq = seq_lens.to(device=dev, dtype=torch.int64)
    ctx = context_lens.to(device=dev, dtype=torch.int64)
    cu = cu_seqlens_q.to(device=dev, dtype=torch.int64)
    state.refresh_from(idx_k, head_cls, block_size, block_table, seq, ctx // block_size)
    P = block_table.shape[1]
    pages = block_table.to(torch.int64).clamp(0, state.kbar.shape[0] - 1)
    kb_seq = state.kbar.index_select(0, pages.reshape(-1)).view(B, P, -1)
    q_lens = cu[1:] - cu[:-1]
    row_seq = torch.repeat_interleave(torch.arange(B, device=dev), q_lens, output_size=T)
    rows = torch.arange(T, device=dev)
    q_pos = (ctx.index_select(0, row_seq) + rows - cu.index_select(0, row_seq)).to(torch.int32)
    z = ops.block_scores(idx_q.reshape(1, T, -1), kb_seq, block_size, local_blocks,
                         q_pos=q_pos, cu_seqlens=cu, max_seqlen=max_query_len, key_lens=seq,
                         S=P * block_size)
    nblk_b = (seq + block_size - 1) // block_size
    width = max(1, min(int(K), int(topm))) if int(topm) > 0 else max(1, int(K))
    idx, bias, valid = ops.route(z, block_cand, idx_scale, floor, sigma, K, topm,
                                 row_nblk=nblk_b.index_select(0, row_seq), width=width)
    out = ops.attn_rows(q, k_cache, v_cache, idx, bias, valid, q_pos, row_seq, block_size,
                        local_blocks * block_size, scale, seq_lens=seq, block_table=block_table,
                        page_size=block_size, out_dtype=out_dtype)
    if return_routing:
        return out, (idx, bias, valid.bool()), q_pos
    return out


def init_decode_state(idx_k, head_cls, block_size, nblk_cap, seq_lens=None, block_table=None,
                      page_size=None):
    kb = ops.kbar(idx_k, head_cls, block_size, seq_lens=seq_lens, nblk_cap=nblk_cap,
                  block_table=block_table, page_size=page_size)
    return DecodeState(kb)


def decode_step(state, q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale,
                floor, sigma, K, topm, scale=None, seq_lens=None, block_table=None,
                page_size=None, out_dtype=torch.float32, nsplit=None, block_cand=None,
                return_routing=False, fused=None, return_scores=False, bounds=None):
    """One decode step for the query at the last cached token of each sequence.
    The newest token is already in k/v and idx_k; its block's summary is refreshed
    inside the fused decode router.  fused (default: whenever nsplit is not given and
    the shapes allow it) runs the window part of the attention beside the router
    (ops.decode_step_fused); otherwise decode_route then attn_decode.  return_scores
    (with return_routing) also returns the block scores [B, nblk_cap] of the router.
    state: a DecodeState (k_bar per sequence) or a KBarPageCache (k_bar per page, read
    through block_table; page_size must equal block_size).  bounds [B, 2]
    (pages.win_bounds_decode of the candidate rows): only those blocks are scored."""
    kbx = {}
    if state.paged:
        if block_table is None or page_size != block_size:
            raise NotImplementedError("a k_bar page pool needs pages of one block")
        kbx["kbar_table"] = block_table
    if bounds is not None:
        kbx["bounds"] = bounds
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    slots = max(1, min(int(K), int(topm))) if int(topm) > 0 else max(1, int(K))
    width = None if seq_lens is None else slots
    if fused is None:
        npw = (local_blocks * block_size + block_size - 1 + 31) // 32
        fused = nsplit is None and D == 128 and slots <= 16 and npw + slots <= 64
    if fused:
        out, (idx, bias, valid), z = ops.decode_step_fused(
            q, k, v, idx_q, idx_k, head_cls, state.kbar, block_size, local_blocks, idx_scale,
            floor, sigma, K, topm, scale, seq_lens=seq_lens, block_table=block_table,
            page_size=page_size, cand=block_cand, width=width, out_dtype=out_dtype,
            return_scores=True, **kbx)
        if return_routing:
            res = (out, (idx, bias, valid.bool()))
            return res + (z,) if return_scores else res
        return out
    idx, bias, valid, z = ops.decode_route(idx_q, idx_k, head_cls, state.kbar, block_size,
                                           local_blocks, idx_scale, floor, sigma, K, topm,
                                           seq_lens=seq_lens, block_table=block_table,
                                           page_size=page_size, cand=block_cand, width=width,
                                           valid_dtype=torch.uint8, return_scores=True, **kbx)
    out = ops.attn_decode(q, k, v, idx[:, 0], bias[:, 0], valid[:, 0], block_size,
                          local_blocks * block_size, scale, seq_lens=seq_lens,
                          block_table=block_table, page_size=page_size, out_dtype=out_dtype,
                          nsplit=nsplit)
    if return_routing:
        res = (out, (idx, bias, valid.bool()))
        return res + (z,) if return_scores else res
    return out


class DecodeGraph:
    """One ``decode_step`` captured into a HIP graph for fixed buffers.

    The router, the split-K attention and the merge of a step (and the small
    tensor ops between them) are recorded once; ``replay()`` relaunches them all
    with one host call, which is what a serving loop does for every token.  The
    inputs are the captured tensors themselves: write the new query (and the new
    cache rows) into them in place before each replay.  Outputs live in buffers
    owned by the graph and are overwritten by the next replay.
    """

    def __init__(self, state, q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks,
                 idx_scale, floor, sigma, K, topm, scale=None, warmup=2, **kw):
        args = (state, q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale,
                floor, sigma, K, topm, scale)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                decode_step(*args, **kw)
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out, self.routing = decode_step(*args, return_routing=True, **kw)

    def replay(self):
        self.graph.replay()
        return self.out
