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

    def __init__(self, kbar):
        self.kbar = kbar


def init_decode_state(idx_k, head_cls, block_size, nblk_cap, seq_lens=None, block_table=None,
                      page_size=None):
    kb = ops.kbar(idx_k, head_cls, block_size, seq_lens=seq_lens, nblk_cap=nblk_cap,
                  block_table=block_table, page_size=page_size)
    return DecodeState(kb)


def decode_step(state, q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale,
                floor, sigma, K, topm, scale=None, seq_lens=None, block_table=None,
                page_size=None, out_dtype=torch.float32, nsplit=None, block_cand=None,
                return_routing=False, fused=None, return_scores=False):
    """One decode step for the query at the last cached token of each sequence.
    The newest token is already in k/v and idx_k; its block's summary is refreshed
    inside the fused decode router.  fused (default: whenever nsplit is not given and
    the shapes allow it) runs the window part of the attention beside the router
    (ops.decode_step_fused); otherwise decode_route then attn_decode.  return_scores
    (with return_routing) also returns the block scores [B, nblk_cap] of the router."""
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
            return_scores=True)
        if return_routing:
            res = (out, (idx, bias, valid.bool()))
            return res + (z,) if return_scores else res
        return out
    idx, bias, valid, z = ops.decode_route(idx_q, idx_k, head_cls, state.kbar, block_size,
                                           local_blocks, idx_scale, floor, sigma, K, topm,
                                           seq_lens=seq_lens, block_table=block_table,
                                           page_size=page_size, cand=block_cand, width=width,
                                           valid_dtype=torch.uint8, return_scores=True)
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
