"""Fused gather attention and block-max scoring on the HIP kernels.

Drop-in counterparts of the reference's Triton entry points, with the same
arguments, shapes and "return None on an unsupported input" behaviour:

* ``triton_gather_attention_e2e`` -- sparse_gather_e2e_triton.py:342-391
* ``triton_gather_attention``     -- sparse_gather_triton.py:343-392 (packing
  ``seg`` start from position_ids, no bias)
* ``triton_block_max_score``      -- sparse_gather_triton.py:431-467

The names are kept so existing call sites import them unchanged; the work runs
in ``libdash_hip.so`` (dash_attn_prefill, dash_block_max_score).  The fused entry
point records autograd when its inputs require grad (the backward runs in
dash_attn_prefill_backward), and so does ``triton_gather_attention`` (no bias;
gradients to q, k and v).
"""

import torch

from . import ops


def gather_attention_e2e(query_states, key_states, value_states, block_indices,
                         blk_bias_slots, position_ids, attention_mask, block_size, scale,
                         local_window=None):
    """[B,HQ,T,D] block-sparse attention with per-slot block bias, or None on an
    unsupported input (attention mask, multi index heads, prefix cache, non-arange
    positions), exactly where the reference returns None.

    block_indices [B,1,T,K] int (-1 = unused slot), blk_bias_slots [B,T,K]."""
    if attention_mask is not None:
        return None
    if block_indices.shape[1] != 1:
        return None
    B, HQ, T, D = query_states.shape
    if key_states.shape[2] != T:
        return None
    if position_ids is None or position_ids.dim() != 2 or position_ids.shape[-1] != T:
        return None
    ar = torch.arange(T, device=position_ids.device)
    if not bool((position_ids == ar).all()):
        return None
    if key_states.shape[1] != HQ:
        rep = HQ // key_states.shape[1]
        key_states = key_states.repeat_interleave(rep, dim=1)
        value_states = value_states.repeat_interleave(rep, dim=1)
    lw = block_size if local_window is None else max(1, int(local_window))
    sel = block_indices[:, 0]
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in
                                       (query_states, key_states, value_states, blk_bias_slots)):
        # gradients to q, k, v and the bias slots (_E2EGatherAttnFn, :288-339)
        return ops.attn_prefill_autograd(query_states, key_states, value_states, sel,
                                         blk_bias_slots, None, block_size, lw, scale)
    return ops.attn_prefill(query_states, key_states, value_states, sel, blk_bias_slots, None,
                            block_size, lw, scale)


def gather_attention(query_states, key_states, value_states, block_indices, position_ids,
                     attention_mask, block_size, scale, local_window=None):
    """[B,HQ,T,D] block-sparse attention without bias; packed rows (position_ids
    restarting at 0) keep every query inside its segment [t - position_ids[t], t].
    block_indices [B,HI,T,S]: query head h uses index head h // (HQ / HI).  Returns
    None where the reference does (mask, prefix cache, index heads that do not divide
    the heads).  Records autograd (q, k, v) when its inputs require grad."""
    if attention_mask is not None:
        return None
    B, HQ, T, D = query_states.shape
    HI = block_indices.shape[1]
    Hkv = key_states.shape[1]
    if HI < 1 or HQ % HI != 0 or Hkv % HI != 0:
        return None
    if key_states.shape[2] != T:
        return None
    if position_ids is None or position_ids.dim() != 2 or position_ids.shape[-1] != T:
        return None
    if Hkv != HQ:
        key_states = key_states.repeat_interleave(HQ // Hkv, dim=1)
        value_states = value_states.repeat_interleave(HQ // Hkv, dim=1)
    # every row's segment start (sparse_gather_triton.py:374), 0 on unpacked rows; the
    # kernels read it per token row b * T + t, so packed rows of any batch size work
    ar = torch.arange(T, device=position_ids.device)
    seg = (ar[None, :] - position_ids).to(torch.int32).expand(B, T)
    lw = block_size if local_window is None else max(1, int(local_window))
    kmin = seg.reshape(-1)
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in
                                           (query_states, key_states, value_states))
    # query head h reads index head h // (HQ / HI) (sparse_gather_triton.py:47)
    G = HQ // HI
    outs = []
    for g in range(HI):
        hs = slice(g * G, (g + 1) * G)
        sel = block_indices[:, g]
        zero_bias = torch.zeros(sel.shape, dtype=torch.float32, device=sel.device)
        args = (query_states[:, hs], key_states[:, hs], value_states[:, hs], sel, zero_bias,
                None, block_size, lw, scale)
        # the unbiased backward of _TritonGatherAttnFn (sparse_gather_triton.py:107-244)
        outs.append(ops.attn_prefill_autograd(*args, kmin=kmin) if grad else
                    ops.attn_prefill(*args, kmin=kmin))
    return outs[0] if HI == 1 else torch.cat(outs, dim=1)


def block_max_score(q, k, pos, seg, block_size, num_key_blocks, local_window=None):
    """[B,C,nblk] fp32: max of q.k over keys seg <= j < max(pos-LW+1, 0), -inf where
    a block has none (sparse_gather_triton.py:431-467)."""
    if q.dim() != 3 or k.dim() != 3:
        raise AssertionError("expects [B, C, D] / [B, Sk, D]")
    if q.shape[-1] > 256:
        raise NotImplementedError(f"index dim D={q.shape[-1]} > 256 not supported")
    return ops.block_max_score(q, k, pos, seg, block_size, num_key_blocks, local_window, mode=1)


# the reference's names, for call sites that import them directly
triton_gather_attention_e2e = gather_attention_e2e
triton_gather_attention = gather_attention
triton_block_max_score = block_max_score
