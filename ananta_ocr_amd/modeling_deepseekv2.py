"""Inference-time DASH helpers with the reference's signatures, on HIP kernels.

Counterparts of modeling_deepseekv2.py:269-500 (the DASH overlay on the
DeepSeek-V2 attention).  Every function keeps the reference's name, argument
order and return shapes, so the overlay's call sites work unchanged:

* ``configure_dash_inference``            -- :269-306
* ``_infer_route_select``                 -- :309-333
* ``_router_qk``                          -- :336-348
* ``_block_scores_infer``                 -- :351-400
* ``_infer_prefill_attend``               -- :403-421 (caches the index keys, and the
                                             block summaries the decode step reuses, on
                                             ``past_kv``)
* ``_decode_attend``                      -- :424-451
* ``_dash_indexer_rope``                  -- :112-130
* ``_dash_decode_forward``                -- :454-500 (projections, RoPE, cache update,
                                             then ``_dash_decode_attend``)

The decode step differs from the reference in one place, with the same result:
the reference concatenates the whole index-key cache and rebuilds every block
summary each step (:485-489); here the index keys live in a growing buffer and
only the summary of the block holding the new token is recomputed (inside the
fused decode launch, ops.decode_step_fused).
"""

import math
import os

import torch

from . import ops, page_rope, pages
from .dash_attention import DashAttention, apply_rotary, checkpoint_sparse_config

_INFER = {"on": False}


def configure_dash_inference(decoder, on, topm=16, page_scope_prefill=True, state=None):
    """Switch inference routing on/off for every DashAttention in ``decoder``
    (modeling_deepseekv2.py:269-306): sets ``_infer_params`` = {idx_scale, floor,
    sigma, K, topm} per router from the checkpoint's sparse_attention_config (the copy
    taken before the routers wrote into it) and its per-layer scale/floor arrays,
    indexed by the layer's slot among the sparse layers (:256-266).  Stage 0 is
    DASH_STAGE0 if set, else the checkpoint's dash_stage0, else "indexer"."""
    if not on:
        if state is not None:
            pages.PAGE_SCOPE["prefill"] = state["page_scope_prefill"]
            for mod, stage0 in state["stage0"]:
                mod.stage0 = stage0
        _INFER["on"] = False
        return None
    state = {"stage0": [], "page_scope_prefill": pages.PAGE_SCOPE["prefill"]}
    cfg = getattr(decoder, "config", None)
    live = (getattr(cfg, "sparse_attention_config", None) or {}) if cfg is not None else {}
    sp = checkpoint_sparse_config(live)
    stage0 = str(os.environ.get("DASH_STAGE0") or sp.get("dash_stage0") or "indexer").lower()
    budget = sp.get("dash_topk_blocks") or sp.get("dash_image_fallback_remote") or 12
    for slot, router in _dash_routers(decoder, sp):
        scale = _per_layer(sp, "dash_scale_per_layer", slot)
        floor = _per_layer(sp, "dash_floor_per_layer", slot)
        if scale is None:
            scale = float(sp.get("dash_scaling_factor", router.scaling_factor))
        if floor is None:
            floor = float(sp.get("dash_prior_floor", router._prior_floor))
        router._infer_params = dict(idx_scale=float(scale) / math.sqrt(router.index_dim),
                                    floor=float(floor),
                                    sigma=float(sp.get("dash_sigma", router.sigma)),
                                    K=int(budget), topm=int(topm))
        state["stage0"].append((router, router.stage0))
        router.stage0 = stage0
    pages.PAGE_SCOPE["prefill"] = bool(page_scope_prefill)
    _INFER["on"] = True
    return state


def _sched_slot(sp, layer_idx):
    """Index of a layer's entry in the per-layer arrays (modeling_deepseekv2.py:256-260):
    its count among the sparse layers of sparse_attention_freq, else the layer index."""
    freq = sp.get("sparse_attention_freq")
    if not isinstance(freq, (list, tuple)) or layer_idx >= len(freq):
        return int(layer_idx)
    return sum(1 for f in freq[:layer_idx] if f)


def _dash_routers(decoder, sp):
    """(slot, router) of every DashAttention of ``decoder``: through decoder.layers[i]
    .self_attn.dash_router with the layer's layer_idx, as the reference walks them;
    a module tree without such layers gives its routers in order, slot = that order."""
    layers = getattr(decoder, "layers", None)
    if layers is not None:
        out = []
        for i, layer in enumerate(layers):
            attn = getattr(layer, "self_attn", None)
            router = getattr(attn, "dash_router", None)
            if isinstance(router, DashAttention):
                out.append((_sched_slot(sp, int(getattr(attn, "layer_idx", i))), router))
        if out:
            return out
    return list(enumerate(m for m in decoder.modules() if isinstance(m, DashAttention)))


def _per_layer(sp, key, slot):
    arr = sp.get(key)
    if not isinstance(arr, (list, tuple)) or not arr:
        return None
    return float(arr[slot]) if 0 <= slot < len(arr) else None


@torch.no_grad()
def _infer_route_select(block_scores, block_cand, p):
    """(topi [B,Lq,K] int64, bias [B,Lq,K] fp32, valid [B,Lq,K] bool) of the inference
    router (modeling_deepseekv2.py:309-333).  Ties go to the lower block id."""
    ti, bi, va = ops.route(block_scores, block_cand, p["idx_scale"], p["floor"], p["sigma"],
                           p["K"], p["topm"])
    return ti.long(), bi, va


def _router_qk(router, hidden_states, pe):
    """Router index q/k [B,S,d] fp32 (modeling_deepseekv2.py:336-348)."""
    return router.router_qk(hidden_states, pe)


@torch.no_grad()
def _block_scores_infer(router, idx_q, idx_k, q_pos, nblk):
    """[B,Lq,nblk] fp32 block scores of queries at q_pos against every key of idx_k
    (modeling_deepseekv2.py:351-400)."""
    return router.block_scores(idx_q, idx_k, q_pos=q_pos.to(torch.int32), nblk=nblk)


# ----------------------------------------------------------------------------- decode state

class DashDecodeCache:
    """Per-layer decode state of one DASH router: the index keys [B, S, d] fp32 in a
    buffer with spare rows, and the block summaries k_bar [B, nblk_cap, d] fp32 of
    stage 0 ``head_cls`` (``None`` for the indexer stage 0, which scores raw keys).

    ``idx_k`` is a view of the first S rows, which is what the reference keeps in
    ``past_kv._dash_idx_k[layer]``.  Appending past the spare rows reallocates both
    buffers at twice the size (amortised O(1) per token; the reference's
    ``torch.cat`` copies the whole cache every step)."""

    def __init__(self, router, idx_k, spare=None):
        B, S, d = idx_k.shape
        self.bs = router.block_size
        self.head_cls = router.head_cls.detach().float()
        cap = self.capacity(S, self.bs, spare)
        self._buf = torch.zeros(B, cap, d, dtype=torch.float32, device=idx_k.device)
        self._buf[:, :S] = idx_k
        self.S = S
        self.kbar = None
        if router.stage0 == "head_cls":
            self.kbar = ops.kbar(self._buf[:, :S], self.head_cls, self.bs,
                                 nblk_cap=cap // self.bs)

    @staticmethod
    def capacity(S, bs, spare=None):
        cap = max(S + (spare if spare is not None else max(S, 1024)), 1)
        return (cap + bs - 1) // bs * bs

    @classmethod
    def buffers(cls, B, S, d, bs, device, head_cls_stage):
        """Zeroed index-key buffer [B, cap, d] and summaries [B, cap // bs, d] (or None)
        for a prefill of S tokens to write into (then ``from_buffers``)."""
        cap = cls.capacity(S, bs)
        buf = torch.zeros(B, cap, d, dtype=torch.float32, device=device)
        kb = torch.zeros(B, cap // bs, d, dtype=torch.float32, device=device) \
            if head_cls_stage else None
        return buf, kb

    @classmethod
    def from_buffers(cls, router, buf, kbar, S):
        """The cache over buffers a prefill wrote: index keys in buf[:, :S] and, for stage
        0 head_cls, the summaries of its blocks in kbar."""
        dc = cls.__new__(cls)
        dc.bs = router.block_size
        dc.head_cls = router.head_cls.detach().float()
        dc._buf, dc.kbar, dc.S = buf, kbar, S
        return dc

    @property
    def idx_k(self):
        return self._buf[:, :self.S]

    def append(self, idx_k_new):
        """Append [B, L, d] index keys (normally L = 1)."""
        L = idx_k_new.shape[1]
        if self.S + L > self._buf.shape[1]:
            B, cap, d = self._buf.shape
            ncap = (max(2 * cap, self.S + L) + self.bs - 1) // self.bs * self.bs
            buf = torch.zeros(B, ncap, d, dtype=torch.float32, device=self._buf.device)
            buf[:, :self.S] = self._buf[:, :self.S]
            self._buf = buf
            if self.kbar is not None:
                kb = torch.zeros(B, ncap // self.bs, d, dtype=torch.float32,
                                 device=buf.device)
                kb[:, :self.kbar.shape[1]] = self.kbar
                self.kbar = kb
        self._buf[:, self.S:self.S + L] = idx_k_new.float()
        self.S += L


def _decode_caches(past_kv):
    if not hasattr(past_kv, "_dash_decode"):
        past_kv._dash_decode = {}
    return past_kv._dash_decode


# ----------------------------------------------------------------------------- prefill

@torch.no_grad()
def _infer_prefill_attend(self, router, hidden_states, q, k, v, idx_pe, pos_ids, block_cand,
                          attn_mask, past_kv):
    """Prefill (q_len > 1) under inference routing (modeling_deepseekv2.py:403-421).

    ``self`` is the attention layer (its ``layer_idx`` keys the caches on
    ``past_kv``).  The index keys are stored in ``past_kv._dash_idx_k[layer_idx]`` as
    the reference does, and the decode state (index-key buffer and block summaries) in
    ``past_kv._dash_decode[layer_idx]``.  Attention goes through
    ``router._forward_triton`` and, where that returns None, ``router._forward_dense``,
    as in the reference."""
    B, H, S, D = q.shape
    nblk = (S + router.block_size - 1) // router.block_size
    p = router._infer_params
    kb = None
    head_cls = router.stage0 == "head_cls"
    if hidden_states.is_cuda and router._front_ok(hidden_states) and \
            (not head_cls or router.block_size in (32, 64)):
        # one launch: projections, norms, RoPE, guards and the block summaries, the index
        # keys and summaries written straight into the decode cache's buffers
        buf = kbuf = None
        if past_kv is not None:
            buf, kbuf = DashDecodeCache.buffers(B, S, router.index_dim, router.block_size,
                                                q.device, head_cls)
        idx_q, idx_k, kb = router.router_front(hidden_states, idx_pe, with_kbar=head_cls,
                                               idx_k_out=buf, kbar_out=kbuf,
                                               nblk_cap=None if kbuf is None else kbuf.shape[1])
        if kb is not None:
            kb = kb[:, :nblk]
        if past_kv is not None:
            dc = DashDecodeCache.from_buffers(router, buf, kbuf, S)
    else:
        idx_q, idx_k = _router_qk(router, hidden_states, idx_pe)
        dc = DashDecodeCache(router, idx_k) if past_kv is not None else None
        if dc is not None:
            kb = dc.kbar                    # the block summaries the scores use
    if past_kv is not None:
        if not hasattr(past_kv, "_dash_idx_k"):
            past_kv._dash_idx_k = {}
        _decode_caches(past_kv)[self.layer_idx] = dc
        past_kv._dash_idx_k[self.layer_idx] = dc.idx_k
    sc = router.block_scores(idx_q, idx_k, q_pos=pos_ids.to(torch.int32), nblk=nblk, kbar=kb)
    topi, bias, valid = _infer_route_select(sc, block_cand, p)
    if router.use_triton and q.is_cuda and attn_mask is None:
        out = router._forward_triton(q, k, v, topi, bias, valid, S, nblk, pos_ids)
        if out is not None:
            return out
    return router._forward_dense(q, k, v, topi, bias, valid, S, nblk, attn_mask)


# ----------------------------------------------------------------------------- decode

@torch.no_grad()
def _decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
    """Decode attention for queries at q_pos [B,Lq] (modeling_deepseekv2.py:424-451).
    q [B,H,Lq,D]; k_all/v_all [B,Hkv,S,D]; topi/bias/valid [B,Lq,K]; row (b, l) attends
    the keys j <= q_pos[b, l] of sequence b.  Returns fp32 [B,H,Lq,D]."""
    B, H, Lq, D = q.shape
    if k_all.shape[1] != H:
        rep = H // k_all.shape[1]
        k_all = k_all.repeat_interleave(rep, dim=1)
        v_all = v_all.repeat_interleave(rep, dim=1)
    if Lq != 1:
        return ops.attn_decode_rows(q, k_all, v_all, topi, bias, valid,
                                    q_pos.reshape(B, Lq), block_size, local_window, scale)
    qp = q_pos.reshape(B).to(torch.int32)
    lens = (qp + 1).clamp(max=k_all.shape[2]).to(torch.int32)
    return ops.attn_decode(q[:, :, 0].to(torch.bfloat16), k_all, v_all, topi[:, 0].to(torch.int32),
                           bias[:, 0], valid[:, 0], block_size, local_window, scale,
                           seq_lens=lens, q_pos=qp)[:, :, None]


def _dash_indexer_rope(self, idx, router, x, pos_ids, coords, main_pe):
    """cos/sin for router scoring (modeling_deepseekv2.py:112-130): the indexer's
    two-axis RoPE when page coordinates exist and index_dim == head_dim, else the
    indexer's 1-D RoPE, else the main branch's (cos, sin)."""
    if idx is not None:
        if coords is not None and getattr(idx, "rotary_emb_2d", None) is not None \
                and router.index_dim == idx.head_dim:
            return idx.rotary_emb_2d(x, coords[0], coords[1])
        if getattr(idx, "rotary_emb_1d", None) is not None:
            return idx.rotary_emb_1d(x, pos_ids)
    return main_pe


@torch.no_grad()
def _dash_decode_attend(self, router, hidden_states, q, k_all, v_all, idx_pe, position_ids,
                        past_kv):
    """The DASH part of one decode step (modeling_deepseekv2.py:480-498) after the cache
    update: router projections of the new tokens, their index keys appended to the
    layer's decode state, block scores, routing (with the layer's page-aware
    ``_dash_dec_allow`` candidates when ``router.image_only``) and attention.  q
    [B,H,Lq,D] (RoPE'd), k_all/v_all [B,Hkv,S,D] the updated cache, position_ids [B,Lq].
    One row per sequence runs as one fused step; several rows per sequence each route
    and attend at their own position.  Returns fp32 [B,H,Lq,D]."""
    B, H, Lq, D = q.shape
    p = router._infer_params
    caches = _decode_caches(past_kv)
    dc = caches.get(self.layer_idx)
    idx_q, idx_k_new = _router_qk(router, hidden_states, idx_pe)
    if dc is None:                       # decode without a DASH prefill: start from here
        dc = DashDecodeCache(router, past_kv._dash_idx_k[self.layer_idx])
        caches[self.layer_idx] = dc
    dc.append(idx_k_new)
    if not hasattr(past_kv, "_dash_idx_k"):
        past_kv._dash_idx_k = {}
    past_kv._dash_idx_k[self.layer_idx] = dc.idx_k
    S = k_all.shape[2]
    if dc.S != S:
        raise ValueError(f"index-key cache holds {dc.S} tokens, KV cache {S}")
    nblk = (S + router.block_size - 1) // router.block_size
    if k_all.shape[1] != H:
        rep = H // k_all.shape[1]
        k_all = k_all.repeat_interleave(rep, dim=1)
        v_all = v_all.repeat_interleave(rep, dim=1)
    cand = None
    allow = getattr(self, "_dash_dec_allow", None)
    if allow is not None and router.image_only:
        if allow.shape[-1] < nblk:
            allow = torch.nn.functional.pad(allow, (0, nblk - allow.shape[-1]), value=False)
        cand = allow[:, :nblk]
    if Lq != 1:
        return _dash_decode_rows(router, dc, q, k_all, v_all, idx_q, cand,
                                 position_ids.reshape(B, Lq), p)
    qpos = position_ids.reshape(B, -1)[:, -1]
    if dc.kbar is not None:
        # fused step: tail summary refresh + scores + routing + attention
        K = int(p["K"])
        out, _ = ops.decode_step_fused(
            q, k_all, v_all, idx_q, dc.idx_k, dc.head_cls, dc.kbar, router.block_size,
            router.local_blocks, p["idx_scale"], p["floor"], p["sigma"], K, p["topm"],
            router._scale, cand=cand, q_pos=qpos)
        return out
    # indexer stage 0: block-max scores over the raw index keys
    sc = _block_scores_infer(router, idx_q, dc.idx_k, qpos[:, None], nblk)
    topi, bias, valid = _infer_route_select(sc, None if cand is None else cand[:, None], p)
    return _decode_attend(q, k_all, v_all, topi, bias, valid, qpos[:, None], router.block_size,
                          router.local_window, router._scale)


@torch.no_grad()
def _dash_decode_rows(router, dc, q, k_all, v_all, idx_q, cand, q_pos, p):
    """Lq > 1 decode rows of one step (modeling_deepseekv2.py:480-498 with q_len rows at
    position_ids [B, Lq]): the block summaries of every block the new tokens touched are
    recomputed, then block scores of each row at its own position, routing, and the
    attention of each row against the cache.  Returns fp32 [B,H,Lq,D]."""
    B, Lq = q_pos.shape
    S = dc.S
    bs = router.block_size
    nblk = (S + bs - 1) // bs
    if dc.kbar is not None:
        c0 = (S - Lq) // bs
        ops.kbar(dc._buf[:, c0 * bs:S], dc.head_cls, bs, nblk_cap=nblk - c0,
                 out=dc.kbar[:, c0:nblk])
        sc = ops.block_scores(idx_q, dc.kbar[:, :nblk], bs, router.local_blocks,
                              q_pos=q_pos.to(torch.int32), S=S)
    else:
        sc = _block_scores_infer(router, idx_q, dc.idx_k, q_pos, nblk)
    if cand is not None:
        cand = cand[:, None, :].expand(B, Lq, nblk)
    topi, bias, valid = _infer_route_select(sc, cand, p)
    return _decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, bs, router.local_window,
                          router._scale)


def _dash_decode_forward(self, hidden_states, position_ids, past_kv):
    """Decode step (q_len == 1) of a DASH layer under inference routing
    (modeling_deepseekv2.py:454-500): q/k/v projections, RoPE (``rotary_emb_2d_main``
    with ``_main_rope_coords`` when ``main_rope_mode == "page2d"``, else
    ``rotary_emb``), cache update, router RoPE, ``_dash_decode_attend``, ``o_proj``.
    Returns (attn_output, None, past_kv, None) like the reference."""
    idx = getattr(self, "indexer", None)
    router = self.dash_router
    nh = self.config.num_attention_heads
    nkv = self.config.num_key_value_heads
    hd = self.head_dim
    bsz, q_len, _ = hidden_states.size()
    if position_ids is None:
        past = past_kv.get_seq_length(self.layer_idx)
        position_ids = torch.arange(past, past + q_len,
                                    device=hidden_states.device)[None].expand(bsz, -1)
    q = self.q_proj(hidden_states).view(bsz, q_len, nh, hd).transpose(1, 2)
    k = self.k_proj(hidden_states).view(bsz, q_len, nkv, hd).transpose(1, 2)
    v = self.v_proj(hidden_states).view(bsz, q_len, nkv, hd).transpose(1, 2)
    coords = None
    if getattr(self, "main_rope_mode", None) == "page2d" and \
            getattr(self, "rotary_emb_2d_main", None) is not None:
        # the page coordinates advanced on the device (page_rope.main_rope_coords)
        coords = page_rope.main_rope_coords(self, q_len, past_kv)
    if coords is not None:
        cos, sin = self.rotary_emb_2d_main(v, coords[0], coords[1])
    else:
        cos, sin = self.rotary_emb(v, position_ids)
    q, k = apply_rotary(q, k, cos, sin)
    k_all, v_all = past_kv.update(k, v, self.layer_idx)
    use_coords = coords if (idx is not None and getattr(idx, "rope_mode", None) == "page2d") \
        else None
    idx_pe = _dash_indexer_rope(self, idx, router, v, position_ids, use_coords, (cos, sin))
    out = _dash_decode_attend(self, router, hidden_states, q, k_all, v_all, idx_pe,
                              position_ids, past_kv)
    out = out.to(hidden_states.dtype).transpose(1, 2).contiguous().reshape(bsz, q_len, -1)
    return self.o_proj(out), None, past_kv, None
