"""Inference-time DASH helpers with the reference's signatures, on HIP kernels.

Counterparts of modeling_deepseekv2.py:269-451 (the DASH overlay on the
DeepSeek-V2 attention): ``configure_dash_inference``, ``_infer_route_select``,
``_block_scores_infer``, ``_infer_prefill_attend`` and ``_decode_attend`` take the
same arguments and return the same shapes; the math runs in libdash_hip.so.
"""

import math

import torch

from . import ops
from .dash_attention import DashAttention

_INFER = {"on": False}


def configure_dash_inference(decoder, on, topm=16, page_scope_prefill=True, state=None):
    """Switch inference routing on/off for every DashAttention in ``decoder``
    (modeling_deepseekv2.py:269-306): sets ``_infer_params`` = {idx_scale, floor,
    sigma, K, topm} per router from the config's per-layer scale/floor arrays."""
    if not on:
        if state is not None:
            for mod, stage0 in state["stage0"]:
                mod.stage0 = stage0
        _INFER["on"] = False
        return None
    state = {"stage0": []}
    cfg = getattr(decoder, "config", None)
    sp = (getattr(cfg, "sparse_attention_config", None) or {}) if cfg is not None else {}
    stage0 = str(sp.get("dash_stage0") or "indexer").lower()
    budget = sp.get("dash_topk_blocks") or sp.get("dash_image_fallback_remote") or 12
    routers = [m for m in decoder.modules() if isinstance(m, DashAttention)]
    for li, router in enumerate(routers):
        scale = _per_layer(sp, "dash_scale_per_layer", li)
        floor = _per_layer(sp, "dash_floor_per_layer", li)
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
    _INFER["on"] = True
    return state


def _per_layer(sp, key, idx):
    arr = sp.get(key)
    if not isinstance(arr, (list, tuple)) or not arr:
        return None
    return float(arr[idx]) if 0 <= idx < len(arr) else None


@torch.no_grad()
def _infer_route_select(block_scores, block_cand, p):
    """(topi [B,Lq,K] int64, bias [B,Lq,K] fp32, valid [B,Lq,K] bool) of the inference
    router (modeling_deepseekv2.py:309-333).  Ties go to the lower block id."""
    ti, bi, va = ops.route(block_scores, block_cand, p["idx_scale"], p["floor"], p["sigma"],
                           p["K"], p["topm"])
    return ti.long(), bi, va


@torch.no_grad()
def _block_scores_infer(router, idx_q, idx_k, q_pos, nblk):
    """[B,Lq,nblk] fp32 block scores of queries at q_pos against every key of idx_k
    (modeling_deepseekv2.py:351-400)."""
    return router.block_scores(idx_q, idx_k, q_pos=q_pos.to(torch.int32), nblk=nblk)


@torch.no_grad()
def _infer_prefill_attend(router, hidden_states, q, k, v, idx_pe, pos_ids, block_cand,
                          attn_mask=None):
    """Prefill under inference routing (modeling_deepseekv2.py:403-421)."""
    if attn_mask is not None:
        raise NotImplementedError("additive attention_mask is not supported by the HIP path")
    B, H, S, D = q.shape
    nblk = (S + router.block_size - 1) // router.block_size
    iq, ik = router.router_qk(hidden_states, idx_pe)
    sc = _block_scores_infer(router, iq, ik, pos_ids, nblk)
    topi, bias, valid = _infer_route_select(sc, block_cand, router._infer_params)
    return ops.attn_prefill(q, k, v, topi, bias, valid, router.block_size, router.local_window,
                            router._scale)


@torch.no_grad()
def _decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
    """Decode attention for Lq == 1 queries at q_pos [B,1] (modeling_deepseekv2.py:424-451).
    q [B,H,1,D]; k_all/v_all [B,Hkv,S,D]; returns fp32 [B,H,1,D]."""
    B, H, Lq, D = q.shape
    if Lq != 1:
        raise NotImplementedError("one decode query per sequence")
    if k_all.shape[1] != H:
        rep = H // k_all.shape[1]
        k_all = k_all.repeat_interleave(rep, dim=1)
        v_all = v_all.repeat_interleave(rep, dim=1)
    qp = q_pos.reshape(B).to(torch.int32)
    lens = (qp + 1).to(torch.int32)
    return ops.attn_decode(q[:, :, 0].to(torch.bfloat16), k_all, v_all, topi[:, 0].to(torch.int32),
                           bias[:, 0], valid[:, 0], block_size, local_window, scale,
                           seq_lens=lens, q_pos=qp)[:, :, None]
