"""DASH attention module on the MI355X HIP kernels.

``DashAttention`` keeps the constructor (``config.sparse_attention_config`` keys)
and the ``forward`` signature of the reference module (dash_attention.py:703-1071)
so that the DeepSeek-V2 decoder can use it unchanged.  The router's index
projections (two 1280->d linears, Gemma RMSNorm, optional RoPE) stay in PyTorch
(dash_attention.py:680-700, :801-852); stage 0 (block summaries and scores),
routing and the block-sparse attention run in ``libdash_hip.so``.

Routing is the inference form (modeling_deepseekv2.py:309-333): top-M by score,
1.5-entmax over the M, first K blocks, centred log-prior bias.  ``_infer_params``
holds {idx_scale, floor, sigma, K, topm} exactly as configure_dash_inference sets
them (modeling_deepseekv2.py:299-301); it defaults to the config's values.
Forward only: no autograd (the reference's backward kernels are not part of this
library), no additive attention_mask, GPU tensors only.
"""

import math

import torch
import torch.nn as nn

from . import ops

ACT_CLAMP = 1.0e4


class GemmaRMSNorm(nn.Module):
    """RMSNorm with scale (1 + weight), fp32 math and the router's finiteness
    guards (dash_attention.py:680-700)."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim))

    def forward(self, x):
        x32 = torch.nan_to_num(x.float(), nan=0.0, posinf=0.0, neginf=0.0)
        x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.eps)
        x32 = x32.clamp(-ACT_CLAMP, ACT_CLAMP)
        return (x32 * (1.0 + self.weight.float())).clamp(-ACT_CLAMP, ACT_CLAMP).to(x.dtype)


def _rotate_half(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary(q, k, cos, sin):
    """Llama RoPE on [B,H,S,d] with cos/sin [B,S,d] (unsqueezed on the head axis)."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    return q * cos + _rotate_half(q) * sin, k * cos + _rotate_half(k) * sin


class DashAttention(nn.Module):
    """Drop-in DASH attention (window + 1.5-entmax routed blocks) on HIP kernels."""

    def __init__(self, config):
        super().__init__()
        sp = getattr(config, "sparse_attention_config", {}) or {}
        self.num_heads = config.num_attention_heads
        self.head_dim = config.hidden_size // config.num_attention_heads
        self.block_size = int(sp.get("sparse_block_size", 128))
        self.local_blocks = max(1, int(sp.get("sparse_local_block", 1)))
        self.local_window = self.local_blocks * self.block_size
        self.scaling_factor = float(sp.get("dash_scaling_factor", 2.0))
        self.q_chunk = int(sp.get("dash_query_chunk", 2048))
        self.image_only = bool(sp.get("dash_image_only", True))
        self._image_token_id = int(sp.get("image_token_id", 128815))
        self.sigma = float(sp.get("dash_sigma", 1.0))
        self._prior_floor = float(sp.get("dash_prior_floor", 1e-2))
        self.topk_blocks = int(sp.get("sparse_topk_blocks", 16))
        self.remote_blocks = max(1, self.topk_blocks - self.local_blocks)
        self.use_triton = bool(sp.get("dash_use_triton", True))   # accepted; always HIP
        self.index_dim = int(sp.get("sparse_index_dim", self.head_dim))
        eps = getattr(config, "rms_norm_eps", 1e-6)
        self.q_proj = nn.Linear(config.hidden_size, self.index_dim, bias=False)
        self.k_proj = nn.Linear(config.hidden_size, self.index_dim, bias=False)
        self.q_norm = GemmaRMSNorm(self.index_dim, eps=eps)
        self.k_norm = GemmaRMSNorm(self.index_dim, eps=eps)
        self.stage0 = str(sp.get("dash_stage0", "indexer")).lower()
        self.head_cls = nn.Parameter(torch.zeros(self.index_dim))
        self._scale = 1.0 / math.sqrt(self.head_dim)
        self._idx_scale = self.scaling_factor / math.sqrt(self.index_dim)
        budget = sp.get("dash_topk_blocks") or sp.get("dash_image_fallback_remote") or 12
        self._infer_params = dict(idx_scale=self._idx_scale, floor=self._prior_floor,
                                  sigma=self.sigma, K=int(budget), topm=16)

    # ---------------------------------------------------------------- router
    def router_qk(self, hidden_states, position_embeddings=None):
        """idx_q/idx_k [B,S,d] fp32 (modeling_deepseekv2.py:336-348)."""
        B, S, _ = hidden_states.shape
        d = self.index_dim
        hs = torch.nan_to_num(hidden_states, nan=0.0, posinf=0.0, neginf=0.0)
        if d == 128 and hs.is_cuda and self.q_norm.eps == self.k_norm.eps:
            # one GEMM for both projections, then the fused norm / RoPE / guards
            w = torch.cat([self.q_proj.weight, self.k_proj.weight], 0)
            proj = torch.nn.functional.linear(hs, w)
            cos = sin = None
            if position_embeddings is not None:
                cos, sin = position_embeddings
                cos, sin = cos[..., :d], sin[..., :d]
            return ops.router_qk_norm(proj, self.q_norm.weight, self.k_norm.weight,
                                      self.q_norm.eps, cos, sin)
        iq = self.q_norm(self.q_proj(hs).view(B, S, 1, d)).transpose(1, 2)
        ik = self.k_norm(self.k_proj(hs).view(B, S, 1, d)).transpose(1, 2)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            iq, ik = apply_rotary(iq, ik, cos[..., :d], sin[..., :d])
        iq = torch.nan_to_num(iq[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
        ik = torch.nan_to_num(ik[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
        return iq, ik

    def block_scores(self, idx_q, idx_k, q_pos=None, nblk=None, kbar=None):
        """[B,Lq,nblk] fp32 remote block scores (modeling_deepseekv2.py:351-400).
        kbar: the block summaries of idx_k when the caller already holds them."""
        B, S, d = idx_k.shape
        if nblk is None:
            nblk = (S + self.block_size - 1) // self.block_size
        if self.stage0 == "head_cls":
            kb = kbar[:, :nblk] if kbar is not None else \
                ops.kbar(idx_k, self.head_cls.detach(), self.block_size, nblk_cap=nblk)
            return ops.block_scores(idx_q, kb, self.block_size, self.local_blocks, q_pos=q_pos,
                                    S=S)
        Lq = idx_q.shape[1]
        if q_pos is None:
            q_pos = torch.arange(Lq, device=idx_q.device)[None].expand(B, -1)
        return ops.block_max_score(idx_q, idx_k, q_pos, None, self.block_size, nblk,
                                   self.local_window, mode=0)

    def route(self, block_scores, block_cand=None):
        """(topi, bias, valid) of the inference router (modeling_deepseekv2.py:309-333)."""
        p = self._infer_params
        return ops.route(block_scores, block_cand, p["idx_scale"], p["floor"], p["sigma"],
                         p["K"], p["topm"])

    # ---------------------------------------------------------------- attend
    def _forward_triton(self, q, k, v, topi, blk_bias, valid, S, nblk, position_ids):
        """Fused block-sparse attention of routed (topi, blk_bias, valid) [B,S,K] plus the
        token window (dash_attention.py:962-978): invalid slots become -1 and the call
        goes to the gather-attention entry point, which returns None on the inputs the
        reference's kernel refuses (non-arange positions, key length != query length)."""
        from .sparse_gather import triton_gather_attention_e2e
        block_indices = topi.masked_fill(~valid.bool(), -1).to(torch.int32).unsqueeze(1)
        if position_ids is None:
            position_ids = torch.arange(S, device=q.device)[None].expand(q.shape[0], -1)
        return triton_gather_attention_e2e(q, k, v, block_indices, blk_bias, position_ids, None,
                                           self.block_size, self._scale, self.local_window)

    def _forward_dense(self, q, k, v, topi, blk_bias, valid, S, nblk, attention_mask):
        """The same attention over token positions 0..S-1 (dash_attention.py:980-1006:
        window keys with bias 0, keys of valid routed blocks below the window with the
        block's bias).  An additive attention_mask is not supported by the kernels and
        raises NotImplementedError (there is no second code path)."""
        if attention_mask is not None:
            raise NotImplementedError("additive attention_mask is not supported by the HIP path")
        if k.shape[2] != S or q.shape[2] != S:
            raise NotImplementedError("query and key lengths must both be S")
        if k.shape[1] != q.shape[1]:
            rep = q.shape[1] // k.shape[1]
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        out = ops.attn_prefill(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16),
                               topi, blk_bias, valid, self.block_size, self.local_window,
                               self._scale)
        return out.to(q.dtype)

    # ---------------------------------------------------------------- forward
    def forward(self, hidden_states, q, k, v, position_embeddings=None, position_ids=None,
                attention_mask=None, image_block_mask=None, block_cand=None, page_ids=None):
        """hidden_states [B,S,hidden]; q,k,v [B,H,S,D] (RoPE'd, GQA-expanded).
        Returns [B,H,S,D] in q.dtype (dash_attention.py:1008-1071).

        The reference's forward routes with its training router: 1.5-entmax over
        every block of the row (dash_attention.py:906-930) and the top k of the masked
        prior under a global k schedule (:932-960).  This module implements the
        inference router only (modeling_deepseekv2.py:403-421, reached through
        ``modeling_deepseekv2._infer_prefill_attend``), so ``forward`` raises
        NotImplementedError instead of silently routing another way."""
        raise NotImplementedError(
            "DashAttention.forward routes with the training router (full-width entmax, "
            "k schedule), which the HIP path does not implement; enable inference routing "
            "(configure_dash_inference) and call _infer_prefill_attend")
