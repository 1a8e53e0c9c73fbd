"""DASH attention module on the MI355X HIP kernels.

``DashAttention`` keeps the constructor (``config.sparse_attention_config`` keys)
and the ``forward`` signature of the reference module (dash_attention.py:703-1071)
so that the DeepSeek-V2 decoder can use it unchanged.

``forward`` is the reference's training forward (dash_attention.py:1008-1071):
stage-0 block scores from the router's index projections (indexer block-max or
head_cls summaries, in PyTorch so that autograd reaches the projections, norms and
head_cls), then the training router in ``libdash_hip.so`` (full-width 1.5-entmax
prior, top-k of the masked prior with k from the global schedule, centred
log-prior bias; dash_train_route with its backward), then the fused block-sparse
attention in ``libdash_hip.so`` with gradients to q, k, v and the bias
(dash_attn_prefill and dash_attn_prefill_backward).

The inference form (modeling_deepseekv2.py:309-333: top-M by score, entmax over
the M, first K) is ``route``; ``_infer_params`` holds {idx_scale, floor, sigma, K,
topm} exactly as configure_dash_inference sets them (modeling_deepseekv2.py:299-301).
An additive attention_mask (padding) is taken as per-row key starts; GPU tensors only.
"""

import copy
import math
import os

import torch
import torch.nn as nn

from . import ops

ACT_CLAMP = 1.0e4
GRAD_CLAMP = 1.0e4
SCORE_NEG = -1.0e9


def _sanitize_grad(g):
    """Gradient hook: non-finite -> 0, clamp +-1e4 (dash_attention.py:607-613)."""
    if g is None:
        return None
    return torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0).clamp(-GRAD_CLAMP, GRAD_CLAMP)


def _env_int(name, default):
    v = os.environ.get(name)
    return default if v is None or v == "" else int(v)


class KSchedule:
    """The global routed-block budget k of training (dash_attention.py:272-341):
    geometric from DASH_K_START (64) to DASH_K_END (12) over DASH_K_ANNEAL_STEPS
    (1000) steps, rounded and clamped to the endpoints.  The clock is the optimizer
    step of an attached trainer state (``attach``, or the first live HF TrainerState
    found on the reference's probe schedule), else the count of training forwards of
    the first registered layer.  A forward replayed inside backward (activation
    checkpointing) does not move it."""

    PROBE_AT = (1, 4, 16, 64, 256)

    def __init__(self):
        self.k_start = _env_int("DASH_K_START", 64)
        self.k_end = _env_int("DASH_K_END", 12)
        self.steps = max(1, _env_int("DASH_K_ANNEAL_STEPS", 1000))
        self.k = self.k_start
        self.micro = 0
        self.step = 0
        self.state = None
        self.leader = None
        self.registered = 0

    def register(self):
        sid = self.registered
        self.registered += 1
        if self.leader is None:
            self.leader = sid
        return sid

    def attach(self, trainer_state):
        """Use trainer_state.global_step as the clock."""
        self.state = trainer_state

    def k_for(self, step):
        frac = min(1.0, max(0.0, step / float(self.steps)))
        k = self.k_start * (self.k_end / float(self.k_start)) ** frac
        lo, hi = sorted((self.k_start, self.k_end))
        return max(lo, min(hi, int(round(k))))

    @staticmethod
    def _find_trainer_state():
        import gc
        for o in gc.get_objects():
            try:
                if type(o).__name__ == "TrainerState" and int(getattr(o, "max_steps", 0) or 0) > 0:
                    return o
            except Exception:
                continue
        return None

    def advance(self, sid, training):
        if not training or sid != self.leader:
            return
        if torch._C._current_graph_task_id() != -1:
            return
        self.micro += 1
        if self.state is None and self.micro in self.PROBE_AT:
            self.state = self._find_trainer_state()
        self.step = int(self.state.global_step) if self.state is not None else self.micro
        self.k = self.k_for(self.step)


K_SCHEDULE = KSchedule()

# sparse_attention_config as the checkpoint gave it, taken before the first router writes
# its parameters into it (the role of modeling_deepseekv2.py:63-64): id of the live dict ->
# (the live dict, its copy).  The live dict is held so that its id is never reused.
CKPT_SP = {}


def checkpoint_sparse_config(live):
    """The copy of ``live`` taken before any router wrote into it, else ``live``."""
    ent = CKPT_SP.get(id(live))
    return ent[1] if ent is not None and ent[0] is live else live


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


MASK_NEG = -1.0e9
# additive-mask entries at or below this exclude a key from a row that keeps another key
# (exp(-1e4) is 0 in fp32 next to the row's own window keys)
MASK_EXCLUDE = -1.0e4
# a row whose every causal key is excluded attends uniformly to all S keys in the
# reference (every logit clamps to -1e9): that needs entries that clamp exactly,
# whatever block bias they add to
MASK_EXCLUDE_ALL = -2.0e9


@torch.no_grad()
def mask_key_starts(attention_mask, B, S, q_chunk=2048):
    """The additive attention mask of _forward_dense (dash_attention.py:1001-1003: added
    to the DASH mask, clamped at -1e9) as per-row key starts.

    attention_mask [B or 1, 1 or H, >= S, >= S]; its [:, :, :S, :S] part is used, as in
    the reference.  Each entry must be 0 (allowed) or <= -1e4 (excluded), equal over
    heads; each row t's allowed keys j <= t must be a suffix [kmin_t, t] (left padding,
    block-diagonal documents), or empty with every causal entry <= -2e9 (a padding row,
    which the reference attends uniformly over all S keys).  Returns (kmin [B, S]
    int32, empty [B, S] bool); empty rows get kmin 0.  Other masks raise
    NotImplementedError (one host synchronisation)."""
    am = attention_mask
    if am.dim() != 4 or am.shape[-2] < S or am.shape[-1] < S:
        raise NotImplementedError(f"attention_mask of shape {tuple(am.shape)}")
    am = am[:, :, :S, :S]
    ok = torch.ones((), dtype=torch.bool, device=am.device)
    if am.shape[1] != 1:
        ok = ok & (am == am[:, :1]).all()
    am = am[:, 0]
    kidx = torch.arange(S, device=am.device)
    kmin = torch.empty(B, S, dtype=torch.int32, device=am.device)
    empty = torch.empty(B, S, dtype=torch.bool, device=am.device)
    for q0 in range(0, S, q_chunk):
        q1 = min(q0 + q_chunk, S)
        a = am[:, q0:q1].float().expand(B, q1 - q0, S)
        qidx = torch.arange(q0, q1, device=am.device)
        causal = kidx[None, None, :] <= qidx[None, :, None]
        zero = a == 0
        allowed = zero & causal
        cnt = allowed.sum(-1)
        first = torch.where(cnt > 0, allowed.to(torch.int8).argmax(-1), qidx[None] + 1)
        e = cnt == 0
        ok = ok & (zero | (a <= MASK_EXCLUDE)).all()
        ok = ok & (cnt == qidx[None] - first + 1).all()
        ok = ok & (~e | ((a <= MASK_EXCLUDE_ALL) | ~causal).all(-1)).all()
        kmin[:, q0:q1] = torch.where(e, torch.zeros_like(first), first).to(torch.int32)
        empty[:, q0:q1] = e
    if not bool(ok):
        raise NotImplementedError(
            "attention_mask rows must allow a suffix [kmin, t] of their causal keys (entries "
            "0 / <= -1e4, equal over heads), or no causal key with entries <= -2e9")
    return kmin, empty


def _fill_empty_rows(out, v, empty):
    """Rows whose causal keys are all masked: the reference's logits there are
    q.k*scale - 1e9 for every one of the S keys, which round to -1e9, so its softmax is
    uniform and the row is the mean of v over all S keys (per head).  The gradient is
    that mean's (to v only).  The reference's own backward of such a row depends on how
    its attention backend rounds -1e9 + s (a backward that recomputes exp(s - lse) with
    both rounded to -1e9 takes every weight as 1), so it has no single value; these are
    padding rows, whose upstream gradient is zero in a padded batch."""
    if empty is None:
        return out
    vm = v.float().mean(2, keepdim=True).to(out.dtype)
    return torch.where(empty[:, None, :, None], vm, out)


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
        # training stage 0 comes from the environment only (dash_attention.py:748);
        # the checkpoint's dash_stage0 is read by configure_dash_inference
        self.stage0 = os.environ.get("DASH_STAGE0", "indexer").lower()
        self.head_cls = nn.Parameter(torch.zeros(self.index_dim))
        self._scale = 1.0 / math.sqrt(self.head_dim)
        self._idx_scale = self.scaling_factor / math.sqrt(self.index_dim)
        budget = sp.get("dash_topk_blocks") or sp.get("dash_image_fallback_remote") or 12
        self._infer_params = dict(idx_scale=self._idx_scale, floor=self._prior_floor,
                                  sigma=self.sigma, K=int(budget), topm=16)
        if isinstance(sp, dict) and id(sp) not in CKPT_SP:
            CKPT_SP[id(sp)] = (sp, copy.deepcopy(sp))
        self._ks_id = K_SCHEDULE.register()
        self._sp = sp if isinstance(sp, dict) else None
        self._persist_router_cfg()

    def _persist_router_cfg(self):
        """Write the router's live parameters into the config's sparse_attention_config
        so that save_pretrained stores them (dash_attention.py:761-774); the first
        registered layer only.  With the per-layer temperature loop off (its default,
        and the only mode here) every layer's scale and floor are the config's."""
        if self._sp is None or self._ks_id != K_SCHEDULE.leader:
            return
        n = K_SCHEDULE.registered
        self._sp["dash_stage0"] = self.stage0
        self._sp["dash_router"] = "entmax_topk_perlayer"
        self._sp["dash_sigma"] = float(self.sigma)
        self._sp["dash_topk_blocks"] = int(K_SCHEDULE.k)
        self._sp["dash_scaling_factor"] = float(
            self.scaling_factor / math.sqrt(self.index_dim) * math.sqrt(self.index_dim))
        self._sp["dash_prior_floor"] = float(self._prior_floor)
        self._sp["dash_scale_per_layer"] = [float(self.scaling_factor)] * n
        self._sp["dash_floor_per_layer"] = [float(self._prior_floor)] * n

    # ---------------------------------------------------------------- router
    # fewest token rows for the fused front end: its work-groups own 64 rows and run
    # the whole hidden width, which loses to the library GEMM for decode-sized batches
    FRONT_MIN_ROWS = 1024

    def _front_ok(self, hidden_states):
        return (self.index_dim == 128 and self.q_norm.eps == self.k_norm.eps
                and hidden_states.shape[0] * hidden_states.shape[1] >= self.FRONT_MIN_ROWS
                and ops.router_front_supported(hidden_states, self.q_proj.weight,
                                               self.k_proj.weight))

    def _front_weights(self):
        """The projection weights in the fused front end's operand order, repacked when
        the weights change."""
        wq, wk = self.q_proj.weight, self.k_proj.weight
        key = (wq.data_ptr(), wk.data_ptr(), wq._version, wk._version)
        cached = getattr(self, "_front_pack", None)
        if cached is None or cached[0] != key:
            cached = (key, ops.router_front_pack(wq.detach(), wk.detach()))
            self._front_pack = cached
        return cached[1]

    def router_front(self, hidden_states, position_embeddings=None, with_kbar=False,
                     idx_k_out=None, kbar_out=None, nblk_cap=None):
        """(idx_q, idx_k, k_bar or None) from bf16 hidden states in one launch: the
        projections, norms, RoPE and guards of router_qk and, with with_kbar (stage 0
        head_cls, blocks of 32 or 64), the block summaries of block_scores."""
        cos = sin = None
        if position_embeddings is not None:
            cos, sin = position_embeddings
        kb = with_kbar and self.stage0 == "head_cls"
        return ops.router_front(hidden_states, self.q_proj.weight.detach(),
                                self.k_proj.weight.detach(), self.q_norm.weight.detach(),
                                self.k_norm.weight.detach(), self.q_norm.eps, cos, sin,
                                head_cls=self.head_cls.detach() if kb else None,
                                block_size=self.block_size if kb else None,
                                idx_k_out=idx_k_out, kbar_out=kbar_out if kb else None,
                                nblk_cap=nblk_cap if kb else None,
                                w_pack=self._front_weights())

    def router_qk(self, hidden_states, position_embeddings=None):
        """idx_q/idx_k [B,S,d] fp32 (modeling_deepseekv2.py:336-348)."""
        B, S, _ = hidden_states.shape
        d = self.index_dim
        if hidden_states.is_cuda and self._front_ok(hidden_states):
            iq, ik, _ = self.router_front(hidden_states, position_embeddings)
            return iq, ik
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
        block's bias).  An additive attention_mask (padding) becomes per-row key starts
        (``mask_key_starts``); a row it masks completely is the mean of v, as the
        reference's clamped softmax gives; a mask of another form raises
        NotImplementedError (there is no second code path)."""
        if k.shape[2] != S or q.shape[2] != S:
            raise NotImplementedError("query and key lengths must both be S")
        kmin = empty = None
        if attention_mask is not None:
            kmin, empty = mask_key_starts(attention_mask, q.shape[0], S)
        if k.shape[1] != q.shape[1]:
            rep = q.shape[1] // k.shape[1]
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        out = ops.attn_prefill(q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16),
                               topi, blk_bias, valid, self.block_size, self.local_window,
                               self._scale, kmin=kmin)
        return _fill_empty_rows(out, v, empty).to(q.dtype)

    # ---------------------------------------------------------------- training stage 0
    def _index_qk_train(self, hidden_states, position_embeddings):
        """idx_q/idx_k [B,S,d] fp32 with autograd to the projections and norms, and
        the gradient sanitizer on both (dash_attention.py:808-821)."""
        B, S, _ = hidden_states.shape
        d = self.index_dim
        hs = torch.nan_to_num(hidden_states, nan=0.0, posinf=0.0, neginf=0.0)
        iq = self.q_norm(self.q_proj(hs).view(B, S, 1, d)).transpose(1, 2)
        ik = self.k_norm(self.k_proj(hs).view(B, S, 1, d)).transpose(1, 2)
        if position_embeddings is not None:
            cos, sin = position_embeddings
            iq, ik = apply_rotary(iq, ik, cos[..., :d], sin[..., :d])
        iq = torch.nan_to_num(iq[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
        ik = torch.nan_to_num(ik[:, 0].float(), nan=0.0, posinf=0.0, neginf=0.0)
        for t in (iq, ik):
            if t.requires_grad:
                t.register_hook(_sanitize_grad)
        return iq, ik

    def _block_scores_train(self, iq, ik, position_ids, nblk):
        """Indexer scores (dash_attention.py:801-835): for query t and block c the max
        over the block's keys j with j <= pos_t - LW of clamp(iq_t . ik_j, +-1e4),
        -1e9 where the block has no such key; chunks of q_chunk queries."""
        B, S, d = ik.shape
        bs = self.block_size
        pad = nblk * bs - S
        kpos = torch.arange(S, device=ik.device)
        rows = []
        for c0 in range(0, S, self.q_chunk):
            c1 = min(c0 + self.q_chunk, S)
            sc = torch.matmul(iq[:, c0:c1], ik.transpose(-1, -2)).clamp(-ACT_CLAMP, ACT_CLAMP)
            reach = position_ids[:, c0:c1, None] - self.local_window      # last remote key
            sc = sc.masked_fill(kpos[None, None, :] > reach, SCORE_NEG)
            if pad > 0:
                sc = torch.nn.functional.pad(sc, (0, pad), value=SCORE_NEG)
            elif pad < 0:
                sc = sc[..., :nblk * bs]
            rows.append(sc.view(B, c1 - c0, nblk, bs).amax(dim=-1))
        return torch.cat(rows, dim=1)

    def _block_scores_headcls_train(self, iq, ik, position_ids, nblk):
        """head_cls scores (dash_attention.py:837-904): per block the softmax over its
        real keys of clamp(ik_j . head_cls / sqrt(d), +-1e4) pools k_bar (the mean when
        head_cls = 0); z = clamp(iq_t . k_bar_c / sqrt(d), +-1e4) for blocks c <=
        pos_t // bs - LB holding a real key, else -1e9."""
        B, S, d = ik.shape
        bs = self.block_size
        inv = 1.0 / math.sqrt(d)
        npad = nblk * bs - S
        real = torch.ones(B, S, dtype=torch.bool, device=ik.device)
        if npad >= 0:
            kk = torch.nn.functional.pad(ik, (0, 0, 0, npad))
            real = torch.nn.functional.pad(real, (0, npad), value=False)
        else:
            kk, real = ik[:, :nblk * bs], real[:, :nblk * bs]
        kk = kk.view(B, nblk, bs, d)
        real = real.view(B, nblk, bs)
        logits = ((kk * self.head_cls.to(kk.dtype)).sum(-1) * inv).clamp(-ACT_CLAMP, ACT_CLAMP)
        lowest = torch.finfo(logits.dtype).min
        top = torch.where(real, logits, logits.new_full((), lowest)).amax(-1, keepdim=True)
        top = torch.where(real.any(-1, keepdim=True), top, torch.zeros_like(top))
        e = torch.exp(logits - top) * real.to(logits.dtype)
        w = e / e.sum(-1, keepdim=True).clamp_min(1e-6)
        kbar = torch.nan_to_num((w.unsqueeze(-1) * kk).sum(2), nan=0.0, posinf=0.0, neginf=0.0)
        has_key = real.any(-1)
        blk = torch.arange(nblk, device=ik.device)
        rows = []
        for c0 in range(0, S, self.q_chunk):
            c1 = min(c0 + self.q_chunk, S)
            z = torch.matmul(iq[:, c0:c1], kbar.transpose(-1, -2))
            if z.requires_grad:
                z.register_hook(_sanitize_grad)
            z = (z * inv).clamp(-ACT_CLAMP, ACT_CLAMP)
            qblk = position_ids[:, c0:c1] // bs
            keep = (blk[None, None, :] <= qblk[:, :, None] - self.local_blocks) & has_key[:, None, :]
            rows.append(z.masked_fill(~keep, SCORE_NEG))
        return torch.cat(rows, dim=1)

    # ---------------------------------------------------------------- forward
    def forward(self, hidden_states, q, k, v, position_embeddings=None, position_ids=None,
                attention_mask=None, image_block_mask=None, block_cand=None, page_ids=None):
        """hidden_states [B,S,hidden]; q,k,v [B,H,S,D] (RoPE'd, GQA-expanded).
        Returns [B,H,S,D] in q.dtype (dash_attention.py:1008-1071).

        Stage-0 scores (indexer, or head_cls when the config's dash_stage0 says so),
        the training router with k = the schedule's current budget (advanced once per
        training forward), and the fused attention over token positions; gradients
        reach q, k, v, the router's projections, norms and head_cls.  block_cand
        [B,S,nblk] takes precedence over image_block_mask [B,nblk] (used when
        dash_image_only); page_ids are diagnostics in the reference and are ignored.
        The reference's per-layer temperature loop (DASH_SPARSITY_SCHED, off by
        default) is not implemented: idx_scale and the prior floor are the config's."""
        B, H, S, D = q.shape
        nblk = (S + self.block_size - 1) // self.block_size
        kmin = empty = None
        if attention_mask is not None:
            # the reference's dense fallback with the mask (dash_attention.py:1064-1071)
            kmin, empty = mask_key_starts(attention_mask, B, S)
        if position_ids is None:
            position_ids = torch.arange(S, device=q.device)[None].expand(B, -1)
        K_SCHEDULE.advance(self._ks_id, self.training)
        self._persist_router_cfg()

        iq, ik = self._index_qk_train(hidden_states, position_embeddings)
        if self.stage0 == "head_cls":
            z = self._block_scores_headcls_train(iq, ik, position_ids, nblk)
        else:
            z = self._block_scores_train(iq, ik, position_ids, nblk)
        if z.requires_grad:
            z.register_hook(_sanitize_grad)
        cand = block_cand
        if cand is None and self.image_only and image_block_mask is not None:
            cand = image_block_mask[:, None, :].expand(B, S, nblk)
        K = max(1, min(int(K_SCHEDULE.k), nblk))
        topi, blk_bias, valid = ops.train_route(z, cand, self._idx_scale, self._prior_floor,
                                                self.sigma, K)
        if k.shape[1] != H:
            rep = H // k.shape[1]
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        bf = torch.bfloat16
        out = ops.attn_prefill_autograd(q.to(bf), k.to(bf), v.to(bf), topi, blk_bias, valid,
                                        self.block_size, self.local_window, self._scale,
                                        kmin=kmin)
        return _fill_empty_rows(out, v, empty).to(q.dtype)
