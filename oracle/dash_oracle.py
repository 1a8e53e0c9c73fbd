"""CPU oracle for the DASH attention hot path.  TEST INFRASTRUCTURE ONLY.

This module is test infrastructure, never the product: only ``tests/``, the entry
point's ``smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it.
The shipped package (``ananta_ocr_amd``) never imports it and has no CPU path.

It restates, op for op in fp32 on the CPU, the reference's PyTorch algorithm
for the path (citations are ``file:line`` in the reference repository):

* router front end (index projections, Gemma RMSNorm, RoPE, guards)
                              -- modeling_deepseekv2.py:336-348, dash_attention.py:684-693
* stage-0 block summaries ``k_bar`` (head_cls softmax pooling; mean pooling when
  ``head_cls == 0``)          -- dash_attention.py:851-888, modeling_deepseekv2.py:362-377
* head_cls block scores       -- dash_attention.py:890-904, modeling_deepseekv2.py:378-386
* indexer (block-max) scores  -- modeling_deepseekv2.py:387-400, dash_attention.py:815-835
* fused block-max scorer      -- sparse_gather_triton.py:395-467 (``-inf`` sentinel, seg)
* 1.5-entmax                  -- dash_attention.py:615-662
* inference routing           -- modeling_deepseekv2.py:309-333
* training routing            -- dash_attention.py:906-960
* prefill attention           -- dash_attention.py:980-1006 (mask algebra + SDPA), with the
                                 fused-kernel set semantics of sparse_gather_e2e_triton.py:34-115
                                 and the segment start of sparse_gather_triton.py:42,63,73
* decode attention            -- modeling_deepseekv2.py:424-451
* packed varlen (cu_seqlens)  -- block-diagonal: each document is run on its own
                                 block grid (the per-request semantics of the serving path)
* page-aware candidates       -- _sparse_base_impl.py:2189-2259 (page ids), :2363-2380 (flat
                                 image mask), :2436-2484 (candidate mask); decode allow row
                                 modeling_anantaocr.py:450-496
* decode window bounds        -- the vendored serving router's route_triton.py:466-505

Deliberate, documented deviation: ``torch.topk`` leaves the order of tied values
unspecified (the CPU kernel returns ties in an arbitrary order).  The oracle
selects with a *stable* descending sort, so ties go to the lower block id.  Tests
compare the oracle with ``torch.topk`` as sets wherever ties straddle the cut.

Parity pinning (what each function is checked against, in tests/):
  router_qk        -> torch's rms_norm (in-range rows), closed forms (constant rows,
                      cos = 1 / sin = 0 identity, cos = 0 / sin = 1 rotate_half), guards
  kbar/scores      -> brute-force float64 loops, closed form (mean pooling)
  entmax15         -> closed forms, invariants, independent float64 bisection
  route            -> brute-force stable ranking, torch.topk as sets
  training route   -> a from-definition row (full-width entmax by bisection); its
                      autograd gradient -> float64 finite differences (gradcheck) and the
                      closed-form entmax Jacobian of dash_attention.py:650-658
  dense_attend     -> brute-force float64 enumeration of the explicit key sets,
                      sliding-window / causal SDPA special cases
  decode_attend    -> the same enumeration at one query; equality with prefill rows
  page candidates  -> known-answer prompts written out by hand, and a token-by-token
                      walk of the prompt (tests/bruteforce.py) on random prompts
  window bounds    -> known-answer rows written out by hand, and a per-row loop from the
                      definition (tests/bruteforce.py:win_bounds_row)
"""

import math

import torch
import torch.nn.functional as F

SCORE_NEG = -1.0e9     # dash_attention.py:602
MASK_NEG = -1.0e9      # dash_attention.py:601
ACT_CLAMP = 1.0e4      # dash_attention.py:604
GRAD_CLAMP = 1.0e4     # dash_attention.py:603
ENTMAX_NEG = -1.0e4    # modeling_deepseekv2.py:56


# ----------------------------------------------------------------------------
# router front end: index q/k projections, Gemma RMSNorm, RoPE
# ----------------------------------------------------------------------------

def gemma_rmsnorm(x, weight, eps):
    """_RMSNorm.forward (dash_attention.py:684-693): fp32 with nan_to_num, x*rsqrt(mean
    x^2 + eps), clamp, scale by (1 + weight), clamp, back to the input dtype."""
    x32 = torch.nan_to_num(x.float(), nan=0.0, posinf=0.0, neginf=0.0)
    x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    x32 = x32.clamp(-ACT_CLAMP, ACT_CLAMP)
    return (x32 * (1.0 + weight.float())).clamp(-ACT_CLAMP, ACT_CLAMP).to(x.dtype)


def rotate_half_rope(x, cos, sin):
    """q * cos + rotate_half(q) * sin (the llama apply_rotary_pos_emb the router calls,
    modeling_deepseekv2.py:345), each op in torch's promoted dtype; cos/sin broadcast
    over x's leading dims."""
    x1, x2 = x.chunk(2, dim=-1)
    return x * cos + torch.cat((-x2, x1), dim=-1) * sin


def router_qk(hidden_states, w_q, w_k, norm_q, norm_k, eps, cos=None, sin=None):
    """_router_qk (modeling_deepseekv2.py:336-348): idx_q, idx_k fp32 [B,S,d].

    The projections are the exact products (float64) rounded once to the hidden
    states' dtype, which is what a linear layer in that dtype returns up to its
    accumulation order.  cos/sin [B or 1, S, >= d]."""
    hs = torch.nan_to_num(hidden_states, nan=0.0, posinf=0.0, neginf=0.0)
    d = w_q.shape[0]
    out = []
    for w, nw in ((w_q, norm_q), (w_k, norm_k)):
        p = (hs.double() @ w.double().t()).to(hs.dtype)
        y = gemma_rmsnorm(p, nw, eps)
        if cos is not None:
            # torch type promotion: bf16 rows with fp32 cos/sin rotate in fp32
            y = rotate_half_rope(y, cos[..., :d], sin[..., :d])
        out.append(torch.nan_to_num(y.float(), nan=0.0, posinf=0.0, neginf=0.0))
    return out[0], out[1]


# ----------------------------------------------------------------------------
# stage 0: block summaries and block scores
# ----------------------------------------------------------------------------

def kbar_headcls(idx_k, head_cls, block_size):
    """k_bar [B,nblk,d] fp32 and chunk_valid [B,nblk] bool.

    Follows modeling_deepseekv2.py:362-377 (== dash_attention.py:851-888):
    zero-pad the key axis to nblk*bs, per-token logit ``k_j.head_cls/sqrt(d)``
    clamped to +-1e4, masked softmax over each block's real tokens (max over
    valid tokens, denominator >= 1e-6), weighted sum, NaN/inf -> 0.
    """
    idx_k = idx_k.float()
    B, S, d = idx_k.shape
    bs = int(block_size)
    nblk = (S + bs - 1) // bs
    Sp = nblk * bs
    inv_sqrt_d = 1.0 / math.sqrt(d)
    if Sp > S:
        kk = F.pad(idx_k, (0, 0, 0, Sp - S))
        real = F.pad(idx_k.new_ones(B, S, dtype=torch.bool), (0, Sp - S), value=False)
    else:
        kk = idx_k[:, :Sp]
        real = idx_k.new_ones(B, Sp, dtype=torch.bool)
    kk = kk.view(B, nblk, bs, d)
    vmask = real.view(B, nblk, bs)
    hc = head_cls.float().view(1, 1, 1, d)
    aw = ((kk * hc).sum(-1) * inv_sqrt_d).clamp(-ACT_CLAMP, ACT_CLAMP)
    neg = torch.finfo(aw.dtype).min
    row_max = torch.where(vmask, aw, aw.new_full((), neg)).amax(dim=-1, keepdim=True)
    row_max = torch.where(vmask.any(dim=-1, keepdim=True), row_max, torch.zeros_like(row_max))
    e = torch.exp(aw - row_max) * vmask.to(aw.dtype)
    w = e / e.sum(dim=-1, keepdim=True).clamp_min(1e-6)
    k_bar = torch.nan_to_num((w.unsqueeze(-1) * kk).sum(dim=2), nan=0.0, posinf=0.0, neginf=0.0)
    chunk_valid = vmask.any(dim=-1)
    return k_bar, chunk_valid


def block_scores_headcls(idx_q, k_bar, chunk_valid, q_pos, block_size, local_blocks,
                         q_chunk=2048):
    """z [B,Lq,nblk] fp32: ``clamp(q.k_bar/sqrt(d), +-1e4)`` where the block is a
    causal remote block (``c <= q_pos//bs - local_blocks``) with a real token,
    else ``SCORE_NEG``.  modeling_deepseekv2.py:378-386."""
    idx_q = idx_q.float()
    B, Lq, d = idx_q.shape
    nblk = k_bar.shape[1]
    inv_sqrt_d = 1.0 / math.sqrt(d)
    blk_ids = torch.arange(nblk)
    out = []
    for c0 in range(0, Lq, q_chunk):
        c1 = min(c0 + q_chunk, Lq)
        z = torch.matmul(idx_q[:, c0:c1], k_bar.transpose(-1, -2)) * inv_sqrt_d
        z = z.clamp(-ACT_CLAMP, ACT_CLAMP)
        qblk = q_pos[:, c0:c1].long() // block_size
        keep = (blk_ids[None, None, :] <= (qblk[:, :, None] - local_blocks)) \
            & chunk_valid[:, None, :]
        out.append(z.masked_fill(~keep, SCORE_NEG))
    return torch.cat(out, dim=1)


def block_scores_indexer(idx_q, idx_k, q_pos, nblk, block_size, local_window, q_chunk=2048):
    """Indexer stage-0: ``max_j clamp(q.k_j, +-1e4)`` over keys with
    ``j <= pos - local_window`` (causal, outside the window); SCORE_NEG where a
    block has no such key.  modeling_deepseekv2.py:387-400."""
    idx_q = idx_q.float()
    idx_k = idx_k.float()
    B, S, d = idx_k.shape
    Sp = nblk * block_size
    kpos = torch.arange(S)
    out = []
    for c0 in range(0, idx_q.shape[1], q_chunk):
        c1 = min(c0 + q_chunk, idx_q.shape[1])
        sc = torch.matmul(idx_q[:, c0:c1], idx_k.transpose(-1, -2)).clamp(-ACT_CLAMP, ACT_CLAMP)
        pos = q_pos[:, c0:c1].long()
        future = kpos[None, None, :] > pos[:, :, None]
        local = (kpos[None, None, :] > (pos[:, :, None] - local_window)) & ~future
        sc = sc.masked_fill(future | local, SCORE_NEG)
        if Sp > S:
            sc = F.pad(sc, (0, Sp - S), value=SCORE_NEG)
        out.append(sc.view(B, c1 - c0, nblk, block_size).amax(dim=-1))
    return torch.cat(out, dim=1)


def block_max_score(q, k, pos, seg, block_size, num_key_blocks, local_window):
    """Fused block-max scorer semantics: ``max_j q.k_j`` over keys
    ``seg <= j < max(pos - LW + 1, 0)``, ``j < Sk``; ``-inf`` where the block has
    no such key; no clamp.  sparse_gather_triton.py:395-428 (kernel), :431-467."""
    q = q.float()
    k = k.float()
    B, C, D = q.shape
    Sk = k.shape[1]
    bs = int(block_size)
    lw = bs if local_window is None else max(1, int(local_window))
    s = torch.matmul(q, k.transpose(-1, -2))
    j = torch.arange(Sk)
    ls = (pos.long() - (lw - 1)).clamp(min=0)
    ok = (j[None, None, :] < ls[:, :, None]) & (j[None, None, :] >= seg.long()[:, :, None])
    s = s.masked_fill(~ok, float("-inf"))
    Sp = num_key_blocks * bs
    if Sp > Sk:
        s = F.pad(s, (0, Sp - Sk), value=float("-inf"))
    else:
        s = s[..., :Sp]
    return s.view(B, C, num_key_blocks, bs).amax(dim=-1)


# ----------------------------------------------------------------------------
# 1.5-entmax and routing
# ----------------------------------------------------------------------------

def _entmax_threshold_and_support(X, dim=-1):
    """Sort-based threshold (dash_attention.py:623-635)."""
    Xsrt, _ = torch.sort(X, descending=True, dim=dim)
    d = X.size(dim)
    rho = torch.arange(1, d + 1, dtype=X.dtype)
    view = [1] * X.dim()
    view[0] = -1
    rho = rho.view(view).transpose(0, dim)
    mean = Xsrt.cumsum(dim) / rho
    mean_sq = (Xsrt ** 2).cumsum(dim) / rho
    ss = rho * (mean_sq - mean ** 2)
    delta = (1 - ss) / rho
    delta_nz = torch.clamp(delta, 0)
    tau = mean - torch.sqrt(delta_nz)
    support_size = (tau <= Xsrt).sum(dim).unsqueeze(dim)
    support_size = support_size.clamp(min=1)
    tau_star = tau.gather(dim, support_size - 1)
    return tau_star, support_size


def sanitize_grad(g):
    """The gradient hook of dash_attention.py:607-613: non-finite -> 0, clamp +-1e4."""
    return torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0).clamp(-GRAD_CLAMP, GRAD_CLAMP)


def entmax15(X, dim=-1):
    """1.5-entmax forward (dash_attention.py:638-662): ``X=(X-max)/2``,
    ``p = clamp(X - tau*, 0)^2``."""
    max_val, _ = X.max(dim=dim, keepdim=True)
    X = X - max_val
    X = X / 2
    tau_star, _ = _entmax_threshold_and_support(X, dim)
    return torch.clamp(X - tau_star, min=0) ** 2


def stable_topk(x, k):
    """Top-k along the last axis ordered by (value desc, index asc).

    Stands in for ``torch.topk`` (whose tie order is unspecified) in
    modeling_deepseekv2.py:322."""
    vals, idx = torch.sort(x, dim=-1, descending=True, stable=True)
    return vals[..., :k], idx[..., :k]


def route_inputs(block_scores, block_cand, idx_scale):
    """``(x, cand)`` exactly as modeling_deepseekv2.py:316-320 builds them."""
    remote = block_scores > (SCORE_NEG * 0.5)
    cand = remote if block_cand is None else (remote & block_cand)
    cand = torch.where(~cand.any(dim=-1, keepdim=True), remote, cand)
    x = torch.where(cand, block_scores * idx_scale, block_scores.new_full((), ENTMAX_NEG))
    x = torch.nan_to_num(x, nan=ENTMAX_NEG, posinf=ENTMAX_NEG, neginf=ENTMAX_NEG)
    return x, cand


def infer_route_select(block_scores, block_cand, idx_scale, floor, sigma, K, topm):
    """Inference routing, modeling_deepseekv2.py:309-333.

    Returns ``(topi [.., K'] int64, bias [.., K'] fp32, valid [.., K'] bool)``
    with ``K' = max(1, min(K, M'))`` and ``M' = max(1, min(topm, nblk))``
    (``nblk`` when ``topm <= 0``).
    """
    block_scores = block_scores.float()
    x, cand = route_inputs(block_scores, block_cand, idx_scale)
    nblk = x.shape[-1]
    M = max(1, min(int(topm), nblk)) if int(topm) > 0 else nblk
    xv, xi = stable_topk(x, M)
    prior = entmax15(xv, dim=-1)
    is_cand = cand.gather(-1, xi)
    Kp = max(1, min(int(K), M))
    xi, prior, valid = xi[..., :Kp], prior[..., :Kp], is_cand[..., :Kp]
    logp = torch.log(prior.clamp_min(floor))
    cnt = valid.sum(dim=-1, keepdim=True).clamp(min=1)
    mu = torch.where(valid, logp, torch.zeros_like(logp)).sum(dim=-1, keepdim=True) / cnt
    bias = torch.where(valid, (logp - mu) * (1.0 / sigma), torch.zeros_like(logp))
    return xi, bias.float(), valid


def train_route_select(block_scores, block_cand, idx_scale, floor, sigma, K):
    """Training-mode routing: full-width entmax prior (dash_attention.py:906-930)
    then top-K of the masked prior with the centred log-prior bias
    (dash_attention.py:932-960).  Ties in the prior are broken by lower block id.

    Differentiable in ``block_scores`` by autograd through the sort-based forward,
    with the prior's gradient hook of dash_attention.py:1045-1046."""
    block_scores = block_scores.float()
    x, cand = route_inputs(block_scores, block_cand, idx_scale)
    prior = entmax15(x, dim=-1)
    if prior.requires_grad:
        prior.register_hook(sanitize_grad)
    nblk = x.shape[-1]
    Kp = max(1, min(int(K), nblk))
    sel_prior = prior.masked_fill(~cand, -1.0)
    topv, topi = stable_topk(sel_prior, Kp)
    valid = topv >= 0.0
    logp = torch.log(topv.clamp_min(floor))
    cnt = valid.sum(dim=-1, keepdim=True).clamp(min=1)
    mu = torch.where(valid, logp, torch.zeros_like(logp)).sum(dim=-1, keepdim=True) / cnt
    bias = (logp - mu) * (1.0 / sigma)
    bias = torch.where(valid, bias, torch.zeros_like(bias)).clamp(-ACT_CLAMP, ACT_CLAMP)
    return topi, bias, valid


# ----------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------

def dense_block_bias(topi, bias, valid, nblk):
    """[..., nblk] fp32 per-block bias, ``MASK_NEG`` for unrouted blocks.

    Slots with ``valid == False`` or a negative index are dropped; a duplicated
    block keeps its first slot (the dedup of sparse_gather_e2e_triton.py:374-384,
    made deterministic).  For the distinct in-range indices routing produces,
    this equals the scatter of dash_attention.py:984-986."""
    topi = topi.long()
    keep = valid & (topi >= 0) & (topi < nblk)
    K = topi.shape[-1]
    if K > 1:
        same = topi[..., :, None] == topi[..., None, :]
        earlier = torch.tril(torch.ones(K, K, dtype=torch.bool), diagonal=-1)
        dup = (same & keep[..., None, :] & earlier).any(-1)
        keep = keep & ~dup
    idx = torch.where(keep, topi, torch.full_like(topi, nblk))
    src = torch.where(keep, bias.float(), torch.full_like(bias.float(), MASK_NEG))
    out = torch.full(topi.shape[:-1] + (nblk + 1,), MASK_NEG, dtype=torch.float32)
    out = out.scatter(-1, idx, src)
    return out[..., :nblk]


def dense_attend(q, k, v, topi, bias, valid, block_size, local_window, scale,
                 q_chunk=2048, kmin=None, rows=None, attention_mask=None):
    """Prefill DASH attention, fp32: dash_attention.py:980-1006.

    Key j is kept for query t when it is causal and either in the token-level
    window ``(t - LW, t]`` (bias 0) or in a routed block (bias of that block);
    the window wins on overlap.  ``kmin`` [B,S] (optional) adds ``j >= kmin[t]``
    (the packing segment start of sparse_gather_triton.py:42,63,73).
    ``attention_mask`` (optional, additive, [B or 1, 1 or H, >= S, >= S]) is added to
    the mask before the clamp at -1e9, as dash_attention.py:1001-1003 does.
    q, k, v: [B,H,S,D]; topi/bias/valid: [B,S,K].  Returns [B,H,S,D] fp32.
    """
    q = q.float(); k = k.float(); v = v.float()
    B, H, S, D = q.shape
    nblk = (S + block_size - 1) // block_size
    kidx = torch.arange(S)
    key_block = kidx // block_size
    logp = dense_block_bias(topi, bias, valid, nblk)
    out_chunks = []
    r0, r1 = (0, S) if rows is None else rows
    for qs in range(r0, r1, q_chunk):
        qe = min(qs + q_chunk, r1)
        qidx = torch.arange(qs, qe)
        base = logp[:, qs:qe].index_select(-1, key_block)[:, None]
        causal = (kidx[None, :] <= qidx[:, None])[None, None]
        local = ((kidx[None, :] <= qidx[:, None]) &
                 (kidx[None, :] > (qidx[:, None] - local_window)))[None, None]
        sel = base > (MASK_NEG * 0.5)
        keep = causal & (local | sel)
        if kmin is not None:
            keep = keep & (kidx[None, None, None, :] >= kmin[:, None, qs:qe, None].long())
        mask = torch.where(local, torch.zeros_like(base), base)
        mask = mask.masked_fill(~keep, MASK_NEG)
        if attention_mask is not None:
            mask = mask + attention_mask[:, :, qs:qe, :S].to(mask.dtype)
        mask = mask.clamp_min(MASK_NEG)
        out_chunks.append(F.scaled_dot_product_attention(
            q[:, :, qs:qe], k, v, attn_mask=mask, is_causal=False, scale=scale))
    return torch.cat(out_chunks, dim=2)


def decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size, local_window, scale):
    """Decode DASH attention, fp32: modeling_deepseekv2.py:424-451.

    q [B,H,Lq,D], k_all/v_all [B,Hkv,S,D], topi/bias/valid [B,Lq,K], q_pos [B,Lq].
    Returns [B,H,Lq,D] fp32."""
    B, H, Lq, D = q.shape
    S = k_all.shape[2]
    nblk = (S + block_size - 1) // block_size
    kpos = torch.arange(S)
    blk = dense_block_bias(topi, bias, valid, nblk)
    base = blk.index_select(-1, kpos // block_size)
    qp = q_pos.long()[:, :, None]
    causal = kpos[None, None, :] <= qp
    local = causal & (kpos[None, None, :] > (qp - local_window))
    keep = causal & (local | (base > MASK_NEG * 0.5))
    m = torch.where(local, torch.zeros_like(base), base).masked_fill(~keep, float("-inf"))
    kk = k_all.float()
    vv = v_all.float()
    if kk.shape[1] != H:
        rep = H // kk.shape[1]
        kk = kk.repeat_interleave(rep, dim=1)
        vv = vv.repeat_interleave(rep, dim=1)
    s = torch.matmul(q.float(), kk.transpose(-1, -2)) * scale + m[:, None]
    return torch.matmul(torch.softmax(s, dim=-1), vv)


# ----------------------------------------------------------------------------
# whole-path pipelines (the CPU baseline and the end-to-end checks)
# ----------------------------------------------------------------------------

def prefill_route(idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale, floor,
                  sigma, K, topm, q_pos=None, block_cand=None):
    """Inference prefill routing: k_bar -> scores -> route
    (modeling_deepseekv2.py:403-416).  Returns (z, topi, bias, valid)."""
    B, S, d = idx_q.shape
    if q_pos is None:
        q_pos = torch.arange(S)[None].expand(B, -1)
    k_bar, cv = kbar_headcls(idx_k, head_cls, block_size)
    z = block_scores_headcls(idx_q, k_bar, cv, q_pos, block_size, local_blocks)
    topi, bias, valid = infer_route_select(z, block_cand, idx_scale, floor, sigma, K, topm)
    return z, topi, bias, valid


def prefill_pipeline(q, k, v, idx_q, idx_k, head_cls, block_size, local_blocks, idx_scale,
                     floor, sigma, K, topm, scale):
    """Full inference prefill (route + dense attend), fp32.  Returns (out, topi, bias, valid)."""
    _, topi, bias, valid = prefill_route(idx_q, idx_k, head_cls, block_size, local_blocks,
                                         idx_scale, floor, sigma, K, topm)
    out = dense_attend(q, k, v, topi, bias, valid, block_size, local_blocks * block_size, scale)
    return out, topi, bias, valid


def prefill_varlen(q, k, v, idx_q, idx_k, cu_seqlens, head_cls, block_size, local_blocks,
                   idx_scale, floor, sigma, K, topm, scale):
    """Packed varlen prefill with block-diagonal semantics: every document is an
    independent DASH prefill on its own block grid.  q/k/v [1,H,T,D];
    idx_q/idx_k [1,T,d]; cu_seqlens [ndoc+1].  Returns (out [1,H,T,D], topi list,
    bias list, valid list)."""
    outs, tis, bis, vas = [], [], [], []
    cu = [int(c) for c in cu_seqlens]
    for d0, d1 in zip(cu[:-1], cu[1:]):
        o, ti, bi, va = prefill_pipeline(q[:, :, d0:d1], k[:, :, d0:d1], v[:, :, d0:d1],
                                         idx_q[:, d0:d1], idx_k[:, d0:d1], head_cls,
                                         block_size, local_blocks, idx_scale, floor, sigma,
                                         K, topm, scale)
        outs.append(o); tis.append(ti); bis.append(bi); vas.append(va)
    return torch.cat(outs, dim=2), tis, bis, vas


def decode_pipeline(q, k_all, v_all, idx_q, idx_k, head_cls, block_size, local_blocks,
                    idx_scale, floor, sigma, K, topm, scale, q_pos=None):
    """One inference decode step for queries at ``q_pos`` (default: the last
    cached token) -- modeling_deepseekv2.py:481-498.  q [B,H,1,D], idx_q [B,1,d],
    idx_k [B,S,d].  Returns (out [B,H,1,D], topi, bias, valid)."""
    B, S, d = idx_k.shape
    if q_pos is None:
        q_pos = torch.full((B, 1), S - 1, dtype=torch.long)
    k_bar, cv = kbar_headcls(idx_k, head_cls, block_size)
    z = block_scores_headcls(idx_q, k_bar, cv, q_pos, block_size, local_blocks)
    topi, bias, valid = infer_route_select(z, None, idx_scale, floor, sigma, K, topm)
    out = decode_attend(q, k_all, v_all, topi, bias, valid, q_pos, block_size,
                        local_blocks * block_size, scale)
    return out, topi, bias, valid


# ----------------------------------------------------------------------------
# page-aware candidate domain (the OCR prompt's pages)
# ----------------------------------------------------------------------------

def _pad_ids(source_input_ids, key_length):
    ids = source_input_ids[..., :key_length].long()
    if ids.shape[-1] < key_length:
        ids = F.pad(ids, (0, key_length - ids.shape[-1]), value=-1)
    return ids


def page_aware_ids(source_input_ids, img_id, page_id, key_length, per_page=273,
                   page_scope_prefill=False):
    """(image_token_mask, image_token_page_ids, query_token_page_ids) [B, key_length],
    or (None, None, None): _sparse_base_impl.py:2189-2259 (diagnostic prints left out)."""
    if source_input_ids is None or img_id is None or page_id is None:
        return None, None, None
    if source_input_ids.ndim != 2:
        return None, None, None
    token_ids = _pad_ids(source_input_ids, key_length)
    image_token_mask = token_ids == img_id
    page_starts = token_ids == page_id
    cum_pages = torch.cumsum(page_starts.long(), dim=-1)
    seq = token_ids.shape[-1]
    ar = torch.arange(seq)
    last_img = (image_token_mask.long() * (ar + 1)).max(dim=-1).values - 1
    prompt_pages = cum_pages.gather(1, last_img.clamp(min=0)[:, None])
    prompt_pages = prompt_pages * (last_img >= 0)[:, None].long()
    marker_mode = prompt_pages > 0
    per_page = max(1, int(per_page))
    img_running = torch.cumsum(image_token_mask.long(), dim=-1) - 1
    image_token_page_ids = torch.where(marker_mode, cum_pages - 1, img_running // per_page)
    image_token_page_ids = image_token_page_ids.masked_fill(~image_token_mask, -1)
    raw_page = cum_pages - 1
    resp_page = raw_page - torch.where(marker_mode, prompt_pages, torch.zeros_like(prompt_pages))
    in_prefill = ar[None, :] <= last_img[:, None]
    query_token_page_ids = torch.where(in_prefill, raw_page, resp_page)
    if not page_scope_prefill:
        query_token_page_ids = query_token_page_ids.masked_fill(in_prefill, -1)
    query_token_page_ids = query_token_page_ids.masked_fill(query_token_page_ids < 0, -1)
    if image_token_mask.sum() == 0 or (query_token_page_ids >= 0).sum() == 0:
        return None, None, None
    return image_token_mask, image_token_page_ids, query_token_page_ids


def flat_image_token_mask(source_input_ids, img_id, key_length):
    """_sparse_base_impl.py:2363-2380."""
    if source_input_ids is None or img_id is None or source_input_ids.ndim != 2:
        return None
    mask = _pad_ids(source_input_ids, key_length) == img_id
    if mask.sum() == 0:
        return None
    return mask


def kl_candidate_mask(pos_chunk, num_key_blocks, image_token_mask, batch, cq, block_size,
                      image_token_page_ids=None, query_token_page_ids=None,
                      image_bucket_constraint=True):
    """[B, 1, cq, nblk] bool: _sparse_base_impl.py:2457-2484 with the page-aware block
    mask of :2436-2455 and the image-block mask of :2173-2183."""
    bs = int(block_size)
    nblk = int(num_key_blocks)
    if image_bucket_constraint and image_token_page_ids is not None \
            and query_token_page_ids is not None:
        k_len = image_token_page_ids.shape[-1]
        pos_clamped = pos_chunk.long().clamp(0, query_token_page_ids.shape[-1] - 1)
        query_pages = query_token_page_ids.gather(1, pos_clamped)
        pad = nblk * bs - k_len
        if pad > 0:
            img_page_padded = F.pad(image_token_page_ids.float(), (0, pad), value=-1).long()
        elif pad < 0:
            img_page_padded = image_token_page_ids[..., :nblk * bs]
        else:
            img_page_padded = image_token_page_ids
        img_page_blocks = img_page_padded.view(batch, nblk, bs)
        qp = query_pages[:, :, None, None]
        kp = img_page_blocks[:, None, :, :]
        same_page = (qp >= 0) & (qp == kp)
        candidate = same_page.any(dim=-1).unsqueeze(1)
    elif image_token_mask is not None:
        B, Sk = image_token_mask.shape
        pad = nblk * bs - Sk
        m = image_token_mask.bool()
        if pad > 0:
            m = F.pad(m, (0, pad), value=False)
        elif pad < 0:
            m = m[..., :nblk * bs]
        img_blk = m.view(B, nblk, bs).any(dim=-1)
        candidate = img_blk[:, None, None, :].expand(batch, 1, cq, nblk).contiguous()
    else:
        candidate = torch.ones(batch, 1, cq, nblk, dtype=torch.bool)
    has_candidate = candidate.any(dim=-1, keepdim=True)
    return torch.where(has_candidate, candidate, torch.ones_like(candidate))


def decode_page_state(input_ids, img_id, pg_id, block_size, per_page=273):
    """Prefill branch of _uocr_dash_decode_allow (modeling_anantaocr.py:465-479)."""
    bs = int(block_size)
    ids = input_ids.long()
    B, L = ids.shape
    img = ids == img_id
    cum = torch.cumsum((ids == pg_id).long(), dim=-1)
    run = torch.cumsum(img.long(), dim=-1)
    per_page = max(1, int(per_page))
    page = torch.where(cum > 0, cum - 1, (run - 1) // per_page)
    page = torch.where(img, page, torch.full_like(page, -1))
    pp = torch.where(img, cum, torch.zeros_like(cum)).cummax(dim=-1).values[:, -1]
    nblk = -(-L // bs)
    pg = F.pad(page, (0, nblk * bs - L), value=-1).view(B, nblk, bs)
    bmax = pg.amax(dim=-1)
    bmin = torch.where(pg >= 0, pg, torch.full_like(pg, 1 << 30)).amin(dim=-1)
    bmin = torch.where(bmax >= 0, bmin, torch.full_like(bmin, -1))
    return {"bmin": bmin, "bmax": bmax, "pp": pp, "mcum": cum[:, -1].clone()}


def decode_allow(state, input_ids, pg_id, total_len, block_size):
    """Decode branch of _uocr_dash_decode_allow (modeling_anantaocr.py:480-496); updates
    state["mcum"].  input_ids [B, 1]; total_len = cached tokens + 1."""
    ids = input_ids.long()
    B = ids.shape[0]
    state["mcum"] = state["mcum"] + (ids[:, -1] == pg_id).long()
    qp = state["mcum"] - 1 - state["pp"]
    qp = torch.where(qp >= 0, qp, torch.full_like(qp, -1))[:, None]
    nblk = -(-int(total_len) // int(block_size))
    bmin, bmax = state["bmin"], state["bmax"]
    same = (bmin >= 0) & (bmin <= qp) & (bmax >= qp) & (qp >= 0)
    open_row = (qp[:, 0] < 0) | ~same.any(dim=-1)
    allow = torch.zeros(B, nblk, dtype=torch.bool)
    n0 = min(nblk, same.shape[-1])
    allow[:, :n0] = same[:, :n0]
    return allow | open_row[:, None]


def decode_win_bounds(allow, seq_lens, max_block, block_size, local_blocks, tile, q_pos=None):
    """Window bounds of decode rows (the serving router's _win_bounds_kernel,
    whl:sglang/srt/layers/attention/unlimited_dash_ops/route_triton.py:466-505, sglang
    0.5.20.dev13+g75b9b06b02, one decode query per sequence).  allow [B, WQ] bool;
    returns (lo, hi, fit) int64/int64/bool [B]."""
    B, WQ = allow.shape
    seq = seq_lens.long()
    qp = seq - 1 if q_pos is None else torch.minimum(q_pos.long(), seq - 1)
    q_blk = torch.div(qp, block_size, rounding_mode="floor")
    W = int(max_block)
    off = torch.arange(min(W, WQ))
    keep = allow[:, :off.numel()].bool() & (off[None, :] <= (q_blk[:, None] - local_blocks)) \
        & (off[None, :] * block_size < seq[:, None])
    big = torch.full_like(off, W)
    lo = torch.where(keep, off[None, :], big[None, :]).min(dim=-1).values
    hi = torch.where(keep, off[None, :], torch.full_like(big, -1)[None, :]).max(dim=-1).values
    any_r = hi >= 0
    n_blk = torch.div(seq + block_size - 1, block_size, rounding_mode="floor")
    w_seq = torch.clamp(n_blk, min=1).clamp(max=W)
    no_remote = (seq <= 0) | ((q_blk - local_blocks) < 0)
    lo_v = torch.where(any_r, lo, torch.zeros_like(lo))
    hi_v = torch.where(any_r, hi + 1, torch.where(no_remote, torch.zeros_like(hi), w_seq))
    return lo_v, hi_v, (hi_v - lo_v) <= tile


# ----------------------------------------------------------------------------
# page2d RoPE: the OCR prompt's two-axis (token, page) coordinates
# ----------------------------------------------------------------------------

def page_rope_pos(source_input_ids, img_id, page_id, key_length, page_span=0):
    """(tok_pos, page_pos, pf_cnt, n_pg) or None: _build_page_rope_pos with
    _page_rope_offsets (_sparse_base_impl.py:2269-2362; the one-shot diagnostic print left
    out).  tok_pos / page_pos [B, key_length] int64, pf_cnt [B, n_pg] int64 (tokens of each
    page up to the last image token), n_pg = 1 + the largest page id.  None where the
    reference falls back to 1-D RoPE: no ids, no image token or no <PAGE> marker in the
    batch, or a row without a marker at or before its last image token."""
    if source_input_ids is None or getattr(source_input_ids, "ndim", 0) != 2:
        return None
    if img_id is None or page_id is None:
        return None
    ids = _pad_ids(source_input_ids, key_length)
    B, S = ids.shape
    ar = torch.arange(S)
    img = ids == img_id
    mk = ids == page_id
    if not bool(img.any()) or not bool(mk.any()):
        return None
    cum = torch.cumsum(mk.long(), dim=-1)
    last_img = (img.long() * (ar + 1)).max(dim=-1).values - 1
    n_pages = cum.gather(1, last_img.clamp(min=0)[:, None])
    n_pages = n_pages * (last_img >= 0)[:, None].long()
    if not bool((n_pages > 0).all()):
        return None
    in_prefill = ar[None, :] <= last_img[:, None]
    page = torch.where(in_prefill, cum, cum - n_pages).clamp(min=0)
    n_pg = int(page.max().item()) + 1
    onehot = F.one_hot(page, num_classes=n_pg).to(torch.int32)
    run = onehot.cumsum(dim=1)
    tok = run.gather(2, page[:, :, None].to(torch.int64)).squeeze(-1).to(torch.int64) - 1
    pf_cnt = (onehot * in_prefill[:, :, None].to(torch.int32)).sum(dim=1)
    pf_k = pf_cnt.gather(1, page.reshape(B, S).to(torch.int64)).to(torch.int64)
    if page_span > 0:
        s_span = float(page_span)
        pre = torch.round(tok.float() * s_span / pf_k.clamp(min=1).float())
        post = s_span + (tok - pf_k).float()
        scaled = torch.where(in_prefill, pre, post).to(torch.int64)
        tok = torch.where(page > 0, scaled, tok)
    return tok, page, pf_cnt.to(torch.int64), n_pg


def rotary2d_inv_freq(dim, base_tok, base_page, page_pairs, tok_freq_mode="resample"):
    """(inv_tok [n_tok], inv_page [page_pairs]) fp32 of the two-axis RoPE:
    DeepseekV2IndexerRotary2D.__init__ (_sparse_base_impl.py:1848-1873)."""
    half = dim // 2
    page_pairs = int(page_pairs)
    if not (0 < page_pairs < half):
        raise ValueError(f"page_pairs={page_pairs} must be in (0, {half})")
    n_tok = half - page_pairs
    ar = torch.arange(0, n_tok, dtype=torch.int64).float()
    if str(tok_freq_mode).lower() == "truncate":
        inv_tok = 1.0 / (base_tok ** (ar * 2 / dim))
    else:
        inv_tok = 1.0 / (base_tok ** (ar / n_tok))
    inv_page = 1.0 / (base_page ** (torch.arange(0, page_pairs, dtype=torch.int64).float()
                                    / page_pairs))
    return inv_tok, inv_page


def rotary2d_cos_sin(tok_pos, page_pos, inv_tok, inv_page, page_mod=0, dtype=torch.float32):
    """cos / sin [B, S, dim] of the two-axis RoPE at (tok_pos, page_pos) [B, S]:
    DeepseekV2IndexerRotary2D.forward (_sparse_base_impl.py:1876-1891)."""
    t = tok_pos.float()[:, :, None]
    p = page_pos
    if page_mod > 0:
        p = torch.remainder(p.to(torch.int64), page_mod)
    p = p.float()[:, :, None]
    a_tok = t * inv_tok.float()[None, None, :]
    a_page = p * inv_page.float()[None, None, :]
    ang = torch.cat((a_tok, a_page), dim=-1)
    emb = torch.cat((ang, ang), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def page_rope_advance(page, tok, pf_cnt, n_pg, new_ids, page_id):
    """The decode step of the page coordinates, one new token per row:
    _main_rope_coords' decode branch (_sparse_base_impl.py:1384-1390).  page / tok [B]
    int64 (the previous token's coordinates), pf_cnt [B, >= n_pg], new_ids [B].  Returns
    the new (tok, page)."""
    is_pg = new_ids == page_id
    page = torch.where(is_pg, (page + 1).clamp(max=n_pg - 1), page)
    pg_start = pf_cnt.gather(1, page[:, None].clamp(min=0)).squeeze(1)
    tok = torch.where(is_pg, pg_start, tok + 1)
    return tok, page
