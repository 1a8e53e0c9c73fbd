"""Torch-facing wrappers of the DASH HIP kernels.

Each function takes device tensors, checks shapes on the host, allocates its
outputs with torch (the library allocates nothing) and calls one C entry point
on the current HIP stream.  CPU tensors are rejected: the product has no CPU path.
"""

import ctypes
import math

import torch

from . import _lib

_NULL = None


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("DASH HIP ops take GPU tensors (no CPU path)")


def _i32(t):
    return None if t is None else t.to(torch.int32).contiguous()


def _u8(t):
    if t is None:
        return None
    if t.dtype == torch.bool:                  # same bytes (0/1): no conversion kernel
        return t.contiguous().view(torch.uint8)
    return t.to(torch.uint8).contiguous()


def _max_len(cu, max_seqlen):
    """Longest document of cu_seqlens: the caller's value, else read from the device
    (one synchronisation; graph capture needs the caller's value)."""
    if max_seqlen is not None:
        return int(max_seqlen)
    return int((cu[1:] - cu[:-1]).max().item()) if cu.numel() > 1 else 0


def _rows(x):
    """bf16 [.., D] tensor whose feature axis is contiguous with 16-byte rows."""
    if x.stride(-1) != 1 or any(s % 8 for s in x.stride()[:-1]) or x.data_ptr() % 16:
        x = x.contiguous()
    return x


def kbar(idx_k, head_cls, block_size, cu_seqlens=None, seq_lens=None, nblk_cap=None,
         tail_only=False, out=None, block_table=None, page_size=None, max_seqlen=None):
    """Stage-0 block summaries.  idx_k fp32 [B,S,d] (or [1,T,d] with cu_seqlens, or
    paged [pages, page_size, d] with block_table).  Returns [B, nblk_cap, d] fp32.
    max_seqlen: the longest cu_seqlens document (read from the device when omitted)."""
    _need_gpu(idx_k, head_cls)
    lib = _lib.load()
    idx_k = idx_k.float()
    if idx_k.stride(-1) != 1:
        idx_k = idx_k.contiguous()
    d = idx_k.shape[-1]
    if cu_seqlens is not None:
        cu = _i32(cu_seqlens)
        B = cu.numel() - 1
        S = _max_len(cu, max_seqlen)
        sb, st, sp = 0, idx_k.stride(-2), 0
    elif block_table is not None:
        cu = None
        B = block_table.shape[0]
        S = block_table.shape[1] * page_size
        sb, st, sp = 0, idx_k.stride(1), idx_k.stride(0)
    else:
        cu = None
        B, S = idx_k.shape[0], idx_k.shape[1]
        sb, st, sp = idx_k.stride(0), idx_k.stride(1), 0
    if seq_lens is not None:
        seq_lens = _i32(seq_lens)
    if nblk_cap is None:
        nblk_cap = (S + block_size - 1) // block_size
    if out is None:
        # every block of every sequence has tokens (and is written) only for full-length
        # contiguous sequences; otherwise the rows past a sequence's blocks stay zero
        full = cu is None and seq_lens is None and block_table is None and not tail_only \
            and nblk_cap == (S + block_size - 1) // block_size
        out = (torch.empty if full else torch.zeros)(B, nblk_cap, d, dtype=torch.float32,
                                                     device=idx_k.device)
    hc = head_cls.float().contiguous()
    bt = _i32(block_table)
    st_ = lib.dash_kbar(_ptr(idx_k), sb, st, sp, _ptr(cu), _ptr(seq_lens), _ptr(bt),
                        0 if bt is None else bt.stride(0), page_size or 0, _ptr(hc), B, S, d,
                        block_size, int(bool(tail_only)), _ptr(out), out.stride(0), nblk_cap,
                        _stream())
    _lib.check(st_, "dash_kbar")
    return out


def block_scores(idx_q, kb, block_size, local_blocks, q_pos=None, cu_seqlens=None,
                 seq_lens=None, S=None, max_seqlen=None, key_lens=None):
    """Block scores z for query rows idx_q fp32 [B,Lq,d] (or [1,T,d] + cu_seqlens)
    against k_bar [B,nblk,d].  Returns [B,Lq,nblk] (or [T,nblk]) fp32.  Key lengths
    per sequence: key_lens [B] when given, else the cu_seqlens documents (or seq_lens,
    else S)."""
    _need_gpu(idx_q, kb)
    lib = _lib.load()
    idx_q = idx_q.float()
    if idx_q.stride(-1) != 1:
        idx_q = idx_q.contiguous()
    kb = kb.contiguous()
    B, nblk, d = kb.shape
    # rows padded to whole 128-byte lines, so that the kernel's 64-block tiles write
    # full lines (returned as a view of the first nblk columns)
    zs = max(32, (nblk + 31) // 32 * 32)
    if cu_seqlens is not None:
        cu = _i32(cu_seqlens)
        T = idx_q.shape[-2]
        Lq = _max_len(cu, max_seqlen)
        z = torch.empty(T, zs, dtype=torch.float32, device=idx_q.device)[:, :nblk]
        sb, st = 0, idx_q.stride(-2)
        Sk = Lq if S is None else S
    else:
        cu = None
        Lq = idx_q.shape[1]
        z = torch.empty(B, Lq, zs, dtype=torch.float32, device=idx_q.device)[:, :, :nblk]
        sb, st = idx_q.stride(0), idx_q.stride(1)
        Sk = Lq if S is None else S
    qp = _i32(q_pos)
    lens = _i32(seq_lens if key_lens is None else key_lens)
    cu_k = cu if key_lens is None else None
    st_ = lib.dash_block_scores(_ptr(idx_q), sb, st, _ptr(cu), Lq, _ptr(qp), _ptr(kb),
                                kb.stride(0), nblk, _ptr(cu_k), _ptr(lens), Sk, B, d, block_size,
                                local_blocks, _ptr(z), zs, _stream())
    _lib.check(st_, "dash_block_scores")
    return z


def block_max_score(q, k, pos, seg, block_size, num_key_blocks, local_window, mode=1):
    """Indexer block-max scores (mode 1: triton_block_max_score semantics, mode 0:
    the torch indexer form).  q [B,C,d], k [B,Sk,d] fp32; pos/seg [B,C]."""
    _need_gpu(q, k, pos)
    lib = _lib.load()
    q = q.float().contiguous()
    k = k.float().contiguous()
    B, C, d = q.shape
    Sk = k.shape[1]
    pos = _i32(pos)
    seg = _i32(seg)
    out = torch.empty(B, C, num_key_blocks, dtype=torch.float32, device=q.device)
    lw = block_size if local_window is None else max(1, int(local_window))
    st_ = lib.dash_block_max_score(_ptr(q), q.stride(0), q.stride(1), C, _ptr(pos), _ptr(seg),
                                   pos.stride(0), _ptr(k), k.stride(0), k.stride(1), Sk, B, d,
                                   block_size, lw, num_key_blocks, mode, _ptr(out),
                                   out.stride(0), out.stride(1), _stream())
    _lib.check(st_, "dash_block_max_score")
    return out


def router_qk_norm(proj, wq, wk, eps, cos=None, sin=None):
    """Gemma RMSNorm (+ RoPE) of the stacked index projections proj [B,S,2d] (q then k,
    bf16 or fp32); cos/sin [B,S,>=d] (or [1,S,>=d]) bf16/fp32 or None.
    Returns (idx_q, idx_k) fp32 [B,S,d] (modeling_deepseekv2.py:336-348)."""
    _need_gpu(proj, wq, wk)
    lib = _lib.load()
    B, S, d2 = proj.shape
    d = d2 // 2
    if proj.dtype not in (torch.bfloat16, torch.float32):
        proj = proj.float()
    if proj.stride(-1) != 1 or proj.stride(0) != S * proj.stride(1):
        proj = proj.contiguous()
    iq = torch.empty(B, S, d, dtype=torch.float32, device=proj.device)
    ik = torch.empty_like(iq)
    wq = wq.float().contiguous()
    wk = wk.float().contiguous()
    cs_bf16, cs_sb, cs_st = 0, 0, 0
    if cos is not None:
        dt = torch.bfloat16 if (cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16) \
            else torch.float32
        cos = cos.to(dt)
        sin = sin.to(dt)
        if cos.stride(-1) != 1 or cos.stride() != sin.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        cs_bf16 = int(dt == torch.bfloat16)
        cs_sb = 0 if cos.shape[0] == 1 else cos.stride(0)
        cs_st = cos.stride(1)
    st_ = lib.dash_router_qk_norm(_ptr(proj), int(proj.dtype == torch.bfloat16), proj.stride(1),
                                  B * S, S, d, _ptr(wq), _ptr(wk), float(eps), _ptr(cos),
                                  _ptr(sin), cs_bf16, cs_sb, cs_st, _ptr(iq), _ptr(ik), _stream())
    _lib.check(st_, "dash_router_qk_norm")
    return iq, ik


def router_front_supported(hs, w_q, w_k, block_size=None):
    """Whether dash_router_front takes these inputs (bf16 hidden states and weights
    [128, hidden], hidden % 64 == 0; block 32 or 64 for the k_bar / scores)."""
    return (hs.is_cuda and hs.dtype == torch.bfloat16 and w_q.dtype == torch.bfloat16
            and w_k.dtype == torch.bfloat16 and w_q.shape == (128, hs.shape[-1])
            and w_k.shape == w_q.shape and hs.shape[-1] % 64 == 0
            and (block_size is None or block_size in (32, 64)))


def router_front_pack(w_q, w_k):
    """The q_proj / k_proj weights bf16 [128, hidden] in the fused front end's operand
    order (dash_router_front_pack_weights); recompute when the weights change."""
    _need_gpu(w_q, w_k)
    lib = _lib.load()
    w_q, w_k = w_q.contiguous(), w_k.contiguous()
    out = torch.empty(w_q.numel() * 2, dtype=torch.bfloat16, device=w_q.device)
    _lib.check(lib.dash_router_front_pack_weights(_ptr(w_q), _ptr(w_k), w_q.shape[1], _ptr(out),
                                                  _stream()), "dash_router_front_pack_weights")
    return out


def router_front(hs, w_q, w_k, nq, nk, eps, cos=None, sin=None, head_cls=None, block_size=None,
                 want_q=True, idx_k_out=None, kbar_out=None, nblk_cap=None, w_pack=None):
    """Fused router front end (one launch) for bf16 hidden states hs [B,S,hidden]:
    projections by w_q / w_k bf16 [128,hidden], Gemma RMSNorm (weights nq / nk [128]),
    RoPE (cos/sin [B or 1,S,>=128] or None) and guards (modeling_deepseekv2.py:336-348);
    with head_cls the block summaries k_bar [B,nblk_cap,128] (:362-379).
    idx_k_out / kbar_out: [B,>=S,128] / [B,>=nblk_cap,128] fp32 views to write into (rows
    contiguous).  w_pack: router_front_pack(w_q, w_k), packed here when omitted.
    Returns (idx_q or None, idx_k, kbar or None)."""
    _need_gpu(hs, w_q, w_k, nq, nk)
    lib = _lib.load()
    B, S, hid = hs.shape
    if not router_front_supported(hs, w_q, w_k, block_size if head_cls is not None else None):
        raise NotImplementedError("dash_router_front: bf16 inputs, hidden % 64 == 0, block 32/64")
    hs = _rows(hs)
    w_q, w_k = w_q.contiguous(), w_k.contiguous()
    if w_pack is None:
        w_pack = router_front_pack(w_q, w_k)
    wq = nq.float().contiguous()
    wk = nk.float().contiguous()
    dev = hs.device

    def _out(t, rows):
        if t is None:
            return torch.empty(B, rows, 128, dtype=torch.float32, device=dev)
        if t.shape[0] != B or t.shape[1] < rows or t.stride(2) != 1 or t.stride(1) != 128:
            raise ValueError("output views need rows of 128 contiguous fp32")
        return t

    iq = torch.empty(B, S, 128, dtype=torch.float32, device=dev) if want_q else None
    ik = _out(idx_k_out, S)
    kb = None
    bs = cap = 0
    if head_cls is not None:
        bs = int(block_size)
        cap = int(nblk_cap) if nblk_cap is not None else (S + bs - 1) // bs
        kb = _out(kbar_out, cap)
        head_cls = head_cls.float().contiguous()
    cs_bf16, cs_sb, cs_st = 0, 0, 0
    if cos is not None:
        if cos.shape[-1] < 128 or cos.shape[-2] != S or cos.shape[0] not in (1, B) \
                or cos.shape != sin.shape:
            raise ValueError("cos/sin must be [B or 1, S, >=128]")
        dt = torch.bfloat16 if (cos.dtype == torch.bfloat16 and sin.dtype == torch.bfloat16) \
            else torch.float32
        cos, sin = cos[..., :128].to(dt), sin[..., :128].to(dt)
        if cos.stride(-1) != 1 or cos.stride() != sin.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        cs_bf16 = int(dt == torch.bfloat16)
        cs_sb = 0 if cos.shape[0] == 1 else cos.stride(0)
        cs_st = cos.stride(1)
    st_ = lib.dash_router_front(
        _ptr(hs), hs.stride(0), hs.stride(1), B, S, hid, _ptr(w_pack), _ptr(w_q), _ptr(w_k),
        _ptr(wq), _ptr(wk), float(eps), _ptr(cos), _ptr(sin), cs_bf16, cs_sb, cs_st,
        _ptr(head_cls), bs, 1.0 / math.sqrt(128), _ptr(iq), 0 if iq is None else iq.stride(0),
        _ptr(ik), ik.stride(0), _ptr(kb), 0 if kb is None else kb.stride(0), cap, _stream())
    _lib.check(st_, "dash_router_front")
    return iq, (ik if idx_k_out is None else ik[:, :S]), kb

def route(z, cand, idx_scale, floor, sigma, K, topm, row_nblk=None, width=None):
    """Inference routing of every row of z [..., nblk] fp32.
    Returns (idx int32 [..., K'], bias fp32, valid bool) with K' = max(1, min(K, M'))."""
    _need_gpu(z)
    lib = _lib.load()
    lead = z.shape[:-1]
    nblk = z.shape[-1]
    z2 = z.reshape(-1, nblk).float()
    if z2.stride(-1) != 1:
        z2 = z2.contiguous()
    rows = z2.shape[0]
    M = max(1, min(int(topm), nblk)) if int(topm) > 0 else nblk
    Kp = max(1, min(int(K), M)) if width is None else int(width)
    idx = torch.empty(rows, Kp, dtype=torch.int32, device=z.device)
    bias = torch.empty(rows, Kp, dtype=torch.float32, device=z.device)
    valid = torch.empty(rows, Kp, dtype=torch.uint8, device=z.device)
    c2 = None
    if cand is not None:
        c2 = _u8(cand.reshape(-1, nblk))
    rn = _i32(row_nblk)
    st_ = lib.dash_route(_ptr(z2), z2.stride(0), rows, nblk, _ptr(rn), _ptr(c2),
                         0 if c2 is None else c2.stride(0), float(idx_scale), float(floor),
                         float(sigma), int(K), int(topm), Kp, _ptr(idx), _ptr(bias),
                         _ptr(valid), _stream())
    _lib.check(st_, "dash_route")
    return idx.view(*lead, Kp), bias.view(*lead, Kp), valid.view(*lead, Kp).view(torch.bool)


TRAIN_MAX_K = 64


def _train_route_inputs(z, cand, row_nblk):
    nblk = z.shape[-1]
    z2 = z.detach().reshape(-1, nblk).float()
    if z2.stride(-1) != 1:
        z2 = z2.contiguous()
    c2 = None if cand is None else _u8(cand.reshape(-1, nblk))
    return z2, c2, _i32(row_nblk)


def train_route_raw(z, cand, idx_scale, floor, sigma, K, row_nblk=None):
    """Training routing of every row of z [..., nblk] fp32 (no autograd).
    Returns (idx int32, bias fp32, valid bool, topv fp32, stat fp32 [rows, 2]) with
    K' = max(1, min(K, nblk)) slots."""
    _need_gpu(z)
    if int(K) > TRAIN_MAX_K:
        raise NotImplementedError(f"training routing supports K <= {TRAIN_MAX_K}, got {K}")
    lib = _lib.load()
    lead = z.shape[:-1]
    nblk = z.shape[-1]
    z2, c2, rn = _train_route_inputs(z, cand, row_nblk)
    rows = z2.shape[0]
    Kp = max(1, min(int(K), nblk))
    idx = torch.empty(rows, Kp, dtype=torch.int32, device=z.device)
    bias = torch.empty(rows, Kp, dtype=torch.float32, device=z.device)
    valid = torch.empty(rows, Kp, dtype=torch.uint8, device=z.device)
    topv = torch.empty(rows, Kp, dtype=torch.float32, device=z.device)
    stat = torch.empty(rows, 2, dtype=torch.float32, device=z.device)
    st_ = lib.dash_train_route(_ptr(z2), z2.stride(0), rows, nblk, _ptr(rn), _ptr(c2),
                               0 if c2 is None else c2.stride(0), float(idx_scale), float(floor),
                               float(sigma), int(K), Kp, _ptr(idx), _ptr(bias), _ptr(valid),
                               _ptr(topv), _ptr(stat), _stream())
    _lib.check(st_, "dash_train_route")
    return (idx.view(*lead, Kp), bias.view(*lead, Kp), valid.view(*lead, Kp).view(torch.bool),
            topv.view(*lead, Kp), stat)


def train_route_backward(z, cand, idx_scale, floor, sigma, idx, valid, topv, stat, dbias,
                         row_nblk=None):
    """dz [..., nblk] fp32 for the bias gradient dbias [..., K'] of train_route_raw."""
    _need_gpu(z, dbias)
    lib = _lib.load()
    nblk = z.shape[-1]
    z2, c2, rn = _train_route_inputs(z, cand, row_nblk)
    rows = z2.shape[0]
    Kp = idx.shape[-1]
    idx2 = _i32(idx.reshape(rows, Kp))
    val2 = _u8(valid.reshape(rows, Kp))
    tv2 = topv.reshape(rows, Kp).float().contiguous()
    db2 = dbias.reshape(rows, Kp).float().contiguous()
    dz = torch.empty(rows, nblk, dtype=torch.float32, device=z.device)
    st_ = lib.dash_train_route_backward(
        _ptr(z2), z2.stride(0), rows, nblk, _ptr(rn), _ptr(c2),
        0 if c2 is None else c2.stride(0), float(idx_scale), float(floor), float(sigma), Kp,
        _ptr(idx2), _ptr(val2), _ptr(tv2), _ptr(stat), _ptr(db2), _ptr(dz), dz.stride(0),
        _stream())
    _lib.check(st_, "dash_train_route_backward")
    return dz.view(z.shape)


class _TrainRouteFn(torch.autograd.Function):
    """_route + _select_and_bias (dash_attention.py:906-960) with the bias
    differentiable in the block scores; topi and valid carry no gradient."""

    @staticmethod
    def forward(ctx, z, cand, idx_scale, floor, sigma, K, row_nblk):
        idx, bias, valid, topv, stat = train_route_raw(z, cand, idx_scale, floor, sigma, K,
                                                       row_nblk)
        ctx.save_for_backward(z, cand, row_nblk, idx, valid, topv, stat)
        ctx.cfg = (idx_scale, floor, sigma)
        ctx.mark_non_differentiable(idx, valid)
        return idx, bias, valid

    @staticmethod
    def backward(ctx, didx, dbias, dvalid):
        z, cand, row_nblk, idx, valid, topv, stat = ctx.saved_tensors
        idx_scale, floor, sigma = ctx.cfg
        if dbias is None:
            return (None,) * 7
        dz = train_route_backward(z, cand, idx_scale, floor, sigma, idx, valid, topv, stat,
                                  dbias, row_nblk)
        return dz.to(z.dtype), None, None, None, None, None, None


def train_route(z, cand, idx_scale, floor, sigma, K, row_nblk=None):
    """Training routing with autograd: (idx int32 [..., K'], bias fp32, valid bool)."""
    return _TrainRouteFn.apply(z, cand, idx_scale, floor, sigma, K, row_nblk)


DENSE_THRESHOLD = 48   # of the 128 queries of a tile; below it a routed block goes sparse
# Small prefills take every routed block with its tile (no plan, no sparse kernel):
# a grid of at most SMALL_TILES 128-query tiles (which the library splits over
# several work-groups each) over sequences of at most SMALL_BLOCKS blocks, so that
# a tile's routed blocks stay few.  The 2,730-token prefill (220 tiles, 43 blocks):
# 64.6 us against 96.2 with the plan at threshold 32 and 80.6 all block-major.
SMALL_TILES = 256
SMALL_BLOCKS = 64

_WORKSPACES = {}


def cached_workspace(key, nbytes, device):
    """A cached device buffer of at least `nbytes` (contents undefined; the kernels
    clear what they count in).  Calls that share it are ordered on the current stream."""
    k = (key, str(device))
    buf = _WORKSPACES.get(k)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            del _WORKSPACES[k]
            del buf
        buf = torch.empty(int(nbytes * 1.1) + 4096, dtype=torch.uint8, device=device)
        _WORKSPACES[k] = buf
    return buf


def release_workspaces(device=None):
    """Drops the cached workspaces (of one device, or of every device) so that their
    memory returns to torch's allocator; the next call that needs one allocates it
    again.  Safe between calls on one stream (torch hands freed memory out again in
    stream order); with work that used a workspace still running on another stream,
    synchronise first."""
    for k in [k for k in _WORKSPACES if device is None or k[1] == str(torch.device(device))]:
        del _WORKSPACES[k]


def cached_workspace_bytes():
    """Total bytes of the cached workspaces."""
    return sum(b.numel() for b in _WORKSPACES.values())


def attn_prefill(q, k, v, idx, bias, valid, block_size, local_window, scale,
                 cu_seqlens=None, kmin=None, return_lse=False, dense_threshold=None,
                 max_seqlen=None, split_tiles=True):
    """Block-sparse prefill attention.  q/k/v bf16 [B,H,S,D] (any strides with a
    contiguous head dim) or [1,H,T,D] with cu_seqlens; idx/bias/valid [B,S,K] (or
    [T,K]).  Returns o [B,H,S,D] bf16 (and lse [B,S,H] fp32).
    dense_threshold: routed blocks shared by fewer queries of a 128-query tile take
    the block-major sparse path (<= 0: all routed blocks with the tile; None: 32, or
    0 for a small prefill, see SMALL_TILES).  split_tiles=False keeps every tile in
    one work-group when all routed blocks go with the tile."""
    _need_gpu(q, k, v)
    lib = _lib.load()
    if q.dtype != torch.bfloat16:
        raise NotImplementedError("dash_attn_prefill computes in bf16")
    q, k, v = _rows(q), _rows(k.to(q.dtype)), _rows(v.to(q.dtype))
    B, H, S, D = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise NotImplementedError("q_len == k_len and equal head counts are required")
    o = torch.empty(B, H, S, D, dtype=q.dtype, device=q.device)
    lse = torch.empty(B, S, H, dtype=torch.float32, device=q.device) if return_lse else None
    K = 0 if idx is None else idx.shape[-1]
    idx_c = None if idx is None else _i32(idx)
    bias_c = None if bias is None else bias.float().contiguous()
    valid_c = _u8(valid)
    cu = _i32(cu_seqlens)
    nb = B
    if cu is not None:
        if B != 1:
            raise ValueError("varlen prefill takes q of shape [1, H, T, D]")
        nb = cu.numel() - 1
        Smax = _max_len(cu, max_seqlen)
        rows = S
    else:
        Smax = S
        rows = B * S
    if dense_threshold is None:
        thr = DENSE_THRESHOLD
        tiles = (Smax + 127) // 128 * H * nb
        if K <= 16 and tiles <= SMALL_TILES and (Smax + block_size - 1) // block_size <= SMALL_BLOCKS:
            thr = 0
    else:
        thr = int(dense_threshold)
    if K > 16:
        thr = max(thr, 129)          # more than 16 slots: every routed pair block-major
    ws, ws_n = None, 0
    nbytes = ctypes.c_int64(0)
    if thr > 0 and K > 0 and block_size <= 64 and rows > 0:
        # the plan of the sparse path
        _lib.check(lib.dash_attn_prefill_workspace_size(nb, H, Smax, rows, K, D, int(block_size),
                                                        nbytes), "workspace")
    elif rows > 0 and split_tiles:
        # every routed block with its tile: the partials of split tiles (small grids)
        _lib.check(lib.dash_attn_prefill_split_workspace_size(nb, H, Smax, D, nbytes), "workspace")
    if nbytes.value > 0:
        ws = cached_workspace("prefill", nbytes.value, q.device)
        ws_n = ws.numel()
    km = _i32(kmin)
    st_ = lib.dash_attn_prefill(
        _ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        _ptr(o), o.stride(0), o.stride(1), o.stride(2),
        _ptr(lse), H, 1,
        _ptr(idx_c), _ptr(valid_c), _ptr(bias_c), K, _ptr(cu), _ptr(km),
        nb, H, Smax, D, int(block_size), int(local_window), float(scale),
        thr, rows, _ptr(ws), ws_n, _stream())
    _lib.check(st_, "dash_attn_prefill")
    return (o, lse) if return_lse else o


def attn_prefill_backward(q, k, v, o, lse, dout, idx, bias, valid, block_size, local_window,
                          scale, cu_seqlens=None, kmin=None, max_seqlen=None, need_dbias=True):
    """Gradients of attn_prefill: (dq, dk, dv) bf16 shaped like q, k, v and the routed
    slots' bias gradient dbias fp32 shaped like bias (or None).  o and lse [B,S,H] (or
    [1,T,H]) are the forward's outputs (attn_prefill(..., return_lse=True))."""
    _need_gpu(q, k, v, o, lse, dout)
    lib = _lib.load()
    q, k, v = _rows(q), _rows(k.to(q.dtype)), _rows(v.to(q.dtype))
    o, dout = _rows(o), _rows(dout.to(q.dtype))
    B, H, S, D = q.shape
    lse = lse.float().contiguous()
    K = 0 if idx is None else idx.shape[-1]
    idx_c = None if idx is None else _i32(idx)
    bias_c = None if bias is None else bias.float().contiguous()
    valid_c = _u8(valid)
    cu = _i32(cu_seqlens)
    nb = B
    if cu is not None:
        nb = cu.numel() - 1
        Smax = _max_len(cu, max_seqlen)
        rows = S
    else:
        Smax = S
        rows = B * S
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dbias = None
    if need_dbias and K > 0:
        dbias = torch.empty(idx.shape, dtype=torch.float32, device=q.device)
    nbytes = ctypes.c_int64(0)
    _lib.check(lib.dash_attn_prefill_backward_workspace_size(nb, H, Smax, rows, K, D,
                                                             int(block_size), nbytes),
               "workspace")
    ws = cached_workspace("prefill_bwd", nbytes.value, q.device)
    km = _i32(kmin)
    st_ = lib.dash_attn_prefill_backward(
        _ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _ptr(v), v.stride(0), v.stride(1), v.stride(2),
        _ptr(o), o.stride(0), o.stride(1), o.stride(2),
        _ptr(dout), dout.stride(0), dout.stride(1), dout.stride(2),
        _ptr(lse), H, 1,
        _ptr(idx_c), _ptr(valid_c), _ptr(bias_c), K, _ptr(cu), _ptr(km),
        nb, H, Smax, D, int(block_size), int(local_window), float(scale),
        _ptr(dq), dq.stride(0), dq.stride(1), dq.stride(2),
        _ptr(dk), dk.stride(0), dk.stride(1), dk.stride(2),
        _ptr(dv), dv.stride(0), dv.stride(1), dv.stride(2),
        _ptr(dbias), rows, _ptr(ws), ws.numel(), _stream())
    _lib.check(st_, "dash_attn_prefill_backward")
    return dq, dk, dv, dbias


class _DashAttnFn(torch.autograd.Function):
    """attn_prefill with gradients to q, k, v and the routed slots' bias (the role of
    _E2EGatherAttnFn, sparse_gather_e2e_triton.py:288-339)."""

    @staticmethod
    def forward(ctx, q, k, v, bias, idx, valid, block_size, local_window, scale, cu_seqlens,
                kmin, max_seqlen):
        out, lse = attn_prefill(q, k, v, idx, bias, valid, block_size, local_window, scale,
                                cu_seqlens=cu_seqlens, kmin=kmin, return_lse=True,
                                max_seqlen=max_seqlen)
        ctx.save_for_backward(q, k, v, out, lse, idx, bias, valid, cu_seqlens, kmin)
        ctx.cfg = (block_size, local_window, scale, max_seqlen)
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse, idx, bias, valid, cu, kmin = ctx.saved_tensors
        block_size, local_window, scale, max_seqlen = ctx.cfg
        dq, dk, dv, dbias = attn_prefill_backward(
            q, k, v, out, lse, dout, idx, bias, valid, block_size, local_window, scale,
            cu_seqlens=cu, kmin=kmin, max_seqlen=max_seqlen,
            need_dbias=bias is not None and ctx.needs_input_grad[3])
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dbias, None, None, None, None,
                None, None, None, None)


def attn_prefill_autograd(q, k, v, idx, bias, valid, block_size, local_window, scale,
                          cu_seqlens=None, kmin=None, max_seqlen=None):
    """attn_prefill recorded for autograd (bf16 q/k/v; the bias gradient is fp32)."""
    return _DashAttnFn.apply(q, k, v, bias, idx, valid, block_size, local_window, scale,
                             cu_seqlens, kmin, max_seqlen)


def default_nsplit(nunits):
    """One unit (key block) per wavefront, at most 64 partials per (b, h)."""
    return int(max(1, min(64, nunits)))


def attn_decode(q, k, v, idx, bias, valid, block_size, local_window, scale, seq_lens=None,
                q_pos=None, block_table=None, page_size=None, out_dtype=torch.float32,
                nsplit=None, return_lse=False):
    """Decode attention for one query per sequence.  q [B,H,D] (or [B,H,1,D]) bf16;
    k/v contiguous [B,H,S,D] or paged [pages, page_size, H, D] with block_table [B,P];
    idx/bias/valid [B,K] (or [B,1,K]).  Returns out [B,H,D] (out_dtype)."""
    _need_gpu(q, k, v)
    lib = _lib.load()
    squeeze = q.dim() == 4
    if squeeze:
        q = q[:, :, 0]
    q = _rows(q.to(torch.bfloat16))
    k = _rows(k.to(torch.bfloat16))
    v = _rows(v.to(torch.bfloat16))
    B, H, D = q.shape
    if block_table is not None:
        bt = _i32(block_table)
        S = bt.shape[1] * page_size
        k_sb, k_sh, k_st, k_sp = 0, k.stride(2), k.stride(1), k.stride(0)
        v_sb, v_sh, v_st, v_sp = 0, v.stride(2), v.stride(1), v.stride(0)
        bt_stride = bt.stride(0)
    else:
        bt = None
        S = k.shape[2]
        k_sb, k_sh, k_st, k_sp = k.stride(0), k.stride(1), k.stride(2), 0
        v_sb, v_sh, v_st, v_sp = v.stride(0), v.stride(1), v.stride(2), 0
        bt_stride = 0
    if idx is not None and idx.dim() == 3:
        idx, bias = idx[:, 0], bias[:, 0]
        valid = None if valid is None else valid[:, 0]
    K = 0 if idx is None else idx.shape[-1]
    idx_c = None if idx is None else _i32(idx)
    bias_c = None if bias is None else bias.float().contiguous()
    valid_c = _u8(valid)
    if nsplit is None:
        nsplit = default_nsplit((local_window + block_size - 1) // block_size + 1 + K)
    ws_bytes = ctypes.c_int64(0)
    _lib.check(lib.dash_attn_decode_workspace_size(B, H, D, nsplit, ws_bytes), "workspace")
    ws = torch.empty((ws_bytes.value + 3) // 4, dtype=torch.float32, device=q.device)
    out = torch.empty(B, H, D, dtype=out_dtype, device=q.device)
    lse = torch.empty(B, H, dtype=torch.float32, device=q.device) if return_lse else None
    lens = _i32(seq_lens)
    qp = _i32(q_pos)
    st_ = lib.dash_attn_decode(
        _ptr(q), q.stride(0), q.stride(1),
        _ptr(k), k_sb, k_sh, k_st, k_sp, _ptr(v), v_sb, v_sh, v_st, v_sp,
        _ptr(bt), bt_stride, int(page_size or 0), _ptr(lens), _ptr(qp),
        _ptr(idx_c), _ptr(valid_c), _ptr(bias_c), K,
        _ptr(out), int(out_dtype == torch.bfloat16), out.stride(0), out.stride(1),
        _ptr(lse), 0 if lse is None else lse.stride(0), 1,
        B, H, S, D, int(block_size), int(local_window), float(scale), int(nsplit),
        _ptr(ws), ws.numel() * 4, _stream())
    _lib.check(st_, "dash_attn_decode")
    if squeeze:
        out = out[:, :, None]
    return (out, lse) if return_lse else out


def attn_rows(q, k, v, idx, bias, valid, q_pos, row_seq, block_size, local_window, scale,
              seq_lens=None, block_table=None, page_size=None, out_dtype=torch.float32):
    """Attention of R query rows, each of its own sequence and position: q [R,H,D] bf16,
    row r of sequence row_seq[r] at position q_pos[r] attends that sequence's window
    (q_pos - LW, q_pos] and the keys below the window of its routed blocks idx[r] (with
    bias[r]).  Cache contiguous [B,H,S,D] or paged [pages, page_size, H, D] with
    block_table [B,P]; seq_lens [B] (default S).  Returns out [R,H,D] (out_dtype).

    Each row runs as one query of dash_attn_decode over a block table whose row r
    addresses sequence row_seq[r]: for a contiguous cache one page per sequence that spans
    its whole length (page b at the sequence's batch offset), so no cache data moves."""
    _need_gpu(q, k, v, q_pos, row_seq)
    lib = _lib.load()
    R, H, D = q.shape
    qr = _rows(q.to(torch.bfloat16))
    k = _rows(k.to(torch.bfloat16))
    v = _rows(v.to(torch.bfloat16))
    rs = row_seq.to(torch.int64)
    if block_table is not None:
        table = _i32(block_table).index_select(0, rs)
        page = int(page_size)
        S = table.shape[1] * page
        k_sp, k_st, k_sh = k.stride(0), k.stride(1), k.stride(2)
        v_sp, v_st, v_sh = v.stride(0), v.stride(1), v.stride(2)
    else:
        S = k.shape[2]
        page = max(block_size, (S + block_size - 1) // block_size * block_size)
        table = row_seq.to(torch.int32).reshape(R, 1).contiguous()
        k_sp, k_st, k_sh = k.stride(0), k.stride(2), k.stride(1)
        v_sp, v_st, v_sh = v.stride(0), v.stride(2), v.stride(1)
    if seq_lens is None:
        lens = torch.full((R,), S, dtype=torch.int32, device=q.device)
    else:
        lens = _i32(seq_lens).index_select(0, rs)
    K = 0 if idx is None else idx.shape[-1]
    idx_c = None if idx is None else _i32(idx.reshape(R, K))
    bias_c = None if bias is None else bias.reshape(R, K).float().contiguous()
    valid_c = None if valid is None else _u8(valid.reshape(R, K))
    qp = _i32(q_pos.reshape(R))
    nsplit = default_nsplit((local_window + block_size - 1) // block_size + 1 + K)
    ws_bytes = ctypes.c_int64(0)
    _lib.check(lib.dash_attn_decode_workspace_size(R, H, D, nsplit, ws_bytes), "workspace")
    ws = torch.empty((ws_bytes.value + 3) // 4, dtype=torch.float32, device=q.device)
    out = torch.empty(R, H, D, dtype=out_dtype, device=q.device)
    if R == 0:
        return out
    st_ = lib.dash_attn_decode(
        _ptr(qr), qr.stride(0), qr.stride(1),
        _ptr(k), 0, k_sh, k_st, k_sp, _ptr(v), 0, v_sh, v_st, v_sp,
        _ptr(table), table.stride(0), page, _ptr(lens), _ptr(qp),
        _ptr(idx_c), _ptr(valid_c), _ptr(bias_c), K,
        _ptr(out), int(out_dtype == torch.bfloat16), out.stride(0), out.stride(1),
        None, 0, 0, R, H, S, D, int(block_size), int(local_window), float(scale), int(nsplit),
        _ptr(ws), ws.numel() * 4, _stream())
    _lib.check(st_, "dash_attn_decode")
    return out


def attn_decode_rows(q, k, v, idx, bias, valid, q_pos, block_size, local_window, scale,
                     seq_lens=None, block_table=None, page_size=None, out_dtype=torch.float32):
    """Decode attention for Lq query rows per sequence, each at its own position.
    q [B,H,Lq,D] bf16; idx/bias/valid [B,Lq,K]; q_pos [B,Lq].  Cache contiguous
    [B,H,S,D] or paged [pages, page_size, H, D] with block_table [B,P] and seq_lens [B].
    Row (b, l) attends keys j <= q_pos[b,l] (and j < the sequence's length) of sequence b.
    Returns out [B,H,Lq,D] (out_dtype)."""
    B, H, Lq, D = q.shape
    qr = q.permute(0, 2, 1, 3).reshape(B * Lq, H, D)
    row_seq = torch.arange(B, device=q.device).repeat_interleave(Lq)
    K = 0 if idx is None else idx.shape[-1]
    out = attn_rows(qr, k, v, None if idx is None else idx.reshape(B * Lq, K),
                    None if bias is None else bias.reshape(B * Lq, K),
                    None if valid is None else valid.reshape(B * Lq, K),
                    q_pos.reshape(B * Lq), row_seq, block_size, local_window, scale,
                    seq_lens=seq_lens, block_table=block_table, page_size=page_size,
                    out_dtype=out_dtype)
    return out.view(B, Lq, H, D).permute(0, 2, 1, 3)


def _kbar_layout(kbar_cache, kbar_table, bounds):
    """(nblk_cap, kb_sb, table int32 or None, kb_ts, bounds int32 or None) of a k_bar
    cache: per sequence [B, nblk_cap, d], or a page pool [pages, d] addressed through
    kbar_table [B, >= nblk_cap] (one page per block)."""
    bnd = None if bounds is None else _i32(bounds.reshape(-1, 2))
    if kbar_table is None:
        return kbar_cache.shape[1], kbar_cache.stride(0), None, 0, bnd
    kbt = _i32(kbar_table)
    return kbt.shape[1], 0, kbt, kbt.stride(0), bnd


def decode_route(idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks, idx_scale,
                 floor, sigma, K, topm, seq_lens=None, block_table=None, page_size=None,
                 cand=None, refresh_tail=True, width=None, return_scores=False,
                 valid_dtype=torch.bool, q_pos=None, kbar_table=None, bounds=None):
    """Decode routing for one query per sequence (at q_pos [B], default the last cached
    token; positions past it are taken as it): refreshes the
    tail block of `kbar_cache` [B, nblk_cap, d] in place, scores and routes.
    idx_q [B,d] or [B,1,d]; idx_k contiguous [B,S,d] or paged [pages, page_size, d].
    Returns idx int32 [B,1,K'], bias fp32, valid (bool, or valid_dtype) and with
    return_scores the scores [B,nblk_cap].
    kbar_table: kbar_cache is a page pool [pages, d] whose row for block c of sequence b is
    kbar_table[b, c]; bounds [B, 2] (win_bounds): only those blocks are scored."""
    _need_gpu(idx_q, idx_k, kbar_cache)
    if _wide_topm(topm):
        return _decode_route_wide(idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks,
                                  idx_scale, floor, sigma, K, topm, seq_lens, block_table,
                                  page_size, cand, refresh_tail, width, return_scores,
                                  valid_dtype, q_pos, kbar_table, bounds)
    lib = _lib.load()
    if idx_q.dim() == 3:
        idx_q = idx_q[:, 0]
    idx_q = idx_q.float().contiguous()
    idx_k = idx_k.float()
    if idx_k.stride(-1) != 1:
        idx_k = idx_k.contiguous()
    B, d = idx_q.shape
    nblk_cap, kb_sb, kbt, kb_ts, bnd = _kbar_layout(kbar_cache, kbar_table, bounds)
    if block_table is not None:
        bt = _i32(block_table)
        S = bt.shape[1] * page_size
        sb, st, sp = 0, idx_k.stride(1), idx_k.stride(0)
    else:
        bt = None
        S = idx_k.shape[1]
        sb, st, sp = idx_k.stride(0), idx_k.stride(1), 0
    Kw = max(1, min(int(K), int(topm))) if width is None else int(width)
    if seq_lens is None and width is None:
        Kw = max(1, min(int(K), max(1, min(int(topm), (S + block_size - 1) // block_size))))
    idx = torch.empty(B, Kw, dtype=torch.int32, device=idx_q.device)
    bias = torch.empty(B, Kw, dtype=torch.float32, device=idx_q.device)
    valid = torch.empty(B, Kw, dtype=torch.uint8, device=idx_q.device)
    z = torch.empty(B, nblk_cap, dtype=torch.float32, device=idx_q.device)
    lens = _i32(seq_lens)
    c2 = None if cand is None else _u8(cand.reshape(B, -1))
    hc = head_cls.float().contiguous()
    qp = None if q_pos is None else _i32(q_pos.reshape(B))
    st_ = lib.dash_decode_route(
        _ptr(idx_q), idx_q.stride(0), _ptr(idx_k), sb, st, sp, _ptr(bt),
        0 if bt is None else bt.stride(0), int(page_size or 0), _ptr(lens), _ptr(qp), S,
        _ptr(hc),
        int(bool(refresh_tail)), _ptr(kbar_cache), kb_sb, nblk_cap, _ptr(kbt), kb_ts, _ptr(bnd),
        _ptr(c2),
        0 if c2 is None else c2.stride(0), B, d, int(block_size), int(local_blocks),
        float(idx_scale), float(floor), float(sigma), int(K), int(topm), Kw, _ptr(idx),
        _ptr(bias), _ptr(valid), _ptr(z), z.stride(0), _stream())
    _lib.check(st_, "dash_decode_route")
    vd = valid[:, None].view(torch.bool) if valid_dtype == torch.bool else valid[:, None].to(valid_dtype)
    res = (idx[:, None], bias[:, None], vd)
    return res + (z,) if return_scores else res


def _wide_topm(topm):
    """Entmax widths the fused decode router does not take (the whole row, or above
    16): those rows are routed by dash_route's one-row-per-wavefront kernel."""
    return int(topm) < 1 or int(topm) > 16


def _decode_route_wide(idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks, idx_scale,
                       floor, sigma, K, topm, seq_lens, block_table, page_size, cand,
                       refresh_tail, width, return_scores, valid_dtype, q_pos, kbar_table=None,
                       bounds=None):
    """decode_route for a wide entmax: the decode router refreshes the tail summary
    and writes the scores (its own one-slot routing is discarded), then dash_route
    routes each sequence's row over its ceil(len / block_size) blocks."""
    _, _, _, z = decode_route(idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks,
                              idx_scale, floor, sigma, 1, 1, seq_lens=seq_lens,
                              block_table=block_table, page_size=page_size, cand=cand,
                              refresh_tail=refresh_tail, width=1, return_scores=True,
                              q_pos=q_pos, kbar_table=kbar_table, bounds=bounds)
    B, nblk_cap = z.shape
    S = block_table.shape[1] * page_size if block_table is not None else idx_k.shape[1]
    if seq_lens is not None:
        lens = seq_lens.reshape(B).to(device=z.device, dtype=torch.int64).clamp(0, S)
    else:
        lens = torch.full((B,), S, dtype=torch.int64, device=z.device)
    nb = ((lens + block_size - 1) // block_size).clamp(max=nblk_cap).to(torch.int32)
    c2 = None
    if cand is not None:
        c2 = cand.reshape(B, -1)
        if c2.shape[1] < nblk_cap:
            c2 = torch.nn.functional.pad(c2.to(torch.uint8), (0, nblk_cap - c2.shape[1]))
        c2 = c2[:, :nblk_cap]
    M = nblk_cap if int(topm) < 1 else min(int(topm), nblk_cap)
    Kw = max(1, min(int(K), M)) if width is None else int(width)
    idx, bias, valid = route(z, c2, idx_scale, floor, sigma, K, topm, row_nblk=nb, width=Kw)
    vd = valid[:, None] if valid_dtype == torch.bool else valid[:, None].to(valid_dtype)
    res = (idx[:, None], bias[:, None], vd)
    return res + (z,) if return_scores else res


def decode_step_fused(q, k, v, idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks,
                      idx_scale, floor, sigma, K, topm, scale, seq_lens=None, block_table=None,
                      page_size=None, cand=None, width=None, out_dtype=torch.float32,
                      return_lse=False, q_pos=None, workspace=None, return_scores=False,
                      no_alloc=False, kbar_table=None, bounds=None):
    """decode_route followed by attn_decode of its routing, in two launches: the window
    part of the attention runs beside the router.  Same arguments and results as those
    two calls (q [B,H,D] or [B,H,1,D]; out [B,H,D]); returns (out, (idx, bias, valid))
    with idx/bias/valid [B,1,K'] (valid uint8), or (out, lse, routing) with return_lse;
    return_scores appends the block scores z [B, nblk_cap] the router computed.
    no_alloc: call dash_decode_step_noalloc, whose partials live in the library's fixed
    per-GPU scratch array (no workspace; the outputs are still allocated here).
    workspace: a caller's buffer instead of the cached one; zero-filled before its first
    step and passed whole on every step (the routing words at its end start at zero,
    and each step leaves them zero).
    A wide entmax (topm <= 0 or > 16) routes through _decode_route_wide and attends
    with attn_decode (three launches instead of two)."""
    _need_gpu(q, k, v, idx_q, idx_k, kbar_cache)
    if _wide_topm(topm):
        if no_alloc:
            raise NotImplementedError("the allocation-free step takes topm in 1..16")
        idx, bias, valid, z = _decode_route_wide(
            idx_q, idx_k, head_cls, kbar_cache, block_size, local_blocks, idx_scale, floor,
            sigma, K, topm, seq_lens, block_table, page_size, cand, True, width, True,
            torch.uint8, q_pos, kbar_table, bounds)
        squeeze = q.dim() == 4
        qq = q[:, :, 0] if squeeze else q
        lw = int(local_blocks) * int(block_size)
        res = attn_decode(qq, k, v, idx[:, 0], bias[:, 0], valid[:, 0], block_size, lw, scale,
                          seq_lens=seq_lens, q_pos=None if q_pos is None else q_pos.reshape(-1),
                          block_table=block_table, page_size=page_size, out_dtype=out_dtype,
                          return_lse=True)
        out, lse = res
        return _step_result(out, lse if return_lse else None, idx[:, 0], bias[:, 0], valid[:, 0],
                            z, squeeze, return_lse, return_scores)
    lib = _lib.load()
    squeeze = q.dim() == 4
    if squeeze:
        q = q[:, :, 0]
    q = _rows(q.to(torch.bfloat16))
    k = _rows(k.to(torch.bfloat16))
    v = _rows(v.to(torch.bfloat16))
    if idx_q.dim() == 3:
        idx_q = idx_q[:, 0]
    idx_q = idx_q.float().contiguous()
    idx_k = idx_k.float()
    if idx_k.stride(-1) != 1:
        idx_k = idx_k.contiguous()
    B, H, D = q.shape
    d = idx_q.shape[1]
    nblk_cap, kb_sb, kbt, kb_ts, bnd = _kbar_layout(kbar_cache, kbar_table, bounds)
    if block_table is not None:
        bt = _i32(block_table)
        S = bt.shape[1] * page_size
        isb, ist, isp = 0, idx_k.stride(1), idx_k.stride(0)
        k_sb, k_sh, k_st, k_sp = 0, k.stride(2), k.stride(1), k.stride(0)
        v_sb, v_sh, v_st, v_sp = 0, v.stride(2), v.stride(1), v.stride(0)
        bt_stride = bt.stride(0)
    else:
        bt = None
        S = idx_k.shape[1]
        isb, ist, isp = idx_k.stride(0), idx_k.stride(1), 0
        k_sb, k_sh, k_st, k_sp = k.stride(0), k.stride(1), k.stride(2), 0
        v_sb, v_sh, v_st, v_sp = v.stride(0), v.stride(1), v.stride(2), 0
        bt_stride = 0
    Kw = max(1, min(int(K), int(topm))) if width is None else int(width)
    if seq_lens is None and width is None:
        Kw = max(1, min(int(K), max(1, min(int(topm), (S + block_size - 1) // block_size))))
    dev = q.device
    idx = torch.empty(B, Kw, dtype=torch.int32, device=dev)
    bias = torch.empty(B, Kw, dtype=torch.float32, device=dev)
    valid = torch.empty(B, Kw, dtype=torch.uint8, device=dev)
    z = torch.empty(B, nblk_cap, dtype=torch.float32, device=dev)
    out = torch.empty(B, H, D, dtype=out_dtype, device=dev)
    lse = torch.empty(B, H, dtype=torch.float32, device=dev) if return_lse else None
    lens = _i32(seq_lens)
    c2 = None if cand is None else _u8(cand.reshape(B, -1))
    hc = head_cls.float().contiguous()
    lw = int(local_blocks) * int(block_size)
    qp = None if q_pos is None else _i32(q_pos.reshape(B))
    if no_alloc:
        st_ = lib.dash_decode_step_noalloc(
            _ptr(idx_q), idx_q.stride(0), _ptr(idx_k), isb, ist, isp, _ptr(bt), bt_stride,
            int(page_size or 0), _ptr(lens), _ptr(qp), S, _ptr(hc), 1, _ptr(kbar_cache),
            kb_sb, nblk_cap, _ptr(kbt), kb_ts, _ptr(bnd), _ptr(c2),
            0 if c2 is None else c2.stride(0), d,
            int(local_blocks), float(idx_scale), float(floor), float(sigma), int(K), int(topm),
            Kw, _ptr(idx), _ptr(bias), _ptr(valid), _ptr(z), z.stride(0),
            _ptr(q), q.stride(0), q.stride(1),
            _ptr(k), k_sb, k_sh, k_st, k_sp, _ptr(v), v_sb, v_sh, v_st, v_sp,
            _ptr(out), int(out_dtype == torch.bfloat16), out.stride(0), out.stride(1),
            _ptr(lse), 0 if lse is None else lse.stride(0), 1,
            B, H, D, int(block_size), lw, float(scale), _stream())
        _lib.check(st_, "dash_decode_step_noalloc")
        return _step_result(out, lse, idx, bias, valid, z, squeeze, return_lse, return_scores)
    ws_bytes = ctypes.c_int64(0)
    _lib.check(lib.dash_decode_step_workspace_size(B, H, D, int(block_size), lw, ws_bytes),
               "workspace")
    if workspace is None:
        ws = _step_workspace(ws_bytes.value, dev)
    else:
        ws = workspace
        if ws.numel() * ws.element_size() < ws_bytes.value:
            raise ValueError("decode step workspace too small")
    st_ = lib.dash_decode_step(
        _ptr(idx_q), idx_q.stride(0), _ptr(idx_k), isb, ist, isp, _ptr(bt), bt_stride,
        int(page_size or 0), _ptr(lens), _ptr(qp), S, _ptr(hc), 1, _ptr(kbar_cache),
        kb_sb, nblk_cap, _ptr(kbt), kb_ts, _ptr(bnd), _ptr(c2),
        0 if c2 is None else c2.stride(0), d, int(local_blocks),
        float(idx_scale), float(floor), float(sigma), int(K), int(topm), Kw, _ptr(idx),
        _ptr(bias), _ptr(valid), _ptr(z), z.stride(0),
        _ptr(q), q.stride(0), q.stride(1),
        _ptr(k), k_sb, k_sh, k_st, k_sp, _ptr(v), v_sb, v_sh, v_st, v_sp,
        _ptr(out), int(out_dtype == torch.bfloat16), out.stride(0), out.stride(1),
        _ptr(lse), 0 if lse is None else lse.stride(0), 1,
        B, H, D, int(block_size), lw, float(scale), _ptr(ws), ws.numel() * ws.element_size(),
        _stream())
    _lib.check(st_, "dash_decode_step")
    return _step_result(out, lse, idx, bias, valid, z, squeeze, return_lse, return_scores)


_STEP_WORKSPACES = {}


def _step_workspace(nbytes, device):
    """The decode step's cached workspace on `device`: zeroed when it is allocated (the
    routing words at its end must start at zero; every step leaves them zero), and
    always passed whole, so those words stay in one place.  Calls that share it are
    ordered on the current stream."""
    k = str(device)
    buf = _STEP_WORKSPACES.get(k)
    if buf is None or buf.numel() * 4 < nbytes:
        if buf is not None:
            del _STEP_WORKSPACES[k]
            del buf
        buf = torch.zeros(((int(nbytes * 1.25) + 4095) // 4096) * 1024, dtype=torch.float32,
                          device=device)
        _STEP_WORKSPACES[k] = buf
    return buf


def _step_result(out, lse, idx, bias, valid, z, squeeze, return_lse, return_scores):
    if squeeze:
        out = out[:, :, None]
    routing = (idx[:, None], bias[:, None], valid[:, None])
    res = (out, lse, routing) if return_lse else (out, routing)
    return res + (z,) if return_scores else res


def inv_sqrt(d):
    return 1.0 / math.sqrt(d)
