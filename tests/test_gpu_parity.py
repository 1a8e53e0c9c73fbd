"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle on the
same seeded inputs.  Integer outputs (routed block ids, validity) must be
bit-exact on identical fp32 scores; floating outputs meet the stated tolerances.
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops
from ananta_ocr_amd import workloads as W
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
# output tolerance of the path (bf16 output, fp32 accumulation)
ATOL, RTOL = 2e-2, 1e-2


def _gen(seed):
    return torch.Generator("cpu").manual_seed(seed)


def _close(out, ref, what, tight=1.5e-2):
    """The output tolerance plus a scale-aware bound: the max error must also be
    below `tight` x max|ref| (bf16 rounding of P and of the output)."""
    out = out.float().cpu()
    ref = ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= ATOL + RTOL * ref.abs()), f"{what}: max err {err.max().item()}"
    scale = ref.abs().max().item()
    assert err.max().item() <= tight * scale + 1e-6, \
        f"{what}: max err {err.max().item():.3e} vs scale {scale:.3e}"


# ------------------------------------------------------------------ stage 0

@pytest.mark.parametrize("S,d,bs,hc", [(2730, 128, 64, 0.0), (1000, 128, 32, 0.7), (77, 64, 64, 2.0)])
def test_kbar_matches_oracle(S, d, bs, hc):
    g = _gen(100 + S)
    ik = torch.randn(2, S, d, generator=g) * 0.1
    head_cls = torch.randn(d, generator=g) * hc
    kb_ref, _ = O.kbar_headcls(ik, head_cls, bs)
    kb = ops.kbar(ik.to(DEV), head_cls.to(DEV), bs)
    torch.testing.assert_close(kb.cpu(), kb_ref, atol=1e-6, rtol=1e-5)


def test_kbar_varlen_and_tail_refresh():
    g = _gen(101)
    cu = [0, 300, 301, 301 + 640]
    ik = torch.randn(1, cu[-1], 128, generator=g)
    hc = torch.randn(128, generator=g)
    kb = ops.kbar(ik.to(DEV), hc.to(DEV), 64, cu_seqlens=torch.tensor(cu).to(DEV))
    for b in range(3):
        ref, _ = O.kbar_headcls(ik[:, cu[b]:cu[b + 1]], hc, 64)
        torch.testing.assert_close(kb[b, :ref.shape[1]].cpu(), ref[0], atol=1e-5, rtol=1e-5)
    # tail refresh on a contiguous cache with per-sequence lengths
    ik2 = torch.randn(3, 500, 128, generator=g)
    lens = torch.tensor([500, 130, 64], dtype=torch.int32)
    kb2 = torch.zeros(3, 8, 128, device=DEV)
    ops.kbar(ik2.to(DEV), hc.to(DEV), 64, seq_lens=lens.to(DEV), nblk_cap=8, tail_only=True,
             out=kb2)
    for b in range(3):
        L = int(lens[b])
        ref, _ = O.kbar_headcls(ik2[b:b + 1, :L], hc, 64)
        c = (L - 1) // 64
        torch.testing.assert_close(kb2[b, c].cpu(), ref[0, c], atol=1e-5, rtol=1e-5)
        assert kb2[b, :c].abs().sum().item() == 0  # only the tail block was written


@pytest.mark.parametrize("S,bs,lb", [(2730, 64, 8), (1000, 32, 4), (5000, 64, 16)])
def test_block_scores_match_oracle(S, bs, lb):
    g = _gen(102 + S)
    q = torch.randn(1, 10, S, 128, generator=g) * 128 ** -0.5
    k = torch.randn(1, 10, S, 128, generator=g) * 128 ** -0.5
    iq, ik = W.router_inputs(q.bfloat16(), k.bfloat16())
    kb_ref, cv = O.kbar_headcls(ik, torch.zeros(128), bs)
    z_ref = O.block_scores_headcls(iq, kb_ref, cv, torch.arange(S)[None], bs, lb)
    kb = ops.kbar(ik.to(DEV), torch.zeros(128, device=DEV), bs)
    z = ops.block_scores(iq.to(DEV), kb, bs, lb).cpu()
    sent = z_ref == O.SCORE_NEG
    assert torch.equal(z == O.SCORE_NEG, sent)
    torch.testing.assert_close(z[~sent], z_ref[~sent], atol=1e-7, rtol=1e-5)


@pytest.mark.parametrize("mode", [0, 1])
def test_block_max_score_matches_oracle(mode):
    g = _gen(103)
    B, C, Sk, d, bs, lw = 2, 300, 300, 128, 64, 100
    q = torch.randn(B, C, d, generator=g)
    k = torch.randn(B, Sk, d, generator=g)
    pos = torch.arange(C)[None].expand(B, -1).contiguous()
    seg = torch.zeros(B, C, dtype=torch.long)
    seg[1, 150:] = 150
    nblk = (Sk + bs - 1) // bs
    out = ops.block_max_score(q.to(DEV), k.to(DEV), pos.to(DEV), seg.to(DEV), bs, nblk, lw,
                              mode=mode).cpu()
    if mode == 1:
        ref = O.block_max_score(q, k, pos, seg, bs, nblk, lw)
    else:
        ref = O.block_scores_indexer(q[:1], k[:1], pos[:1], nblk, bs, lw)
        out = out[:1]
    fin = torch.isfinite(ref) & (ref > -5e8)
    assert torch.equal(fin, torch.isfinite(out) & (out > -5e8))
    torch.testing.assert_close(out[fin], ref[fin], atol=2e-5, rtol=1e-5)
    assert torch.equal(out[~fin], ref[~fin])


# ------------------------------------------------------------------ routing

def _route_check(z, cand, idx_scale, K, topm):
    ti_r, bi_r, va_r = O.infer_route_select(z, cand, idx_scale, W.FLOOR, W.SIGMA, K, topm)
    ti, bi, va = ops.route(z.to(DEV), None if cand is None else cand.to(DEV), idx_scale,
                           W.FLOOR, W.SIGMA, K, topm)
    ti, bi, va = ti.cpu().long(), bi.cpu(), va.cpu()
    assert ti.shape == ti_r.shape
    assert torch.equal(va, va_r), "valid mismatch"
    mism = (ti != ti_r).nonzero()
    assert mism.numel() == 0, f"routed ids differ at {mism[:5].tolist()}"
    torch.testing.assert_close(bi, bi_r, atol=2e-5, rtol=1e-5)


def _scores(S, nblk, bs, lb, seed, scale, quant=None, nan_frac=0.0):
    g = _gen(seed)
    z = torch.randn(1, S, nblk, generator=g) * scale
    if quant:
        z = torch.round(z * quant) / quant           # many exact ties
    t = torch.arange(S)[None, :, None]
    keep = torch.arange(nblk)[None, None, :] <= (t // bs - lb)
    if nan_frac:
        z = z.masked_fill((torch.rand(z.shape, generator=g) < nan_frac) & keep, float("nan"))
    return z.masked_fill(~keep, O.SCORE_NEG)


@pytest.mark.parametrize("nblk,scale,K,topm", [
    (43, 1e-4, 8, 8),          # prefill at 2,730 tokens: full support
    (427, 1e-3, 16, 16),       # 27,300 tokens
    (427, 0.5, 16, 16),        # partial entmax support
    (100, 3.0, 5, 12),         # K < M, narrow support
    (2048, 0.2, 16, 16),       # widest row the kernel takes
    (7, 1.0, 16, 16),          # M' = nblk < topm
])
def test_route_bit_exact_on_identical_scores(nblk, scale, K, topm):
    bs, lb = 64, 8
    S = min((nblk + lb + 1) * bs, 6000)
    z = _scores(S, nblk, bs, lb, 200 + nblk, scale)
    _route_check(z, None, W.IDX_SCALE, K, topm)


def test_route_ties_nans_and_candidates():
    bs, lb, nblk, S = 16, 2, 150, 2600
    z = _scores(S, nblk, bs, lb, 210, 1.0, quant=4.0, nan_frac=0.01)
    g = _gen(211)
    cand = torch.rand(1, S, nblk, generator=g) < 0.3
    cand[:, ::5] = False                      # rows that fall back to `remote`
    _route_check(z, cand, W.IDX_SCALE, 8, 16)
    _route_check(z, None, 40.0, 16, 16)


def test_route_on_gpu_scores_end_to_end():
    """scores -> route on the GPU, the oracle routing the GPU's own scores."""
    d = W.make_prefill(W.PREFILL_2730)
    kb = ops.kbar(d["idx_k"].to(DEV), torch.zeros(128, device=DEV), 64)
    z = ops.block_scores(d["idx_q"].to(DEV), kb, 64, 8)
    _route_check(z.cpu(), None, W.IDX_SCALE, 8, 8)


# ------------------------------------------------------------------ prefill attention

def _attn_inputs(seed, B, H, S, bs, lw, K, qscale=1.0, dup=False):
    g = _gen(seed)
    q = (torch.randn(B, H, S, 128, generator=g) * qscale * 0.3).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.3).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    nblk = (S + bs - 1) // bs
    lb = (lw + bs - 1) // bs
    qblk = torch.arange(S)[None, :, None] // bs
    # random remote blocks (as routing returns), some invalid / -1 slots
    hi = (qblk - lb).clamp(min=0).float()
    idx = (torch.rand(B, S, K, generator=g) * (hi + 1)).floor().long()
    valid = (torch.rand(B, S, K, generator=g) < 0.85) & (qblk - lb >= 0)
    if dup:
        idx[..., 1] = idx[..., 0]
    else:
        # distinct ids per row like topk
        for j in range(1, K):
            same = (idx[..., j:j + 1] == idx[..., :j]).any(-1)
            valid[..., j] &= ~same
    idx = torch.where(torch.rand(B, S, K, generator=g) < 0.05, torch.full_like(idx, -1), idx)
    bias = torch.randn(B, S, K, generator=g) * 2
    return q, k, v, idx.clamp(max=nblk - 1), bias, valid


@pytest.mark.parametrize("thr", [0, 1, 24, 129])   # all tile / mixed / all sparse
@pytest.mark.parametrize("B,H,S,bs,lw,K,qs", [
    (1, 2, 300, 64, 128, 4, 3.0),
    (2, 3, 700, 64, 512, 8, 1.0),
    (1, 2, 513, 32, 100, 6, 3.0),     # window not a block multiple, bs 32
    (1, 1, 1100, 128, 256, 3, 2.0),   # bs 128 (tile path only)
    # 128-key blocks, window 31: the last block is routed and its second 64-key item lies
    # wholly past the end of the 43 tokens (its rows were once addressed out of bounds)
    (1, 1, 43, 128, 31, 4, 2.0),
    (1, 2, 64, 64, 512, 4, 1.0),      # window covers everything
    (1, 2, 3000, 64, 256, 16, 2.0),   # many remote blocks per tile
])
def test_prefill_attention_matches_oracle(B, H, S, bs, lw, K, qs, thr):
    _prefill_check(B, H, S, bs, lw, K, qs, thr)


@pytest.mark.parametrize("B,H,S,bs,lw,K,qs", [
    (1, 2, 2000, 32, 128, 64, 2.0),   # the training schedule's first k, block 32
    (2, 2, 1500, 64, 256, 33, 2.0),   # three slot groups, the last one partial
    (1, 3, 900, 64, 128, 24, 1.0),
])
def test_prefill_attention_more_than_16_slots(B, H, S, bs, lw, K, qs):
    """K > 16: every routed pair goes block-major whatever the threshold asks."""
    for thr in (24, 129):
        _prefill_check(B, H, S, bs, lw, K, qs, thr)


def _prefill_check(B, H, S, bs, lw, K, qs, thr):
    q, k, v, idx, bias, valid = _attn_inputs(300 + S, B, H, S, bs, lw, K, qscale=qs)
    scale = 1 / math.sqrt(128)
    ref = O.dense_attend(q, k, v, idx, bias, valid, bs, lw, scale)
    out, lse = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV),
                                valid.to(DEV), bs, lw, scale, return_lse=True,
                                dense_threshold=thr)
    _close(out, ref, f"prefill thr={thr}")
    assert torch.isfinite(lse).all()


@pytest.mark.parametrize("thr", [0, 1, 129])
def test_prefill_duplicates_and_strided_inputs(thr):
    B, H, S, bs, lw, K = 1, 2, 400, 64, 128, 4
    q, k, v, idx, bias, valid = _attn_inputs(310, B, H, S, bs, lw, K, qscale=2.0, dup=True)
    scale = 1 / math.sqrt(128)
    ref = O.dense_attend(q, k, v, idx, bias, valid, bs, lw, scale)
    # [B,S,H,D] storage viewed as [B,H,S,D]
    qs_, ks_, vs_ = (t.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for t in (q, k, v))
    out = ops.attn_prefill(qs_, ks_, vs_, idx.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, scale,
                           dense_threshold=thr)
    _close(out, ref, "prefill strided")


@pytest.mark.parametrize("thr", [0, 129])
def test_prefill_segment_start(thr):
    B, H, S, bs, lw, K = 1, 2, 600, 64, 128, 5
    q, k, v, idx, bias, valid = _attn_inputs(320, B, H, S, bs, lw, K, qscale=2.0)
    kmin = torch.zeros(1, S, dtype=torch.long)
    kmin[0, 250:] = 250
    scale = 1 / math.sqrt(128)
    ref = O.dense_attend(q, k, v, idx, bias, valid, bs, lw, scale, kmin=kmin)
    out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV),
                           valid.to(DEV), bs, lw, scale, kmin=kmin.to(DEV), dense_threshold=thr)
    _close(out, ref, "prefill kmin")


@pytest.mark.parametrize("thr", [0, 24, 129])
def test_prefill_varlen_block_diagonal(thr):
    g = _gen(330)
    cu = [0, 273, 273 + 819, 273 + 819 + 64, 273 + 819 + 64 + 1000]
    T, H, bs, lw, K = cu[-1], 2, 64, 256, 4
    q, k, v, idx, bias, valid = _attn_inputs(331, 1, H, T, bs, lw, K, qscale=2.0)
    scale = 1 / math.sqrt(128)
    # per-document routing on each document's own grid
    for b in range(len(cu) - 1):
        L = cu[b + 1] - cu[b]
        t = torch.arange(L)
        lb = lw // bs
        hi = (t // bs - lb).clamp(min=0)
        i2 = (torch.rand(L, K, generator=g) * (hi[:, None] + 1)).floor().long()
        idx[0, cu[b]:cu[b + 1]] = i2
        valid[0, cu[b]:cu[b + 1]] &= (t // bs - lb >= 0)[:, None]
    out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx[0].to(DEV), bias[0].to(DEV),
                           valid[0].to(DEV), bs, lw, scale,
                           cu_seqlens=torch.tensor(cu, dtype=torch.int32).to(DEV),
                           dense_threshold=thr)
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        ref = O.dense_attend(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1], idx[:, s0:s1],
                             bias[:, s0:s1], valid[:, s0:s1], bs, lw, scale)
        _close(out[:, :, s0:s1], ref, f"varlen doc {b}")


@pytest.mark.parametrize("thr", [24, 129])
def test_prefill_varlen_many_documents(thr):
    """1,100 packed documents: more sequences than one work-group scans at once
    (the chunk-count prefix over sequences runs in two passes), documents with and
    without sparse chunks."""
    g = _gen(340)
    lens = (torch.rand(1100, generator=g) * 90 + 20).long().tolist()
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    T, H, bs, lw, K = cu[-1], 1, 32, 16, 3
    q, k, v, idx, bias, valid = _attn_inputs(341, 1, H, T, bs, lw, K)
    for b in range(len(lens)):
        L = lens[b]
        t = torch.arange(L)
        lb = (lw + bs - 1) // bs
        hi = (t // bs - lb).clamp(min=0)
        idx[0, cu[b]:cu[b + 1]] = (torch.rand(L, K, generator=g) * (hi[:, None] + 1)).floor().long()
        valid[0, cu[b]:cu[b + 1]] &= (t // bs - lb >= 0)[:, None]
    out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx[0].to(DEV), bias[0].to(DEV),
                           valid[0].to(DEV), bs, lw, 1 / math.sqrt(128),
                           cu_seqlens=torch.tensor(cu, dtype=torch.int32).to(DEV),
                           dense_threshold=thr).cpu()
    for b in range(len(lens)):
        s0, s1 = cu[b], cu[b + 1]
        ref = O.dense_attend(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1], idx[:, s0:s1],
                             bias[:, s0:s1], valid[:, s0:s1], bs, lw, 1 / math.sqrt(128))
        _close(out[:, :, s0:s1], ref, f"document {b}")


@pytest.mark.parametrize("thr", [0, 24])
@pytest.mark.parametrize("K", [0, 4])
def test_prefill_empty_documents_single_tokens_no_routing(thr, K):
    """Packed documents of 0, 5, 0, 295, 1 and 0 tokens; with and without routed slots."""
    g = _gen(350 + K)
    cu = [0, 0, 5, 5, 300, 301, 301]
    T, H, bs, lw = cu[-1], 2, 64, 128
    q, k, v, idx, bias, valid = _attn_inputs(351 + K, 1, H, T, bs, lw, max(K, 1))
    if K == 0:
        idx, bias, valid = idx[..., :0], bias[..., :0], valid[..., :0]
    else:
        for b in range(len(cu) - 1):
            L = cu[b + 1] - cu[b]
            t = torch.arange(L)
            hi = (t // bs - lw // bs).clamp(min=0)
            idx[0, cu[b]:cu[b + 1]] = (torch.rand(L, K, generator=g) * (hi[:, None] + 1)).floor().long()
            valid[0, cu[b]:cu[b + 1]] &= (t // bs - lw // bs >= 0)[:, None]
    scale = 1 / math.sqrt(128)
    out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx[0].to(DEV), bias[0].to(DEV),
                           valid[0].to(DEV), bs, lw, scale,
                           cu_seqlens=torch.tensor(cu, dtype=torch.int32).to(DEV),
                           dense_threshold=thr).cpu()
    assert out.shape == (1, H, T, 128)
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        if s1 == s0:
            continue
        ref = O.dense_attend(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1], idx[:, s0:s1],
                             bias[:, s0:s1], valid[:, s0:s1], bs, lw, scale)
        _close(out[:, :, s0:s1], ref, f"document {b}")


@pytest.mark.parametrize("B,H,S,bs,lw,K,qs,km", [
    (1, 2, 300, 64, 128, 4, 3.0, False),     # 6 tiles: 8 parts each, most of them empty
    (2, 3, 700, 64, 512, 8, 1.0, True),      # 36 tiles, segment starts
    (1, 1, 1100, 128, 256, 3, 2.0, False),   # 128-key blocks: parts cut at block boundaries
    (1, 10, 2730, 64, 512, 8, 1.0, False),   # 220 tiles: 2 parts
])
def test_prefill_split_tiles(B, H, S, bs, lw, K, qs, km):
    """Every routed block with its tile, the tiles of a small grid split over several
    work-groups (their partials merged by a second launch) and unsplit: both against
    the oracle, and their log-sum-exps against each other."""
    q, k, v, idx, bias, valid = _attn_inputs(360 + S, B, H, S, bs, lw, K, qscale=qs)
    kmin = None
    if km:
        kmin = torch.zeros(B, S, dtype=torch.long)
        kmin[:, 250:] = 250
        kmin[1:, 480:] = 480
    scale = 1 / math.sqrt(128)
    ref = O.dense_attend(q, k, v, idx, bias, valid, bs, lw, scale, kmin=kmin)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw,
            scale)
    kw = dict(return_lse=True, dense_threshold=0,
              kmin=None if kmin is None else kmin.to(DEV))
    o_split, l_split = ops.attn_prefill(*args, **kw)
    o_one, l_one = ops.attn_prefill(*args, split_tiles=False, **kw)
    _close(o_split, ref, "split tiles")
    _close(o_one, ref, "one work-group per tile")
    # each side sums bf16-rounded probabilities (relative error <= 2^-9 per term, so
    # <= 2^-9 in the sum and in the log-sum-exp) against its own running maxima
    torch.testing.assert_close(l_split.cpu(), l_one.cpu(), atol=2 * 2.0 ** -9, rtol=0)


def test_prefill_workspace_any_contents():
    """The sparse path's workspace may hold anything, as a cached buffer last used by a
    call of another shape does: the call clears its own counters first."""
    g = _gen(345)
    lens = (torch.rand(300, generator=g) * 90 + 20).long().tolist()
    cu = [0]
    for L in lens:
        cu.append(cu[-1] + L)
    T, H, bs, lw, K = cu[-1], 1, 32, 16, 3
    q, k, v, idx, bias, valid = _attn_inputs(346, 1, H, T, bs, lw, K)
    for b in range(len(lens)):
        L = lens[b]
        t = torch.arange(L)
        lb = (lw + bs - 1) // bs
        hi = (t // bs - lb).clamp(min=0)
        idx[0, cu[b]:cu[b + 1]] = (torch.rand(L, K, generator=g) * (hi[:, None] + 1)).floor().long()
        valid[0, cu[b]:cu[b + 1]] &= (t // bs - lb >= 0)[:, None]
    qd = q.to(DEV)
    ws = ops.cached_workspace("prefill", 256 << 20, qd.device)     # the buffer the call takes
    ws.fill_(0x5A)                       # every counter starts at 0x5A5A5A5A
    out = ops.attn_prefill(qd, k.to(DEV), v.to(DEV), idx[0].to(DEV), bias[0].to(DEV),
                           valid[0].to(DEV), bs, lw, 1 / math.sqrt(128),
                           cu_seqlens=torch.tensor(cu, dtype=torch.int32).to(DEV),
                           dense_threshold=24).cpu()
    for b in range(len(lens)):
        s0, s1 = cu[b], cu[b + 1]
        ref = O.dense_attend(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1], idx[:, s0:s1],
                             bias[:, s0:s1], valid[:, s0:s1], bs, lw, 1 / math.sqrt(128))
        _close(out[:, :, s0:s1], ref, f"document {b}")


def test_prefill_pipeline_2730_tokens():
    """Prefill at 2,730 tokens (10 pages): GPU k_bar -> scores -> route -> attention.
    Routing is bit-exact against the oracle on the GPU's scores; the attention is
    compared with the oracle on the same routing."""
    cfg = W.PREFILL_2730
    d = W.make_prefill(cfg)
    kb = ops.kbar(d["idx_k"].to(DEV), torch.zeros(128, device=DEV), cfg.bs)
    z = ops.block_scores(d["idx_q"].to(DEV), kb, cfg.bs, cfg.lw // cfg.bs)
    ti, bi, va = ops.route(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap)
    ti_r, bi_r, va_r = O.infer_route_select(z.cpu(), None, W.IDX_SCALE, W.FLOOR, W.SIGMA,
                                            cfg.cap, cfg.cap)
    assert torch.equal(ti.cpu().long(), ti_r) and torch.equal(va.cpu(), va_r)
    scale = 1 / math.sqrt(128)
    out = ops.attn_prefill(d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV), ti, bi, va,
                           cfg.bs, cfg.lw, scale)
    ref = O.dense_attend(d["q"], d["k"], d["v"], ti_r, bi_r, va_r, cfg.bs, cfg.lw, scale)
    _close(out, ref, "prefill 2730")


# ------------------------------------------------------------------ decode attention

def _decode_inputs(seed, B, H, S, bs, lw, K, lens=None):
    g = _gen(seed)
    q = (torch.randn(B, H, 128, generator=g) * 0.6).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.3).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    if lens is None:
        lens = torch.full((B,), S, dtype=torch.int32)
    idx = torch.zeros(B, K, dtype=torch.long)
    valid = torch.zeros(B, K, dtype=torch.bool)
    for b in range(B):
        L = int(lens[b])
        hi = (L - 1) // bs - (lw + bs - 1) // bs
        if hi >= 0:
            perm = torch.randperm(hi + 1, generator=g)[:K]
            idx[b, :perm.numel()] = perm
            valid[b, :perm.numel()] = True
    bias = torch.randn(B, K, generator=g)
    return q, k, v, idx, bias, valid, lens


def _decode_ref(q, k, v, idx, bias, valid, lens, bs, lw, scale):
    outs = []
    for b in range(q.shape[0]):
        L = int(lens[b])
        o = O.decode_attend(q[b:b + 1, :, None], k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                            idx[b:b + 1, None], bias[b:b + 1, None], valid[b:b + 1, None],
                            torch.tensor([[L - 1]]), bs, lw, scale)
        outs.append(o[:, :, 0])
    return torch.cat(outs)


@pytest.mark.parametrize("nsplit", [None, 1, 3, 20, 64])
def test_decode_contiguous_matches_oracle(nsplit):
    B, H, S, bs, lw, K = 3, 2, 3000, 64, 1024, 16
    lens = torch.tensor([3000, 1500, 1100], dtype=torch.int32)
    q, k, v, idx, bias, valid, lens = _decode_inputs(400, B, H, S, bs, lw, K, lens)
    scale = 1 / math.sqrt(128)
    ref = _decode_ref(q, k, v, idx, bias, valid, lens, bs, lw, scale)
    out = ops.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV),
                          valid.to(DEV), bs, lw, scale, seq_lens=lens.to(DEV), nsplit=nsplit)
    _close(out, ref, "decode")


def test_decode_without_routed_blocks_and_single_token():
    B, H, bs, lw = 3, 2, 64, 512
    lens = torch.tensor([1, 64, 1500], dtype=torch.int32)
    q, k, v, idx, bias, valid, lens = _decode_inputs(420, B, H, 1500, bs, lw, 1, lens)
    idx, bias, valid = idx[:, :0], bias[:, :0], valid[:, :0]
    scale = 1 / math.sqrt(128)
    ref = _decode_ref(q, k, v, idx, bias, valid, lens, bs, lw, scale)
    out = ops.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), None, None, None, bs, lw, scale,
                          seq_lens=lens.to(DEV))
    _close(out, ref, "decode, window only")
    torch.testing.assert_close(out[0].cpu(), v[0, :, 0].float(), atol=1e-6, rtol=0)   # one key


def test_decode_paged_matches_contiguous_oracle():
    B, H, bs, lw, K = 4, 2, 64, 512, 8
    lens = torch.tensor([2000, 700, 1300, 65], dtype=torch.int32)
    S = int(lens.max())
    q, k, v, idx, bias, valid, lens = _decode_inputs(410, B, H, S, bs, lw, K, lens)
    g = _gen(411)
    npg = [(int(L) + bs - 1) // bs for L in lens]
    perm = torch.randperm(sum(npg), generator=g)
    table = torch.zeros(B, max(npg), dtype=torch.int32)
    kp = torch.zeros(sum(npg), bs, H, 128, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    o = 0
    for b in range(B):
        for p in range(npg[b]):
            phys = int(perm[o + p])
            table[b, p] = phys
            seg = slice(p * bs, min((p + 1) * bs, int(lens[b])))
            n = seg.stop - seg.start
            kp[phys, :n] = k[b, :, seg].transpose(0, 1)
            vp[phys, :n] = v[b, :, seg].transpose(0, 1)
        o += npg[b]
    scale = 1 / math.sqrt(128)
    ref = _decode_ref(q, k, v, idx, bias, valid, lens, bs, lw, scale)
    out = ops.attn_decode(q.to(DEV), kp.to(DEV), vp.to(DEV), idx.to(DEV), bias.to(DEV),
                          valid.to(DEV), bs, lw, scale, seq_lens=lens.to(DEV),
                          block_table=table.to(DEV), page_size=bs)
    _close(out, ref, "decode paged")


def _pages_of(k, v, lens, page, seed):
    """k/v [B,H,S,D] -> pages [n, page, H, D] in a random order, and the block table."""
    B = k.shape[0]
    g = _gen(seed)
    npg = [(int(L) + page - 1) // page for L in lens]
    perm = torch.randperm(sum(npg), generator=g)
    table = torch.zeros(B, max(npg), dtype=torch.int32)
    kp = torch.zeros(sum(npg), page, k.shape[1], 128, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    o = 0
    for b in range(B):
        for p_ in range(npg[b]):
            phys = int(perm[o + p_])
            table[b, p_] = phys
            seg = slice(p_ * page, min((p_ + 1) * page, int(lens[b])))
            n = seg.stop - seg.start
            kp[phys, :n] = k[b, :, seg].transpose(0, 1)
            vp[phys, :n] = v[b, :, seg].transpose(0, 1)
        o += npg[b]
    return kp, vp, table


@pytest.mark.parametrize("bs,mult", [(64, 2), (64, 4), (32, 3)])
def test_decode_pages_of_several_blocks_equal_contiguous(bs, mult):
    """Pages holding several key blocks (page = mult * block): the split-K decode and the
    fused decode step give the contiguous cache's results bit for bit.  A round trip's
    block-table entry is read once and its rows are addressed from the page's first key,
    so every row offset inside a page goes through that arithmetic."""
    B, H, lw, K = 3, 2, 256, 4
    lens = torch.tensor([1500, 333, 900], dtype=torch.int32)
    S = int(lens.max())
    q, k, v, idx, bias, valid, lens = _decode_inputs(430 + mult + bs, B, H, S, bs, lw, K, lens)
    page = mult * bs
    kp, vp, table = _pages_of(k, v, lens, page, 440 + mult)
    scale = 1 / math.sqrt(128)
    args = (idx.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, scale)
    cont = ops.attn_decode(q.to(DEV), k.to(DEV), v.to(DEV), *args, seq_lens=lens.to(DEV)).cpu()
    paged = ops.attn_decode(q.to(DEV), kp.to(DEV), vp.to(DEV), *args, seq_lens=lens.to(DEV),
                            block_table=table.to(DEV), page_size=page).cpu()
    assert torch.equal(cont, paged)
    _close(paged, _decode_ref(q, k, v, idx, bias, valid, lens, bs, lw, scale), "decode, pages of blocks")
    # the fused step (routing beside the window part) over the same two layouts
    g = _gen(450 + mult)
    iq = torch.randn(B, 1, 128, generator=g)
    ik = torch.randn(B, S, 128, generator=g)
    ik_pages = torch.zeros(kp.shape[0], page, 128)
    for b in range(B):
        for p_ in range((int(lens[b]) + page - 1) // page):
            seg = slice(p_ * page, min((p_ + 1) * page, int(lens[b])))
            ik_pages[int(table[b, p_]), :seg.stop - seg.start] = ik[b, seg]
    hc = torch.zeros(128, device=DEV)
    nblk_cap = table.shape[1] * page // bs          # the summaries cover the table's pages
    outs = []
    for kk, vv, ikk, kw in ((k, v, ik, {}), (kp, vp, ik_pages,
                                             dict(block_table=table.to(DEV), page_size=page))):
        kb = ops.kbar(ikk.to(DEV), hc, bs, seq_lens=lens.to(DEV), nblk_cap=nblk_cap, **kw)
        o, _ = ops.decode_step_fused(q.to(DEV), kk.to(DEV), vv.to(DEV), iq.to(DEV), ikk.to(DEV), hc,
                                     kb, bs, lw // bs, W.IDX_SCALE, W.FLOOR, W.SIGMA, K, K, scale,
                                     seq_lens=lens.to(DEV), **kw)
        outs.append(o.cpu())
    assert torch.equal(outs[0], outs[1])


def test_decode_equals_prefill_last_row():
    B, H, S, bs, lw, K = 1, 2, 900, 64, 256, 4
    q, k, v, idx, bias, valid = _attn_inputs(420, B, H, S, bs, lw, K, qscale=2.0)
    scale = 1 / math.sqrt(128)
    pre = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV),
                           valid.to(DEV), bs, lw, scale).float().cpu()
    dec = ops.attn_decode(q[:, :, -1].to(DEV), k.to(DEV), v.to(DEV), idx[:, -1].to(DEV),
                          bias[:, -1].to(DEV), valid[:, -1].to(DEV), bs, lw, scale).cpu()
    _close(dec, pre[:, :, -1], "decode vs prefill", tight=2e-2)


# ------------------------------------------------------------------ fused decode router

def _decode_route_check(ik_seq, iq, lens, bs, lb, K, topm, hc, cand=None, paged=None):
    """ik_seq: list of per-sequence idx_k [L_b, d] (CPU).  The k_bar cache starts from
    the summaries of all complete blocks (the tail block is left stale on purpose)."""
    B = len(ik_seq)
    d = iq.shape[-1]
    nblk_cap = max((int(L) + bs - 1) // bs for L in lens)
    kb0 = torch.zeros(B, nblk_cap, d)
    refs = []
    for b in range(B):
        kb_r, _ = O.kbar_headcls(ik_seq[b][None], hc, bs)
        refs.append(kb_r[0])
        n = kb_r.shape[1]
        kb0[b, :n - 1] = kb_r[0, :n - 1]          # tail block stale (zeros)
    if paged is None:
        S = max(int(L) for L in lens)
        ik = torch.zeros(B, S, d)
        for b in range(B):
            ik[b, :int(lens[b])] = ik_seq[b]
        kw = {}
        ik_dev = ik.to(DEV)
    else:
        pages, table = paged
        ik_dev = pages.to(DEV)
        kw = dict(block_table=table.to(DEV), page_size=bs)
    kb = kb0.to(DEV)
    ti, bi, va, z = ops.decode_route(iq.to(DEV), ik_dev, hc.to(DEV), kb, bs, lb, W.IDX_SCALE,
                                     W.FLOOR, W.SIGMA, K, topm,
                                     seq_lens=torch.tensor(lens, dtype=torch.int32).to(DEV),
                                     cand=None if cand is None else cand.to(DEV),
                                     return_scores=True, **kw)
    ti, bi, va, z, kb = ti.cpu(), bi.cpu(), va.cpu(), z.cpu(), kb.cpu()
    for b in range(B):
        L = int(lens[b])
        n = (L + bs - 1) // bs
        torch.testing.assert_close(kb[b, n - 1], refs[b][n - 1], atol=1e-5, rtol=1e-5)
        zr = O.block_scores_headcls(iq[b:b + 1, None], refs[b][None], torch.ones(1, n, dtype=torch.bool),
                                    torch.tensor([[L - 1]]), bs, lb)[0, 0]
        sent = zr == O.SCORE_NEG
        assert torch.equal(z[b, :n] == O.SCORE_NEG, sent)
        torch.testing.assert_close(z[b, :n][~sent], zr[~sent], atol=1e-7, rtol=1e-5)
        # routing bit-exact on the kernel's own scores
        cb = None if cand is None else cand[b:b + 1, None, :n]
        t_r, b_r, v_r = O.infer_route_select(z[b:b + 1, None, :n], cb, W.IDX_SCALE, W.FLOOR,
                                             W.SIGMA, K, topm)
        kp = t_r.shape[-1]
        assert torch.equal(va[b, 0, :kp], v_r[0, 0]), b
        assert torch.equal(ti[b, 0, :kp].long(), t_r[0, 0]), b
        torch.testing.assert_close(bi[b, 0, :kp], b_r[0, 0], atol=2e-5, rtol=1e-5)
        assert (ti[b, 0, kp:] == -1).all() and not va[b, 0, kp:].any()


@pytest.mark.parametrize("hc_scale,scale", [(0.0, 1.0), (1.5, 30.0)])
def test_decode_route_contiguous(hc_scale, scale):
    g = _gen(500)
    lens = [27300, 5000, 1100, 640, 1]
    d, bs, lb = 128, 64, 16
    ik_seq = [torch.randn(L, d, generator=g) * 0.1 for L in lens]
    iq = torch.randn(len(lens), d, generator=g) * scale
    hc = torch.randn(d, generator=g) * hc_scale
    _decode_route_check(ik_seq, iq, lens, bs, lb, 16, 16, hc)


def test_decode_route_ties():
    """Block-constant keys from three levels (many exactly tied scores) and one
    sequence where every remote block ties: ids must follow (score desc, id asc)."""
    g = _gen(502)
    lens = [5000, 2000, 64 * 20]
    d, bs, lb = 128, 64, 2
    base = torch.randn(3, d, generator=g) * 0.1
    ik_seq = []
    for L in lens:
        lvl = torch.randint(0, 3, ((L + bs - 1) // bs,), generator=g)
        ik_seq.append(base[lvl].repeat_interleave(bs, 0)[:L].contiguous())
    ik_seq[2] = torch.full((lens[2], d), 0.05)
    iq = torch.randn(len(lens), d, generator=g)
    _decode_route_check(ik_seq, iq, lens, bs, lb, 16, 16, torch.zeros(d))


def test_decode_route_paged_with_candidates():
    g = _gen(501)
    lens = [3000, 2049, 700]
    d, bs, lb = 128, 64, 4
    ik_seq = [torch.randn(L, d, generator=g) for L in lens]
    iq = torch.randn(len(lens), d, generator=g) * 10
    npg = [(L + bs - 1) // bs for L in lens]
    perm = torch.randperm(sum(npg), generator=g)
    table = torch.zeros(len(lens), max(npg), dtype=torch.int32)
    pages = torch.zeros(sum(npg), bs, d)
    o = 0
    for b, L in enumerate(lens):
        for p in range(npg[b]):
            ph = int(perm[o + p])
            table[b, p] = ph
            seg = ik_seq[b][p * bs:min((p + 1) * bs, L)]
            pages[ph, :seg.shape[0]] = seg
        o += npg[b]
    cand = torch.rand(len(lens), max(npg), generator=g) < 0.3
    cand[2] = False                             # falls back to every remote block
    _decode_route_check(ik_seq, iq, lens, bs, lb, 8, 12, torch.zeros(d), cand=cand,
                        paged=(pages, table))


def test_decode_step_pipeline_matches_oracle():
    """decode_step (fused router + split-K attention) against the oracle decode path."""
    from ananta_ocr_amd import pipeline
    cfg = W.Decode("small", 3, 4000, 64, 1024, 16, seed=9)
    d = W.make_decode(cfg)
    hc = torch.zeros(128)
    nblk = (cfg.S + cfg.bs - 1) // cfg.bs
    st = pipeline.init_decode_state(d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, nblk)
    scale = 1 / math.sqrt(128)
    out, (ti, bi, va) = pipeline.decode_step(
        st, d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV), d["idx_q"].to(DEV),
        d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE * 50, W.FLOOR,
        W.SIGMA, cfg.cap, cfg.cap, scale, return_routing=True)
    ref, t_r, b_r, v_r = O.decode_pipeline(d["q"][:, :, None], d["k"], d["v"], d["idx_q"],
                                           d["idx_k"], hc, cfg.bs, cfg.lw // cfg.bs,
                                           W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap,
                                           scale)
    # the oracle routes its own scores: compare ids as sets where both are valid
    assert torch.equal(va.cpu(), v_r)
    assert torch.equal(ti.cpu().long(), t_r)
    _close(out, ref[:, :, 0], "decode step")


@pytest.mark.parametrize("paged", [False, True])
@pytest.mark.parametrize("bs", [32, 64, 128])
def test_decode_step_fused_matches_two_launch_path(paged, bs):
    """The fused decode step (window attention beside the router, routed blocks and
    merge in a second launch) against decode_route + attn_decode: routing bit for bit,
    outputs to fp32 rounding (the window is cut into 32-key pieces instead of blocks)."""
    from ananta_ocr_amd import pipeline
    H, d, lw, K = 3, 128, 512, 8
    lens = [2900, 1, 33, 511, 1300]
    B, S = len(lens), max(lens)
    g = _gen(470 + bs + int(paged))
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    ik = torch.randn(B, S, d, generator=g)
    iq = torch.randn(B, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.1
    nblk = (S + bs - 1) // bs
    kw = dict(seq_lens=torch.tensor(lens, dtype=torch.int32).to(DEV))
    if paged:
        npg = [(L + bs - 1) // bs for L in lens]
        perm = torch.randperm(sum(npg), generator=g)
        table = torch.zeros(B, max(npg), dtype=torch.int32)
        kp = torch.zeros(sum(npg), bs, H, 128, dtype=torch.bfloat16)
        vp = torch.zeros_like(kp)
        ikp = torch.zeros(sum(npg), bs, d)
        o = 0
        for b in range(B):
            for pg in range(npg[b]):
                phys = int(perm[o + pg])
                table[b, pg] = phys
                seg = slice(pg * bs, min((pg + 1) * bs, lens[b]))
                n = seg.stop - seg.start
                kp[phys, :n] = k[b, :, seg].transpose(0, 1)
                vp[phys, :n] = v[b, :, seg].transpose(0, 1)
                ikp[phys, :n] = ik[b, seg]
            o += npg[b]
        kd, vd, ikd = kp.to(DEV), vp.to(DEV), ikp.to(DEV)
        kw.update(block_table=table.to(DEV), page_size=bs)
        nblk = max(npg)
    else:
        kd, vd, ikd = k.to(DEV), v.to(DEV), ik.to(DEV)
    st = pipeline.init_decode_state(ikd, hc.to(DEV), bs, nblk, **kw)
    args = (hc.to(DEV), bs, lw // bs, W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, K, K, 1 / math.sqrt(128))
    out_f, (ti_f, bi_f, va_f) = pipeline.decode_step(st, q.to(DEV), kd, vd, iq.to(DEV), ikd, *args,
                                                     return_routing=True, fused=True, **kw)
    out_s, (ti_s, bi_s, va_s) = pipeline.decode_step(st, q.to(DEV), kd, vd, iq.to(DEV), ikd, *args,
                                                     return_routing=True, fused=False, **kw)
    assert torch.equal(ti_f, ti_s) and torch.equal(va_f, va_s) and torch.equal(bi_f, bi_s)
    assert va_f.any()
    torch.testing.assert_close(out_f, out_s, atol=2e-5, rtol=2e-5)


@pytest.mark.parametrize("B", [5, 40])
def test_decode_step_workspace_reuse(B):
    """The fused step's routers hand their slots to the window wavefronts of the same
    launch through words at the end of the workspace, which start at zero and which
    every step zeroes again.  Steps whose routing changes, run on one reused buffer,
    give the results of a freshly zeroed buffer bit for bit, and match decode_route +
    attn_decode; so does a smaller batch on the same buffer.  B = 5 takes the routed
    slots in the first launch; B = 40 (a grid of several rounds) in a launch of their
    own."""
    import ctypes
    from ananta_ocr_amd import _lib, pipeline
    H, d, bs, lw, K = 10, 128, 64, 1024, 16
    g = _gen(900 + B)
    lens = torch.randint(1100, 3000, (B,), generator=g)
    S = int(lens.max())
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16().to(DEV)
    v = torch.randn(B, H, S, 128, generator=g).bfloat16().to(DEV)
    ik = torch.randn(B, S, d, generator=g).to(DEV)
    hc = (torch.randn(d, generator=g) * 0.1).to(DEV)
    L = lens.to(torch.int32).to(DEV)
    st = pipeline.init_decode_state(ik, hc, bs, (S + bs - 1) // bs, seq_lens=L)
    need = ctypes.c_int64(0)
    assert _lib.load().dash_decode_step_workspace_size(B, H, 128, bs, lw, need) == 0
    nf = (need.value + 3) // 4 + 1000            # not a multiple of 256 bytes
    reused = torch.zeros(nf, dtype=torch.float32, device=DEV)
    args = (hc, bs, lw // bs, W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, K, K, 1 / math.sqrt(128))
    prev = None
    for step in range(3):
        q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16().to(DEV)
        iq = torch.randn(B, d, generator=g).to(DEV)
        res = [ops.decode_step_fused(q, k, v, iq, ik, hc, st.kbar, *args[1:], seq_lens=L,
                                     workspace=ws)
               for ws in (reused, torch.zeros(nf, device=DEV))]
        for a_, b_ in zip(res[0][1], res[1][1]):
            assert torch.equal(a_, b_), step
        assert torch.equal(res[0][0], res[1][0]), step
        out_s, (ti_s, bi_s, va_s) = pipeline.decode_step(st, q, k, v, iq, ik, *args,
                                                         return_routing=True, fused=False,
                                                         seq_lens=L)
        out, (ti, bi, va) = res[0]
        assert torch.equal(ti[:, 0], ti_s[:, 0]) and torch.equal(bi[:, 0], bi_s[:, 0])
        assert bool(va.bool().any())
        torch.testing.assert_close(out, out_s, atol=2e-5, rtol=2e-5)
        if prev is not None:
            assert not torch.equal(ti, prev), step        # the routing changed
        prev = ti.clone()
    # every step left the words zero
    assert not bool(reused.view(torch.int64)[-(B * 32 + 64):].ne(0).any())
    # a smaller batch on the same buffer
    Bs = B // 2 + 1
    sub = dict(seq_lens=L[:Bs])
    st_s = pipeline.init_decode_state(ik[:Bs], hc, bs, (S + bs - 1) // bs, **sub)
    res = [ops.decode_step_fused(q[:Bs], k[:Bs], v[:Bs], iq[:Bs], ik[:Bs], hc, st_s.kbar,
                                 *args[1:], workspace=ws, **sub)
           for ws in (reused, torch.zeros(nf, device=DEV))]
    assert torch.equal(res[0][0], res[1][0])
    for a_, b_ in zip(res[0][1], res[1][1]):
        assert torch.equal(a_, b_)


def test_decode_graph_replays_match_eager():
    """decode_step captured in a HIP graph: every replay (with eager work and
    synchronisations between replays, and after the query buffer is rewritten in
    place) equals the eager step bit for bit."""
    from ananta_ocr_amd import pipeline
    cfg = W.Decode("small", 3, 4000, 64, 1024, 16, seed=12)
    d = W.make_decode(cfg)
    hc = torch.zeros(128, device=DEV)
    nblk = (cfg.S + cfg.bs - 1) // cfg.bs
    q, k, v = d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV)
    iq, ik = d["idx_q"].to(DEV), d["idx_k"].to(DEV)
    st = pipeline.init_decode_state(ik, hc, cfg.bs, nblk)
    args = (hc, cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap,
            1 / math.sqrt(128))
    eager = pipeline.decode_step(st, q, k, v, iq, ik, *args).clone()
    g = pipeline.DecodeGraph(st, q, k, v, iq, ik, *args)
    for i in range(4):
        out = g.replay().clone()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        again = pipeline.decode_step(st, q, k, v, iq, ik, *args)      # eager work in between
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    # a new query written into the captured buffer
    gen = torch.Generator().manual_seed(13)
    q2 = (torch.randn(q.shape, generator=gen) * 0.5).to(DEV, q.dtype)
    iq2 = torch.randn(iq.shape, generator=gen).to(DEV, iq.dtype)
    ref2 = pipeline.decode_step(st, q2, k, v, iq2, ik, *args).clone()
    q.copy_(q2)
    iq.copy_(iq2)
    for i in range(2):
        out = g.replay().clone()
        torch.cuda.synchronize()
        assert torch.equal(out, ref2), f"replay with new query {i}"


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("paged", [False, True])
def test_decode_checkpoint_config_matches_oracle(paged, fused):
    """Decode at the shipped checkpoint's router configuration (config.json: block 32,
    local blocks 4 = window 128, dash_topk_blocks 12, topm 16, learned head_cls) on
    sequences of several lengths, contiguous or paged (pages of 32 tokens in a random
    physical order), fused step or router + split-K: block summaries and scores within
    fp32 tolerance, routing bit for bit on the GPU's own scores, attention within the
    output tolerance."""
    from ananta_ocr_amd import pipeline
    bs, lb, K, topm, H, d = 32, 4, 12, 16, 4, 128
    lw = lb * bs
    lens = [5000, 97, 129, 1, 2048, 3333]
    B, S = len(lens), max(lens)
    g = _gen(880 + 2 * int(paged) + int(fused))
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    ik = torch.randn(B, S, d, generator=g)
    iq = torch.randn(B, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.3
    lens_t = torch.tensor(lens, dtype=torch.int32)
    kw = dict(seq_lens=lens_t.to(DEV))
    nblk = (S + bs - 1) // bs
    if paged:
        npg = [(L + bs - 1) // bs for L in lens]
        perm = torch.randperm(sum(npg), generator=g)
        table = torch.zeros(B, max(npg), dtype=torch.int32)
        kp = torch.zeros(sum(npg), bs, H, 128, dtype=torch.bfloat16)
        vp = torch.zeros_like(kp)
        ikp = torch.zeros(sum(npg), bs, d)
        o = 0
        for b in range(B):
            for pg in range(npg[b]):
                phys = int(perm[o + pg])
                table[b, pg] = phys
                seg = slice(pg * bs, min((pg + 1) * bs, lens[b]))
                n = seg.stop - seg.start
                kp[phys, :n] = k[b, :, seg].transpose(0, 1)
                vp[phys, :n] = v[b, :, seg].transpose(0, 1)
                ikp[phys, :n] = ik[b, seg]
            o += npg[b]
        kd, vd, ikd = kp.to(DEV), vp.to(DEV), ikp.to(DEV)
        kw.update(block_table=table.to(DEV), page_size=bs)
        nblk = max(npg)
    else:
        kd, vd, ikd = k.to(DEV), v.to(DEV), ik.to(DEV)
    st = pipeline.init_decode_state(ikd, hc.to(DEV), bs, nblk, **kw)
    idx_scale = 128.0 / math.sqrt(128)
    out, (ti, bi, va), z = pipeline.decode_step(
        st, q.to(DEV), kd, vd, iq.to(DEV), ikd, hc.to(DEV), bs, lb, idx_scale, 1e-4, 1.0, K,
        topm, 1 / math.sqrt(128), return_routing=True, fused=fused, return_scores=True, **kw)
    out, ti, bi, va, z, kbar = out.cpu(), ti.cpu().long(), bi.cpu(), va.cpu(), z.cpu(), \
        st.kbar.cpu()
    Kp = ti.shape[-1]
    for b, L in enumerate(lens):
        kb_r, cv = O.kbar_headcls(ik[b:b + 1, :L], hc, bs)
        nb = kb_r.shape[1]
        torch.testing.assert_close(kbar[b:b + 1, :nb], kb_r, atol=1e-5, rtol=1e-5)
        z_r = O.block_scores_headcls(iq[b:b + 1, None], kb_r, cv, torch.tensor([[L - 1]]), bs,
                                     lb)
        zb = z[b:b + 1, None, :nb]
        sent = z_r < -5e8
        assert torch.equal(zb < -5e8, sent), f"sequence {b}: sentinel pattern"
        torch.testing.assert_close(zb[~sent], z_r[~sent], atol=2e-5, rtol=2e-5)
        t_r, b_r, v_r = O.infer_route_select(zb, None, idx_scale, 1e-4, 1.0, K, topm)
        kp_ = t_r.shape[-1]
        assert torch.equal(ti[b:b + 1, :, :kp_], t_r), f"sequence {b}: routed ids"
        assert torch.equal(va[b:b + 1, :, :kp_], v_r), f"sequence {b}: validity"
        torch.testing.assert_close(bi[b:b + 1, :, :kp_], b_r, atol=2e-5, rtol=1e-5)
        assert bool((ti[b, :, kp_:Kp] == -1).all())
        ref = O.decode_attend(q[b:b + 1, :, None].float(), k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                              t_r, b_r, v_r, torch.tensor([[L - 1]]), bs, lw, 1 / math.sqrt(128))
        _close(out[b:b + 1], ref[:, :, 0], f"decode bs 32 sequence {b} ({L} tokens)")


@pytest.mark.parametrize("nblk,scale,K,topm,quant,with_cand", [
    (427, 0.5, 16, 0, None, False),     # entmax over the whole row (topm <= 0)
    (100, 3.0, 12, 40, None, True),     # topm above 16
    (2048, 0.2, 64, 0, None, False),    # widest row, 64 slots
    (300, 1.0, 24, 64, 4.0, True),      # exact ties in x
    (43, 1e-4, 8, -1, None, False),
])
def test_route_wide_entmax_matches_oracle(nblk, scale, K, topm, quant, with_cand):
    """dash_route with topm <= 0 or > 16 (modeling_deepseekv2.py:323): ids and validity
    bit for bit (they depend on the ranking of x only), bias within 2e-3 (the oracle's
    threshold comes from float32 cumulative sums, the kernel's from float64)."""
    S = 600 if nblk < 1000 else 80
    bs, lb = (4, 2) if nblk < 1000 else (1, 1 - nblk + S)
    z = _scores(S, nblk, bs, lb, 700 + nblk + K, scale, quant=quant, nan_frac=0.005)
    cand = None
    if with_cand:
        cand = torch.rand(1, S, nblk, generator=_gen(701)) < 0.4
        cand[:, ::6] = False
    ti_r, bi_r, va_r = O.infer_route_select(z, cand, W.IDX_SCALE, W.FLOOR, W.SIGMA, K, topm)
    ti, bi, va = ops.route(z.to(DEV), None if cand is None else cand.to(DEV), W.IDX_SCALE,
                           W.FLOOR, W.SIGMA, K, topm)
    ti, bi, va = ti.cpu().long(), bi.cpu(), va.cpu()
    assert ti.shape == ti_r.shape
    assert torch.equal(ti, ti_r), f"routed ids differ at {(ti != ti_r).nonzero()[:5].tolist()}"
    assert torch.equal(va, va_r)
    torch.testing.assert_close(bi, bi_r, atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("topm,K", [(0, 24), (40, 20)])
def test_decode_wide_entmax_matches_oracle(topm, K):
    """Decode with a wide entmax: routing on the GPU's own scores equals the oracle's
    (ids and validity exactly), attention within the output tolerance."""
    from ananta_ocr_amd import pipeline
    bs, lb, H, d = 64, 4, 2, 128
    lens = [3000, 700, 1, 2222]
    B, S = len(lens), max(lens)
    g = _gen(990 + topm)
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    ik = torch.randn(B, S, d, generator=g)
    iq = torch.randn(B, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.3
    lens_t = torch.tensor(lens, dtype=torch.int32).to(DEV)
    nblk = (S + bs - 1) // bs
    st = pipeline.init_decode_state(ik.to(DEV), hc.to(DEV), bs, nblk, seq_lens=lens_t)
    idx_scale = 4.0 / math.sqrt(128)
    out, (ti, bi, va), z = pipeline.decode_step(
        st, q.to(DEV), k.to(DEV), v.to(DEV), iq.to(DEV), ik.to(DEV), hc.to(DEV), bs, lb,
        idx_scale, 1e-4, 1.0, K, topm, 1 / math.sqrt(128), return_routing=True, fused=True,
        return_scores=True, seq_lens=lens_t)
    out, ti, bi, va, z = out.cpu(), ti.cpu().long(), bi.cpu(), va.cpu().bool(), z.cpu()
    for b, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        zb = z[b:b + 1, None, :nb]
        t_r, b_r, v_r = O.infer_route_select(zb, None, idx_scale, 1e-4, 1.0, K, topm)
        kp_ = t_r.shape[-1]
        assert torch.equal(ti[b:b + 1, :, :kp_], t_r), f"sequence {b}: routed ids"
        assert torch.equal(va[b:b + 1, :, :kp_], v_r), f"sequence {b}: validity"
        torch.testing.assert_close(bi[b:b + 1, :, :kp_], b_r, atol=2e-3, rtol=1e-3)
        ref = O.decode_attend(q[b:b + 1, :, None].float(), k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                              t_r, b_r, v_r, torch.tensor([[L - 1]]), bs, lb * bs,
                              1 / math.sqrt(128))
        _close(out[b:b + 1], ref[:, :, 0], f"decode wide entmax sequence {b}")


def test_packed_prefill_graph_replays_match_eager():
    """A packed (cu_seqlens) prefill pass (k_bar, scores, routing, attention) given
    max_seqlen makes no host synchronisation, so it is captured in a HIP graph; every
    replay (with eager work and synchronisations between replays, and after new
    inputs are written into the captured buffers) equals the eager pass bit for bit."""
    from ananta_ocr_amd import pipeline
    cfg = W.Prefill("graph_packed", 1, 0, 64, 512, 8, seed=21, doc_pages=[3, 1, 7, 2])
    d = W.make_prefill(cfg, device=DEV)
    cu, cl = d["cu_seqlens"], d["cu_list"]
    maxlen = max(b - a for a, b in zip(cl[:-1], cl[1:]))
    hc = torch.zeros(128, device=DEV)
    args = (hc, cfg.bs, cfg.lw // cfg.bs, W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap,
            1 / math.sqrt(128))
    ins = [d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"]]

    def run():
        return pipeline.prefill(*ins, *args, cu_seqlens=cu, max_seqlen=maxlen)

    eager = run().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        again = run()                                  # eager work in between
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    d2 = W.make_prefill(W.Prefill("graph_packed2", 1, 0, 64, 512, 8, seed=22,
                                  doc_pages=[3, 1, 7, 2]), device=DEV)
    for dst, key in zip(ins, ["q", "k", "v", "idx_q", "idx_k"]):
        dst.copy_(d2[key])
    ref2 = run().clone()
    assert not torch.equal(ref2, eager)
    for i in range(2):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref2), f"replay with new inputs {i}"
    # and the pass against the oracle on the new inputs, document by document
    ref = O.prefill_varlen(d2["q"].cpu(), d2["k"].cpu(), d2["v"].cpu(), d2["idx_q"].cpu(),
                           d2["idx_k"].cpu(), cu.cpu(), torch.zeros(128), cfg.bs,
                           cfg.lw // cfg.bs, W.IDX_SCALE * 50, W.FLOOR, W.SIGMA, cfg.cap,
                           cfg.cap, 1 / math.sqrt(128))[0]
    _close(out, ref, "captured packed prefill")
