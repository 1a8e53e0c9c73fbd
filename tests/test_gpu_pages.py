"""Page-aware candidates on the GPU (csrc/dash_pages.hip through the C ABI) against the
oracle: page ids, per-query candidate rows, the decode allow row, and routing and
attention restricted by them."""

import math
import random
from types import SimpleNamespace

import pytest
import torch

from ananta_ocr_amd import ops, pages, pipeline
from ananta_ocr_amd import workloads as W
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
IMG, PG, TXT, BOS = 5, 9, 7, 1


def _prompt(rng, L, per_page_mode, img_run=(1, 9)):
    ids = [BOS]
    while len(ids) < L:
        if not per_page_mode and rng.random() < 0.15:
            ids.append(PG)
        if rng.random() < 0.6:
            ids.extend([IMG] * rng.randint(*img_run))
        else:
            ids.extend([TXT] * rng.randint(1, 4))
        if rng.random() < 0.1:
            ids.append(PG)
    return ids[:L]


def _ocr_prompt(pages_n, per_page, resp_tokens, rng):
    """An OCR prompt: BOS, then per page a marker and per_page image tokens, an
    instruction, then the response: per page a marker and some text."""
    ids = [BOS]
    for _ in range(pages_n):
        ids += [PG] + [IMG] * per_page
    ids += [TXT] * 5
    for _ in range(pages_n):
        ids += [PG] + [TXT] * rng.randint(1, resp_tokens)
    return ids


@pytest.mark.parametrize("seed,L", [(0, 700), (1, 5000), (2, 30000)])
def test_page_ids_match_oracle(seed, L):
    rng = random.Random(seed)
    rows = [_prompt(rng, L, per_page_mode=(b == 1)) for b in range(3)]
    rows.append(_ocr_prompt(pages_n=max(1, L // 400), per_page=273 if L > 5000 else 60,
                            resp_tokens=30, rng=rng)[:L])
    rows[-1] += [TXT] * (L - len(rows[-1]))
    ids = torch.tensor(rows)
    for scope in (False, True):
        for per_page in (3, 273):
            itm, ipi, qpi, en = pages.page_ids(ids.to(DEV), IMG, PG, L + 5, per_page, scope)
            r = O.page_aware_ids(ids, IMG, PG, L + 5, per_page, scope)
            if r[0] is None:
                assert not bool(en.cpu().any(0).all())
                continue
            assert torch.equal(itm.cpu(), r[0])
            assert torch.equal(ipi.cpu().long(), r[1]), f"image pages scope={scope}"
            assert torch.equal(qpi.cpu().long(), r[2]), f"query pages scope={scope}"
            assert bool(en.cpu().any(0).all())


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_block_cand_matches_oracle(bs):
    rng = random.Random(bs)
    B, L = 3, 9000
    rows = [_prompt(rng, L, per_page_mode=False), _prompt(rng, L, per_page_mode=True),
            _ocr_prompt(20, 273, 40, rng)[:L]]
    rows[2] += [TXT] * (L - len(rows[2]))
    ids = torch.tensor(rows)
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, L, 3, page_scope_prefill=True)
    nblk = (L + bs - 1) // bs
    g = torch.Generator().manual_seed(bs)
    pos = torch.randint(-5, L + 5, (B, 2000), generator=g)
    for mode, args in [("page", (itm, ipi, qpi)), ("flat", (itm, None, None)),
                       ("all", (None, None, None))]:
        got = pages.block_cand(pos.to(DEV), nblk, bs, *[None if a is None else a.to(DEV)
                                                         for a in args])
        ref = O.kl_candidate_mask(pos, nblk, args[0], B, 2000, bs, args[1], args[2])[:, 0]
        assert torch.equal(got.cpu(), ref), f"{mode} candidates"


def test_block_cand_wide_blocks():
    """Blocks holding image tokens of more than 64 pages (one image token per page):
    the kernel scans such blocks instead of using its 64-page bits."""
    L, bs = 1280, 256
    ids = torch.tensor([[IMG] * 880 + [PG, TXT] * 200])
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, L, per_page=1)
    pos = torch.arange(L)[None]
    nblk = L // bs
    got = pages.block_cand(pos.to(DEV), nblk, bs, itm.to(DEV), ipi.to(DEV), qpi.to(DEV))
    ref = O.kl_candidate_mask(pos, nblk, itm, 1, L, bs, ipi, qpi)[:, 0]
    assert torch.equal(got.cpu(), ref)
    assert not bool(ref[0, -1].all())          # some rows really are restricted


def test_overlay_functions_match_reference_calls():
    rng = random.Random(3)
    L = 3000
    ids = torch.tensor([_ocr_prompt(6, 273, 30, rng)[:L] + [TXT] * 0])
    L = ids.shape[1]
    idx = SimpleNamespace(image_bucket_constraint=True, image_token_id=IMG, page_token_id=PG,
                          per_page_image_tokens=273, page_scope_prefill=True, block_size=64)
    itm, ipi, qpi = pages._dash_page_ids(None, idx, ids.to(DEV), L)
    r = O.page_aware_ids(ids, IMG, PG, L, 273, True)
    assert torch.equal(ipi.cpu(), r[1]) and torch.equal(qpi.cpu(), r[2])
    pos = torch.arange(L)[None]
    nblk = (L + 63) // 64
    cand = pages._dash_block_cand(None, idx, None, pos.to(DEV), itm, ipi, qpi, nblk, 1, L)
    ref = O.kl_candidate_mask(pos, nblk, r[0], 1, L, 64, r[1], r[2])[:, 0]
    assert torch.equal(cand.cpu(), ref)
    idx.image_bucket_constraint = False
    itm2, ipi2, qpi2 = pages._dash_page_ids(None, idx, ids.to(DEV), L)
    assert ipi2 is None and qpi2 is None and torch.equal(itm2.cpu(), r[0])
    assert pages._dash_block_cand(None, idx, None, pos.to(DEV), None, None, None, nblk, 1, L) \
        is None


@pytest.mark.parametrize("bs", [32, 64])
def test_decode_allow_matches_oracle(bs):
    rng = random.Random(40 + bs)
    B, L = 4, 4000
    rows = [_ocr_prompt(8, 273, 30, rng)[:L], _prompt(rng, L, False), _prompt(rng, L, True),
            _ocr_prompt(3, 100, 10, rng)[:L]]
    rows = [r + [TXT] * (L - len(r)) for r in rows]
    ids = torch.tensor(rows)
    st = pages.DecodePageState(ids.to(DEV), IMG, PG, bs, per_page_image_tokens=50)
    ref = O.decode_page_state(ids, IMG, PG, bs, per_page=50)
    assert torch.equal(st.bmin.cpu().long(), ref["bmin"])
    assert torch.equal(st.bmax.cpu().long(), ref["bmax"])
    assert torch.equal(st.pp.cpu().long(), ref["pp"])
    assert torch.equal(st.markers.cpu().long(), ref["mcum"])
    for step in range(30):
        new = torch.tensor([[PG if rng.random() < 0.2 else TXT] for _ in range(B)])
        total = L + step + 1
        a = st.allow(new.to(DEV), total)
        r = O.decode_allow(ref, new, PG, total, bs)
        assert torch.equal(a.cpu(), r), f"step {step}"


def test_page_aware_prefill_routing_and_attention():
    """An OCR prompt of 10 pages x 273 image tokens (markers, instruction, response text)
    with page-aware candidates: routing bit-exact against the oracle on the same scores
    and candidates, attention within tolerance."""
    rng = random.Random(9)
    ids = _ocr_prompt(10, 273, 40, rng)
    S = len(ids)
    itm, ipi, qpi = O.page_aware_ids(torch.tensor([ids]), IMG, PG, S, 273, True)
    bs, lb, K = 64, 4, 8
    nblk = (S + bs - 1) // bs
    pos = torch.arange(S)[None]
    cand = pages.block_cand(pos.to(DEV), nblk, bs, itm.to(DEV), ipi.to(DEV), qpi.to(DEV))
    cand_r = O.kl_candidate_mask(pos, nblk, itm, 1, S, bs, ipi, qpi)[:, 0]
    assert torch.equal(cand.cpu(), cand_r)
    cfg = W.Prefill("pages", 1, S, bs, lb * bs, K, seed=31)
    d = W.make_prefill(cfg)
    hc = torch.zeros(128)
    out, (ti, bi, va) = pipeline.prefill(d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV),
                                         d["idx_q"].to(DEV), d["idx_k"].to(DEV), hc.to(DEV), bs,
                                         lb, W.IDX_SCALE * 20, W.FLOOR, W.SIGMA, K, 16,
                                         block_cand=cand, return_routing=True)
    kb, cv = O.kbar_headcls(d["idx_k"], hc, bs)
    z = ops.block_scores(d["idx_q"].to(DEV), ops.kbar(d["idx_k"].to(DEV), hc.to(DEV), bs), bs,
                         lb).cpu()
    t_r, b_r, v_r = O.infer_route_select(z, cand_r, W.IDX_SCALE * 20, W.FLOOR, W.SIGMA, K, 16)
    assert torch.equal(ti.cpu().long(), t_r) and torch.equal(va.cpu(), v_r)
    torch.testing.assert_close(bi.cpu(), b_r, atol=2e-5, rtol=1e-5)
    # the candidates change the routing of text queries (their own page's blocks only)
    t_free, _, _ = O.infer_route_select(z, None, W.IDX_SCALE * 20, W.FLOOR, W.SIGMA, K, 16)
    assert not torch.equal(t_free, t_r)
    ref = O.dense_attend(d["q"], d["k"], d["v"], t_r, b_r, v_r, bs, lb * bs, 1 / math.sqrt(128))
    err = (out.float().cpu() - ref).abs()
    assert bool((err <= 2e-2 + 1e-2 * ref.abs()).all()), err.max().item()


def test_page_aware_decode_step():
    """A decode step restricted by the allow row of its page, fused and two-launch,
    against the oracle routing with the same candidates."""
    rng = random.Random(12)
    ids = _ocr_prompt(12, 273, 20, rng)
    L = len(ids)
    B, bs, lb, K, H = 2, 64, 4, 8, 4
    rows = torch.tensor([ids, ids[:L]])
    st = pages.DecodePageState(rows.to(DEV), IMG, PG, bs)
    ref_st = O.decode_page_state(rows, IMG, PG, bs)
    new = torch.tensor([[TXT], [PG]])
    S = L + 1
    allow = st.allow(new.to(DEV), S)
    allow_r = O.decode_allow(ref_st, new, PG, S, bs)
    assert torch.equal(allow.cpu(), allow_r)
    g = torch.Generator().manual_seed(13)
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    ik = torch.randn(B, S, 128, generator=g)
    iq = torch.randn(B, 128, generator=g)
    hc = torch.zeros(128)
    nblk = (S + bs - 1) // bs
    for fused in (True, False):
        dst = pipeline.init_decode_state(ik.to(DEV), hc.to(DEV), bs, nblk)
        out, (ti, bi, va) = pipeline.decode_step(
            dst, q.to(DEV), k.to(DEV), v.to(DEV), iq.to(DEV), ik.to(DEV), hc.to(DEV), bs, lb,
            W.IDX_SCALE * 20, W.FLOOR, W.SIGMA, K, 16, 1 / math.sqrt(128), block_cand=allow,
            return_routing=True, fused=fused)
        ref, t_r, b_r, v_r = O.decode_pipeline(q.float()[:, :, None], k, v, iq[:, None], ik, hc,
                                               bs, lb, W.IDX_SCALE * 20, W.FLOOR, W.SIGMA, K, 16,
                                               1 / math.sqrt(128))
        # the oracle pipeline routes without candidates: route its scores with them
        kb, cv = O.kbar_headcls(ik, hc, bs)
        z = O.block_scores_headcls(iq[:, None], kb, cv, torch.full((B, 1), S - 1), bs, lb)
        t_c, b_c, v_c = O.infer_route_select(z, allow_r[:, None], W.IDX_SCALE * 20, W.FLOOR,
                                             W.SIGMA, K, 16)
        assert torch.equal(ti.cpu().long(), t_c) and torch.equal(va.cpu(), v_c), f"fused={fused}"
        ref = O.decode_attend(q.float()[:, :, None], k, v, t_c, b_c, v_c, torch.full((B, 1), S - 1),
                              bs, lb * bs, 1 / math.sqrt(128))[:, :, 0]
        err = (out.cpu() - ref).abs()
        assert bool((err <= 2e-2 + 1e-2 * ref.abs()).all()), err.max().item()
