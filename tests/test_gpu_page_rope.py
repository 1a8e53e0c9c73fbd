"""Page2D RoPE state on the GPU (dash_page_rope_pos, dash_rope2d_cos_sin,
dash_page_rope_advance through the C ABI) against the oracle: prompt coordinates (exact),
two-axis cos/sin (fp32 within 1e-6, bf16 within one bf16 step), the per-token decode
advance (exact); then a multi-page OCR prompt through the reference's call order with
page2d RoPE on the main branch and the router: the prefill (coordinates, router cos/sin,
page-aware candidates, _infer_prefill_attend) and decode steps with <PAGE> markers in the
response (_dash_decode_forward, the coordinates advanced on the device), each against the
oracle."""

import math
import random
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from ananta_ocr_amd import modeling_deepseekv2 as MD
from ananta_ocr_amd import page_rope as PR
from ananta_ocr_amd import pages
from ananta_ocr_amd.dash_attention import DashAttention, apply_rotary
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
IMG, PG, TXT, BOS = 5, 9, 7, 1


def _ocr(rng, pages_n, per_page, resp, instr=5):
    ids = [BOS] + [TXT] * rng.randint(0, 3)
    for _ in range(pages_n):
        ids += [PG] + [IMG] * (per_page if per_page else rng.randint(2, 40))
    ids += [TXT] * instr
    for _ in range(resp):
        ids += [PG] + [TXT] * rng.randint(0, 30)
    return ids


def _batch(rows, L=None):
    L = L or max(len(r) for r in rows)
    ids = torch.full((len(rows), L), TXT, dtype=torch.long)
    for b, r in enumerate(rows):
        ids[b, :min(L, len(r))] = torch.tensor(r[:L])
    return ids


@pytest.mark.parametrize("seed,pages_n,per_page,span", [
    (0, 3, 0, 0), (1, 12, 0, 7), (2, 40, 273, 0), (3, 100, 273, 512),
])
def test_page_rope_pos_matches_oracle(seed, pages_n, per_page, span):
    rng = random.Random(seed)
    rows = [_ocr(rng, rng.randint(1, pages_n), per_page, rng.randint(0, pages_n))
            for _ in range(3)]
    ids = _batch(rows)
    L = ids.shape[1] + 3                      # padded with -1 up to the key length
    pos = PR.build_page_rope_pos(ids.to(DEV), L, IMG, PG, span)
    tok, page, pf, n_pg = O.page_rope_pos(ids, IMG, PG, L, span)
    assert torch.equal(pos.tok.cpu(), tok) and torch.equal(pos.page.cpu(), page)
    assert pos.meta.cpu().tolist() == [n_pg, 1]
    assert torch.equal(pos.pf_cnt.cpu()[:, :n_pg], pf)
    assert not pos.pf_cnt.cpu()[:, n_pg:].any()
    idx = SimpleNamespace(image_token_id=IMG, page_token_id=PG, rope_page_span=span)
    t2, p2 = PR._build_page_rope_pos(idx, ids.to(DEV), L)
    assert torch.equal(t2.cpu(), tok) and int(idx._page_rope_meta["n_pg"]) == n_pg


def test_page_rope_pos_fallback_flag():
    """Where the reference falls back to 1-D (a row whose last image token has no marker
    before it, no image, no marker) the flag is 0 and the reference wrapper returns None."""
    cases = [[[PG, IMG, TXT], [IMG, PG, TXT]], [[TXT, PG, TXT]], [[TXT, IMG, IMG]],
             [[IMG, IMG, PG, TXT]]]
    idx = SimpleNamespace(image_token_id=IMG, page_token_id=PG, rope_page_span=0)
    for rows in cases:
        ids = torch.tensor(rows)
        assert O.page_rope_pos(ids, IMG, PG, ids.shape[1]) is None
        pos = PR.build_page_rope_pos(ids.to(DEV), ids.shape[1], IMG, PG)
        assert int(pos.meta[1]) == 0
        assert PR._build_page_rope_pos(idx, ids.to(DEV), ids.shape[1]) is None


@pytest.mark.parametrize("pairs,mod,mode,theta", [
    (1, 2, "resample", 10000.0),               # the checkpoint's router (config.json)
    (8, 0, "truncate", 500000.0),
    (3, 5, "resample", 10000.0),
])
def test_rope2d_cos_sin_matches_oracle(pairs, mod, mode, theta):
    rng = random.Random(7)
    ids = _batch([_ocr(rng, 60, 273, 30), _ocr(rng, 20, 273, 80)])
    L = ids.shape[1]
    tok, page, _, _ = O.page_rope_pos(ids, IMG, PG, L)
    mod_ = PR.PageRope2D(128, theta, 256.0, pairs, mode, mod).to(DEV)
    it, ip = O.rotary2d_inv_freq(128, theta, 256.0, pairs, mode)
    assert torch.equal(mod_.inv_tok.cpu(), it) and torch.equal(mod_.inv_page.cpu(), ip)
    x32 = torch.zeros(1, device=DEV)
    c, s = mod_(x32, tok.to(DEV), page.to(DEV))
    rc, rs = O.rotary2d_cos_sin(tok, page, it, ip, mod)
    torch.testing.assert_close(c.cpu(), rc, atol=1e-6, rtol=0)
    torch.testing.assert_close(s.cpu(), rs, atol=1e-6, rtol=0)
    cb, sb = mod_(x32.bfloat16(), tok.to(DEV), page.to(DEV))
    rcb, rsb = O.rotary2d_cos_sin(tok, page, it, ip, mod, dtype=torch.bfloat16)
    for got, want in ((cb.cpu(), rcb), (sb.cpu(), rsb)):
        diff = (got.float() - want.float()).abs()
        step = want.float().abs().clamp_min(2 ** -126) * 2 ** -7
        assert torch.all(diff <= step)
        assert (diff > 0).float().mean().item() < 1e-3


def test_page_rope_advance_matches_oracle():
    rng = random.Random(11)
    rows = [_ocr(rng, n, 0, 0) for n in (2, 5, 9, 1)]
    ids = _batch(rows)
    L = ids.shape[1]
    pos = PR.build_page_rope_pos(ids.to(DEV), L, IMG, PG)
    tok, page, pf, n_pg = O.page_rope_pos(ids, IMG, PG, L)
    st = PR.PageRopeState(page=pos.page[:, -1].clone(), tok=pos.tok[:, -1].clone(),
                          pf_cnt=pos.pf_cnt, n_pg=pos.n_pg)
    t, p = tok[:, -1], page[:, -1]
    for step in range(60):
        new = torch.tensor([PG if rng.random() < 0.3 else TXT for _ in rows])
        gt, gp = PR.page_rope_advance(st, new.to(DEV), PG)
        t, p = O.page_rope_advance(p, t, pf, n_pg, new, PG)
        assert gt[:, 0].cpu().tolist() == t.tolist() and gp[:, 0].cpu().tolist() == p.tolist()
    assert (p == n_pg - 1).any()             # the clamp at the last page was reached
    # the reference's dict form of the state advances the same way
    dst = {"page": pos.page[:, -1].clone(), "tok": pos.tok[:, -1].clone(),
           "pf_cnt": pos.pf_cnt, "n_pg": int(n_pg)}
    gt, gp = PR.page_rope_advance(dst, torch.full((4,), PG, device=DEV), PG)
    t1, p1 = O.page_rope_advance(page[:, -1], tok[:, -1], pf, n_pg, torch.full((4,), PG), PG)
    assert gt[:, 0].cpu().tolist() == t1.tolist() and dst["page"].cpu().tolist() == p1.tolist()


class _Cache:
    def __init__(self):
        self.k, self.v = {}, {}

    def update(self, k, v, li):
        if li in self.k:
            self.k[li] = torch.cat([self.k[li], k], 2)
            self.v[li] = torch.cat([self.v[li], v], 2)
        else:
            self.k[li], self.v[li] = k, v
        return self.k[li], self.v[li]

    def get_seq_length(self, li=0):
        return self.k[li].shape[2] if li in self.k else 0


def _close(out, ref, what, tight=1.5e-2):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"{what}: {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, f"{what}: {err.max().item()}"


def test_ocr_prompt_through_prefill_and_decode_with_page2d_rope(monkeypatch):
    """The checkpoint's router (block 32, window 128, K 12, topm 16, stage 0 head_cls;
    page2d RoPE with one page pair folded mod 2, page theta 256, token theta 1e4) on a
    two-row OCR prompt of 273-token pages: the prefill as _dash_attn_forward runs it
    (coordinates from the prompt ids, main-branch RoPE from them, the router's cos/sin,
    page-aware candidates, _infer_prefill_attend), then decode steps (_dash_decode_forward)
    whose tokens include <PAGE> markers."""
    monkeypatch.setenv("DASH_STAGE0", "head_cls")
    torch.manual_seed(0)
    rng = random.Random(3)
    heads, bs, lb, budget = 2, 32, 4, 12
    hidden = heads * 128
    rows = [_ocr(rng, 5, 273, 1, instr=9), _ocr(rng, 3, 273, 2, instr=30)]
    ids = _batch(rows)
    B, S = ids.shape
    sp = dict(sparse_block_size=bs, sparse_local_block=lb, dash_scaling_factor=128.0,
              dash_prior_floor=1e-4, dash_sigma=1.0, dash_topk_blocks=budget,
              sparse_index_dim=128, dash_image_only=True, dash_stage0="head_cls")
    cfg = SimpleNamespace(num_attention_heads=heads, num_key_value_heads=heads,
                          hidden_size=hidden, rms_norm_eps=1e-6, sparse_attention_config=sp)
    router = DashAttention(cfg)
    with torch.no_grad():
        router.head_cls.normal_(0, 0.5)
    router = router.to(DEV).bfloat16()
    idx = SimpleNamespace(image_token_id=IMG, page_token_id=PG, rope_page_span=0, head_dim=128,
                          rope_mode="page2d", image_bucket_constraint=True, block_size=bs,
                          rotary_emb_2d=PR.PageRope2D(128, 10000.0, 256.0, 1, "resample",
                                                      2).to(DEV),
                          rotary_emb_1d=None)
    layer = SimpleNamespace(
        config=cfg, head_dim=128, layer_idx=2, dash_router=router, indexer=idx,
        main_rope_mode="page2d", _main_rope_pos_2d=None, _sparse_source_input_ids=ids.to(DEV),
        rotary_emb_2d_main=PR.PageRope2D(128, 10000.0, 256.0, 1, "resample", 2).to(DEV),
        q_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        k_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        v_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        o_proj=nn.Identity(), rotary_emb=None)
    decoder = nn.Module()
    decoder.router = router
    decoder.config = cfg
    MD.configure_dash_inference(decoder, True)
    p = router._infer_params
    scale = 1 / math.sqrt(128)
    steps = [TXT, TXT, PG, TXT, PG, TXT, TXT, PG, PG, TXT]
    g = torch.Generator(device=DEV).manual_seed(4)
    hs = torch.randn(B, S + len(steps), hidden, device=DEV, generator=g).bfloat16()
    cache = _Cache()
    with torch.no_grad():
        # ---- prefill, as _dash_attn_forward does it ----
        coords = PR._build_page_rope_pos(idx, layer._sparse_source_input_ids, S)
        assert coords is not None
        tok_r, page_r, pf_r, n_pg = O.page_rope_pos(ids, IMG, PG, S)
        assert torch.equal(coords[0].cpu(), tok_r) and torch.equal(coords[1].cpu(), page_r)
        layer._main_rope_pos_2d = coords
        assert PR.main_rope_coords(layer, S, cache) is coords
        x = hs[:, :S]
        q = layer.q_proj(x).view(B, S, heads, 128).transpose(1, 2)
        k = layer.k_proj(x).view(B, S, heads, 128).transpose(1, 2)
        v = layer.v_proj(x).view(B, S, heads, 128).transpose(1, 2)
        cos, sin = layer.rotary_emb_2d_main(v, coords[0], coords[1])
        q, k = apply_rotary(q, k, cos, sin)
        k_all, v_all = cache.update(k, v, layer.layer_idx)
        pos_ids = torch.arange(S, device=DEV)[None].expand(B, -1)
        pe = MD._dash_indexer_rope(layer, idx, router, v, pos_ids, coords, (cos, sin))
        it, ip = O.rotary2d_inv_freq(128, 10000.0, 256.0, 1)
        rc, _ = O.rotary2d_cos_sin(tok_r, page_r, it, ip, 2, dtype=torch.bfloat16)
        assert (pe[0].cpu().float() - rc.float()).abs().max().item() <= 2 ** -8
        itm, ipi, qpi = pages._dash_page_ids(layer, idx, layer._sparse_source_input_ids, S)
        nblk = (S + bs - 1) // bs
        cand = pages._dash_block_cand(layer, idx, router, pos_ids, itm, ipi, qpi, nblk, B, S)
        out = MD._infer_prefill_attend(layer, router, x, q, k_all, v_all, pe, pos_ids, cand,
                                       None, cache)
        # the oracle from the router's index keys on: candidates, summaries, scores,
        # routing, attention
        iq, ik = router.router_qk(x, pe)
        # configure_dash_inference turns page_scope_prefill on (its default)
        it_o, ip_o, qp_o = O.page_aware_ids(ids, IMG, PG, S, page_scope_prefill=True)
        cand_o = O.kl_candidate_mask(torch.arange(S)[None].expand(B, -1), nblk, it_o, B, S, bs,
                                     ip_o, qp_o)[:, 0]
        assert torch.equal(cand.cpu(), cand_o)
        kb, cv = O.kbar_headcls(ik.cpu(), router.head_cls.float().cpu(), bs)
        z = O.block_scores_headcls(iq.cpu(), kb, cv, torch.arange(S)[None].expand(B, -1), bs, lb)
        ti, bi, va = O.infer_route_select(z, cand_o, p["idx_scale"], p["floor"], p["sigma"],
                                          p["K"], p["topm"])
        ref = O.dense_attend(q.cpu(), k_all.cpu(), v_all.cpu(), ti, bi, va, bs, bs * lb, scale)
        _close(out, ref, "prefill")
        # ---- decode steps: the coordinates advance on the device ----
        st = cache._page_rope_state[layer.layer_idx]
        t_o, p_o = tok_r[:, -1], page_r[:, -1]
        idx_keys = [ik]
        for i, x_id in enumerate(steps):
            t = S + i
            new = torch.full((B, 1), x_id, dtype=torch.long)
            layer._sparse_source_input_ids = torch.cat(
                [layer._sparse_source_input_ids, new.to(DEV)], 1)
            pos_t = torch.full((B, 1), t, device=DEV)
            out_t, _, _, _ = MD._dash_decode_forward(layer, hs[:, t:t + 1], pos_t, cache)
            t_o, p_o = O.page_rope_advance(p_o, t_o, pf_r, n_pg, new[:, 0], PG)
            assert st.tok.cpu().tolist() == t_o.tolist() and st.page.cpu().tolist() == p_o.tolist()
            ct, stn = layer.rotary_emb_2d_main(hs, t_o[:, None].to(DEV), p_o[:, None].to(DEV))
            xt = hs[:, t:t + 1]
            qd = layer.q_proj(xt).view(B, 1, heads, 128).transpose(1, 2)
            qd, _ = apply_rotary(qd, qd, ct, stn)
            pe_t = idx.rotary_emb_2d(hs, t_o[:, None].to(DEV), p_o[:, None].to(DEV))
            iq_t, ik_t = router.router_qk(xt, pe_t)
            idx_keys.append(ik_t)
            ik_all = torch.cat(idx_keys, 1)
            assert torch.equal(cache._dash_idx_k[layer.layer_idx], ik_all)
            k_all, v_all = cache.k[layer.layer_idx], cache.v[layer.layer_idx]
            ref_t = O.decode_pipeline(qd.cpu(), k_all.cpu(), v_all.cpu(), iq_t.cpu(), ik_all.cpu(),
                                      router.head_cls.float().cpu(), bs, lb, p["idx_scale"],
                                      p["floor"], p["sigma"], p["K"], p["topm"], scale)[0]
            _close(out_t.view(B, 1, heads, 128).transpose(1, 2), ref_t, f"decode step {i}")
    MD.configure_dash_inference(decoder, False)
