"""GPU parity at the workloads' full sizes: the 27,300-token prefill (block 64,
window 1,024, cap 16, 5 % offset key blocks), the 16-document packed prefill
(78,078 tokens for seed 4, block-diagonal varlen), the 32-sequence paged decode
(lengths 2,730..27,300, pages of 64 tokens in a random physical order: every sequence
of one layer, and all 12 layers run back to back with three sequences of each
checked) and the 8 x 27,300 contiguous decode.

Every stage is checked against the CPU oracle on the same inputs: the block
summaries and scores within fp32 tolerance, the routing bit-exact on the GPU's own
scores, the attention on every query row (prefill) or sequence (decode) within the
output tolerance.
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops, pipeline
from ananta_ocr_amd import workloads as W
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2          # bf16 output, fp32 accumulation
SCALE = 1 / math.sqrt(128)


def _close(out, ref, what, tight=1.5e-2):
    out = out.float().cpu()
    ref = ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= ATOL + RTOL * ref.abs()), f"{what}: max err {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, \
        f"{what}: max err {err.max().item():.3e}"


def _scores_close(z, z_ref, what):
    sent = z_ref < -5e8
    assert torch.equal(z < -5e8, sent), f"{what}: sentinel pattern differs"
    torch.testing.assert_close(z[~sent], z_ref[~sent], atol=2e-5, rtol=2e-5)


def _route_equal(z, ti, bi, va, K, topm, what):
    """GPU routing of z against the oracle routing of the same fp32 scores."""
    t_r, b_r, v_r = O.infer_route_select(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, K, topm)
    kp = t_r.shape[-1]
    assert torch.equal(va[..., :kp], v_r), f"{what}: valid differs"
    mism = (ti[..., :kp] != t_r).nonzero()
    assert mism.numel() == 0, f"{what}: routed ids differ at {mism[:5].tolist()}"
    torch.testing.assert_close(bi[..., :kp], b_r, atol=2e-5, rtol=1e-5)
    # slots past K' = min(K, M') are empty
    assert bool((ti[..., kp:] == -1).all()) and not bool(va[..., kp:].any())
    return t_r, b_r, v_r


def test_prefill_27300_tokens_full_size():
    cfg = W.PREFILL_27300
    d = W.make_prefill(cfg)
    S, lb = d["S"], cfg.lw // cfg.bs
    hc = torch.zeros(128)
    print(f"prefill {cfg.name}: S={S}", flush=True)
    kb = ops.kbar(d["idx_k"].to(DEV), hc.to(DEV), cfg.bs)
    z = ops.block_scores(d["idx_q"].to(DEV), kb, cfg.bs, lb)
    ti, bi, va = ops.route(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap)
    out = ops.attn_prefill(d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV), ti, bi, va,
                           cfg.bs, cfg.lw, SCALE)
    kb_r, cv = O.kbar_headcls(d["idx_k"], hc, cfg.bs)
    torch.testing.assert_close(kb.cpu(), kb_r, atol=1e-6, rtol=1e-5)
    pos = torch.arange(S)[None]
    z_r = O.block_scores_headcls(d["idx_q"], kb_r, cv, pos, cfg.bs, lb)
    z = z.cpu()
    _scores_close(z, z_r, "scores")
    t_r, b_r, v_r = _route_equal(z, ti.cpu().long(), bi.cpu(), va.cpu(), cfg.cap, cfg.cap,
                                 "route")
    # the offset blocks must actually be routed (the workload's point)
    assert int(v_r.sum()) > 0
    ref = O.dense_attend(d["q"], d["k"], d["v"], t_r, b_r, v_r, cfg.bs, cfg.lw, SCALE,
                         q_chunk=1024)
    _close(out, ref, "prefill 27300")


def test_packed_16_documents_full_size():
    cfg = W.PACKED_16DOC
    d = W.make_prefill(cfg)
    cu = d["cu_list"]
    T, lb = d["S"], cfg.lw // cfg.bs
    hc = torch.zeros(128)
    print(f"packed {cfg.name}: T={T}, docs={len(cu) - 1}", flush=True)
    out, (ti, bi, va) = pipeline.prefill(
        d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV), d["idx_q"].to(DEV),
        d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, lb, W.IDX_SCALE, W.FLOOR, W.SIGMA,
        cfg.cap, cfg.cap, SCALE, cu_seqlens=d["cu_seqlens"].to(DEV), return_routing=True)
    # the GPU's own scores, to route them on the CPU as well
    kb = ops.kbar(d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, cu_seqlens=d["cu_seqlens"].to(DEV))
    z = ops.block_scores(d["idx_q"].to(DEV), kb, cfg.bs, lb,
                         cu_seqlens=d["cu_seqlens"].to(DEV)).cpu()
    kb = kb.cpu()
    out = out.cpu()
    ti, bi, va = ti.cpu().long(), bi.cpu(), va.cpu()
    for b in range(len(cu) - 1):
        s0, s1 = cu[b], cu[b + 1]
        L = s1 - s0
        nblk = (L + cfg.bs - 1) // cfg.bs
        kb_r, cv = O.kbar_headcls(d["idx_k"][:, s0:s1], hc, cfg.bs)
        torch.testing.assert_close(kb[b:b + 1, :nblk], kb_r, atol=1e-6, rtol=1e-5)
        zd = z[s0:s1, :nblk][None]
        z_r = O.block_scores_headcls(d["idx_q"][:, s0:s1], kb_r, cv, torch.arange(L)[None],
                                     cfg.bs, lb)
        _scores_close(zd, z_r, f"scores doc {b}")
        t_r, b_r, v_r = _route_equal(zd, ti[None, s0:s1], bi[None, s0:s1], va[None, s0:s1],
                                     cfg.cap, cfg.cap, f"route doc {b}")
        ref = O.dense_attend(d["q"][:, :, s0:s1], d["k"][:, :, s0:s1], d["v"][:, :, s0:s1],
                             t_r, b_r, v_r, cfg.bs, cfg.lw, SCALE, q_chunk=1024)
        _close(out[:, :, s0:s1], ref, f"document {b} ({L} tokens)")


def _gather_pages(x, table_row, L):
    """[pages, bs, ...] paged tensor -> [L, ...] contiguous rows of one sequence."""
    npg = (L + x.shape[1] - 1) // x.shape[1]
    return x[table_row[:npg].long()].reshape(-1, *x.shape[2:])[:L]


def _check_paged_sequences(cfg, d, lens, table, out, ti, bi, va, seqs, what):
    """Oracle check of the given sequences of one paged decode step: routing on the
    oracle's own scores (only blocks tied with the last selected one to fp32 rounding
    may differ), attention on the GPU's routing.  Pages are gathered on the GPU, so that
    only the checked sequences travel to the host.  Returns the near-tie count."""
    lb = cfg.lw // cfg.bs
    hc = torch.zeros(128)
    out = out.float().cpu()
    ti, bi, va = ti.cpu().long(), bi.cpu(), va.cpu()
    ties = 0
    for b in seqs:
        L = int(lens[b])
        row = table[b].to(d["k"].device)
        ik = _gather_pages(d["idx_k"], row, L)[None].cpu()                   # [1, L, d]
        k = _gather_pages(d["k"], row, L).permute(1, 0, 2)[None].cpu()      # [1, H, L, D]
        v = _gather_pages(d["v"], row, L).permute(1, 0, 2)[None].cpu()
        q, iq = d["q"][b:b + 1].cpu(), d["idx_q"][b:b + 1].cpu()
        kb_r, cv = O.kbar_headcls(ik, hc, cfg.bs)
        z_r = O.block_scores_headcls(iq, kb_r, cv, torch.tensor([[L - 1]]), cfg.bs, lb)
        t_r, b_r, v_r = O.infer_route_select(z_r, None, W.IDX_SCALE, W.FLOOR, W.SIGMA,
                                             cfg.cap, cfg.cap)
        kp_ = t_r.shape[-1]
        g_ids = set(ti[b, 0, :kp_][va[b, 0, :kp_]].tolist())
        r_ids = set(t_r[0, 0][v_r[0, 0]].tolist())
        if g_ids != r_ids:
            # scores are computed in a different order on the two sides: only blocks
            # tied with the last selected one (to fp32 rounding) may swap
            zz = z_r[0, 0]
            edge = zz[t_r[0, 0, kp_ - 1]].item()
            for c in g_ids ^ r_ids:
                assert abs(zz[c].item() - edge) <= 1e-5 * abs(edge) + 1e-6, \
                    f"{what}, sequence {b}: block {c} routed on one side only"
            ties += 1
        else:
            assert torch.equal(ti[b, 0, :kp_], t_r[0, 0]), f"{what}, sequence {b}: slot order"
            torch.testing.assert_close(bi[b, 0, :kp_], b_r[0, 0], atol=1e-4, rtol=1e-4)
        # attention on the GPU's routing
        ref = O.decode_attend(q[:, :, None], k, v, ti[b:b + 1, :, :kp_],
                              bi[b:b + 1, :, :kp_], va[b:b + 1, :, :kp_],
                              torch.tensor([[L - 1]]), cfg.bs, cfg.lw, SCALE)
        _close(out[b:b + 1], ref[:, :, 0], f"{what}, sequence {b} ({L} tokens)")
    return ties


def _paged_step(cfg, d, st):
    hc = torch.zeros(128, device=DEV)
    return pipeline.decode_step(
        st, d["q"], d["k"], d["v"], d["idx_q"], d["idx_k"], hc, cfg.bs, cfg.lw // cfg.bs,
        W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap, cfg.cap, SCALE, seq_lens=d["seq_lens"],
        block_table=d["block_table"], page_size=cfg.bs, return_routing=True)


def _paged_state(cfg, d, table):
    return pipeline.init_decode_state(d["idx_k"], torch.zeros(128, device=DEV), cfg.bs,
                                      table.shape[1], seq_lens=d["seq_lens"],
                                      block_table=d["block_table"], page_size=cfg.bs)


def test_paged_decode_32_sequences_full_size():
    cfg = W.PAGED_12L
    lens, table = W.paged_layout(cfg)
    d = W.make_paged_decode(cfg, DEV, 0, lens, table)
    print(f"paged decode {cfg.name}: B={cfg.B}, tokens={int(lens.sum())}", flush=True)
    st = _paged_state(cfg, d, table)
    out, (ti, bi, va) = _paged_step(cfg, d, st)
    ties = _check_paged_sequences(cfg, d, lens, table, out, ti, bi, va, range(cfg.B), "layer 0")
    assert ties <= 2, f"{ties} sequences with near-tied routing"


def test_paged_decode_12_layers_stacked():
    """The 12-layer paged decode as the benchmark runs it: every layer's cache and state
    made first, then the 12 fused steps back to back on one stream, then each layer
    checked against the oracle on three of its 32 sequences (layer l: sequences l,
    l + 12 and l + 24 mod 32, so that every sequence is checked in some layer)."""
    cfg = W.PAGED_12L
    lens, table = W.paged_layout(cfg)
    layers = []
    for layer in range(cfg.layers):
        d = W.make_paged_decode(cfg, DEV, layer, lens, table)
        layers.append((d, _paged_state(cfg, d, table)))
    print(f"paged decode {cfg.name}: {cfg.layers} layers made", flush=True)
    results = [_paged_step(cfg, d, st) for d, st in layers]
    torch.cuda.synchronize()
    ties = 0
    for layer, ((d, _), (out, (ti, bi, va))) in enumerate(zip(layers, results)):
        seqs = sorted({(layer + 12 * j) % cfg.B for j in range(3)})
        ties += _check_paged_sequences(cfg, d, lens, table, out, ti, bi, va, seqs,
                                       f"layer {layer}")
        print(f"layer {layer}: sequences {seqs} match", flush=True)
    assert ties <= 3, f"{ties} sequences with near-tied routing"


def test_decode_b8_27300_full_size():
    """The B = 8 decode step at its full size (8 x 27,300 contiguous cached tokens,
    block 64, window 1,024, cap 16) through pipeline.decode_step, the fused step the
    benchmark times: block summaries and scores within fp32 tolerance, routing bit for
    bit on the GPU's own scores, attention within the output tolerance."""
    cfg = W.DECODE_B8
    d = W.make_decode(cfg)
    lb = cfg.lw // cfg.bs
    hc = torch.zeros(128)
    nblk = (cfg.S + cfg.bs - 1) // cfg.bs
    print(f"decode {cfg.name}: B={cfg.B}, S={cfg.S}", flush=True)
    st = pipeline.init_decode_state(d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, nblk)
    out, (ti, bi, va), z = pipeline.decode_step(
        st, d["q"].to(DEV), d["k"].to(DEV), d["v"].to(DEV), d["idx_q"].to(DEV),
        d["idx_k"].to(DEV), hc.to(DEV), cfg.bs, lb, W.IDX_SCALE, W.FLOOR, W.SIGMA, cfg.cap,
        cfg.cap, SCALE, return_routing=True, return_scores=True)
    kb_r, cv = O.kbar_headcls(d["idx_k"], hc, cfg.bs)
    torch.testing.assert_close(st.kbar.cpu(), kb_r, atol=1e-6, rtol=1e-5)
    qpos = torch.full((cfg.B, 1), cfg.S - 1)
    z_r = O.block_scores_headcls(d["idx_q"], kb_r, cv, qpos, cfg.bs, lb)
    zg = z.cpu()[:, None, :nblk]
    _scores_close(zg, z_r, "decode scores")
    t_r, b_r, v_r = _route_equal(zg, ti.cpu().long(), bi.cpu(), va.cpu(), cfg.cap, cfg.cap,
                                 "decode routing")
    assert v_r.any()
    ref = O.decode_attend(d["q"][:, :, None], d["k"], d["v"], t_r, b_r, v_r, qpos, cfg.bs,
                          cfg.lw, SCALE)
    _close(out, ref[:, :, 0], "decode B=8 x 27,300")
