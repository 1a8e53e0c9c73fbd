"""Serving-side decode state on the GPU: the k_bar page pool (one summary per physical
KV page, read through the block table), the window bounds of decode rows from their
allow rows, and decode scans restricted to those bounds.

The pool path is compared with the per-sequence k_bar cache (identical routing,
scores and outputs, bit for bit), including a reordered batch that reuses the pool
unchanged; the bounds with the oracle's restatement of the serving router's rule;
the bounded scan with the unbounded one (identical routing and outputs; scores equal
inside the span)."""

import math
import random

import pytest
import torch

from ananta_ocr_amd import pages, pipeline
from ananta_ocr_amd import workloads as W
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _paged(seed, lens, bs, H=2, d=128, spare=7):
    """A paged cache: K/V [pages, bs, H, 128] bf16, index keys [pages, bs, d] fp32, the
    block table with physical pages in random order (and spare unused pages)."""
    g = torch.Generator().manual_seed(seed)
    B = len(lens)
    npg = [(L + bs - 1) // bs for L in lens]
    total = sum(npg) + spare
    perm = torch.randperm(total, generator=g)
    table = torch.zeros(B, max(npg), dtype=torch.int32)
    o = 0
    for b in range(B):
        table[b, :npg[b]] = perm[o:o + npg[b]].int()
        o += npg[b]
    k = (torch.randn(total, bs, H, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(total, bs, H, 128, generator=g).bfloat16()
    ik = torch.randn(total, bs, d, generator=g)
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    iq = torch.randn(B, d, generator=g)
    hc = torch.randn(d, generator=g) * 0.3
    return dict(k=k.to(DEV), v=v.to(DEV), ik=ik.to(DEV), q=q.to(DEV), iq=iq.to(DEV),
                hc=hc.to(DEV), table=table.to(DEV), lens=torch.tensor(lens, dtype=torch.int32).to(DEV),
                total=total)


def _step(state, d, bs, lb, K, topm, fused, cand=None, bounds=None, order=None):
    sel = slice(None) if order is None else order
    kw = dict(seq_lens=d["lens"][sel], block_table=d["table"][sel], page_size=bs,
              block_cand=None if cand is None else cand[sel], bounds=bounds,
              return_routing=True, return_scores=True, fused=fused)
    return pipeline.decode_step(state, d["q"][sel], d["k"], d["v"], d["iq"][sel], d["ik"],
                                d["hc"], bs, lb, W.IDX_SCALE * 4, W.FLOOR, W.SIGMA, K, topm,
                                1 / math.sqrt(128), **kw)


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("bs", [32, 64])
def test_kbar_page_pool_equals_per_sequence_cache(fused, bs):
    lens = [3000, 1, 777, 64 * 20, 2049]
    d = _paged(40 + bs, lens, bs)
    lb, K, topm = 4, 12, 16
    nblk = d["table"].shape[1]
    seq_state = pipeline.init_decode_state(d["ik"], d["hc"], bs, nblk, seq_lens=d["lens"],
                                           block_table=d["table"], page_size=bs)
    pool = pipeline.KBarPageCache(d["total"], 128, DEV)
    pool.put_sequences(d["ik"], d["hc"], bs, d["table"], d["lens"])
    o1, (i1, b1, v1), z1 = _step(seq_state, d, bs, lb, K, topm, fused)
    o2, (i2, b2, v2), z2 = _step(pool, d, bs, lb, K, topm, fused)
    torch.cuda.synchronize()
    assert torch.equal(i1, i2) and torch.equal(v1, v2) and torch.equal(b1, b2)
    assert torch.equal(o1, o2)
    # scores (written for each sequence's blocks) and every used page's row equal the
    # sequence's block summary (tail included)
    tab = d["table"].long().cpu()
    for b, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        assert torch.equal(z1[b, :nb], z2[b, :nb])
        assert torch.equal(pool.kbar[tab[b, :nb].to(DEV)], seq_state.kbar[b, :nb])


def test_kbar_page_pool_survives_batch_reordering():
    """The batch reordered (as continuous batching does): the same pool serves it
    without moving any summary, and every sequence gets the output it got before."""
    bs, lb, K, topm = 64, 4, 12, 16
    lens = [1500, 4000, 300, 2222]
    d = _paged(51, lens, bs)
    pool = pipeline.KBarPageCache(d["total"], 128, DEV)
    pool.put_sequences(d["ik"], d["hc"], bs, d["table"], d["lens"])
    o1, (i1, _, _), _ = _step(pool, d, bs, lb, K, topm, True)
    order = torch.tensor([2, 0, 3, 1], device=DEV)
    o2, (i2, _, _), _ = _step(pool, d, bs, lb, K, topm, True, order=order)
    torch.cuda.synchronize()
    assert torch.equal(o1[order], o2) and torch.equal(i1[order], i2)


def test_kbar_page_pool_refresh_tail_matches_oracle():
    bs = 64
    lens = [1000, 130, 64 * 7]
    d = _paged(52, lens, bs)
    pool = pipeline.KBarPageCache(d["total"], 128, DEV)
    pool.refresh_tail(d["ik"], d["hc"], bs, d["table"], d["lens"], tail_pages=2)
    tab = d["table"].long().cpu()
    ik = d["ik"].cpu()
    for b, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        keys = ik[tab[b, :nb]].reshape(-1, 128)[:L][None]
        kb_r, _ = O.kbar_headcls(keys, d["hc"].cpu(), bs)
        for c in range(max(0, nb - 2), nb):
            torch.testing.assert_close(pool.kbar[tab[b, c]].cpu(), kb_r[0, c], atol=1e-5, rtol=1e-5)
        untouched = tab[b, :max(0, nb - 2)]
        assert bool((pool.kbar[untouched.to(DEV)] == 0).all())


@pytest.mark.parametrize("seed", [0, 1])
def test_win_bounds_match_oracle(seed):
    g = torch.Generator().manual_seed(seed)
    B, W_, bs, lb = 300, 430, 64, 16
    allow = torch.rand(B, W_ + 1, generator=g) < torch.rand(B, 1, generator=g) * 0.05
    allow[::9] = False                                # rows with nothing allowed
    seq = torch.randint(0, W_ * bs + 1, (B,), generator=g)
    bounds, fit = pages.win_bounds_decode(allow.to(DEV), seq.to(DEV), W_, bs, lb, tile=128)
    lo, hi, fit_r = O.decode_win_bounds(allow, seq, W_, bs, lb, 128)
    assert torch.equal(bounds[:, 0].cpu().long(), lo) and torch.equal(bounds[:, 1].cpu().long(), hi)
    assert torch.equal(fit.cpu(), fit_r)


@pytest.mark.parametrize("paged_pool", [False, True])
def test_bounded_decode_scan_equals_full_scan(paged_pool):
    """Candidates confined to a few blocks per sequence (a page's image blocks): the
    scan restricted to their bounds routes and attends exactly as the full scan."""
    bs, lb, K, topm = 64, 4, 12, 16
    lens = [27300, 9000, 513, 20000]
    d = _paged(60, lens, bs)
    B = len(lens)
    nblk = d["table"].shape[1]
    rng = random.Random(61)
    cand = torch.zeros(B, nblk, dtype=torch.bool)
    for b, L in enumerate(lens):
        nb = (L + bs - 1) // bs
        if b == 2:
            continue                                  # no candidate: falls back to all remote
        c0 = rng.randrange(0, max(1, nb - 30))
        cand[b, c0:c0 + rng.randint(1, 6)] = True
    cand = cand.to(DEV)
    bounds, fit = pages.win_bounds_decode(cand, d["lens"], nblk, bs, lb, tile=128)
    if paged_pool:
        state = pipeline.KBarPageCache(d["total"], 128, DEV)
        state.put_sequences(d["ik"], d["hc"], bs, d["table"], d["lens"])
        state2 = pipeline.KBarPageCache(d["total"], 128, DEV)
        state2.kbar.copy_(state.kbar)
    else:
        mk = lambda: pipeline.init_decode_state(d["ik"], d["hc"], bs, nblk, seq_lens=d["lens"],
                                                block_table=d["table"], page_size=bs)
        state, state2 = mk(), mk()
    for fused in (True, False):
        o1, (i1, b1, v1), z1 = _step(state, d, bs, lb, K, topm, fused, cand=cand)
        o2, (i2, b2, v2), z2 = _step(state2, d, bs, lb, K, topm, fused, cand=cand, bounds=bounds)
        torch.cuda.synchronize()
        assert torch.equal(i1, i2) and torch.equal(v1, v2) and torch.equal(b1, b2), fused
        assert torch.equal(o1, o2), fused
        bc = bounds.cpu()
        for b in range(B):
            lo, hi = int(bc[b, 0]), int(bc[b, 1])
            assert torch.equal(z1[b, lo:hi], z2[b, lo:hi])
            assert bool((z2[b, :lo] < -5e8).all()) and bool((z2[b, hi:(lens[b] + bs - 1) // bs] < -5e8).all())
