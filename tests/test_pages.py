"""The oracle's page-aware candidate domain (oracle/dash_oracle.py: page_aware_ids,
kl_candidate_mask, decode_page_state, decode_allow) pinned by prompts whose pages
are written out by hand and by a token-by-token walk of random prompts
(tests/bruteforce.py).  CPU only."""

import random

import pytest
import torch

import bruteforce as BF
from oracle import dash_oracle as O

IMG, PG, TXT, BOS = 5, 9, 7, 1
# <PAGE> I I I <PAGE> I I <PAGE> I I I T T <PAGE> T <PAGE> T
PROMPT = [BOS, PG, IMG, IMG, IMG, PG, IMG, IMG, PG, IMG, IMG, IMG, TXT, TXT, PG, TXT, PG, TXT]


def test_flat_image_token_mask_known_answer():
    """The flat (any page) image-token mask of _build_flat_image_token_mask
    (_sparse_base_impl.py:2363-2380): ids == image id over key_length tokens, the ids
    cut or padded with -1, None without an image token or for ids that are not 2-D;
    and the product's torch function (pages.build_flat_image_token_mask) equals it."""
    from ananta_ocr_amd import pages as P
    ids = torch.tensor([PROMPT, [TXT] * len(PROMPT)])
    want = [[x == IMG for x in PROMPT], [False] * len(PROMPT)]
    for L in (len(PROMPT), 10, len(PROMPT) + 5):
        m = O.flat_image_token_mask(ids, IMG, L)
        exp = [r[:L] + [False] * max(0, L - len(r)) for r in want]
        assert m.tolist() == exp, L
        assert torch.equal(P.build_flat_image_token_mask(ids, IMG, L), m), L
    # the ids are padded with -1 before the comparison, so an image id of -1 matches the
    # padding, as in the reference
    assert O.flat_image_token_mask(torch.tensor([[TXT, TXT]]), -1, 4).tolist() == \
        [[False, False, True, True]]
    assert O.flat_image_token_mask(torch.tensor([[TXT, TXT]]), IMG, 2) is None
    assert O.flat_image_token_mask(torch.tensor([IMG, IMG]), IMG, 2) is None
    assert O.flat_image_token_mask(None, IMG, 2) is None
    assert P.build_flat_image_token_mask(torch.tensor([[TXT, TXT]]), IMG, 2) is None


def test_page_ids_marker_mode_known_answer():
    ids = torch.tensor([PROMPT])
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, len(PROMPT), per_page=3)
    assert itm[0].tolist() == [x == IMG for x in PROMPT]
    assert ipi[0].tolist() == [-1, -1, 0, 0, 0, -1, 1, 1, -1, 2, 2, 2, -1, -1, -1, -1, -1, -1]
    assert qpi[0].tolist() == [-1] * 14 + [0, 0, 1, 1]
    _, _, qpi_s = O.page_aware_ids(ids, IMG, PG, len(PROMPT), per_page=3,
                                   page_scope_prefill=True)
    assert qpi_s[0].tolist() == [-1, 0, 0, 0, 0, 1, 1, 1, 2, 2, 2, 2, -1, -1, 0, 0, 1, 1]


def test_page_ids_per_page_mode_known_answer():
    # no marker before the last image token: pages of 3 image tokens; response pages are
    # opened by markers and counted from 0
    ids = torch.tensor([[IMG] * 7 + [PG, TXT, TXT, PG, TXT]])
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, 12, per_page=3)
    assert ipi[0].tolist() == [0, 0, 0, 1, 1, 1, 2] + [-1] * 5
    assert qpi[0].tolist() == [-1] * 7 + [0, 0, 0, 1, 1]
    # no marker at all: no query page, so no page-aware ids
    assert O.page_aware_ids(torch.tensor([[IMG] * 7 + [TXT] * 3]), IMG, PG, 10, 3) == \
        (None, None, None)
    # padding to key_length with -1, and cutting
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, 14, per_page=3)
    assert ipi.shape == (1, 14) and qpi[0, 12:].tolist() == [1, 1]


def test_candidate_mask_known_answer():
    ids = torch.tensor([PROMPT])
    itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, 18, per_page=3)
    pos = torch.tensor([[14, 16, 12, 0]])
    c = O.kl_candidate_mask(pos, 5, itm, 1, 4, 4, ipi, qpi)[0, 0]
    assert c[0].tolist() == [True, True, False, False, False]      # page 0: blocks 0, 1
    assert c[1].tolist() == [False, True, False, False, False]     # page 1: block 1
    assert c[2].tolist() == [True] * 5                              # no page: fallback
    assert c[3].tolist() == [True] * 5
    flat = O.kl_candidate_mask(pos, 5, itm, 1, 4, 4, None, None)[0, 0]
    assert flat[0].tolist() == [True, True, True, False, False]    # every image block
    none = O.kl_candidate_mask(pos, 5, None, 1, 4, 4)[0, 0]
    assert bool(none.all())


def test_decode_allow_known_answer():
    ids = torch.tensor([PROMPT])
    st = O.decode_page_state(ids, IMG, PG, 4, per_page=3)
    assert st["bmin"][0].tolist() == [0, 0, 2, -1, -1]
    assert st["bmax"][0].tolist() == [0, 1, 2, -1, -1]
    assert int(st["pp"][0]) == 3 and int(st["mcum"][0]) == 5
    a = O.decode_allow(st, torch.tensor([[TXT]]), PG, 19, 4)       # page 5 - 1 - 3 = 1
    assert a[0].tolist() == [False, True, False, False, False]
    a = O.decode_allow(st, torch.tensor([[PG]]), PG, 20, 4)        # a marker: page 2
    assert a[0].tolist() == [False, False, True, False, False]
    a = O.decode_allow(st, torch.tensor([[PG]]), PG, 21, 4)        # page 3: no image block
    assert a[0].tolist() == [True] * 6


def _random_prompt(rng, L, per_page_mode):
    ids = [BOS]
    while len(ids) < L:
        if not per_page_mode and rng.random() < 0.15:
            ids.append(PG)
        r = rng.random()
        ids.extend([IMG] * rng.randint(1, 9) if r < 0.6 else [TXT] * rng.randint(1, 4))
        if rng.random() < 0.1:
            ids.append(PG)
    return ids[:L]


@pytest.mark.parametrize("seed", range(6))
def test_page_ids_and_candidates_match_token_walk(seed):
    rng = random.Random(seed)
    B, L, per_page, bs = 3, 300, rng.choice([3, 7, 16]), rng.choice([4, 8, 32])
    rows = [_random_prompt(rng, L, per_page_mode=(b == 1 and seed % 2 == 0)) for b in range(B)]
    ids = torch.tensor(rows)
    for scope in (False, True):
        itm, ipi, qpi = O.page_aware_ids(ids, IMG, PG, L, per_page, scope)
        if itm is None:
            continue
        for b in range(B):
            f, ip, qp = BF.walk_pages(rows[b], IMG, PG, per_page, scope)
            assert itm[b].tolist() == f and ipi[b].tolist() == ip and qpi[b].tolist() == qp
        nblk = (L + bs - 1) // bs
        pos = torch.randint(-3, L + 3, (B, 50), generator=torch.Generator().manual_seed(seed))
        cm = O.kl_candidate_mask(pos, nblk, itm, B, 50, bs, ipi, qpi)[:, 0]
        for b in range(B):
            for i in range(50):
                qpage = qpi[b, min(max(int(pos[b, i]), 0), L - 1)].item()
                assert cm[b, i].tolist() == BF.candidates_row(qpage, ipi[b].tolist(), nblk, bs)


@pytest.mark.parametrize("seed", range(4))
def test_decode_allow_matches_token_walk(seed):
    rng = random.Random(100 + seed)
    B, L, per_page, bs = 3, 257, rng.choice([3, 10]), rng.choice([4, 16, 64])
    rows = [_random_prompt(rng, L, per_page_mode=(b == 2)) for b in range(B)]
    st = O.decode_page_state(torch.tensor(rows), IMG, PG, bs, per_page)
    walks = [BF.walk_decode_pages(r, IMG, PG, per_page, bs) for r in rows]
    for b in range(B):
        bmin, bmax, pp, m = walks[b]
        assert st["bmin"][b].tolist() == bmin and st["bmax"][b].tolist() == bmax
        assert int(st["pp"][b]) == pp and int(st["mcum"][b]) == m
    marks = [w[3] for w in walks]
    for step in range(12):
        new = [PG if rng.random() < 0.3 else TXT for _ in range(B)]
        total = L + step + 1
        a = O.decode_allow(st, torch.tensor(new)[:, None], PG, total, bs)
        nblk = (total + bs - 1) // bs
        for b in range(B):
            row, marks[b] = BF.decode_allow_row(walks[b][0], walks[b][1], walks[b][2], marks[b],
                                                new[b] == PG, nblk)
            assert a[b].tolist() == row, (seed, step, b)


def test_win_bounds_known_answers():
    """Block 4, one local block: the query at 29 sits in block 7, so blocks <= 6 are
    remote.  Rows: allowed {2, 5} -> [2, 6); allowed only beyond the remote range ->
    the live width [0, 8); a query in block 0 -> nothing; allowed {6} with a tile of
    0 blocks -> does not fit."""
    allow = torch.zeros(4, 10, dtype=torch.bool)
    allow[0, [2, 5]] = True
    allow[1, [7, 9]] = True
    allow[2, [0]] = True
    allow[3, [6]] = True
    seq = torch.tensor([30, 30, 3, 30])
    lo, hi, fit = O.decode_win_bounds(allow, seq, 10, 4, 1, 2)
    assert lo.tolist() == [2, 0, 0, 6]
    assert hi.tolist() == [6, 8, 0, 7]
    assert fit.tolist() == [False, False, True, True]
    lo, hi, fit = O.decode_win_bounds(allow, seq, 10, 4, 1, 0)
    assert fit.tolist() == [False, False, True, False]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_win_bounds_match_definition(seed):
    g = torch.Generator().manual_seed(seed)
    B, W, bs, lb = 64, 40, 8, 2
    allow = torch.rand(B, W + 3, generator=g) < torch.rand(B, 1, generator=g) * 0.3
    seq = torch.randint(0, W * bs + 1, (B,), generator=g)
    lo, hi, fit = O.decode_win_bounds(allow, seq, W, bs, lb, 6)
    for b in range(B):
        assert (int(lo[b]), int(hi[b]), bool(fit[b])) == \
            BF.win_bounds_row(allow[b].tolist(), int(seq[b]), W, bs, lb, 6), b


# ---------------------------------------------------------------- page2d RoPE coordinates

def test_page_rope_pos_known_answer():
    """_build_page_rope_pos / _page_rope_offsets on a hand-worked prompt: page = markers so
    far up to the last image, markers after it afterwards (page 0 = the text before the first
    marker and the instruction after the last image); tok = running count in the page; the
    span scaling rounds half to even."""
    ids = torch.tensor([PROMPT])
    tok, page, pf, n_pg = O.page_rope_pos(ids, IMG, PG, len(PROMPT))
    assert page[0].tolist() == [0, 1, 1, 1, 1, 2, 2, 2, 3, 3, 3, 3, 0, 0, 1, 1, 2, 2]
    assert tok[0].tolist() == [0, 0, 1, 2, 3, 0, 1, 2, 0, 1, 2, 3, 1, 2, 4, 5, 3, 4]
    assert pf[0].tolist() == [1, 4, 3, 4] and n_pg == 4
    tok, page, _, _ = O.page_rope_pos(ids, IMG, PG, len(PROMPT), page_span=10)
    assert tok[0].tolist() == [0, 0, 2, 5, 8, 0, 3, 7, 0, 2, 5, 8, 1, 2, 10, 11, 10, 11]
    # padded to a longer key length with -1: the padding continues the last page
    tok, page, _, _ = O.page_rope_pos(ids, IMG, PG, len(PROMPT) + 2)
    assert page[0].tolist()[-3:] == [2, 2, 2] and tok[0].tolist()[-3:] == [4, 5, 6]


def test_page_rope_pos_falls_back_where_the_reference_does():
    assert O.page_rope_pos(torch.tensor([[TXT, PG, TXT]]), IMG, PG, 3) is None     # no image
    assert O.page_rope_pos(torch.tensor([[TXT, IMG, IMG]]), IMG, PG, 3) is None    # no marker
    # a marker only after the last image token: not marker mode
    assert O.page_rope_pos(torch.tensor([[IMG, IMG, PG, TXT]]), IMG, PG, 4) is None
    # one row of the batch without a prompt page: the whole batch falls back
    two = torch.tensor([[PG, IMG, TXT], [IMG, PG, TXT]])
    assert O.page_rope_pos(two, IMG, PG, 3) is None
    assert O.page_rope_pos(None, IMG, PG, 3) is None
    assert O.page_rope_pos(torch.tensor([PG, IMG]), IMG, PG, 2) is None


def _random_ocr_prompt(rng, pages, resp_pages, per_page=(2, 9), prefix=3):
    ids = [BOS] + [TXT] * rng.randint(0, prefix)
    for _ in range(pages):
        ids += [PG] + [IMG] * rng.randint(*per_page)
    ids += [TXT] * rng.randint(0, 4)
    for _ in range(resp_pages):
        ids += [PG] + [TXT] * rng.randint(0, 6)
    return ids


@pytest.mark.parametrize("seed", range(6))
def test_page_rope_pos_matches_token_walk(seed):
    rng = random.Random(seed)
    B = 3
    rows = [_random_ocr_prompt(rng, rng.randint(1, 6), rng.randint(0, 5)) for _ in range(B)]
    L = max(len(r) for r in rows) + rng.randint(0, 3)
    ids = torch.full((B, L), -1, dtype=torch.long)
    for b, r in enumerate(rows):
        ids[b, :len(r)] = torch.tensor(r)
    tok, page, pf, n_pg = O.page_rope_pos(ids, IMG, PG, L)
    maxp = 0
    for b in range(B):
        wt, wp, wpf, n = BF.walk_page_rope(ids[b].tolist(), IMG, PG)
        assert tok[b].tolist() == wt and page[b].tolist() == wp
        maxp = max(maxp, max(wp))
        for p in range(n_pg):
            assert int(pf[b, p]) == wpf.get(p, 0)
    assert n_pg == maxp + 1


@pytest.mark.parametrize("seed", range(4))
def test_page_rope_decode_advance_equals_recompute(seed):
    """Stepping the coordinates one generated token at a time equals recomputing them on
    the longer prompt while the page stays within the prompt's pages; a further <PAGE>
    stays on the last page and restarts at its prefill count (the reference's clamp)."""
    rng = random.Random(100 + seed)
    prompt = _random_ocr_prompt(rng, rng.randint(3, 6), 0)
    tok, page, pf, n_pg = O.page_rope_pos(torch.tensor([prompt]), IMG, PG, len(prompt))
    t, p = tok[:, -1], page[:, -1]
    seq = list(prompt)
    for step in range(30):
        x = PG if rng.random() < 0.25 else TXT
        seq.append(x)
        t, p = O.page_rope_advance(p, t, pf, n_pg, torch.tensor([x]), PG)
        if int(p) < n_pg - 1 or x != PG:
            ref = O.page_rope_pos(torch.tensor([seq]), IMG, PG, len(seq))
            if ref[3] == n_pg:
                assert int(t) == int(ref[0][0, -1]) and int(p) == int(ref[1][0, -1]), step
    # the clamp, by hand: at the last page a <PAGE> keeps the page and restarts the count
    last = torch.tensor([n_pg - 1])
    t2, p2 = O.page_rope_advance(last, torch.tensor([50]), pf, n_pg, torch.tensor([PG]), PG)
    assert int(p2) == n_pg - 1 and int(t2) == int(pf[0, n_pg - 1])


def test_rotary2d_frequencies_and_angles():
    """DeepseekV2IndexerRotary2D: inverse frequencies base ** -(j / n) (resample) or
    base ** -(2 j / dim) (truncate) for the token pairs and base_page ** -(i / pairs) for
    the page pairs; cos/sin [.., dim] with the first n_tok pairs turned by tok only, the
    rest by page (mod page_mod), both halves equal; against float64 closed forms."""
    dim, bt, bp = 128, 10000.0, 256.0
    for mode in ("resample", "truncate"):
        it, ip = O.rotary2d_inv_freq(dim, bt, bp, 1, mode)
        n = dim // 2 - 1
        j = torch.arange(n, dtype=torch.float64)
        exp = bt ** (-(j / n) if mode == "resample" else -(2 * j / dim))
        torch.testing.assert_close(it.double(), exp, atol=0, rtol=1e-6)
        assert ip.tolist() == [1.0]
    it, ip = O.rotary2d_inv_freq(dim, bt, bp, 4)
    torch.testing.assert_close(ip.double(), bp ** -(torch.arange(4).double() / 4), rtol=1e-6,
                               atol=0)
    with pytest.raises(ValueError):
        O.rotary2d_inv_freq(dim, bt, bp, 64)
    tok = torch.tensor([[0, 1, 7, 2730]])
    page = torch.tensor([[0, 3, 4, 5]])
    c, s = O.rotary2d_cos_sin(tok, page, it, ip, page_mod=2)
    assert c.shape == (1, 4, dim)
    torch.testing.assert_close(c[..., :64], c[..., 64:], atol=0, rtol=0)
    # the angles are fp32 products (an angle of ~800 rad carries a 6e-5 rounding step);
    # cos / sin of those fp32 angles in float64
    ang_t = (tok.float()[..., None] * it[None, None]).double()
    ang_p = ((page % 2).float()[..., None] * ip[None, None]).double()
    ang = torch.cat([ang_t, ang_p], -1)
    torch.testing.assert_close(c[..., :64].double(), ang.cos(), atol=2e-6, rtol=0)
    torch.testing.assert_close(s[..., :64].double(), ang.sin(), atol=2e-6, rtol=0)
    assert c[0, 0].eq(1).all() and s[0, 0].eq(0).all()
    # page 3 and 5 fold to the same parity: equal page part, different token part
    torch.testing.assert_close(c[0, 1, 60:64], c[0, 3, 60:64], atol=0, rtol=0)
    c0, _ = O.rotary2d_cos_sin(tok, page, it, ip, page_mod=0)
    assert not torch.equal(c0[0, 1, 60:64], c0[0, 3, 60:64])
