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
