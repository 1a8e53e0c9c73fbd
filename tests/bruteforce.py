"""Independent float64 brute-force formulations used to pin the oracle.

These are written from the mathematical definition of each quantity (explicit
key-set enumeration, bisection for the entmax threshold, plain ranking), not by
retyping the oracle's tensor algebra, so a dropped term, a wrong sign or an
off-by-one in the oracle fails a comparison against them.
"""

import math

import numpy as np


def entmax15_bisect(x, iters=200):
    """1.5-entmax by bisection on tau: p_i = max(x_i/2 - tau, 0)^2 with sum 1
    (Peters, Niculae & Martins 2019, eq. for alpha = 1.5).  float64."""
    x = np.asarray(x, dtype=np.float64)
    X = (x - x.max()) / 2.0
    lo, hi = X.max() - 1.0, X.max()          # f(lo) >= 1, f(hi) = 0
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        f = np.sum(np.maximum(X - mid, 0.0) ** 2)
        if f >= 1.0:
            lo = mid
        else:
            hi = mid
    tau = 0.5 * (lo + hi)
    return np.maximum(X - tau, 0.0) ** 2


def rank_desc(values):
    """Indices ordered by (value desc, index asc), by plain Python sorting."""
    return sorted(range(len(values)), key=lambda i: (-values[i], i))


def route_row(z_row, cand_row, idx_scale, floor, sigma, K, topm):
    """Inference routing of one query row from the definition.
    z_row: float32 numpy [nblk]; cand_row: bool numpy [nblk] or None.
    Returns (idx list, valid list, bias list [float64])."""
    nblk = len(z_row)
    remote = [float(z) > -5.0e8 for z in z_row]
    cand = list(remote) if cand_row is None else [r and bool(c) for r, c in zip(remote, cand_row)]
    if not any(cand):
        cand = list(remote)
    x = []
    for i in range(nblk):
        if cand[i]:
            v = np.float32(z_row[i]) * np.float32(idx_scale)
            if not np.isfinite(v):
                v = np.float32(-1.0e4)
        else:
            v = np.float32(-1.0e4)
        x.append(float(v))
    M = max(1, min(topm, nblk)) if topm > 0 else nblk
    order = rank_desc(x)[:M]
    prior = entmax15_bisect([x[i] for i in order])
    Kp = max(1, min(K, M))
    idx = order[:Kp]
    valid = [cand[i] for i in idx]
    logp = [math.log(max(p, floor)) for p in prior[:Kp]]
    cnt = max(1, sum(valid))
    mu = sum(lp for lp, va in zip(logp, valid) if va) / cnt
    bias = [((lp - mu) / sigma) if va else 0.0 for lp, va in zip(logp, valid)]
    return idx, valid, bias


def train_route_row(z_row, cand_row, idx_scale, floor, sigma, K):
    """Training routing of one query row from the definition: the 1.5-entmax prior over
    every block (bisection on its threshold, float64), the K highest candidate priors
    (non-candidates ranked below every candidate), the centred log-prior bias over the
    candidates among them, clamped to +-1e4.  Returns (idx, valid, bias)."""
    nblk = len(z_row)
    remote = [float(z) > -5.0e8 for z in z_row]
    cand = list(remote) if cand_row is None else [r and bool(c) for r, c in zip(remote, cand_row)]
    if not any(cand):
        cand = list(remote)
    x = []
    for i in range(nblk):
        v = np.float32(z_row[i]) * np.float32(idx_scale) if cand[i] else np.float32(-1.0e4)
        x.append(float(v) if np.isfinite(v) else -1.0e4)
    prior = entmax15_bisect(x)
    masked = [float(prior[i]) if cand[i] else -1.0 for i in range(nblk)]
    Kp = max(1, min(K, nblk))
    idx = rank_desc(masked)[:Kp]
    valid = [masked[i] >= 0.0 for i in idx]
    logp = [math.log(max(masked[i], floor)) if valid[j] else math.log(floor)
            for j, i in enumerate(idx)]
    cnt = max(1, sum(valid))
    mu = sum(lp for lp, va in zip(logp, valid) if va) / cnt
    bias = [max(-1e4, min(1e4, (lp - mu) / sigma)) if va else 0.0 for lp, va in zip(logp, valid)]
    return idx, valid, bias


def key_sets(t, S, topi_row, bias_row, valid_row, block_size, local_window, kmin=0):
    """Explicit key set of query t: dict key -> additive bias.

    Window keys: max(t - LW + 1, kmin) <= j <= t, bias 0.
    Routed keys: j in a valid routed block, j <= t, kmin <= j < t - LW + 1,
    bias of the block (first slot wins on a duplicated block)."""
    ls = t - local_window + 1
    keys = {}
    for j in range(max(ls, kmin, 0), t + 1):
        keys[j] = 0.0
    seen = set()
    for c, b, va in zip(topi_row, bias_row, valid_row):
        c = int(c)
        if not va or c < 0 or c in seen:
            continue
        seen.add(c)
        for j in range(c * block_size, min((c + 1) * block_size, S)):
            if j <= t and j < ls and j >= kmin:
                keys[j] = float(b)
    return keys


def attend_row(qv, K, V, keys, scale):
    """softmax over an explicit key set, float64.  qv [D], K/V [S,D]."""
    js = sorted(keys)
    if not js:
        return np.zeros(V.shape[1])
    s = np.array([scale * float(np.dot(qv, K[j])) + keys[j] for j in js])
    s -= s.max()
    p = np.exp(s)
    p /= p.sum()
    return p @ V[js]


def attend_brute(q, k, v, topi, bias, valid, block_size, local_window, scale, rows=None,
                 kmin=None):
    """q,k,v float64 numpy [B,H,S,D]; topi/bias/valid [B,S,K].
    Returns {(b,h,t): out[D]} for the requested rows (default all)."""
    B, H, S, D = q.shape
    out = {}
    for b in range(B):
        for t in (range(S) if rows is None else rows):
            km = 0 if kmin is None else int(kmin[b, t])
            keys = key_sets(t, S, topi[b, t], bias[b, t], valid[b, t], block_size,
                            local_window, km)
            for h in range(H):
                out[(b, h, t)] = attend_row(q[b, h, t], k[b, h], v[b, h], keys, scale)
    return out


# ---------------------------------------------------------------- OCR pages

def walk_pages(ids, img_id, page_id, per_page, page_scope_prefill):
    """Token-by-token page assignment of one prompt row, from the definitions: an image
    token belongs to the page of the last <PAGE> marker before it when the prompt has a
    marker before its last image token, else to (its index among image tokens) //
    per_page; a query token belongs to the page of the last marker before it, counted
    from the first marker after the prompt's last image (response pages restart at 0)
    when the prompt is in marker mode, and has no page inside the prompt unless
    page_scope_prefill.  Returns (image flags, image pages, query pages), lists."""
    L = len(ids)
    last = max([t for t in range(L) if ids[t] == img_id], default=-1)
    prompt_markers = sum(1 for t in range(last + 1) if ids[t] == page_id)
    marker_mode = prompt_markers > 0
    markers = nimg = 0
    flags, ipages, qpages = [], [], []
    for t in range(L):
        if ids[t] == page_id:
            markers += 1
        if ids[t] == img_id:
            ipages.append(markers - 1 if marker_mode else nimg // per_page)
            nimg += 1
            flags.append(True)
        else:
            ipages.append(-1)
            flags.append(False)
        if t <= last:
            q = markers - 1 if page_scope_prefill else -1
        else:
            q = markers - 1 - (prompt_markers if marker_mode else 0)
        qpages.append(q if q >= 0 else -1)
    return flags, ipages, qpages


def candidates_row(qp, ipages, nblk, bs):
    """Candidate blocks of a query of page qp: blocks with an image token of page qp,
    or every block when there is none."""
    L = len(ipages)
    row = [qp >= 0 and any(ipages[j] == qp for j in range(c * bs, min(c * bs + bs, L)))
           for c in range(nblk)]
    return row if any(row) else [True] * nblk


def walk_decode_pages(ids, img_id, page_id, per_page, bs):
    """Decode page state of one prompt row: each image token's page (the last marker
    before it - 1 once a marker was seen, else its index among image tokens // per_page),
    per key block the smallest and largest such page (-1 without image tokens), the
    markers up to the last image token and all markers."""
    L = len(ids)
    markers = nimg = 0
    pages = []
    pp = 0
    for t in range(L):
        if ids[t] == page_id:
            markers += 1
        if ids[t] == img_id:
            pages.append(markers - 1 if markers > 0 else nimg // per_page)
            nimg += 1
            pp = markers
        else:
            pages.append(-1)
    nblk = (L + bs - 1) // bs
    bmin, bmax = [], []
    for c in range(nblk):
        ps = [p for p in pages[c * bs:(c + 1) * bs] if p >= 0]
        bmin.append(min(ps) if ps else -1)
        bmax.append(max(ps) if ps else -1)
    return bmin, bmax, pp, markers


def decode_allow_row(bmin, bmax, pp, markers, new_is_marker, nblk):
    """Allow row of one decode step: the query's page is (markers after this token) - 1 -
    pp; blocks whose [bmin, bmax] holds it; every block when none does or there is no
    page.  Returns (row, updated markers)."""
    m = markers + (1 if new_is_marker else 0)
    qp = m - 1 - pp
    same = [qp >= 0 and c < len(bmin) and bmin[c] >= 0 and bmin[c] <= qp <= bmax[c]
            for c in range(nblk)]
    if qp < 0 or not any(same):
        return [True] * nblk, m
    return same, m


def win_bounds_row(allow, seq, max_block, bs, lb, tile):
    """(lo, hi, fit) of one decode row from the definition: the allowed blocks that are
    remote for the query at seq - 1 and hold a live key; with none, the live width (or
    nothing when the query has no remote block)."""
    q_blk = (seq - 1) // bs if seq > 0 else -1
    live = [c for c in range(min(max_block, len(allow)))
            if allow[c] and c <= q_blk - lb and c * bs < seq]
    if live:
        lo, hi = min(live), max(live) + 1
    elif seq <= 0 or q_blk - lb < 0:
        lo, hi = 0, 0
    else:
        lo, hi = 0, min(max_block, max((seq + bs - 1) // bs, 1))
    return lo, hi, hi - lo <= tile


def walk_page_rope(ids_row, img_id, page_id):
    """Two-axis coordinates of one prompt row from the definition, token by token:
    page = markers so far (up to the last image token), else markers after it; tok = how
    many earlier tokens share the page.  Returns (tok list, page list, prefill count per
    page dict, prompt pages)."""
    last = max((i for i, x in enumerate(ids_row) if x == img_id), default=-1)
    n = sum(1 for x in ids_row[:last + 1] if x == page_id)
    seen, pf = {}, {}
    toks, pages = [], []
    marks = 0
    for i, x in enumerate(ids_row):
        if x == page_id:
            marks += 1
        p = marks if i <= last else marks - n
        toks.append(seen.get(p, 0))
        seen[p] = seen.get(p, 0) + 1
        pages.append(p)
        if i <= last:
            pf[p] = pf.get(p, 0) + 1
    return toks, pages, pf, n
