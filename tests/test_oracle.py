"""Pins the CPU oracle (oracle/dash_oracle.py) to independent formulations:
closed forms, invariants, float64 brute force and bisection.  CPU only."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import bruteforce as bf
from oracle import dash_oracle as O


def _rng(seed):
    return torch.Generator().manual_seed(seed)


# ---------------------------------------------------------------- entmax15

def test_entmax_two_point_closed_form():
    # x = [a, 0]: support 1 (p = [1, 0]) iff a >= 2; otherwise tau solves
    # 2 tau^2 + a tau + a^2/4 - 1 = 0 with X = [0, -a/2].
    for a in [0.0, 0.3, 1.0, 1.7, 1.999, 2.0, 2.5, 10.0]:
        p = O.entmax15(torch.tensor([[a, 0.0]], dtype=torch.float64))[0].numpy()
        if a >= 2.0:
            exp = np.array([1.0, 0.0])
        else:
            tau = (-a - math.sqrt(8.0 - a * a)) / 4.0
            exp = np.array([tau * tau, (a / 2.0 + tau) ** 2])
        np.testing.assert_allclose(p, exp, atol=1e-12)


def test_entmax_uniform_and_invariants():
    for n in [1, 2, 5, 16]:
        p = O.entmax15(torch.full((1, n), 3.25))[0]
        torch.testing.assert_close(p, torch.full((n,), 1.0 / n), atol=1e-6, rtol=0)
    x = torch.randn(64, 16, generator=_rng(0)) * 3
    p = O.entmax15(x)
    assert (p >= 0).all()
    torch.testing.assert_close(p.sum(-1), torch.ones(64), atol=1e-5, rtol=0)
    torch.testing.assert_close(O.entmax15(x + 7.5), p, atol=1e-5, rtol=0)
    # order-equivariance: permuting the input permutes the output
    perm = torch.randperm(16, generator=_rng(1))
    torch.testing.assert_close(O.entmax15(x[:, perm]), p[:, perm], atol=1e-6, rtol=0)


@pytest.mark.parametrize("scale", [0.1, 1.0, 4.0, 30.0])
def test_entmax_matches_bisection(scale):
    x = torch.randn(200, 16, generator=_rng(2)) * scale
    p = O.entmax15(x.double()).numpy()
    for r in range(x.shape[0]):
        np.testing.assert_allclose(p[r], bf.entmax15_bisect(x[r].double().numpy()), atol=1e-9)
    # fp32 path stays within fp32 tolerance of the exact threshold
    p32 = O.entmax15(x).numpy()
    for r in range(x.shape[0]):
        np.testing.assert_allclose(p32[r], bf.entmax15_bisect(x[r].double().numpy()), atol=2e-5)


def test_entmax_sentinel_entries_get_zero():
    x = torch.tensor([[0.5, 0.2, -1.0e4, -1.0e4]])
    p = O.entmax15(x)[0]
    assert p[2] == 0 and p[3] == 0
    torch.testing.assert_close(p[:2].sum(), torch.tensor(1.0))


# ---------------------------------------------------------------- routing

def test_stable_topk_is_plain_ranking():
    x = torch.randint(-3, 4, (50, 40), generator=_rng(3)).float()  # many ties
    v, i = O.stable_topk(x, 12)
    for r in range(50):
        exp = bf.rank_desc(x[r].tolist())[:12]
        assert i[r].tolist() == exp


def test_idx_scale_multiply_is_single_fp32_rounding():
    z = torch.randn(10000, generator=_rng(4)) * 1e-3
    s = 128.0 / math.sqrt(128.0)
    a = (z * s).numpy()
    b = z.numpy() * np.float32(s)
    assert np.array_equal(a, b)


def _route_case(seed, B, S, nblk, scale_z, with_cand, nan_frac=0.0):
    g = _rng(seed)
    z = torch.randn(B, S, nblk, generator=g) * scale_z
    # remote mask pattern like the real scores: block c remote iff c <= t//bs - LB
    bs, lb = 4, 2
    t = torch.arange(S)[None, :, None]
    keep = torch.arange(nblk)[None, None, :] <= (t // bs - lb)
    z = z.masked_fill(~keep, O.SCORE_NEG)
    if nan_frac:
        m = torch.rand(B, S, nblk, generator=g) < nan_frac
        z = z.masked_fill(m & keep, float("nan"))
    cand = None
    if with_cand:
        cand = torch.rand(B, S, nblk, generator=g) < 0.4
        cand[:, ::7] = False          # rows that fall back to `remote`
    return z, cand


@pytest.mark.parametrize("with_cand", [False, True])
@pytest.mark.parametrize("scale_z,K,topm", [(1e-3, 8, 8), (1.0, 4, 16), (0.3, 16, 16), (5.0, 3, 0)])
def test_infer_route_matches_definition(with_cand, scale_z, K, topm):
    z, cand = _route_case(11, 2, 60, 15, scale_z, with_cand, nan_frac=0.02)
    idx_scale, floor, sigma = 128 / math.sqrt(128), 1e-4, 1.0
    ti, bi, va = O.infer_route_select(z, cand, idx_scale, floor, sigma, K, topm)
    for b in range(2):
        for t in range(60):
            e_idx, e_val, e_bias = bf.route_row(
                z[b, t].numpy(), None if cand is None else cand[b, t].numpy(),
                idx_scale, floor, sigma, K, topm)
            assert ti[b, t].tolist() == e_idx, (b, t)
            assert va[b, t].tolist() == e_val, (b, t)
            np.testing.assert_allclose(bi[b, t].numpy(), e_bias, atol=2e-4)


def test_infer_route_sets_match_torch_topk_without_ties():
    z, _ = _route_case(12, 2, 80, 19, 0.5, False)
    idx_scale = 128 / math.sqrt(128)
    ti, _, va = O.infer_route_select(z, None, idx_scale, 1e-4, 1.0, 6, 8)
    x, cand = O.route_inputs(z, None, idx_scale)
    xv, xi = x.topk(8, dim=-1)
    for b in range(2):
        for t in range(80):
            vals = xv[b, t]
            cut_tie = (vals[5] == vals[6]).item() or (vals[7] == x[b, t].sort(descending=True)[0][8]).item()
            if not cut_tie:
                assert set(ti[b, t].tolist()) == set(xi[b, t, :6].tolist())


def test_route_no_remote_rows_are_invalid():
    z = torch.full((1, 3, 5), O.SCORE_NEG)
    ti, bi, va = O.infer_route_select(z, None, 2.0, 1e-4, 1.0, 4, 4)
    assert not va.any()
    assert (bi == 0).all()


@pytest.mark.parametrize("seed,scale,with_cand,K", [(21, 11.3, False, 5), (22, 0.7, True, 8),
                                                    (23, 40.0, True, 12), (24, 11.3, True, 30)])
def test_train_route_matches_definition(seed, scale, with_cand, K):
    """Ids, validity and bias of the training router against the from-definition row
    (full-width entmax by bisection): wide and narrow support, candidate masks, and
    K above the number of candidates (the remaining slots are non-candidates)."""
    z, cand = _route_case(seed, 1, 40, 37, 0.5, with_cand)
    ti, bi, va = O.train_route_select(z, cand, scale, 1e-4, 1.0, K)
    for t in range(40):
        idx, valid, bias = bf.train_route_row(z[0, t].numpy(), None if cand is None else
                                              cand[0, t].numpy(), scale, 1e-4, 1.0, K)
        assert va[0, t].tolist() == valid, t
        nv = sum(valid)
        assert ti[0, t, :nv].tolist() == idx[:nv], t
        torch.testing.assert_close(bi[0, t].double(), torch.tensor(bias, dtype=torch.float64),
                                   atol=2e-4, rtol=1e-4)


def test_train_route_selects_top_prior():
    z, cand = _route_case(13, 1, 50, 13, 0.5, True)
    ti, bi, va = O.train_route_select(z, cand, 11.3, 1e-4, 1.0, 5)
    x, c = O.route_inputs(z, cand, 11.3)
    prior = O.entmax15(x)
    for t in range(50):
        pr = prior[0, t].masked_fill(~c[0, t], -1.0).tolist()
        assert ti[0, t].tolist() == bf.rank_desc(pr)[:5]


def test_entmax15_gradient_is_the_closed_form_jacobian():
    """Autograd through the sort-based forward equals float64 finite differences
    (gradcheck) and the closed-form backward of dash_attention.py:650-658,
    dX = dY*sqrt(Y) - sqrt(Y) * sum(dY*sqrt(Y)) / sum(sqrt(Y))."""
    g = _rng(31)
    X = (torch.randn(6, 19, generator=g, dtype=torch.float64) * 1.5).requires_grad_()
    assert torch.autograd.gradcheck(lambda t: O.entmax15(t, dim=-1), (X,), eps=1e-7, atol=1e-6)
    Y = O.entmax15(X, dim=-1)
    assert ((Y > 0).sum(-1) < 19).all() and ((Y > 0).sum(-1) > 1).all()   # partial support
    dY = torch.randn(6, 19, generator=g, dtype=torch.float64)
    (gx,) = torch.autograd.grad(Y, X, dY)
    gp = Y.detach().sqrt()
    closed = dY * gp - gp * (dY * gp).sum(-1, keepdim=True) / gp.sum(-1, keepdim=True)
    torch.testing.assert_close(gx, closed, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("with_cand", [False, True])
def test_train_route_gradient_central_differences(with_cand):
    """d(sum(w * bias))/dz of the training router by autograd against central
    differences of the forward (selection fixed: a small step keeps the top-K set)."""
    z, cand = _route_case(41, 1, 24, 19, 0.5, with_cand)
    remote = z > O.SCORE_NEG * 0.5
    w = torch.randn(1, 24, 5, generator=_rng(42))

    def f(zz):
        _, b, _ = O.train_route_select(zz, cand, 3.0, 1e-2, 1.0, 5)
        return (w * b).sum()

    zg = z.clone().requires_grad_()
    f(zg).backward()
    grad = zg.grad
    d = torch.randn(z.shape, generator=_rng(43)) * remote
    eps = 1e-3
    num = (f(z + eps * d) - f(z - eps * d)).item() / (2 * eps)
    ana = (grad * d).sum().item()
    assert abs(num - ana) <= 2e-2 * max(abs(ana), 1.0), (num, ana)
    assert (grad[~remote] == 0).all()


def test_sanitize_grad_bounds_and_zeroes_nonfinite():
    g = torch.tensor([float("nan"), float("inf"), -float("inf"), 3e4, -2e5, 7.0])
    assert O.sanitize_grad(g).tolist() == [0.0, 0.0, 0.0, 1e4, -1e4, 7.0]


# ---------------------------------------------------------------- router front end

def test_gemma_rmsnorm_is_rms_norm_with_one_plus_weight():
    x = torch.randn(5, 9, 128, generator=_rng(30)) * 3
    w = torch.randn(128, generator=_rng(31)) * 0.3
    ref = F.rms_norm(x.double(), (128,), weight=1.0 + w.double(), eps=1e-6)
    torch.testing.assert_close(O.gemma_rmsnorm(x, w, 1e-6).double(), ref, atol=2e-6, rtol=2e-6)


def test_gemma_rmsnorm_constant_rows_clamps_and_guards():
    w = torch.linspace(-0.5, 0.5, 128)
    x = torch.full((3, 128), 2.5)
    x[1] = -7.0
    x[2, :] = float("nan")                                  # nan -> 0 -> the zero row
    y = O.gemma_rmsnorm(x, w, 1e-6)                          # c / sqrt(c^2 + eps) = 1 - O(1e-7)
    torch.testing.assert_close(y[0], 1.0 + w, atol=1e-6, rtol=0)
    torch.testing.assert_close(y[1], -(1.0 + w), atol=1e-6, rtol=0)
    assert (y[2] == 0).all()
    big = torch.zeros(1, 128)
    big[0, 0] = 1.0                                          # one hot: sqrt(128) before clamp
    y = O.gemma_rmsnorm(big, torch.full((128,), 1e4), 1e-6)  # (1 + w) * sqrt(128) > 1e4
    assert y[0, 0].item() == 1e4 and (y[0, 1:] == 0).all()


def test_rope_identity_and_rotate_half():
    x = torch.randn(2, 7, 128, generator=_rng(32))
    one, zero = torch.ones(1, 7, 128), torch.zeros(1, 7, 128)
    assert torch.equal(O.rotate_half_rope(x, one, zero), x)
    rot = O.rotate_half_rope(x, zero, one)
    assert torch.equal(rot[..., :64], -x[..., 64:]) and torch.equal(rot[..., 64:], x[..., :64])


def test_router_qk_projection_and_guards():
    g = _rng(33)
    hs = torch.randn(2, 11, 256, generator=g)
    hs[0, 3, 5] = float("inf")                              # nan_to_num before the projection
    wq, wk = torch.randn(128, 256, generator=g) * 0.1, torch.randn(128, 256, generator=g) * 0.1
    nq, nk = torch.randn(128, generator=g) * 0.2, torch.randn(128, generator=g) * 0.2
    ang = torch.arange(11)[:, None] * (1e4 ** (-torch.arange(0, 128, 2) / 128))[None]
    emb = torch.cat([ang, ang], -1)[None]
    iq, ik = O.router_qk(hs, wq, wk, nq, nk, 1e-6, emb.cos(), emb.sin())
    clean = torch.nan_to_num(hs, posinf=0.0)
    for got, w, nw in ((iq, wq, nq), (ik, wk, nk)):
        p = (clean.double() @ w.double().t())
        y = F.rms_norm(p, (128,), weight=1.0 + nw.double(), eps=1e-6)
        y1, y2 = y[..., :64], y[..., 64:]
        ref = torch.cat([y1 * emb.cos()[..., :64] - y2 * emb.sin()[..., :64],
                         y2 * emb.cos()[..., 64:] + y1 * emb.sin()[..., 64:]], -1)
        torch.testing.assert_close(got.double(), ref, atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- stage 0

def test_kbar_zero_headcls_is_block_mean():
    idx_k = torch.randn(2, 37, 8, generator=_rng(5))
    kb, cv = O.kbar_headcls(idx_k, torch.zeros(8), 8)
    assert kb.shape == (2, 5, 8) and cv.all()
    k64 = idx_k.double()
    for c in range(5):
        exp = k64[:, c * 8:min((c + 1) * 8, 37)].mean(1)
        torch.testing.assert_close(kb[:, c].double(), exp, atol=1e-6, rtol=0)


def test_kbar_headcls_softmax_pooling():
    idx_k = torch.randn(1, 21, 6, generator=_rng(6))
    hc = torch.randn(6, generator=_rng(7)) * 3
    kb, _ = O.kbar_headcls(idx_k, hc, 4)
    k = idx_k[0].double().numpy()
    h = hc.double().numpy()
    for c in range(6):
        rows = k[c * 4:min(c * 4 + 4, 21)]
        aw = rows @ h / math.sqrt(6)
        w = np.exp(aw - aw.max())
        w /= w.sum()
        np.testing.assert_allclose(kb[0, c].numpy(), w @ rows, atol=1e-5)


def test_block_scores_headcls_definition():
    B, S, d, bs, lb = 2, 45, 8, 4, 3
    iq = torch.randn(B, S, d, generator=_rng(8))
    ik = torch.randn(B, S, d, generator=_rng(9))
    kb, cv = O.kbar_headcls(ik, torch.zeros(d), bs)
    pos = torch.arange(S)[None].expand(B, -1)
    z = O.block_scores_headcls(iq, kb, cv, pos, bs, lb, q_chunk=7)
    nblk = kb.shape[1]
    for b in range(B):
        for t in range(S):
            for c in range(nblk):
                if c <= t // bs - lb:
                    e = float(np.dot(iq[b, t].double().numpy(), kb[b, c].double().numpy())) / math.sqrt(d)
                    assert abs(z[b, t, c].item() - e) < 1e-5
                else:
                    assert z[b, t, c].item() == O.SCORE_NEG


def test_block_scores_indexer_definition():
    B, S, d, bs, lw = 1, 30, 4, 4, 6
    iq = torch.randn(B, S, d, generator=_rng(10))
    ik = torch.randn(B, S, d, generator=_rng(11))
    nblk = 8
    pos = torch.arange(S)[None]
    z = O.block_scores_indexer(iq, ik, pos, nblk, bs, lw, q_chunk=9)
    for t in range(S):
        for c in range(nblk):
            js = [j for j in range(c * bs, min(c * bs + bs, S)) if j <= t - lw]
            if js:
                e = max(float(np.dot(iq[0, t].double().numpy(), ik[0, j].double().numpy())) for j in js)
                assert abs(z[0, t, c].item() - e) < 1e-5
            else:
                assert z[0, t, c].item() == O.SCORE_NEG


def test_block_max_score_definition():
    B, C, D, Sk, bs, lw = 1, 20, 4, 24, 4, 5
    q = torch.randn(B, C, D, generator=_rng(12))
    k = torch.randn(B, Sk, D, generator=_rng(13))
    pos = torch.arange(C)[None] + 3
    seg = torch.tensor([[0] * 10 + [9] * 10])
    out = O.block_max_score(q, k, pos, seg, bs, 6, lw)
    for t in range(C):
        ls = max(int(pos[0, t]) - lw + 1, 0)
        for c in range(6):
            js = [j for j in range(c * bs, c * bs + bs) if j < ls and j >= seg[0, t] and j < Sk]
            if js:
                e = max(float(np.dot(q[0, t].double().numpy(), k[0, j].double().numpy())) for j in js)
                assert abs(out[0, t, c].item() - e) < 1e-5
            else:
                assert out[0, t, c].item() == float("-inf")


# ---------------------------------------------------------------- attention

def _attn_case(seed, B=1, H=2, S=70, D=16, bs=8, lb=2, K=3, qscale=2.0):
    g = _rng(seed)
    q = torch.randn(B, H, S, D, generator=g) * qscale
    k = torch.randn(B, H, S, D, generator=g)
    v = torch.randn(B, H, S, D, generator=g)
    nblk = (S + bs - 1) // bs
    topi = torch.randint(0, nblk, (B, S, K), generator=g)
    bias = torch.randn(B, S, K, generator=g)
    valid = torch.rand(B, S, K, generator=g) < 0.8
    # routed blocks are remote, as the router guarantees; a few -1 slots
    qblk = torch.arange(S)[None, :, None] // bs
    valid &= topi <= qblk - lb
    topi = torch.where(torch.rand(B, S, K, generator=g) < 0.1, torch.full_like(topi, -1), topi)
    return q, k, v, topi, bias, valid, bs, lb * bs


@pytest.mark.parametrize("seed", [0, 1])
def test_dense_attend_matches_key_set_enumeration(seed):
    q, k, v, topi, bias, valid, bs, lw = _attn_case(20 + seed)
    scale = 1.0 / math.sqrt(q.shape[-1])
    out = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale, q_chunk=17)
    ref = bf.attend_brute(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                          topi.numpy(), bias.numpy(), valid.numpy(), bs, lw, scale)
    for (b, h, t), o in ref.items():
        np.testing.assert_allclose(out[b, h, t].double().numpy(), o, atol=2e-5)


def test_dense_attend_with_segment_start():
    q, k, v, topi, bias, valid, bs, lw = _attn_case(30, S=50)
    kmin = torch.tensor([[0] * 20 + [20] * 30])
    scale = 0.25
    out = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale, kmin=kmin)
    ref = bf.attend_brute(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                          topi.numpy(), bias.numpy(), valid.numpy(), bs, lw, scale,
                          kmin=kmin.numpy())
    for (b, h, t), o in ref.items():
        np.testing.assert_allclose(out[b, h, t].double().numpy(), o, atol=2e-5)


def test_dense_attend_reduces_to_sliding_window_and_causal():
    q, k, v, topi, bias, valid, bs, lw = _attn_case(31, S=64)
    scale = 0.25
    S = 64
    none = torch.zeros_like(valid)
    out = O.dense_attend(q, k, v, topi, bias, none, bs, lw, scale)
    i = torch.arange(S)
    win = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - lw)
    exp = F.scaled_dot_product_attention(q, k, v, attn_mask=win, scale=scale)
    torch.testing.assert_close(out, exp, atol=1e-5, rtol=1e-5)
    out2 = O.dense_attend(q, k, v, topi, bias, none, bs, 10 * S, scale)
    exp2 = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
    torch.testing.assert_close(out2, exp2, atol=1e-5, rtol=1e-5)
    # every remote block routed with zero bias -> plain causal attention
    nblk = S // bs
    allb = torch.arange(nblk)[None, None, :].expand(1, S, nblk)
    qblk = torch.arange(S)[None, :, None] // bs
    out3 = O.dense_attend(q, k, v, allb, torch.zeros(1, S, nblk), allb <= qblk - lw // bs,
                          bs, lw, scale)
    torch.testing.assert_close(out3, exp2, atol=1e-5, rtol=1e-5)
    # row 0 attends only key 0
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0], atol=1e-6, rtol=0)


def test_decode_attend_equals_prefill_last_row_and_brute_force():
    q, k, v, topi, bias, valid, bs, lw = _attn_case(32, S=77, K=4)
    scale = 0.3
    S = 77
    full = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale)
    for t in [S - 1, 40, 17]:
        dec = O.decode_attend(q[:, :, t:t + 1], k[:, :, :t + 1], v[:, :, :t + 1],
                              topi[:, t:t + 1], bias[:, t:t + 1], valid[:, t:t + 1],
                              torch.tensor([[t]]), bs, lw, scale)
        torch.testing.assert_close(dec[:, :, 0], full[:, :, t], atol=1e-5, rtol=1e-5)


def _left_pad_mask(B, S, pads, fill):
    """HF-style 4-D additive mask: causal, and keys before the row's left padding end
    excluded, with ``fill`` for excluded entries."""
    i = torch.arange(S)
    m = torch.zeros(B, 1, S, S)
    for b, p in enumerate(pads):
        bad = (i[None, :] > i[:, None]) | (i[None, :] < p)
        m[b, 0] = torch.where(bad, torch.full((), fill), torch.zeros(()))
    return m


def test_dense_attend_attention_mask_left_padding():
    """The additive mask term (dash_attention.py:1001-1003): an all-zero mask changes
    nothing; with left padding, a row past the padding attends the key-set enumeration
    with segment start = the padding length; a row whose causal keys are all padding
    gets every logit clamped to -1e9, so the mean of v over all S keys."""
    B, S = 2, 60
    q, k, v, topi, bias, valid, bs, lw = _attn_case(33, B=B, S=S)
    scale = 0.3
    plain = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale)
    zero = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale,
                          attention_mask=torch.zeros(1, 1, S, S))
    assert torch.equal(plain, zero)
    pads = [0, 23]
    am = _left_pad_mask(B, S, pads, torch.finfo(torch.float32).min)
    out = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale, q_chunk=19,
                         attention_mask=am)
    kmin = torch.tensor(pads)[:, None].expand(B, S)
    ref = bf.attend_brute(q.double().numpy(), k.double().numpy(), v.double().numpy(),
                          topi.numpy(), bias.numpy(), valid.numpy(), bs, lw, scale,
                          kmin=kmin.numpy())
    for (b, h, t), o in ref.items():
        if t >= pads[b]:
            np.testing.assert_allclose(out[b, h, t].double().numpy(), o, atol=2e-5)
    vm = v[1].mean(1)                                   # [H, D]
    for t in range(pads[1]):
        torch.testing.assert_close(out[1, :, t], vm, atol=1e-5, rtol=1e-5)
    # -1e4 excludes a key as well as the dtype minimum on rows that keep a key
    out2 = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale,
                          attention_mask=_left_pad_mask(B, S, pads, -1e4))
    torch.testing.assert_close(out2[1, :, pads[1]:], out[1, :, pads[1]:], atol=1e-6, rtol=0)


def test_decode_attend_several_rows_per_sequence():
    """Lq > 1 decode rows (modeling_deepseekv2.py:424-451 with q_pos [B, Lq]): each row
    equals the prefill row at its position."""
    q, k, v, topi, bias, valid, bs, lw = _attn_case(34, B=2, S=90, K=4)
    scale = 0.3
    full = O.dense_attend(q, k, v, topi, bias, valid, bs, lw, scale)
    pos = torch.tensor([[89, 40, 41], [7, 88, 60]])
    qs = torch.stack([q[b][:, pos[b]] for b in range(2)])
    sel = [torch.stack([x[b][pos[b]] for b in range(2)]) for x in (topi, bias, valid)]
    dec = O.decode_attend(qs, k, v, *sel, pos, bs, lw, scale)
    for b in range(2):
        torch.testing.assert_close(dec[b], full[b][:, pos[b]], atol=1e-5, rtol=1e-5)


def test_varlen_documents_are_isolated():
    g = _rng(40)
    H, D, d = 2, 16, 8
    cu = [0, 37, 37 + 61, 37 + 61 + 20]
    T = cu[-1]
    q = torch.randn(1, H, T, D, generator=g)
    k = torch.randn(1, H, T, D, generator=g)
    v = torch.randn(1, H, T, D, generator=g)
    iq = torch.randn(1, T, d, generator=g)
    ik = torch.randn(1, T, d, generator=g)
    args = (torch.zeros(d), 4, 2, 3.0, 1e-4, 1.0, 3, 3, 0.25)
    out, *_ = O.prefill_varlen(q, k, v, iq, ik, cu, *args)
    k2, v2, ik2 = k.clone(), v.clone(), ik.clone()
    k2[:, :, cu[1]:cu[2]] += 5
    v2[:, :, cu[1]:cu[2]] -= 3
    ik2[:, cu[1]:cu[2]] *= -2
    out2, *_ = O.prefill_varlen(q, k2, v2, iq, ik2, cu, *args)
    torch.testing.assert_close(out[:, :, :cu[1]], out2[:, :, :cu[1]])
    torch.testing.assert_close(out[:, :, cu[2]:], out2[:, :, cu[2]:])
    # the middle document alone equals a standalone run on its own grid
    alone, *_ = O.prefill_pipeline(q[:, :, cu[1]:cu[2]], k[:, :, cu[1]:cu[2]], v[:, :, cu[1]:cu[2]],
                                   iq[:, cu[1]:cu[2]], ik[:, cu[1]:cu[2]], *args)
    torch.testing.assert_close(out[:, :, cu[1]:cu[2]], alone)
