"""Training routing (dash_train_route / dash_train_route_backward through the C ABI)
against the oracle's train_route_select (dash_attention.py:906-960) and its
autograd gradient (the entmax backward of dash_attention.py:650-658 with the
prior's gradient hook).

Indices and validity are compared exactly on rows whose masked prior has no
near-tie at the cut (the kernel's prior comes from a float64 threshold, the
oracle's from float32 cumulative sums, so values within ~1e-6 may swap); such
rows are compared as sets of near-equal values.  Bias and dz within tolerances
stated per test.
"""

import pytest
import torch

from ananta_ocr_amd import ops
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, B, S, nblk, bs, lb, scale_z, with_cand, nan_frac=0.0):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(B, S, nblk, generator=g) * scale_z
    t = torch.arange(S)[None, :, None]
    keep = torch.arange(nblk)[None, None, :] <= (t // bs - lb)
    z = z.masked_fill(~keep, O.SCORE_NEG)
    if nan_frac:
        m = torch.rand(B, S, nblk, generator=g) < nan_frac
        z = z.masked_fill(m & keep, float("nan"))
    cand = None
    if with_cand:
        cand = torch.rand(B, S, nblk, generator=g) < 0.4
        cand[:, ::7] = False
    return z, cand


def _masked_prior(z, cand, scale):
    x, c = O.route_inputs(z.float(), cand, scale)
    return O.entmax15(x, dim=-1).masked_fill(~c, -1.0)


def _check_forward(z, cand, scale, floor, sigma, K, got, bias_atol=1e-3):
    ti, bi, va = O.train_route_select(z, cand, scale, floor, sigma, K)
    gi, gb, gv = (t.cpu() for t in got)
    assert gi.shape == ti.shape
    sp = _masked_prior(z, cand, scale)
    Kp = ti.shape[-1]
    srt = torch.sort(sp, dim=-1, descending=True).values[..., :Kp + 1]
    # rows with no near-tie among the first K'+1 masked priors: adjacent values that
    # differ by less than 1e-5 without being equal, or a prior just inside the support
    # (exact ties, e.g. candidates at prior 0, go to the lower id on both sides)
    d = srt[..., :-1] - srt[..., 1:]
    near = ((d > 0) & (d < 1e-5)).any(-1) | ((srt > 0) & (srt < 1e-5)).any(-1)
    clean = ~near
    assert clean.float().mean() > 0.9
    assert torch.equal(gi.long()[clean], ti[clean])
    assert torch.equal(gv[clean], va[clean])
    torch.testing.assert_close(gb[clean], bi[clean], atol=bias_atol, rtol=1e-4)
    # near-tie rows: the selected masked priors agree as values
    vals_got = sp.gather(-1, gi.long().clamp_min(0))
    torch.testing.assert_close(torch.sort(vals_got, -1).values,
                               torch.sort(sp.gather(-1, ti), -1).values, atol=2e-5, rtol=0)
    return ti, bi, va


@pytest.mark.parametrize("B,S,nblk,scale,with_cand,K", [
    (2, 300, 43, 11.313708, False, 8),        # 128/sqrt(128): the configs' idx_scale
    (1, 400, 97, 40.0, True, 12),             # narrow support, candidate masks
    (1, 200, 60, 0.7, True, 16),              # wide support
    (1, 260, 130, 3.0, False, 64),            # the schedule's starting k
    (2, 90, 20, 11.313708, True, 33),         # K above the candidates: trailing non-candidates
    (1, 64, 2048, 5.0, False, 24),            # 2048 blocks (32 columns per lane)
    (1, 64, 700, 5.0, True, 1),
])
def test_train_route_forward_matches_oracle(B, S, nblk, scale, with_cand, K):
    # wide rows: row t has nblk - S + t + 1 remote blocks
    bs, lb = (1, S - nblk) if nblk > S // 2 else (4, 2)
    z, cand = _case(100 + nblk + K, B, S, nblk, bs, lb, 0.5, with_cand)
    got = ops.train_route_raw(z.to(DEV), None if cand is None else cand.to(DEV), scale, 1e-2,
                              1.0, K)
    _check_forward(z, cand, scale, 1e-2, 1.0, K, got[:3])
    # topv is the masked prior of each selected slot
    sp = _masked_prior(z, cand, scale)
    torch.testing.assert_close(got[3].cpu(), sp.gather(-1, got[0].cpu().long()), atol=2e-6,
                               rtol=1e-5)


def test_train_route_nonfinite_scores_and_empty_rows():
    """NaN scores are not remote (x -> -1e4); rows with no remote block are all invalid
    with bias 0; floor 1e-4 and sigma 0.5 reach the bias."""
    z, cand = _case(7, 1, 160, 40, 4, 2, 0.5, True, nan_frac=0.1)
    got = ops.train_route_raw(z.to(DEV), cand.to(DEV), 11.313708, 1e-4, 0.5, 8)
    _, bi, va = _check_forward(z, cand, 11.313708, 1e-4, 0.5, 8, got[:3], bias_atol=4e-3)
    empty = ~(z > O.SCORE_NEG * 0.5).any(-1)
    assert empty.any()
    assert not got[2].cpu()[empty].any()
    assert (got[1].cpu()[empty] == 0).all()


def test_train_route_row_nblk_is_the_truncated_row():
    """row_nblk[r] = n runs the row as if it had n columns."""
    z, cand = _case(9, 1, 120, 50, 2, 1, 0.5, False)
    g = torch.Generator().manual_seed(10)
    nb = torch.randint(1, 51, (120,), generator=g, dtype=torch.int32)
    got = ops.train_route_raw(z.to(DEV), None, 11.313708, 1e-2, 1.0, 6, row_nblk=nb.to(DEV))
    gi, gb, gv = (t.cpu()[0] for t in got[:3])
    for r in range(120):
        n = int(nb[r])
        zr = z[:, r:r + 1, :n]
        ti, bi, va = O.train_route_select(zr, None, 11.313708, 1e-2, 1.0, 6)
        kp = ti.shape[-1]
        sp = _masked_prior(zr, None, 11.313708)[0, 0]
        assert torch.allclose(torch.sort(sp[gi[r, :kp].long()]).values,
                              torch.sort(sp[ti[0, 0]]).values, atol=2e-5)
        assert torch.equal(gv[r, :kp], va[0, 0])
        assert (gi[r, kp:] == -1).all() and (gb[r, kp:] == 0).all()
        torch.testing.assert_close(torch.sort(gb[r, :kp]).values, torch.sort(bi[0, 0]).values,
                                   atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("nblk,scale,with_cand,K,floor", [
    (43, 11.313708, False, 8, 1e-2),
    (97, 40.0, True, 12, 1e-2),
    (60, 0.7, True, 16, 1e-4),
    (130, 3.0, False, 64, 1e-2),
])
def test_train_route_backward_matches_oracle_autograd(nblk, scale, with_cand, K, floor):
    """dz of the kernel pair against autograd through the oracle's forward (fp32),
    tolerance 2e-3 of the largest |dz| plus 1e-5."""
    z, cand = _case(200 + nblk, 1, 300, nblk, 4, 2, 0.5, with_cand)
    zr = z.clone().requires_grad_()
    ti, bi, va = O.train_route_select(zr, cand, scale, floor, 1.0, K)
    g = torch.Generator().manual_seed(nblk)
    dbias = torch.randn(bi.shape, generator=g)
    bi.backward(dbias)
    zd = z.to(DEV).requires_grad_()
    idx, bias, valid = ops.train_route(zd, None if cand is None else cand.to(DEV), scale, floor,
                                       1.0, K)
    # same selection as the oracle on the compared rows
    sp = _masked_prior(z, cand, scale)
    same = (idx.cpu().long() == ti).all(-1)
    assert same.float().mean() > 0.9
    bias.backward(dbias.to(DEV))
    got = zd.grad.cpu()
    ref = zr.grad
    tol = 2e-3 * ref.abs().max().item() + 1e-5
    err = (got - ref).abs()[same]
    assert err.max().item() <= tol, (err.max().item(), tol)
    # columns that are not candidates get no gradient
    x, c = O.route_inputs(z, cand, scale)
    assert (got[~c] == 0).all()
    assert sp.shape == z.shape


def test_train_route_autograd_equals_raw_backward():
    z, cand = _case(5, 2, 150, 40, 4, 2, 0.5, True)
    zd, cd = z.to(DEV), cand.to(DEV)
    zg = zd.clone().requires_grad_()
    idx, bias, valid = ops.train_route(zg, cd, 11.313708, 1e-2, 1.0, 8)
    dbias = torch.randn(bias.shape, device=DEV)
    bias.backward(dbias)
    i2, b2, v2, tv, st = ops.train_route_raw(zd, cd, 11.313708, 1e-2, 1.0, 8)
    dz = ops.train_route_backward(zd, cd, 11.313708, 1e-2, 1.0, i2, v2, tv, st, dbias)
    assert torch.equal(idx, i2) and torch.equal(valid, v2) and torch.equal(bias, b2)
    assert torch.equal(zg.grad, dz)


def test_train_route_rejects_k_above_64():
    z, _ = _case(1, 1, 16, 80, 1, 1, 0.5, False)
    with pytest.raises(NotImplementedError):
        ops.train_route_raw(z.to(DEV), None, 1.0, 1e-2, 1.0, 65)
