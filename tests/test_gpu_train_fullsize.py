"""The training step the benchmark times (train_s27300_lw1024_k16: one sequence of
27,300 tokens, 10 heads, block 64, window 1,024, k = 16, 427 blocks), at that size, on
the GPU against the oracle:

* training routing of the block scores (dash_train_route; dash_attention.py:906-960):
  ids, validity and bias (1e-3) slot for slot on every row whose top-K+1 masked priors
  are separated by more than 1e-7, as sets on every row whose cut is, and the selected
  priors equal as values on every row;
* attention forward and backward (dash_attn_prefill / dash_attn_prefill_backward; the
  routed pairs of the forward split between the tile kernel's dense blocks and the
  block-major path, the backward's all block-major) against torch autograd of the
  oracle's explicit-softmax attention (dense_attend, fp32) on a sample of query rows:
  the upstream gradient is zero outside the sample, so the full-size dq, dk, dv and
  bias gradient equal the reference's over the sampled rows alone, and dk / dv are
  compared on every key;
* routing backward to the scores (dash_train_route_backward) against autograd through
  the oracle's training routing, on the rows both select alike.

Tolerances (bf16 operands, fp32 accumulation): outputs 2e-2 abs / 1e-2 rel per element
and 1.5 % of the output scale; gradients the same 1.5 % of each gradient's largest
magnitude (max) and 0.3 % of its mean magnitude (mean); routing gradient 2e-3 of its
scale.
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops
from ananta_ocr_amd import workloads as W
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
GRAD_MAX = 1.5e-2
GRAD_MEAN = 3e-3


def _rows_sample(S):
    """Contiguous query ranges: the last 512 rows and four 128-row ranges spread over the
    sequence (early rows with a short remote range, middle, late)."""
    return [(1100, 1228), (9000, 9128), (17000, 17128), (23500, 23628), (S - 512, S)]


def _masked_prior(z, scale):
    x, c = O.route_inputs(z.float(), None, scale)
    return O.entmax15(x, dim=-1).masked_fill(~c, -1.0)


def test_training_step_at_benchmark_size():
    cfg = W.PREFILL_27300
    d = W.make_prefill(cfg)
    S, K, bs, lw = d["S"], cfg.cap, cfg.bs, cfg.lw
    lb = lw // bs
    nblk = (S + bs - 1) // bs
    assert (S, K, nblk) == (27300, 16, 427)
    scale = 1.0 / math.sqrt(W.D)
    q, k, v = (d[n].to(DEV) for n in ("q", "k", "v"))
    hc = torch.zeros(W.D, device=DEV)
    kb = ops.kbar(d["idx_k"].to(DEV), hc, bs)
    z = ops.block_scores(d["idx_q"].to(DEV), kb, bs, lb)

    # ---- training routing at full size ----
    idx, bias, valid, topv, stat = ops.train_route_raw(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, K)
    zc = z.cpu()
    ti, bi, va = O.train_route_select(zc, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, K)
    gi, gb, gv = idx.cpu().long(), bias.cpu(), valid.cpu()
    sp = _masked_prior(zc, W.IDX_SCALE)
    srt = torch.sort(sp, dim=-1, descending=True).values[..., :K + 1]
    # at this size the priors are near 1/400 each and adjacent ones often lie within
    # 1e-6 of each other; the two sides' priors agree to ~1e-9 (fp32 cumulative sums
    # against a float64 threshold), so a gap above 1e-7 decides the order
    dd = srt[..., :-1] - srt[..., 1:]
    sep = (dd > 1e-7) | (dd == 0)
    cut = sep[..., K - 1]                       # the selected set is decided
    order = sep[..., :K].all(-1)                # ... and so is the slot order
    print(f"routing: set decided on {int(cut.sum())}, order on {int(order.sum())} of "
          f"{cut.numel()} rows", flush=True)
    assert cut.float().mean() > 0.9 and order.float().mean() > 0.3
    assert torch.equal(gi[order], ti[order]) and torch.equal(gv[order], va[order])
    torch.testing.assert_close(gb[order], bi[order], atol=1e-3, rtol=1e-4)
    # rows whose set is decided: the same (block, validity, bias) slots in any order
    key_g, pg = torch.sort(gi, -1)
    key_t, pt = torch.sort(ti, -1)
    assert torch.equal(key_g[cut], key_t[cut])
    assert torch.equal(gv.gather(-1, pg)[cut], va.gather(-1, pt)[cut])
    torch.testing.assert_close(gb.gather(-1, pg)[cut], bi.gather(-1, pt)[cut], atol=1e-3,
                               rtol=1e-4)
    # every row: the selected priors agree as values
    vals_got = sp.gather(-1, gi.clamp_min(0))
    torch.testing.assert_close(torch.sort(vals_got, -1).values,
                               torch.sort(sp.gather(-1, ti), -1).values, atol=1e-6, rtol=0)

    # ---- attention forward and backward, upstream gradient on the sampled rows ----
    out, lse = ops.attn_prefill(q, k, v, idx, bias, valid, bs, lw, scale, return_lse=True)
    ranges = _rows_sample(S)
    g = torch.Generator().manual_seed(12)
    dout = torch.zeros(1, W.H, S, W.D)
    for r0, r1 in ranges:
        dout[:, :, r0:r1] = torch.randn(1, W.H, r1 - r0, W.D, generator=g)
    dout = dout.bfloat16()
    dq, dk, dv, db = ops.attn_prefill_backward(q, k, v, out, lse, dout.to(DEV), idx, bias,
                                               valid, bs, lw, scale)
    torch.cuda.synchronize()
    qr, kr, vr = (t.float().requires_grad_() for t in (d["q"], d["k"], d["v"]))
    br = gb.clone().requires_grad_()
    for r0, r1 in ranges:
        ref = O.dense_attend(qr, kr, vr, gi, br, gv, bs, lw, scale, q_chunk=128, rows=(r0, r1))
        got = out[:, :, r0:r1].float().cpu()
        err = (got - ref.detach()).abs()
        assert torch.all(err <= 2e-2 + 1e-2 * ref.detach().abs()), (r0, err.max().item())
        assert err.max().item() <= 1.5e-2 * ref.detach().abs().max().item(), (r0, err.max())
        (ref * dout[:, :, r0:r1].float()).sum().backward()
    sample = torch.zeros(S, dtype=torch.bool)
    for r0, r1 in ranges:
        sample[r0:r1] = True
    assert (dq.cpu()[:, :, ~sample] == 0).all()
    assert (db.cpu()[:, ~sample] == 0).all()
    for got, want, what in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv"),
                            (db, br.grad, "dbias")):
        got = got.float().cpu()
        scale_ = want.abs().max().item()
        err = (got - want).abs()
        print(f"{what}: max err {err.max().item():.3e} ({err.max().item() / scale_:.4f} of "
              f"scale), mean {err.mean().item() / want.abs().mean().item():.4f} of the mean",
              flush=True)
        assert err.max().item() <= GRAD_MAX * scale_ + 1e-6, what
        # the absolute slack is far below the bar: the gradients' mean magnitudes here
        # are ~1e-5 .. 1e-3, so a slack of 1e-7 would be ~1 % of them
        assert err.mean().item() <= GRAD_MEAN * want.abs().mean().item() + 1e-10, what

    # ---- routing backward to the scores, on rows whose selected set both sides share ----
    dz = ops.train_route_backward(z, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, idx, valid, topv, stat,
                                  db).cpu()
    zr = zc.clone().requires_grad_()
    _, bi2, _ = O.train_route_select(zr, None, W.IDX_SCALE, W.FLOOR, W.SIGMA, K)
    # the bias gradient of each oracle slot: that of the kernel's slot holding its block
    dbc = db.cpu()
    match = (ti[..., :, None] == gi[..., None, :]).float()
    bi2.backward((match * dbc[..., None, :]).sum(-1))
    rows = (key_g == key_t).all(-1)[0] & sample
    assert rows.sum() > 0.9 * sample.sum()
    ref = zr.grad[0][rows]
    err = (dz[0][rows] - ref).abs()
    assert err.max().item() <= 2e-3 * ref.abs().max().item() + 1e-5, err.max().item()
