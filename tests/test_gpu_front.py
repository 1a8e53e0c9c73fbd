"""Fused router front end (dash_router_front through the C ABI): projection, Gemma
RMSNorm, RoPE and guards against the oracle's router_qk; the block summaries against
the oracle's kbar_headcls on the kernel's own index keys, and the block scores of those
summaries against the oracle's block_scores_headcls.

Tolerance of idx_q / idx_k: the projection is rounded to bf16 as the bf16 linear layer
rounds it, from an fp32 accumulation whose order differs from the exact product's; a
value within that error of a rounding boundary rounds the other way, and the bf16
steps after it (the normed row, the RoPE products and sum) carry the difference as at
most a few bf16 ulps.  So: >= 98 % of the elements bit-equal to the oracle, and every
element within 2^-6 * (|ref| + 1).
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(seed, B, S, hid, cs_dtype=torch.bfloat16, cs_batch=1, nonfinite=False):
    g = torch.Generator().manual_seed(seed)
    hs = torch.randn(B, S, hid, generator=g).bfloat16()
    if nonfinite:
        hs[0, min(5, S - 1), 3] = float("nan")
        hs[-1, S // 2, 100] = float("inf")
        hs[-1, S - 1, 7] = -float("inf")
    w = (torch.randn(256, hid, generator=g) / math.sqrt(hid)).bfloat16()
    nq = torch.randn(128, generator=g) * 0.3
    nk = torch.randn(128, generator=g) * 0.3
    cos = sin = None
    if cs_dtype is not None:
        off = torch.randint(0, 5000, (cs_batch, 1, 1), generator=g).float()
        ang = (torch.arange(S)[None, :, None] + off) * \
            (5e5 ** (-torch.arange(0, 128, 2) / 128))[None, None]
        emb = torch.cat([ang, ang, ang[..., :16]], -1)          # [.., S, 144]: 128 used
        cos, sin = emb.cos().to(cs_dtype), emb.sin().to(cs_dtype)
    hc = torch.randn(128, generator=g) * 0.5
    return hs, w, nq, nk, cos, sin, hc


def _check_idx(got, ref, what):
    got = got.float().cpu()
    exact = (got == ref).float().mean().item()
    err = (got - ref).abs()
    tol = 2.0 ** -6 * (ref.abs() + 1.0)
    assert exact >= 0.98, f"{what}: only {exact:.4f} bit-equal"
    assert bool((err <= tol).all()), f"{what}: max err {err.max().item():.3e}"


def _run(hs, w, nq, nk, cos, sin, hc, bs, with_kbar=True):
    dv = lambda t: None if t is None else t.to(DEV)
    return ops.router_front(hs.to(DEV), w[:128].to(DEV), w[128:].to(DEV), nq.to(DEV), nk.to(DEV),
                            1e-6, dv(cos), dv(sin), head_cls=dv(hc) if with_kbar else None,
                            block_size=bs if with_kbar else None, want_q=True)


@pytest.mark.parametrize("B,S,hid,bs,lb,cs,cs_batch", [
    (1, 1000, 1280, 32, 4, torch.bfloat16, 1),     # the checkpoint's block 32, window 128
    (2, 777, 1280, 64, 2, torch.bfloat16, 2),      # per-sequence cos/sin, partial last tile
    (1, 37, 256, 32, 1, torch.float32, 1),         # one partial tile; fp32 cos/sin
    (2, 130, 512, 32, 1, None, 1),                 # no RoPE; own-tile blocks (bs * lb < 64)
    (1, 64, 1280, 64, 16, torch.bfloat16, 1),      # one full tile, nothing remote
])
def test_router_front_matches_oracle(B, S, hid, bs, lb, cs, cs_batch):
    hs, w, nq, nk, cos, sin, hc = _inputs(S + hid + bs, B, S, hid, cs, cs_batch, nonfinite=True)
    iq, ik, kb = _run(hs, w, nq, nk, cos, sin, hc, bs)
    torch.cuda.synchronize()
    rq, rk = O.router_qk(hs, w[:128], w[128:], nq, nk, 1e-6, cos, sin)
    _check_idx(iq, rq, "idx_q")
    _check_idx(ik, rk, "idx_k")
    # k_bar: the oracle's pooling of the kernel's own index keys
    kb_r, cv = O.kbar_headcls(ik.cpu(), hc, bs)
    torch.testing.assert_close(kb.cpu(), kb_r, atol=2e-5, rtol=2e-5)
    # the scores of the fused outputs against the oracle's
    z = ops.block_scores(iq, kb, bs, lb)
    pos = torch.arange(S)[None].expand(B, -1)
    z_r = O.block_scores_headcls(iq.cpu(), kb.cpu(), cv, pos, bs, lb)
    torch.testing.assert_close(z.cpu(), z_r, atol=1e-4, rtol=1e-4)


def test_router_front_nonfinite_hidden_rows():
    """Rows with nan / inf hidden states (the GEMM's non-finite rows, recomputed from the
    sanitized row): several in one tile, at both tile edges, a whole row of inf, and a
    row of huge finite values (its sum of squares overflows: the row norms to 0)."""
    hs, w, nq, nk, cos, sin, hc = _inputs(21, 1, 300, 1280)
    for r in (0, 1, 63, 64, 127, 200):
        hs[0, r, (r * 37) % 1280] = float("nan") if r % 2 else float("inf")
    hs[0, 150] = float("inf")
    hs[0, 151] = 1.0e30                                     # the sum of squares overflows
    iq, ik, kb = _run(hs, w, nq, nk, cos, sin, hc, 32)
    torch.cuda.synchronize()
    rq, rk = O.router_qk(hs, w[:128], w[128:], nq, nk, 1e-6, cos, sin)
    _check_idx(iq, rq, "idx_q")
    _check_idx(ik, rk, "idx_k")
    assert bool(torch.isfinite(iq).all()) and bool(torch.isfinite(kb).all())


def test_router_front_without_kbar_gives_the_same_index_keys():
    hs, w, nq, nk, cos, sin, hc = _inputs(3, 2, 300, 1280)
    iq, ik, kb = _run(hs, w, nq, nk, cos, sin, hc, 32)
    iq2, ik2, kb2 = _run(hs, w, nq, nk, cos, sin, hc, 32, with_kbar=False)
    assert kb2 is None
    assert torch.equal(iq, iq2) and torch.equal(ik, ik2)


def test_router_front_matches_unfused_router():
    """Against the GEMM + norm kernel path (the projection from the library GEMM):
    the same tolerance, as both round an fp32 accumulation to bf16."""
    hs, w, nq, nk, cos, sin, _ = _inputs(4, 1, 513, 1280)
    proj = torch.nn.functional.linear(hs.to(DEV), w.to(DEV))
    uq, uk = ops.router_qk_norm(proj, nq.to(DEV), nk.to(DEV), 1e-6, cos.to(DEV)[..., :128],
                                sin.to(DEV)[..., :128])
    iq, ik, _ = _run(hs, w, nq, nk, cos, sin, None, None, with_kbar=False)
    _check_idx(iq, uq.cpu(), "idx_q vs unfused")
    _check_idx(ik, uk.cpu(), "idx_k vs unfused")


@pytest.mark.parametrize("bs", [32, 64])
def test_router_front_full_size(bs):
    """27,300 tokens, hidden 1280 (427 tiles): k_bar against the standalone pooling
    kernel on the same index keys, and the index keys of a slice of rows against the
    oracle (the projection of 4,096 rows)."""
    S = 27300
    hs, w, nq, nk, cos, sin, hc = _inputs(11, 1, S, 1280)
    iq, ik, kb = _run(hs, w, nq, nk, cos, sin, hc, bs)
    kb_sa = ops.kbar(ik, hc.to(DEV), bs)
    torch.cuda.synchronize()
    torch.testing.assert_close(kb, kb_sa, atol=2e-5, rtol=2e-5)
    rq, rk = O.router_qk(hs[:, -4096:], w[:128], w[128:], nq, nk, 1e-6, cos[:, -4096:],
                         sin[:, -4096:])
    _check_idx(iq[:, -4096:], rq, "idx_q tail")
    _check_idx(ik[:, -4096:], rk, "idx_k tail")


def test_router_front_writes_into_decode_buffers():
    """idx_k and k_bar written into larger buffers (the decode cache's spare rows)."""
    hs, w, nq, nk, cos, sin, hc = _inputs(5, 2, 400, 1280)
    ikb = torch.full((2, 512, 128), 7.0, device=DEV)
    kbb = torch.full((2, 16, 128), 7.0, device=DEV)
    dv = lambda t: t.to(DEV)
    iq, ik, kb = ops.router_front(dv(hs), dv(w[:128]), dv(w[128:]), dv(nq), dv(nk), 1e-6,
                                  dv(cos), dv(sin), head_cls=dv(hc), block_size=32,
                                  idx_k_out=ikb, kbar_out=kbb, nblk_cap=16)
    iq2, ik2, kb2 = _run(hs, w, nq, nk, cos, sin, hc, 32)
    assert torch.equal(ik, ik2) and torch.equal(ikb[:, :400], ik2)
    assert bool((ikb[:, 400:] == 7.0).all()) and bool((kbb[:, 13:] == 7.0).all())
    assert torch.equal(kbb[:, :13], kb2)


def test_router_front_rejects_unsupported():
    hs, w, nq, nk, _, _, hc = _inputs(6, 1, 100, 1280)
    dv = lambda t: t.to(DEV)
    with pytest.raises(NotImplementedError):
        ops.router_front(dv(hs).float(), dv(w[:128]), dv(w[128:]), dv(nq), dv(nk), 1e-6)
    with pytest.raises(NotImplementedError):
        ops.router_front(dv(hs), dv(w[:128]), dv(w[128:]), dv(nq), dv(nk), 1e-6, head_cls=dv(hc),
                         block_size=128)
