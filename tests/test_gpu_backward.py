"""Backward of the prefill attention (dash_attn_prefill_backward through the C ABI)
against a plain PyTorch fp32 reference of the same attention, differentiated by
autograd: dq, dk, dv and the routed slots' bias gradient.

The reference attends, for query t, the window keys (t - LW, t] with bias 0 and the
keys below t - LW + 1 of its routed blocks with the slot's bias (first valid slot of
a block; duplicates and invalid slots get no gradient), with softmax over those
keys -- the math of _forward_dense (dash_attention.py:980-1006) written with an
explicit softmax so that autograd reaches the bias.  Inputs are the bf16 values
upcast to fp32, so the comparison measures the kernels' bf16 operands (P and dS are
rounded to bf16 for the matrix cores) and fp32 accumulation.
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops
from ananta_ocr_amd import sparse_gather as SG
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ref(q, k, v, topi, bias, valid, bs, lw, scale, kmin=None):
    """fp32 [B,H,S,D] attention with the DASH key sets; differentiable in q, k, v, bias."""
    B, H, S, D = q.shape
    nblk = (S + bs - 1) // bs
    blk = O.dense_block_bias(topi, bias, valid, nblk)           # [B, S, nblk], scatter
    kidx = torch.arange(S)
    base = blk.index_select(-1, kidx // bs)                       # [B, S, S]
    t = kidx[:, None]
    causal = kidx[None, :] <= t
    local = causal & (kidx[None, :] > t - lw)
    keep = causal & (local[None] | (base > O.MASK_NEG * 0.5))
    if kmin is not None:
        keep = keep & (kidx[None, None, :] >= kmin[:, :, None])
    m = torch.where(local[None], torch.zeros_like(base), base)
    m = m.masked_fill(~keep, float("-inf"))
    s = torch.matmul(q, k.transpose(-1, -2)) * scale + m[:, None]
    return torch.matmul(torch.softmax(s, dim=-1), v)


def _close_grad(got, ref, what, frac=1.5e-2):
    got, ref = got.float().cpu(), ref.float().cpu()
    scale = ref.abs().max().item()
    err = (got - ref).abs()
    assert err.max().item() <= frac * scale + 1e-6, \
        f"{what}: max err {err.max().item():.3e} vs max |ref| {scale:.3e}"
    assert err.mean().item() <= 4e-3 * scale + 1e-7, f"{what}: mean err {err.mean().item():.3e}"


def _case(seed, B, H, S, bs, lw, K, dup=True):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.6).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.6).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    nblk = (S + bs - 1) // bs
    topi = torch.randint(0, nblk, (B, S, K), generator=g)
    if dup and K > 1:
        topi[:, ::5, 1] = topi[:, ::5, 0]                          # duplicated blocks
    bias = torch.randn(B, S, K, generator=g) * 0.7
    valid = torch.rand(B, S, K, generator=g) < 0.85
    dout = torch.randn(B, H, S, 128, generator=g).bfloat16()
    return q, k, v, topi, bias, valid, dout


@pytest.mark.parametrize("B,H,S,bs,lw,K", [
    (1, 2, 700, 64, 256, 6),
    (2, 2, 1000, 32, 128, 12),          # the shipped checkpoint's block 32, window 128, K 12
    (1, 3, 1300, 64, 512, 16),
    (1, 2, 333, 128, 200, 4),           # window not a block multiple, 128-key blocks
    (1, 2, 1200, 32, 128, 64),          # the training schedule's first k
    (1, 2, 900, 64, 256, 20),           # two slot groups, the last one partial
    (1, 2, 800, 96, 288, 8),            # 96-key blocks: key stages that span two blocks
    (1, 2, 1100, 256, 512, 4),          # 256-key blocks: four key stages per block
    (1, 1, 43, 128, 31, 4),             # routed last block whose second key stage is past the end
])
def test_backward_matches_torch_autograd(B, H, S, bs, lw, K):
    q, k, v, topi, bias, valid, dout = _case(10 + S + bs, B, H, S, bs, lw, K)
    scale = 1 / math.sqrt(128)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    br = bias.clone().requires_grad_()
    out_r = _ref(qr, kr, vr, topi, br, valid, bs, lw, scale)
    out_r.backward(dout.float())
    args = [t.to(DEV) for t in (q, k, v)]
    out, lse = ops.attn_prefill(*args, topi.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, scale,
                                return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), topi.to(DEV),
                                               bias.to(DEV), valid.to(DEV), bs, lw, scale)
    torch.cuda.synchronize()
    _close_grad(out, out_r.detach(), "out")
    _close_grad(dq, qr.grad, "dq")
    _close_grad(dk, kr.grad, "dk")
    _close_grad(dv, vr.grad, "dv")
    _close_grad(db, br.grad, "dbias")
    # slots that are not the first valid occurrence of their block get no gradient
    assert bool((db.cpu()[br.grad == 0] == 0).all())


@pytest.mark.parametrize("gscale", [1e6, 1e-6])
def test_backward_gradient_magnitudes(gscale):
    """Output gradients far from 1: the routed pairs' dQ partials pass through fp16 with a
    power-of-two scale per 32-dim piece, which must neither overflow (partials far above
    fp16's 65,504 at the large scale) nor lose the small ones to fp16's subnormal range."""
    B, H, S, bs, lw, K = 1, 2, 700, 64, 128, 8
    q, k, v, topi, bias, valid, dout = _case(91, B, H, S, bs, lw, K)
    dout = (dout.float() * gscale).bfloat16()
    scale = 1 / math.sqrt(128)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    br = bias.clone().requires_grad_()
    out_r = _ref(qr, kr, vr, topi, br, valid, bs, lw, scale)
    out_r.backward(dout.float())
    args = [t.to(DEV) for t in (q, k, v)]
    out, lse = ops.attn_prefill(*args, topi.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, scale,
                                return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), topi.to(DEV),
                                               bias.to(DEV), valid.to(DEV), bs, lw, scale)
    torch.cuda.synchronize()
    for got, ref, what in ((dq, qr.grad, "dq"), (dk, kr.grad, "dk"), (dv, vr.grad, "dv"),
                           (db, br.grad, "dbias")):
        assert torch.isfinite(got.float()).all(), what
        _close_grad(got, ref, what)


def test_backward_segment_starts():
    """kmin (packed segments inside one sequence, packing_patch.py): keys before a
    row's segment start are invisible to it, in the window and in routed blocks."""
    B, H, S, bs, lw, K = 1, 2, 1000, 64, 256, 8
    q, k, v, topi, bias, valid, dout = _case(77, B, H, S, bs, lw, K)
    starts = torch.tensor([0, 130, 131, 420, 777])
    kmin = torch.zeros(B, S, dtype=torch.int32)
    for s0, s1 in zip(starts.tolist(), starts.tolist()[1:] + [S]):
        kmin[:, s0:s1] = s0
    scale = 1 / math.sqrt(128)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    br = bias.clone().requires_grad_()
    out_r = _ref(qr, kr, vr, topi, br, valid, bs, lw, scale, kmin=kmin)
    out_r.backward(dout.float())
    args = [t.to(DEV) for t in (q, k, v)]
    km = kmin.to(DEV)
    out, lse = ops.attn_prefill(*args, topi.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, scale,
                                kmin=km, return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), topi.to(DEV),
                                               bias.to(DEV), valid.to(DEV), bs, lw, scale, kmin=km)
    torch.cuda.synchronize()
    _close_grad(out, out_r.detach(), "out")
    _close_grad(dq, qr.grad, "dq")
    _close_grad(dk, kr.grad, "dk")
    _close_grad(dv, vr.grad, "dv")
    _close_grad(db, br.grad, "dbias")


def test_backward_without_routing_is_sliding_window():
    q, k, v, _, _, _, dout = _case(3, 1, 2, 900, 64, 256, 1)
    scale = 1 / math.sqrt(128)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    none = torch.zeros(1, 900, 1, dtype=torch.long)
    out_r = _ref(qr, kr, vr, none, torch.zeros(1, 900, 1), torch.zeros(1, 900, 1, dtype=torch.bool),
                 64, 256, scale)
    out_r.backward(dout.float())
    args = [t.to(DEV) for t in (q, k, v)]
    out, lse = ops.attn_prefill(*args, None, None, None, 64, 256, scale, return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), None, None, None, 64,
                                               256, scale)
    assert db is None
    _close_grad(dq, qr.grad, "dq")
    _close_grad(dk, kr.grad, "dk")
    _close_grad(dv, vr.grad, "dv")


def test_backward_varlen_documents():
    """cu_seqlens: every document's gradients equal a standalone run's."""
    cu = [0, 400, 401, 401 + 777]
    T = cu[-1]
    q, k, v, topi, bias, valid, dout = _case(5, 1, 2, T, 64, 256, 6, dup=False)
    scale = 1 / math.sqrt(128)
    # per-document routing indices (each document on its own block grid)
    g = torch.Generator().manual_seed(6)
    for d0, d1 in zip(cu[:-1], cu[1:]):
        nb = (d1 - d0 + 63) // 64
        topi[:, d0:d1] = torch.randint(0, nb, (1, d1 - d0, 6), generator=g)
    args = [t.to(DEV) for t in (q, k, v)]
    cu_t = torch.tensor(cu, dtype=torch.int32, device=DEV)
    out, lse = ops.attn_prefill(*args, topi[0].to(DEV), bias[0].to(DEV), valid[0].to(DEV), 64, 256,
                                scale, cu_seqlens=cu_t, return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), topi[0].to(DEV),
                                               bias[0].to(DEV), valid[0].to(DEV), 64, 256, scale,
                                               cu_seqlens=cu_t)
    for d0, d1 in zip(cu[:-1], cu[1:]):
        sl = slice(d0, d1)
        qr, kr, vr = (t[:, :, sl].float().requires_grad_() for t in (q, k, v))
        br = bias[:, sl].clone().requires_grad_()
        out_r = _ref(qr, kr, vr, topi[:, sl], br, valid[:, sl], 64, 256, scale)
        out_r.backward(dout[:, :, sl].float())
        _close_grad(dq[:, :, sl], qr.grad, f"dq doc {d0}")
        _close_grad(dk[:, :, sl], kr.grad, f"dk doc {d0}")
        _close_grad(dv[:, :, sl], vr.grad, f"dv doc {d0}")
        _close_grad(db[sl][None], br.grad, f"dbias doc {d0}")


def test_gather_attention_e2e_autograd():
    """The reference's fused entry point with autograd: gradients reach q, k, v and the
    bias slots (blk_bias_slots), as _E2EGatherAttnFn's do."""
    B, H, S, bs, lw, K = 1, 2, 640, 64, 256, 6
    q, k, v, topi, bias, valid, dout = _case(8, B, H, S, bs, lw, K, dup=False)
    scale = 1 / math.sqrt(128)
    sel = topi.masked_fill(~valid, -1)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    br = bias.clone().requires_grad_()
    out_r = _ref(qr, kr, vr, topi, br, valid, bs, lw, scale)
    out_r.backward(dout.float())
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    bg = bias.to(DEV).requires_grad_()
    pos = torch.arange(S, device=DEV)[None]
    out = SG.triton_gather_attention_e2e(qg, kg, vg, sel[:, None].to(DEV).int(), bg, pos, None, bs,
                                         scale, lw)
    out.backward(dout.to(DEV))
    _close_grad(out.detach(), out_r.detach(), "out")
    _close_grad(qg.grad, qr.grad, "dq")
    _close_grad(kg.grad, kr.grad, "dk")
    _close_grad(vg.grad, vr.grad, "dv")
    _close_grad(bg.grad, br.grad, "dbias")
