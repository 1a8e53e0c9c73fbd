"""DashAttention.forward (the reference's training forward, dash_attention.py:1008-1071)
on the GPU, with autograd, against the oracle chain on the CPU in fp32: stage-0
scores (block_scores_indexer, or kbar_headcls + block_scores_headcls), the
training router (train_route_select, differentiable) and the dense attention
(dense_attend), differentiated by torch autograd.

Compared: the output, the gradients of q, k, v and of the router's parameters
(index projections, norm weights, head_cls), which reach them only through the
routed blocks' bias.  The router inputs use a wide entmax support (idx_scale well
below the checkpoint's) so that the masked priors have no near-ties: the test
asserts the gap, so that both sides select the same blocks.
"""

import math
from types import SimpleNamespace

import pytest
import torch

from ananta_ocr_amd import dash_attention as DA
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _config(H, bs, lb, stage0, scaling):
    sp = dict(sparse_block_size=bs, sparse_local_block=lb, dash_scaling_factor=scaling,
              dash_sigma=1.0, dash_prior_floor=1e-2, dash_image_only=False,
              sparse_index_dim=128)
    return SimpleNamespace(num_attention_heads=H, hidden_size=H * 128, rms_norm_eps=1e-6,
                           sparse_attention_config=sp)


def _rope(B, S, d, g):
    inv = 1.0 / (10000 ** (torch.arange(0, d, 2).float() / d))
    ang = torch.arange(S).float()[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)[None].expand(B, -1, -1)
    return emb.cos().contiguous(), emb.sin().contiguous()


def _grad_close(got, ref, what, frac):
    got, ref = got.float().cpu(), ref.float().cpu()
    scale = ref.abs().max().item()
    err = (got - ref).abs().max().item()
    assert err <= frac * scale + 1e-6, f"{what}: max err {err:.3e} vs max |ref| {scale:.3e}"


@pytest.mark.parametrize("stage0,H,S,bs,lb,K", [
    ("indexer", 2, 700, 64, 2, 8),
    ("head_cls", 2, 1200, 32, 4, 64),      # k above 16: the block-major path, 38 blocks
])
def test_training_forward_and_gradients_match_oracle(stage0, H, S, bs, lb, K, monkeypatch):
    # the schedule is global (its clock follows the first layer created in the
    # process): pin its k for this test
    monkeypatch.setattr(DA.K_SCHEDULE, "k", K)
    monkeypatch.setattr(DA.K_SCHEDULE, "advance", lambda sid, training: None)
    monkeypatch.setenv("DASH_STAGE0", stage0)          # read by the constructor only
    g = torch.Generator().manual_seed(S + bs)
    cfg = _config(H, bs, lb, stage0, scaling=0.35)
    torch.manual_seed(S)
    mod = DA.DashAttention(cfg)
    with torch.no_grad():
        mod.q_proj.weight.normal_(0, 0.05, generator=g)
        mod.k_proj.weight.normal_(0, 0.05, generator=g)
        mod.q_norm.weight.normal_(0, 0.2, generator=g)
        mod.k_norm.weight.normal_(0, 0.2, generator=g)
        mod.head_cls.normal_(0, 1.0, generator=g)
    mod.train()
    B = 1
    hs = torch.randn(B, S, H * 128, generator=g)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    w = torch.randn(B, H, S, 128, generator=g)
    cos, sin = _rope(B, S, 128, g)

    # ---- GPU: the module ----
    mg = mod.to(DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = mg(hs.to(DEV), qg, kg, vg, position_embeddings=(cos.to(DEV), sin.to(DEV)))
    (out.float() * w.to(DEV)).sum().backward()
    got = {n: p.grad.detach().cpu() for n, p in mg.named_parameters() if p.grad is not None}

    # ---- CPU: the oracle chain in fp32 ----
    mc = DA.DashAttention(cfg)
    mc.load_state_dict({n: t.cpu() for n, t in mg.state_dict().items()})
    iq, ik = mc._index_qk_train(hs, (cos, sin))
    nblk = (S + bs - 1) // bs
    pos = torch.arange(S)[None]
    if stage0 == "head_cls":
        kbar, cv = O.kbar_headcls(ik, mc.head_cls, bs)
        z = O.block_scores_headcls(iq, kbar, cv, pos, bs, lb)
    else:
        z = O.block_scores_indexer(iq, ik, pos, nblk, bs, bs * lb)
    idx_scale = 0.35 / math.sqrt(128)
    Kp = min(K, nblk)
    # no near-tie at the cut of the masked prior: both sides select the same set
    if Kp < nblk:
        x, c = O.route_inputs(z.detach(), None, idx_scale)
        sp = O.entmax15(x).masked_fill(~c, -1.0)
        srt = torch.sort(sp, -1, descending=True).values
        a, b = srt[..., Kp - 1], srt[..., Kp]
        assert not (((a - b) > 0) & ((a - b) < 1e-5)).any()
        assert not (((b > 0) & (b < 1e-5)) | ((a > 0) & (a < 1e-5))).any()
    topi, bias, valid = O.train_route_select(z, None, idx_scale, 1e-2, 1.0, Kp)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    ref = O.dense_attend(qr, kr, vr, topi, bias, valid, bs, bs * lb, 1 / math.sqrt(128))
    (ref * w).sum().backward()

    o32 = out.detach().float().cpu()
    assert (o32 - ref.detach()).abs().max().item() <= 2e-2 * ref.abs().max().item() + 1e-3
    _grad_close(qg.grad, qr.grad, "dq", 1.5e-2)
    _grad_close(kg.grad, kr.grad, "dk", 1.5e-2)
    _grad_close(vg.grad, vr.grad, "dv", 1.5e-2)
    ref_p = {n: p.grad for n, p in mc.named_parameters() if p.grad is not None}
    names = ["q_proj.weight", "k_proj.weight", "q_norm.weight", "k_norm.weight"]
    if stage0 == "head_cls":
        names.append("head_cls")
    for n in names:
        assert n in got and n in ref_p, n
        assert ref_p[n].abs().max() > 0, n
        _grad_close(got[n], ref_p[n], n, 5e-2)


def test_training_forward_rejects_unsupported_attention_mask():
    """A right-padded mask (pad query rows keep keys [0, len), not a suffix of their
    causal range) is refused before any kernel runs."""
    mod = DA.DashAttention(_config(2, 64, 2, "indexer", 1.0)).to(DEV)
    q = torch.zeros(1, 2, 128, 128, dtype=torch.bfloat16, device=DEV)
    i = torch.arange(128, device=DEV)
    right = torch.where((i[None, :] <= i[:, None]) & (i[None, :] < 100), 0.0, -1e30)
    with pytest.raises(NotImplementedError):
        mod(torch.zeros(1, 128, 256, device=DEV), q, q, q, attention_mask=right[None, None])
