"""The drop-in Python interfaces (DashAttention, the inference helpers and the
fused gather-attention entry points) against the CPU oracle."""

import math
from types import SimpleNamespace

import pytest
import torch

from ananta_ocr_amd import modeling_deepseekv2 as MD
from ananta_ocr_amd import sparse_gather as SG
from ananta_ocr_amd.dash_attention import DashAttention
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(out, ref, what, tight=1.5e-2):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"{what}: {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, f"{what}: {err.max().item()}"


def _config(stage0, bs=64, lb=4, budget=6, scale=128.0, hidden=256, heads=2):
    sp = dict(sparse_block_size=bs, sparse_local_block=lb, dash_scaling_factor=scale,
              dash_prior_floor=1e-4, dash_sigma=1.0, dash_topk_blocks=budget,
              sparse_index_dim=128, dash_stage0=stage0, dash_image_only=True)
    return SimpleNamespace(num_attention_heads=heads, hidden_size=heads * 128,
                           rms_norm_eps=1e-6, sparse_attention_config=sp)


@pytest.mark.parametrize("stage0", ["head_cls", "indexer"])
def test_dash_attention_forward_matches_oracle(stage0, monkeypatch):
    monkeypatch.setenv("DASH_STAGE0", stage0)
    torch.manual_seed(0)
    cfg = _config(stage0)
    mod = DashAttention(cfg).eval()
    with torch.no_grad():
        mod.head_cls.normal_(0, 0.5)
        mod.q_norm.weight.normal_(0, 0.1)
    B, S, H = 1, 900, 2
    g = torch.Generator().manual_seed(1)
    hs = torch.randn(B, S, cfg.hidden_size, generator=g)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    mod_gpu = mod.to(DEV)
    layer = SimpleNamespace(layer_idx=0)
    pos = torch.arange(S, device=DEV)[None]
    with torch.no_grad():
        out = MD._infer_prefill_attend(layer, mod_gpu, hs.to(DEV), q.to(DEV), k.to(DEV),
                                       v.to(DEV), None, pos, None, None, None)
        iq, ik = mod_gpu.router_qk(hs.to(DEV))
        sc = mod_gpu.block_scores(iq, ik)
        ti, bi, va = mod_gpu.route(sc)
    iq, ik, sc = iq.cpu(), ik.cpu(), sc.cpu()
    nblk = (S + 63) // 64
    pos = torch.arange(S)[None]
    if stage0 == "head_cls":
        kb, cv = O.kbar_headcls(ik, mod.head_cls.detach().cpu(), 64)
        sc_r = O.block_scores_headcls(iq, kb, cv, pos, 64, 4)
    else:
        sc_r = O.block_scores_indexer(iq, ik, pos, nblk, 64, 256)
    sent = sc_r < -5e8
    assert torch.equal(sc < -5e8, sent)
    torch.testing.assert_close(sc[~sent], sc_r[~sent], atol=2e-5, rtol=2e-5)
    p = mod._infer_params
    t_r, b_r, v_r = O.infer_route_select(sc, None, p["idx_scale"], p["floor"], p["sigma"],
                                         p["K"], p["topm"])
    assert torch.equal(ti.cpu().long(), t_r) and torch.equal(va.cpu(), v_r)
    ref = O.dense_attend(q, k, v, t_r, b_r, v_r, 64, 256, 1 / math.sqrt(128))
    _close(out, ref, f"DashAttention {stage0}")


def test_dash_attention_candidate_mask_and_errors():
    torch.manual_seed(2)
    cfg = _config("head_cls")
    mod = DashAttention(cfg).eval().to(DEV)
    B, S, H = 1, 700, 2
    hs = torch.randn(B, S, cfg.hidden_size, device=DEV)
    q = torch.randn(B, H, S, 128, device=DEV).bfloat16()
    k = torch.randn(B, H, S, 128, device=DEV).bfloat16()
    v = torch.randn(B, H, S, 128, device=DEV).bfloat16()
    nblk = (S + 63) // 64
    cand = torch.rand(B, S, nblk, device=DEV) < 0.5
    layer = SimpleNamespace(layer_idx=0)
    pos = torch.arange(S, device=DEV)[None]
    with torch.no_grad():
        out = MD._infer_prefill_attend(layer, mod, hs, q, k, v, None, pos, cand, None, None)
        iq, ik = mod.router_qk(hs)
        sc = mod.block_scores(iq, ik)
    p = mod._infer_params
    t_r, b_r, v_r = O.infer_route_select(sc.cpu(), cand.cpu(), p["idx_scale"], p["floor"],
                                         p["sigma"], p["K"], p["topm"])
    ref = O.dense_attend(q.cpu(), k.cpu(), v.cpu(), t_r, b_r, v_r, 64, 256, 1 / math.sqrt(128))
    _close(out, ref, "DashAttention block_cand")
    # an all-open additive mask is the plain path; a right-padded one (pad query rows
    # keep keys that are not a suffix of their causal range) is refused
    out_m = MD._infer_prefill_attend(layer, mod, hs, q, k, v, None, pos, cand,
                                     torch.zeros(1, 1, S, S, device=DEV), None)
    _close(out_m, ref, "DashAttention block_cand, open mask")
    i = torch.arange(S, device=DEV)
    right = torch.where((i[None, :] <= i[:, None]) & (i[None, :] < 600), 0.0, -1e30)
    with pytest.raises(NotImplementedError):
        MD._infer_prefill_attend(layer, mod, hs, q, k, v, None, pos, None,
                                 right[None, None], None)
    with pytest.raises(NotImplementedError):
        mod(hs, q, k, v, attention_mask=right[None, None])


def test_gather_attention_e2e_matches_oracle_and_returns_none():
    g = torch.Generator().manual_seed(3)
    B, H, T, bs, lw, K = 2, 2, 500, 64, 128, 5
    q = (torch.randn(B, H, T, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, T, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, T, 128, generator=g).bfloat16()
    nblk = (T + bs - 1) // bs
    sel = torch.randint(-1, nblk, (B, 1, T, K), generator=g, dtype=torch.int32)
    bias = torch.randn(B, T, K, generator=g)
    pos = torch.arange(T)[None].expand(B, -1)
    out = SG.triton_gather_attention_e2e(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV),
                                         bias.to(DEV), pos.to(DEV), None, bs, 0.1, lw)
    ref = O.dense_attend(q, k, v, sel[:, 0].long(), bias, sel[:, 0] >= 0, bs, lw, 0.1)
    _close(out, ref, "gather e2e")
    assert SG.triton_gather_attention_e2e(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV),
                                          bias.to(DEV), pos.to(DEV), torch.zeros(1, device=DEV),
                                          bs, 0.1, lw) is None
    assert SG.triton_gather_attention_e2e(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV),
                                          bias.to(DEV), (pos + 1).to(DEV), None, bs, 0.1,
                                          lw) is None


def test_gather_attention_packed_segments():
    g = torch.Generator().manual_seed(4)
    H, bs, lw, K = 2, 64, 128, 4
    lens = [300, 200, 150]
    T = sum(lens)
    pos = torch.cat([torch.arange(L) for L in lens])[None]
    q = (torch.randn(1, H, T, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(1, H, T, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(1, H, T, 128, generator=g).bfloat16()
    nblk = (T + bs - 1) // bs
    sel = torch.randint(-1, nblk, (1, 1, T, K), generator=g, dtype=torch.int32)
    out = SG.triton_gather_attention(q.to(DEV), k.to(DEV), v.to(DEV), sel.to(DEV), pos.to(DEV),
                                     None, bs, 0.1, lw)
    kmin = torch.arange(T)[None] - pos
    ref = O.dense_attend(q, k, v, sel[:, 0].long(), torch.zeros(1, T, K), sel[:, 0] >= 0, bs, lw,
                         0.1, kmin=kmin)
    _close(out, ref, "gather packed")


def test_gather_attention_index_heads_packed_with_gradients():
    """Several index heads (query head h reads index head h // (HQ / HI), with GQA kv
    heads), packed segments, and gradients to q, k, v against autograd through the
    oracle (the unbiased backward of _TritonGatherAttnFn)."""
    g = torch.Generator().manual_seed(6)
    HQ, Hkv, HI, bs, lw, K = 4, 2, 2, 32, 96, 5
    lens = [260, 333, 90]
    T = sum(lens)
    pos = torch.cat([torch.arange(L) for L in lens])[None]
    q = (torch.randn(1, HQ, T, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(1, Hkv, T, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(1, Hkv, T, 128, generator=g).bfloat16()
    dout = torch.randn(1, HQ, T, 128, generator=g).bfloat16()
    nblk = (T + bs - 1) // bs
    sel = torch.randint(-1, nblk, (1, HI, T, K), generator=g, dtype=torch.int32)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = SG.triton_gather_attention(qg, kg, vg, sel.to(DEV), pos.to(DEV), None, bs, 0.1, lw)
    out.backward(dout.to(DEV))
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    ke, ve = kr.repeat_interleave(HQ // Hkv, 1), vr.repeat_interleave(HQ // Hkv, 1)
    kmin = torch.arange(T)[None] - pos
    G = HQ // HI
    refs = []
    for hi in range(HI):
        hs = slice(hi * G, (hi + 1) * G)
        refs.append(O.dense_attend(qr[:, hs], ke[:, hs], ve[:, hs], sel[:, hi].long(),
                                   torch.zeros(1, T, K), sel[:, hi] >= 0, bs, lw, 0.1, kmin=kmin))
    ref = torch.cat(refs, 1)
    ref.backward(dout.float())
    _close(out.detach(), ref.detach(), "gather index heads")
    for got, want, what in ((qg.grad, qr.grad, "dq"), (kg.grad, kr.grad, "dk"),
                            (vg.grad, vr.grad, "dv")):
        err = (got.float().cpu() - want).abs().max().item()
        assert err <= 1.5e-2 * want.abs().max().item() + 1e-6, f"{what}: {err:.3e}"


def test_decode_attend_helper_matches_oracle():
    g = torch.Generator().manual_seed(5)
    B, H, S, bs, lw, K = 2, 2, 2000, 64, 512, 6
    q = (torch.randn(B, H, 1, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    qp = torch.tensor([[S - 1], [1500]])
    topi = torch.stack([torch.randperm(20, generator=g)[:K] for _ in range(B)])[:, None]
    bias = torch.randn(B, 1, K, generator=g)
    valid = torch.rand(B, 1, K, generator=g) < 0.8
    out = MD._decode_attend(q.to(DEV), k.to(DEV), v.to(DEV), topi.to(DEV), bias.to(DEV),
                            valid.to(DEV), qp.to(DEV), bs, lw, 0.1)
    ref = O.decode_attend(q, k, v, topi, bias, valid, qp, bs, lw, 0.1)
    _close(out, ref, "decode helper")


def _qk_norm_ref(x, w, eps, cos, sin):
    """Plain torch restatement of the router's index path for one side
    (GemmaRMSNorm dash_attention.py:680-700, rotate-half RoPE, finiteness guards),
    on the CPU in the projection's dtype."""
    x32 = torch.nan_to_num(x.float(), nan=0.0, posinf=0.0, neginf=0.0)
    x32 = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + eps)
    x32 = x32.clamp(-1e4, 1e4)
    y = (x32 * (1.0 + w.float())).clamp(-1e4, 1e4).to(x.dtype)
    if cos is not None:
        y1, y2 = y.chunk(2, dim=-1)
        y = y * cos + torch.cat((-y2, y1), dim=-1) * sin
    return torch.nan_to_num(y.float(), nan=0.0, posinf=0.0, neginf=0.0)


@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cdt", [None, torch.float32, torch.bfloat16])
def test_router_qk_norm_matches_torch(pdt, cdt):
    from ananta_ocr_amd import ops
    g = torch.Generator().manual_seed(7)
    B, S, d = 2, 301, 128
    proj = torch.randn(B, S, 2 * d, generator=g) * 3
    proj[0, 5, 7] = float("nan")
    proj[1, 9, 130] = float("inf")
    proj[0, 11] *= 1e6                                  # norm clamps
    proj = proj.to(pdt)
    wq = torch.randn(d, generator=g) * 0.3
    wk = torch.randn(d, generator=g) * 0.3
    cos = sin = None
    if cdt is not None:
        ang = torch.arange(S)[:, None] * (1e4 ** (-torch.arange(0, 160, 2) / 160))[None]
        emb = torch.cat([ang, ang], -1)                 # [S, 160]: the first d dims are used
        cos, sin = emb.cos()[None].to(cdt), emb.sin()[None].to(cdt)
    iq, ik = ops.router_qk_norm(proj.to(DEV), wq.to(DEV), wk.to(DEV), 1e-6,
                                None if cos is None else cos[..., :d].to(DEV),
                                None if sin is None else sin[..., :d].to(DEV))
    c = None if cos is None else cos[..., :d]
    s = None if sin is None else sin[..., :d]
    for side, (out, w) in enumerate(((iq, wq), (ik, wk))):
        ref = _qk_norm_ref(proj[..., side * d:(side + 1) * d], w, 1e-6, c, s)
        out = out.cpu()
        assert torch.isfinite(out).all()
        if pdt == torch.float32:
            torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
        else:
            # one bf16 rounding may flip on the ulp-level difference of the row norm
            err = (out - ref).abs()
            assert torch.all(err <= 2 ** -7 * ref.abs() + 1e-6), f"side {side}: {err.max().item()}"
            assert (err > 0).float().mean().item() < 0.01


def test_router_qk_fused_matches_unfused_module_path():
    torch.manual_seed(3)
    cfg = _config("head_cls")
    mod = DashAttention(cfg).eval().to(DEV)
    with torch.no_grad():
        mod.q_norm.weight.normal_(0, 0.2)
        mod.k_norm.weight.normal_(0, 0.2)
        hs = torch.randn(1, 257, cfg.hidden_size, device=DEV)
        iq, ik = mod.router_qk(hs)
        d = mod.index_dim
        hq = mod.q_norm(mod.q_proj(hs).view(1, 257, 1, d))[:, :, 0].float()
        hk = mod.k_norm(mod.k_proj(hs).view(1, 257, 1, d))[:, :, 0].float()
    torch.testing.assert_close(iq, hq, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(ik, hk, atol=2e-5, rtol=2e-5)
