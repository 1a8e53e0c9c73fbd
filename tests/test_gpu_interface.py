"""Boundary cases of the reference's interface that go beyond one plain sequence, on the
GPU against the oracle:

* an additive padding mask in prefill, inference (_forward_dense, dash_attention.py:
  980-1006; _infer_prefill_attend, modeling_deepseekv2.py:403-421) and training
  (DashAttention.forward with autograd): left padding as per-row key starts, rows
  whose causal keys are all padding as the reference's uniform average;
* several decode rows per sequence (_decode_attend with q [B,H,Lq,D] and q_pos [B,Lq],
  modeling_deepseekv2.py:424-451), alone and through _dash_decode_forward;
* packed rows (position_ids restarting inside a row) at batch > 1 in
  triton_gather_attention (sparse_gather_triton.py:343-392), with gradients.
"""

import math
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from ananta_ocr_amd import dash_attention as DA
from ananta_ocr_amd import modeling_deepseekv2 as MD
from ananta_ocr_amd import sparse_gather as SG
from ananta_ocr_amd.dash_attention import apply_rotary
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(out, ref, what, tight=1.5e-2):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"{what}: {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, f"{what}: {err.max().item()}"


def _config(heads, bs, lb, budget=6, scale=128.0):
    sp = dict(sparse_block_size=bs, sparse_local_block=lb, dash_scaling_factor=scale,
              dash_prior_floor=1e-4, dash_sigma=1.0, dash_topk_blocks=budget,
              sparse_index_dim=128, dash_image_only=True)
    return SimpleNamespace(num_attention_heads=heads, num_key_value_heads=heads,
                           hidden_size=heads * 128, rms_norm_eps=1e-6,
                           sparse_attention_config=sp)


def _left_pad_mask(pads, S, fill):
    """HF-style [B, 1, S, S] additive mask: causal, keys before the row's padding end
    excluded (``fill``)."""
    i = torch.arange(S)
    m = torch.zeros(len(pads), 1, S, S)
    for b, p in enumerate(pads):
        bad = (i[None, :] > i[:, None]) | (i[None, :] < p)
        m[b, 0] = torch.where(bad, torch.full((), fill), torch.zeros(()))
    return m


@pytest.mark.parametrize("stage0,bs,lb,S,pads", [
    ("head_cls", 64, 4, 900, [0, 173]),
    ("indexer", 32, 4, 700, [300, 64]),
])
def test_prefill_padding_mask_matches_oracle(stage0, bs, lb, S, pads, monkeypatch):
    monkeypatch.setenv("DASH_STAGE0", stage0)
    torch.manual_seed(1)
    B, H = len(pads), 2
    mod = DA.DashAttention(_config(H, bs, lb)).eval().to(DEV)
    with torch.no_grad():
        mod.head_cls.normal_(0, 0.5)
    g = torch.Generator().manual_seed(2)
    hs = torch.randn(B, S, H * 128, generator=g)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    am = _left_pad_mask(pads, S, torch.finfo(torch.float32).min)
    pos = torch.arange(S)[None].expand(B, -1)
    layer = SimpleNamespace(layer_idx=0)
    with torch.no_grad():
        out = MD._infer_prefill_attend(layer, mod, hs.to(DEV), q.to(DEV), k.to(DEV),
                                       v.to(DEV), None, pos.to(DEV), None, am.to(DEV), None)
        iq, ik = mod.router_qk(hs.to(DEV))
        sc = mod.block_scores(iq, ik, q_pos=pos.to(DEV).to(torch.int32))
    p = mod._infer_params
    t_r, b_r, v_r = O.infer_route_select(sc.cpu(), None, p["idx_scale"], p["floor"],
                                         p["sigma"], p["K"], p["topm"])
    ref = O.dense_attend(q, k, v, t_r, b_r, v_r, bs, bs * lb, 1 / math.sqrt(128),
                         attention_mask=am)
    _close(out, ref, "padded prefill")
    # the padding rows are the mean of v over the whole sequence
    for b, pd in enumerate(pads):
        if pd:
            vm = v[b].float().mean(1)
            _close(out[b, :, :pd].float().cpu(), vm[:, None].expand(-1, pd, -1), "pad rows")
    # the attention mask of _unmask_unattended (padding rows opened to every key) and a
    # mask whose excluded entries are -1e4: the rows past the padding are the same
    am2 = _left_pad_mask(pads, S, -1e4)
    for b, pd in enumerate(pads):
        am2[b, 0, :pd] = 0.0
    with torch.no_grad():
        out2 = MD._infer_prefill_attend(layer, mod, hs.to(DEV), q.to(DEV), k.to(DEV),
                                        v.to(DEV), None, pos.to(DEV), None, am2.to(DEV), None)
    ref2 = O.dense_attend(q, k, v, t_r, b_r, v_r, bs, bs * lb, 1 / math.sqrt(128),
                          attention_mask=am2)
    _close(out2, ref2, "padded prefill, opened pad rows")


def test_training_forward_with_padding_mask(monkeypatch):
    """DashAttention.forward with a left-padding mask, gradients included, against the
    oracle chain (indexer stage 0, train_route_select, dense_attend with the mask)."""
    monkeypatch.setenv("DASH_STAGE0", "indexer")
    monkeypatch.setattr(DA.K_SCHEDULE, "k", 8)
    monkeypatch.setattr(DA.K_SCHEDULE, "advance", lambda sid, training: None)
    H, S, bs, lb, K = 2, 640, 64, 2, 8
    pads = [0, 150]
    B = len(pads)
    cfg = _config(H, bs, lb, scale=0.35)
    cfg.sparse_attention_config["dash_prior_floor"] = 1e-2
    cfg.sparse_attention_config["dash_image_only"] = False
    torch.manual_seed(3)
    mod = DA.DashAttention(cfg)
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        mod.q_proj.weight.normal_(0, 0.05, generator=g)
        mod.k_proj.weight.normal_(0, 0.05, generator=g)
    mod.train()
    hs = torch.randn(B, S, H * 128, generator=g)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    w = torch.randn(B, H, S, 128, generator=g)
    # the padding rows' upstream gradient is zero, as in a padded batch (their outputs
    # reach no loss); the reference's gradient through such a row is a rounding artefact
    for b, pd in enumerate(pads):
        w[b, :, :pd] = 0
    am = _left_pad_mask(pads, S, torch.finfo(torch.float32).min)
    mg = mod.to(DEV)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = mg(hs.to(DEV), qg, kg, vg, attention_mask=am.to(DEV))
    (out.float() * w.to(DEV)).sum().backward()
    got = {n: p.grad.detach().cpu() for n, p in mg.named_parameters() if p.grad is not None}

    mc = DA.DashAttention(cfg)
    mc.load_state_dict({n: t.cpu() for n, t in mg.state_dict().items()})
    iq, ik = mc._index_qk_train(hs, None)
    nblk = (S + bs - 1) // bs
    z = O.block_scores_indexer(iq, ik, torch.arange(S)[None].expand(B, -1), nblk, bs, bs * lb)
    idx_scale = 0.35 / math.sqrt(128)
    x, c = O.route_inputs(z.detach(), None, idx_scale)
    sp = O.entmax15(x).masked_fill(~c, -1.0)
    srt = torch.sort(sp, -1, descending=True).values
    a_, b_ = srt[..., K - 1], srt[..., K]
    assert not (((a_ - b_) > 0) & ((a_ - b_) < 1e-5)).any()
    topi, bias, valid = O.train_route_select(z, None, idx_scale, 1e-2, 1.0, K)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    ref = O.dense_attend(qr, kr, vr, topi, bias, valid, bs, bs * lb, 1 / math.sqrt(128),
                         attention_mask=am)
    (ref * w).sum().backward()
    o32 = out.detach().float().cpu()
    assert (o32 - ref.detach()).abs().max().item() <= 2e-2 * ref.abs().max().item() + 1e-3
    for gg, rr, what in ((qg.grad, qr.grad, "dq"), (kg.grad, kr.grad, "dk"),
                         (vg.grad, vr.grad, "dv")):
        err = (gg.float().cpu() - rr).abs().max().item()
        assert err <= 1.5e-2 * rr.abs().max().item() + 1e-6, f"{what}: {err:.3e}"
    ref_p = {n: p.grad for n, p in mc.named_parameters() if p.grad is not None}
    for n in ["q_proj.weight", "k_proj.weight"]:
        err = (got[n] - ref_p[n]).abs().max().item()
        assert err <= 5e-2 * ref_p[n].abs().max().item() + 1e-6, n


@pytest.mark.parametrize("paged", [False, True])
def test_decode_attend_several_rows(paged):
    g = torch.Generator().manual_seed(5)
    B, H, S, bs, lw, K, Lq = 2, 2, 1500, 64, 256, 6, 3
    q = (torch.randn(B, H, Lq, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    qp = torch.tensor([[S - 1, S - 2, 700], [5, 1200, S - 1]])
    nblk = (S + bs - 1) // bs
    topi = torch.randint(0, nblk, (B, Lq, K), generator=g)
    bias = torch.randn(B, Lq, K, generator=g)
    valid = torch.rand(B, Lq, K, generator=g) < 0.8
    ref = O.decode_attend(q, k, v, topi, bias, valid, qp, bs, lw, 0.1)
    if not paged:
        out = MD._decode_attend(q.to(DEV), k.to(DEV), v.to(DEV), topi.to(DEV), bias.to(DEV),
                                valid.to(DEV), qp.to(DEV), bs, lw, 0.1)
    else:
        from ananta_ocr_amd import ops
        P = nblk
        perm = torch.randperm(B * P, generator=g)
        table = perm.view(B, P).to(torch.int32)
        kc = torch.zeros(B * P, bs, H, 128, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        for b in range(B):
            for c in range(P):
                n = min(bs, S - c * bs)
                kc[table[b, c], :n] = k[b, :, c * bs:c * bs + n].transpose(0, 1)
                vc[table[b, c], :n] = v[b, :, c * bs:c * bs + n].transpose(0, 1)
        out = ops.attn_decode_rows(q.to(DEV), kc.to(DEV), vc.to(DEV), topi.to(DEV),
                                   bias.to(DEV), valid.to(DEV), qp.to(DEV), bs, lw, 0.1,
                                   seq_lens=torch.full((B,), S).to(DEV),
                                   block_table=table.to(DEV), page_size=bs)
    _close(out, ref, f"decode rows paged={paged}")


class _Cache:
    def __init__(self):
        self.k, self.v = {}, {}

    def update(self, k, v, li):
        if li in self.k:
            self.k[li] = torch.cat([self.k[li], k], 2)
            self.v[li] = torch.cat([self.v[li], v], 2)
        else:
            self.k[li], self.v[li] = k, v
        return self.k[li], self.v[li]

    def get_seq_length(self, li=0):
        return self.k[li].shape[2] if li in self.k else 0


class _Rope(nn.Module):
    def __init__(self, dim, theta=10000.0):
        super().__init__()
        self.inv = 1.0 / theta ** (torch.arange(0, dim, 2).float() / dim)

    def forward(self, x, position_ids):
        f = position_ids.float()[..., None] * self.inv.to(x.device)
        emb = torch.cat([f, f], -1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


@pytest.mark.parametrize("stage0,bs,lb,budget,S,chunks", [
    ("head_cls", 32, 4, 12, 1000, [3, 1, 40, 2]),     # the checkpoint's router; 40 rows
    ("indexer", 64, 2, 5, 600, [4, 70]),              # span three blocks
])
def test_decode_forward_several_rows(stage0, bs, lb, budget, S, chunks, monkeypatch):
    """_dash_decode_forward with q_len rows after an _infer_prefill_attend, against the
    oracle's decode step at position_ids [B, Lq] on the whole cache."""
    monkeypatch.setenv("DASH_STAGE0", stage0)
    torch.manual_seed(7)
    B, heads = 2, 2
    hidden = heads * 128
    cfg = _config(heads, bs, lb, budget)
    router = DA.DashAttention(cfg)
    with torch.no_grad():
        router.head_cls.normal_(0, 0.5)
    layer = SimpleNamespace(
        config=cfg, head_dim=128, layer_idx=1, dash_router=router.to(DEV).bfloat16(),
        indexer=None, main_rope_mode="1d",
        q_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        k_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        v_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        o_proj=nn.Identity(), rotary_emb=_Rope(128))
    decoder = nn.Module()
    decoder.router = router
    decoder.config = cfg
    MD.configure_dash_inference(decoder, True)
    p = router._infer_params
    scale = 1 / math.sqrt(128)
    total = S + sum(chunks)
    g = torch.Generator(device=DEV).manual_seed(8)
    hs = torch.randn(B, total, hidden, device=DEV, generator=g).bfloat16()
    cache = _Cache()

    def qkv(h, pos):
        L = h.shape[1]
        q = layer.q_proj(h).view(B, L, heads, 128).transpose(1, 2)
        k = layer.k_proj(h).view(B, L, heads, 128).transpose(1, 2)
        v = layer.v_proj(h).view(B, L, heads, 128).transpose(1, 2)
        cos, sin = layer.rotary_emb(v, pos)
        q, k = apply_rotary(q, k, cos, sin)
        return q, k, v, (cos, sin)

    with torch.no_grad():
        pos = torch.arange(S, device=DEV)[None].expand(B, -1)
        q, k, v, pe = qkv(hs[:, :S], pos)
        k_all, v_all = cache.update(k, v, layer.layer_idx)
        MD._infer_prefill_attend(layer, router, hs[:, :S], q, k_all, v_all, pe, pos, None,
                                 None, cache)
        t = S
        for L in chunks:
            pos_t = torch.arange(t, t + L, device=DEV)[None].expand(B, -1)
            out_t, _, _, _ = MD._dash_decode_forward(layer, hs[:, t:t + L], pos_t, cache)
            qd, _, _, pe_t = qkv(hs[:, t:t + L], pos_t)
            iq_t, _ = router.router_qk(hs[:, t:t + L], pe_t)
            ik_all = cache._dash_idx_k[layer.layer_idx]
            assert ik_all.shape[1] == t + L
            k_all, v_all = cache.k[layer.layer_idx], cache.v[layer.layer_idx]
            if stage0 == "head_cls":
                ref = O.decode_pipeline(qd.cpu(), k_all.cpu(), v_all.cpu(), iq_t.cpu(),
                                        ik_all.cpu(), router.head_cls.float().cpu(), bs, lb,
                                        p["idx_scale"], p["floor"], p["sigma"], p["K"],
                                        p["topm"], scale, q_pos=pos_t.cpu())[0]
            else:
                nblk = (t + L + bs - 1) // bs
                z = O.block_scores_indexer(iq_t.cpu(), ik_all.cpu(), pos_t.cpu(), nblk, bs,
                                           lb * bs)
                ti, bi, va = O.infer_route_select(z, None, p["idx_scale"], p["floor"],
                                                  p["sigma"], p["K"], p["topm"])
                ref = O.decode_attend(qd.cpu(), k_all.cpu(), v_all.cpu(), ti, bi, va,
                                      pos_t.cpu(), bs, lb * bs, scale)
            _close(out_t.view(B, L, heads, 128).transpose(1, 2), ref, f"decode rows t={t} L={L}")
            t += L
    MD.configure_dash_inference(decoder, False)


def test_gather_attention_packed_rows_batch_two():
    """Packed rows at batch 2 (each row with its own segments) in triton_gather_attention,
    output and gradients to q, k, v."""
    g = torch.Generator().manual_seed(9)
    B, H, bs, lw, K = 2, 2, 32, 96, 5
    T = 480
    segs = [[200, 150, 130], [480]]
    pos = torch.stack([torch.cat([torch.arange(L) for L in sg]) for sg in segs])
    q = (torch.randn(B, H, T, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, T, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, T, 128, generator=g).bfloat16()
    dout = torch.randn(B, H, T, 128, generator=g).bfloat16()
    nblk = (T + bs - 1) // bs
    sel = torch.randint(-1, nblk, (B, 1, T, K), generator=g, dtype=torch.int32)
    qg, kg, vg = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = SG.triton_gather_attention(qg, kg, vg, sel.to(DEV), pos.to(DEV), None, bs, 0.1, lw)
    out.backward(dout.to(DEV))
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    kmin = torch.arange(T)[None] - pos
    ref = O.dense_attend(qr, kr, vr, sel[:, 0].long(), torch.zeros(B, T, K), sel[:, 0] >= 0,
                         bs, lw, 0.1, kmin=kmin)
    ref.backward(dout.float())
    _close(out.detach(), ref.detach(), "gather packed batch 2")
    for got, want, what in ((qg.grad, qr.grad, "dq"), (kg.grad, kr.grad, "dk"),
                            (vg.grad, vr.grad, "dv")):
        err = (got.float().cpu() - want).abs().max().item()
        assert err <= 1.5e-2 * want.abs().max().item() + 1e-6, f"{what}: {err:.3e}"
