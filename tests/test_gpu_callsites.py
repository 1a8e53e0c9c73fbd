"""The reference's own call sequence through this library's functions: a prefill
through ``_infer_prefill_attend`` (modeling_deepseekv2.py:403-421, called from the
overlay's attention forward with the layer as ``self`` and the KV cache as
``past_kv``), then decode steps through ``_dash_decode_forward`` (:454-500) on the
same cache, with a stub layer and a stub cache that behave like the transformers
ones the overlay uses.  Each step is compared with the oracle run from scratch on
the whole cache (what the reference's decode step computes every step)."""

import math
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from ananta_ocr_amd import modeling_deepseekv2 as MD
from ananta_ocr_amd.dash_attention import DashAttention, apply_rotary
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(out, ref, what, tight=1.5e-2):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"{what}: {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, f"{what}: {err.max().item()}"


class _Cache:
    """transformers-style KV cache: update() appends along the token axis."""

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
    """1-D rotary embedding: (cos, sin) [B, L, D] for position_ids [B, L]."""

    def __init__(self, dim, theta=10000.0):
        super().__init__()
        self.inv = 1.0 / theta ** (torch.arange(0, dim, 2).float() / dim)

    def forward(self, x, position_ids):
        f = position_ids.float()[..., None] * self.inv.to(x.device)
        emb = torch.cat([f, f], -1)
        return emb.cos().to(x.dtype), emb.sin().to(x.dtype)


def _layer(stage0, bs, lb, budget, heads, layer_idx=3, seed=0):
    torch.manual_seed(seed)
    hidden = heads * 128
    sp = dict(sparse_block_size=bs, sparse_local_block=lb, dash_scaling_factor=128.0,
              dash_prior_floor=1e-4, dash_sigma=1.0, dash_topk_blocks=budget,
              sparse_index_dim=128, dash_stage0=stage0, dash_image_only=True)
    cfg = SimpleNamespace(num_attention_heads=heads, num_key_value_heads=heads,
                          hidden_size=hidden, rms_norm_eps=1e-6, sparse_attention_config=sp)
    router = DashAttention(cfg)
    with torch.no_grad():
        router.head_cls.normal_(0, 0.5)
        router.q_norm.weight.normal_(0, 0.1)
    layer = SimpleNamespace(
        config=cfg, head_dim=128, layer_idx=layer_idx, dash_router=router.to(DEV).bfloat16(),
        indexer=None, main_rope_mode="1d",
        q_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        k_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        v_proj=nn.Linear(hidden, hidden, bias=False).to(DEV).bfloat16(),
        o_proj=nn.Identity(), rotary_emb=_Rope(128))
    decoder = nn.Module()
    decoder.router = layer.dash_router
    decoder.config = cfg
    return layer, decoder


def _qkv(layer, hs, pos):
    """RoPE'd q, k and v of the layer, and the (cos, sin) the router also uses (the
    layer has no indexer RoPE of its own, so _dash_indexer_rope returns the main one)."""
    B, L, _ = hs.shape
    H = layer.config.num_attention_heads
    q = layer.q_proj(hs).view(B, L, H, 128).transpose(1, 2)
    k = layer.k_proj(hs).view(B, L, H, 128).transpose(1, 2)
    v = layer.v_proj(hs).view(B, L, H, 128).transpose(1, 2)
    cos, sin = layer.rotary_emb(v, pos)
    q, k = apply_rotary(q, k, cos, sin)
    return q, k, v, (cos, sin)


@pytest.mark.parametrize("stage0,bs,lb,budget,S,steps", [
    ("head_cls", 32, 4, 12, 1000, 40),      # the shipped checkpoint's router (config.json)
    ("head_cls", 64, 4, 6, 700, 70),        # crosses a block boundary and a buffer growth
    ("indexer", 64, 2, 5, 600, 5),
])
def test_prefill_then_decode_in_reference_call_order(stage0, bs, lb, budget, S, steps):
    B, heads = 2, 2
    layer, decoder = _layer(stage0, bs, lb, budget, heads)
    router = layer.dash_router
    state = MD.configure_dash_inference(decoder, True, topm=16)
    p = router._infer_params
    assert p["K"] == budget and p["topm"] == 16
    g = torch.Generator(device=DEV).manual_seed(11)
    hs = torch.randn(B, S + steps, heads * 128, device=DEV, generator=g).bfloat16()
    cache = _Cache()
    scale = 1.0 / math.sqrt(128)
    with torch.no_grad():
        # ---- prefill, as _dash_attn_forward calls it (cache updated first) ----
        pos = torch.arange(S, device=DEV)[None].expand(B, -1)
        q, k, v, pe = _qkv(layer, hs[:, :S], pos)
        k_all, v_all = cache.update(k, v, layer.layer_idx)
        out = MD._infer_prefill_attend(layer, router, hs[:, :S], q, k_all, v_all, pe, pos,
                                       None, None, cache)
        iq, ik = router.router_qk(hs[:, :S], pe)
        assert torch.equal(cache._dash_idx_k[layer.layer_idx], ik)
        if stage0 == "head_cls":
            ref = O.prefill_pipeline(q.cpu(), k.cpu(), v.cpu(), iq.cpu(), ik.cpu(),
                                     router.head_cls.float().cpu(), bs, lb, p["idx_scale"],
                                     p["floor"], p["sigma"], p["K"], p["topm"], scale)[0]
            _close(out, ref, "prefill")
        idx_keys = [ik]
        # ---- decode steps, as _patched_forward calls them (q_len == 1) ----
        for t in range(S, S + steps):
            pos_t = torch.full((B, 1), t, device=DEV)
            out_t, _, cache_out, _ = MD._dash_decode_forward(layer, hs[:, t:t + 1], pos_t,
                                                             cache)
            assert cache_out is cache
            qd, _, _, pe_t = _qkv(layer, hs[:, t:t + 1], pos_t)
            iq_t, ik_t = router.router_qk(hs[:, t:t + 1], pe_t)
            idx_keys.append(ik_t)
            ik_all = torch.cat(idx_keys, 1)
            assert torch.equal(cache._dash_idx_k[layer.layer_idx], ik_all)
            k_all, v_all = cache.k[layer.layer_idx], cache.v[layer.layer_idx]
            if (t - S) % 7 == 0 or t == S + steps - 1:
                if stage0 == "head_cls":
                    ref_t = O.decode_pipeline(qd.cpu(), k_all.cpu(), v_all.cpu(), iq_t.cpu(),
                                              ik_all.cpu(), router.head_cls.float().cpu(), bs,
                                              lb, p["idx_scale"], p["floor"], p["sigma"],
                                              p["K"], p["topm"], scale)[0]
                else:
                    nblk = (t + 1 + bs - 1) // bs
                    z = O.block_scores_indexer(iq_t.cpu(), ik_all.cpu(),
                                               torch.full((B, 1), t), nblk, bs, lb * bs)
                    ti, bi, va = O.infer_route_select(z, None, p["idx_scale"], p["floor"],
                                                      p["sigma"], p["K"], p["topm"])
                    ref_t = O.decode_attend(qd.cpu(), k_all.cpu(), v_all.cpu(), ti, bi, va,
                                            torch.full((B, 1), t), bs, lb * bs, scale)
                # out_t [B, 1, H*D] (o_proj = identity) vs the oracle's [B, H, 1, D]
                _close(out_t.view(B, 1, heads, 128).transpose(1, 2), ref_t, f"decode t={t}")
    MD.configure_dash_inference(decoder, False, state=state)
    assert not MD._INFER["on"]


def test_forward_triton_and_dense_match_reference_semantics():
    layer, _ = _layer("head_cls", 64, 4, 6, 2)
    router = layer.dash_router
    g = torch.Generator().manual_seed(4)
    B, H, S, K = 1, 2, 640, 6
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    topi = torch.randint(0, 10, (B, S, K), generator=g)
    bias = torch.randn(B, S, K, generator=g)
    valid = torch.rand(B, S, K, generator=g) < 0.7
    nblk = (S + 63) // 64
    ref = O.dense_attend(q, k, v, topi, bias, valid, 64, 256, 1 / math.sqrt(128))
    pos = torch.arange(S)[None]
    a = [t.to(DEV) for t in (q, k, v, topi, bias, valid)]
    with torch.no_grad():
        o1 = router._forward_triton(*a, S, nblk, pos.to(DEV))
        o2 = router._forward_dense(*a, S, nblk, None)
        _close(o1, ref, "_forward_triton")
        _close(o2, ref, "_forward_dense")
        # non-arange positions: the fused entry point declines, as the reference's does
        assert router._forward_triton(*a, S, nblk, (pos + 1).to(DEV)) is None
        # an all-open additive mask: the same attention; a mask with a hole is refused
        o3 = router._forward_dense(*a, S, nblk, torch.zeros(1, 1, S, S, device=DEV))
        _close(o3, ref, "_forward_dense, open mask")
        hole = torch.zeros(1, 1, S, S, device=DEV)
        hole[..., 5] = -1e30
        with pytest.raises(NotImplementedError):
            router._forward_dense(*a, S, nblk, hole)
        with pytest.raises(NotImplementedError):
            router(torch.zeros(B, S, 256, device=DEV), *a[:3], attention_mask=hole)


def test_decode_position_before_cache_end():
    """position_ids below the cache length (left-padded rows): window, causal limit and
    remote blocks follow the position, as in the reference's _decode_attend."""
    layer, decoder = _layer("head_cls", 64, 2, 4, 2, seed=3)
    router = layer.dash_router
    MD.configure_dash_inference(decoder, True)
    p = router._infer_params
    B, S = 2, 900
    g = torch.Generator(device=DEV).manual_seed(5)
    hs = torch.randn(B, S + 1, 256, device=DEV, generator=g).bfloat16()
    cache = _Cache()
    with torch.no_grad():
        pos = torch.arange(S, device=DEV)[None].expand(B, -1)
        q, k, v, pe = _qkv(layer, hs[:, :S], pos)
        k_all, v_all = cache.update(k, v, layer.layer_idx)
        MD._infer_prefill_attend(layer, router, hs[:, :S], q, k_all, v_all, pe, pos, None,
                                 None, cache)
        pos_t = torch.tensor([[S], [700]], device=DEV)
        out_t, _, _, _ = MD._dash_decode_forward(layer, hs[:, S:S + 1], pos_t, cache)
        qd, _, _, pe_t = _qkv(layer, hs[:, S:S + 1], pos_t)
        iq_t, ik_t = router.router_qk(hs[:, S:S + 1], pe_t)
        ik_all = cache._dash_idx_k[layer.layer_idx]
        assert torch.equal(ik_all[:, -1:], ik_t)
        k_all, v_all = cache.k[layer.layer_idx], cache.v[layer.layer_idx]
        ref = O.decode_pipeline(qd.cpu(), k_all.cpu(), v_all.cpu(), iq_t.cpu(), ik_all.cpu(),
                                router.head_cls.float().cpu(), 64, 2, p["idx_scale"],
                                p["floor"], p["sigma"], p["K"], p["topm"], 1 / math.sqrt(128),
                                q_pos=pos_t.cpu())[0]
    MD.configure_dash_inference(decoder, False)
    _close(out_t.view(B, 1, 2, 128).transpose(1, 2), ref, "decode at q_pos")
