"""Router configuration at the module boundary, on the CPU (no kernels run).

* Stage 0 of the training forward comes from DASH_STAGE0 only, default "indexer"
  (dash_attention.py:748), whatever the checkpoint's dash_stage0 says.
* configure_dash_inference takes DASH_STAGE0 first, then the checkpoint's dash_stage0,
  then "indexer" (modeling_deepseekv2.py:285), reading the checkpoint's copy of the
  config, not what the routers wrote into it.
* The first router writes its live parameters into sparse_attention_config
  (_persist_router_cfg, dash_attention.py:761-774) at construction and in forward.

The checkpoint's sparse_attention_config is the committed fixture
tests/golden/checkpoint_sparse_config.json (values of the reference's config.json).
"""

import copy
import json
import math
import os
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from ananta_ocr_amd import dash_attention as DA
from ananta_ocr_amd import modeling_deepseekv2 as MD

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "checkpoint_sparse_config.json")


def _shipped():
    with open(GOLDEN) as f:
        c = json.load(f)
    sp = copy.deepcopy(c["sparse_attention_config"])
    cfg = SimpleNamespace(num_attention_heads=c["num_attention_heads"],
                          hidden_size=c["hidden_size"], rms_norm_eps=c["rms_norm_eps"],
                          sparse_attention_config=sp)
    return cfg, c


def _decoder(cfg, n_layers):
    """A decoder shaped like DeepseekV2Model: layers[i].self_attn.dash_router."""
    dec = nn.Module()
    dec.config = cfg
    dec.layers = nn.ModuleList()
    for i in range(n_layers):
        layer = nn.Module()
        layer.self_attn = nn.Module()
        layer.self_attn.layer_idx = i
        layer.self_attn.dash_router = DA.DashAttention(cfg)
        dec.layers.append(layer)
    return dec


@pytest.fixture
def fresh_schedule(monkeypatch):
    """A fresh global k schedule (its leader is the first router made in the test)."""
    monkeypatch.setattr(DA, "K_SCHEDULE", DA.KSchedule())
    return DA.K_SCHEDULE


def test_shipped_config_trains_with_indexer_stage0_unless_env(monkeypatch, fresh_schedule):
    monkeypatch.delenv("DASH_STAGE0", raising=False)
    cfg, raw = _shipped()
    assert raw["sparse_attention_config"]["dash_stage0"] == "head_cls"
    mod = DA.DashAttention(cfg)
    assert mod.stage0 == "indexer"
    monkeypatch.setenv("DASH_STAGE0", "HEAD_CLS")
    cfg2, _ = _shipped()
    assert DA.DashAttention(cfg2).stage0 == "head_cls"
    monkeypatch.setenv("DASH_STAGE0", "")             # set but empty: not head_cls
    cfg3, _ = _shipped()
    assert DA.DashAttention(cfg3).stage0 == ""


def test_configure_inference_stage0_order(monkeypatch, fresh_schedule):
    monkeypatch.delenv("DASH_STAGE0", raising=False)
    cfg, raw = _shipped()
    dec = _decoder(cfg, 3)
    routers = [l.self_attn.dash_router for l in dec.layers]
    assert all(r.stage0 == "indexer" for r in routers)
    # the constructor wrote its stage 0 into the live config; the checkpoint's copy wins
    assert cfg.sparse_attention_config["dash_stage0"] == "indexer"
    state = MD.configure_dash_inference(dec, True, topm=16)
    assert all(r.stage0 == "head_cls" for r in routers)
    sp = raw["sparse_attention_config"]
    for r in routers:
        p = r._infer_params
        assert p["K"] == sp["dash_topk_blocks"] == 12 and p["topm"] == 16
        assert p["idx_scale"] == 128.0 / math.sqrt(128) and p["floor"] == 1e-4
        assert p["sigma"] == 1.0
    MD.configure_dash_inference(dec, False, state=state)
    assert all(r.stage0 == "indexer" for r in routers)
    # the environment variable wins over the checkpoint
    monkeypatch.setenv("DASH_STAGE0", "indexer")
    MD.configure_dash_inference(dec, True)
    assert all(r.stage0 == "indexer" for r in routers)
    # with neither, "indexer"
    monkeypatch.delenv("DASH_STAGE0")
    cfg4, _ = _shipped()
    del cfg4.sparse_attention_config["dash_stage0"]
    dec4 = _decoder(cfg4, 1)
    MD.configure_dash_inference(dec4, True)
    assert dec4.layers[0].self_attn.dash_router.stage0 == "indexer"
    MD.configure_dash_inference(dec4, False)


def test_configure_inference_per_layer_slots(monkeypatch, fresh_schedule):
    """Per-layer arrays are indexed by the layer's count among the sparse layers of
    sparse_attention_freq (modeling_deepseekv2.py:256-266)."""
    monkeypatch.delenv("DASH_STAGE0", raising=False)
    cfg, _ = _shipped()
    sp = cfg.sparse_attention_config
    dec = _decoder(cfg, 4)
    ck = DA.checkpoint_sparse_config(sp)
    ck["sparse_attention_freq"] = [0, 1, 0, 1]
    ck["dash_scale_per_layer"] = [10.0, 20.0]
    ck["dash_floor_per_layer"] = [1e-3, 2e-3]
    MD.configure_dash_inference(dec, True)
    got = [(l.self_attn.dash_router._infer_params["idx_scale"] * math.sqrt(128),
            l.self_attn.dash_router._infer_params["floor"]) for l in dec.layers]
    # layer 0 -> slot 0, 1 -> 0, 2 -> 1, 3 -> 1
    assert [round(a, 6) for a, _ in got] == [10.0, 10.0, 20.0, 20.0]
    assert [b for _, b in got] == [1e-3, 1e-3, 2e-3, 2e-3]
    # no freq array: the slot is the layer index; past the array's end, the scalar
    del ck["sparse_attention_freq"]
    MD.configure_dash_inference(dec, True)
    got = [l.self_attn.dash_router._infer_params["floor"] for l in dec.layers]
    assert got == [1e-3, 2e-3, ck["dash_prior_floor"], ck["dash_prior_floor"]]
    MD.configure_dash_inference(dec, False)


def test_persist_router_cfg_writes_leader_parameters(monkeypatch, fresh_schedule):
    monkeypatch.delenv("DASH_STAGE0", raising=False)
    sp = dict(sparse_block_size=64, sparse_local_block=4, dash_scaling_factor=0.7,
              dash_prior_floor=3e-3, dash_sigma=2.0, sparse_index_dim=128)
    cfg = SimpleNamespace(num_attention_heads=2, hidden_size=256, rms_norm_eps=1e-6,
                          sparse_attention_config=sp)
    a = DA.DashAttention(cfg)
    assert sp["dash_stage0"] == "indexer"
    assert sp["dash_router"] == "entmax_topk_perlayer"
    assert sp["dash_sigma"] == 2.0 and sp["dash_prior_floor"] == 3e-3
    assert sp["dash_topk_blocks"] == fresh_schedule.k == 64
    assert sp["dash_scaling_factor"] == 0.7 / math.sqrt(128) * math.sqrt(128)
    assert sp["dash_scale_per_layer"] == [0.7] and sp["dash_floor_per_layer"] == [3e-3]
    # a second router: not the leader, writes nothing; the leader's next write lists both
    sp2 = dict(sp, dash_scaling_factor=5.0)
    cfg2 = SimpleNamespace(num_attention_heads=2, hidden_size=256, rms_norm_eps=1e-6,
                           sparse_attention_config=sp2)
    DA.DashAttention(cfg2)
    assert sp2["dash_scale_per_layer"] == [0.7]          # copied from sp, untouched
    fresh_schedule.k = 17
    a._persist_router_cfg()
    assert sp["dash_topk_blocks"] == 17
    assert sp["dash_scale_per_layer"] == [0.7, 0.7] and len(sp["dash_floor_per_layer"]) == 2
    # the checkpoint's copy is the dict as it was before the first write
    assert "dash_router" not in DA.checkpoint_sparse_config(sp)
    # a config that is not a dict is left alone
    cfg3 = SimpleNamespace(num_attention_heads=2, hidden_size=256, rms_norm_eps=1e-6)
    DA.DashAttention(cfg3)


def _mask(rows, S, fill):
    """[B, 1, S, S] additive mask: 0 where rows[b](t, j) allows key j, else fill."""
    i = torch.arange(S)
    m = torch.zeros(len(rows), 1, S, S)
    for b, allow in enumerate(rows):
        ok = allow(i[:, None], i[None, :])
        m[b, 0] = torch.where(ok, torch.zeros(()), torch.full((), fill))
    return m


def test_mask_key_starts_left_padding_and_documents():
    S = 40
    causal = lambda t, j: j <= t
    mn = torch.finfo(torch.float32).min
    m = _mask([causal, lambda t, j: (j <= t) & (j >= 11),
               lambda t, j: (j <= t) & (j >= torch.where(t >= 25, 25, 0))], S, mn)
    kmin, empty = DA.mask_key_starts(m, 3, S)
    t = torch.arange(S)
    assert kmin[0].tolist() == [0] * S and not empty[0].any()
    # rows before the padding end have no causal key: empty, kmin 0
    assert empty[1].tolist() == (t < 11).tolist()
    assert kmin[1].tolist() == torch.where(t < 11, 0, 11).tolist()
    assert kmin[2].tolist() == torch.where(t >= 25, 25, 0).tolist() and not empty[2].any()
    # a mask of batch 1 and larger than S broadcasts; the rows of _unmask_unattended
    # (all zero) allow everything
    big = torch.zeros(1, 1, S + 5, S + 7)
    kmin, empty = DA.mask_key_starts(big, 2, S)
    assert not kmin.any() and not empty.any()
    # identical heads are accepted
    kmin, _ = DA.mask_key_starts(m[1:2].expand(1, 4, S, S), 1, S)
    assert kmin[0].tolist() == torch.where(t < 11, 0, 11).tolist()


@pytest.mark.parametrize("case", ["right_pad", "hole", "partial_value", "heads",
                                  "fp16_min_empty_row", "shape"])
def test_mask_key_starts_refuses_other_masks(case):
    S = 32
    if case == "right_pad":      # pad query rows keep keys [0, 20): not a suffix of [0, t]
        m = _mask([lambda t, j: (j <= t) & (j < 20)], S, -1e30)
    elif case == "hole":
        m = _mask([lambda t, j: (j <= t) & (j != 5)], S, -1e30)
    elif case == "partial_value":
        m = _mask([lambda t, j: j <= t], S, -1e30)
        m[0, 0, 10, 3] = -3.0
    elif case == "heads":
        m = _mask([lambda t, j: j <= t], S, -1e30).expand(1, 2, S, S).clone()
        m[0, 1, 20, 20] = -1e30
    elif case == "fp16_min_empty_row":   # a fully masked row whose entries do not clamp
        m = _mask([lambda t, j: (j <= t) & (j >= 8)], S, -65504.0)
    else:
        m = torch.zeros(1, S, S)
    with pytest.raises(NotImplementedError):
        DA.mask_key_starts(m, 1, S)
