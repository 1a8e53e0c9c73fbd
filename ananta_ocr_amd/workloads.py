"""Synthetic DASH workloads (seeded), shared by the benchmark and the tests.

Inputs follow one rule: a CPU ``torch.Generator`` seeded per workload draws Q,
K, V (in that order) as ``randn * 128**-0.5`` in fp32, cast to bf16; the router
inputs are the head means of Q and K in fp32 (``idx_q``/``idx_k`` [B, S, 128]);
stage 0 uses ``head_cls = 0`` (mean pooling), ``idx_scale = 128/sqrt(128)``,
``floor = 1e-4``, ``sigma = 1``, ``M = K = cap``.
"""

import math
from dataclasses import dataclass, field

import torch

D = 128
H = 10
IDX_SCALE = 128.0 / math.sqrt(128.0)
FLOOR = 1e-4
SIGMA = 1.0
PAGE_TOKENS = 273


@dataclass
class Prefill:
    name: str
    B: int
    S: int
    bs: int
    lw: int
    cap: int
    seed: int
    offset_frac: float = 0.0      # fraction of key blocks given a +2.0 mean offset
    doc_pages: list = field(default_factory=list)   # packed varlen documents (pages each)


@dataclass
class Decode:
    name: str
    B: int
    S: int
    bs: int
    lw: int
    cap: int
    seed: int
    layers: int = 1
    paged: bool = False
    len_lo: int = 0
    len_hi: int = 0


PREFILL_2730 = Prefill("prefill_s2730_lw512_cap8", 1, 2730, 64, 512, 8, seed=1)
DECODE_B8 = Decode("decode_b8_kv27300_lw1024_cap16", 8, 27300, 64, 1024, 16, seed=2)
PREFILL_27300 = Prefill("prefill_s27300_lw1024_cap16", 1, 27300, 64, 1024, 16, seed=3,
                        offset_frac=0.05)
PACKED_16DOC = Prefill("packed16_pages1to40_lw512_cap8", 1, 0, 64, 512, 8, seed=4)
PAGED_12L = Decode("paged_decode_12l_b32", 32, 27300, 64, 1024, 16, seed=5, layers=12,
                   paged=True, len_lo=2730, len_hi=27300)


def router_inputs(q, k):
    """idx_q/idx_k: head means of Q and K in fp32, [B,S,D]."""
    return q.float().mean(1), k.float().mean(1)


def make_prefill(cfg, device="cpu"):
    """Returns dict with q,k,v bf16 [B,H,S,D], idx_q/idx_k fp32 [B,S,D] on `device`
    (and cu_seqlens for packed workloads)."""
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    cu = None
    if cfg is PACKED_16DOC or cfg.doc_pages:
        pages = cfg.doc_pages or torch.randint(1, 41, (16,), generator=g).tolist()
        lens = [p * PAGE_TOKENS for p in pages]
        cu = [0]
        for L in lens:
            cu.append(cu[-1] + L)
        B, S = 1, cu[-1]
    else:
        B, S = cfg.B, cfg.S
    shape = (B, H, S, D)
    sc = D ** -0.5
    q = torch.randn(shape, generator=g) * sc
    k = torch.randn(shape, generator=g) * sc
    v = torch.randn(shape, generator=g) * sc
    if cfg.offset_frac > 0:
        nblk = (S + cfg.bs - 1) // cfg.bs
        n = int(math.floor(cfg.offset_frac * nblk))
        blocks = torch.randperm(nblk, generator=g)[:n]
        u = torch.randn(D, generator=g)
        u = u / u.norm()
        for c in blocks.tolist():
            k[:, :, c * cfg.bs:(c + 1) * cfg.bs] += 2.0 * u
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    iq, ik = router_inputs(q, k)
    out = dict(q=q.to(device), k=k.to(device), v=v.to(device), idx_q=iq.to(device),
               idx_k=ik.to(device), B=B, S=S)
    if cu is not None:
        out["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32, device=device)
        out["cu_list"] = cu
    return out


def make_decode(cfg, device="cpu", layer=0):
    """Contiguous decode workload: the query is the last cached token of every
    sequence.  Returns q [B,H,D], k/v [B,H,S,D] bf16, idx_q [B,1,D], idx_k [B,S,D]."""
    g = torch.Generator("cpu").manual_seed(cfg.seed + 498 * layer if layer else cfg.seed)
    shape = (cfg.B, H, cfg.S, D)
    sc = D ** -0.5
    q = (torch.randn((cfg.B, H, D), generator=g) * sc).bfloat16()
    k = (torch.randn(shape, generator=g) * sc).bfloat16()
    v = (torch.randn(shape, generator=g) * sc).bfloat16()
    iq = q.float().mean(1)[:, None]
    ik = k.float().mean(1)
    return dict(q=q.to(device), k=k.to(device), v=v.to(device), idx_q=iq.to(device),
                idx_k=ik.to(device))


def make_paged_decode(cfg, device, layer, lengths=None, table=None):
    """Paged decode workload for one layer.  Lengths and the page permutation come
    from a CPU generator seeded with cfg.seed; layer l draws its Q/K/V on the
    device from seed 500+l.  Returns q [B,H,D], k/v [pages, bs, H, D] bf16,
    idx_q [B,1,D], idx_k paged [pages, bs, D] fp32, block_table, seq_lens."""
    if lengths is None or table is None:
        lengths, table = paged_layout(cfg)
    pages = int(table.max().item()) + 1 if table.numel() else 0
    g = torch.Generator(device).manual_seed(500 + layer)
    sc = D ** -0.5
    q = (torch.randn((cfg.B, H, D), generator=g, device=device) * sc).bfloat16()
    k = (torch.randn((pages, cfg.bs, H, D), generator=g, device=device) * sc).bfloat16()
    v = (torch.randn((pages, cfg.bs, H, D), generator=g, device=device) * sc).bfloat16()
    iq = q.float().mean(1)[:, None]
    ik = k.float().mean(2)
    return dict(q=q, k=k, v=v, idx_q=iq, idx_k=ik, block_table=table.to(device),
                seq_lens=lengths.to(device))


def paged_layout(cfg):
    """Per-sequence lengths U[len_lo, len_hi] and a random physical page permutation."""
    g = torch.Generator("cpu").manual_seed(cfg.seed)
    lengths = torch.randint(cfg.len_lo, cfg.len_hi + 1, (cfg.B,), generator=g)
    npg = [(int(L) + cfg.bs - 1) // cfg.bs for L in lengths]
    perm = torch.randperm(sum(npg), generator=g)
    maxp = max(npg)
    table = torch.zeros(cfg.B, maxp, dtype=torch.int32)
    o = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[o:o + n].to(torch.int32)
        o += n
    return lengths.to(torch.int32), table


# Router front end: the index projections of the checkpoint's shape (hidden 1280,
# index dim 128, bf16), its block size 32 and stage 0 head_cls, over 27,300 tokens.
FRONT_NAME = "router_front_s27300_h1280_bs32"
FRONT_S, FRONT_HIDDEN, FRONT_BS = 27300, 1280, 32


def make_front(S=FRONT_S, hidden=FRONT_HIDDEN, seed=8, device="cpu"):
    """Synthetic router inputs: hidden states randn bf16 [1, S, hidden], q/k projection
    weights randn/sqrt(hidden) bf16 [128, hidden], Gemma norm weights randn*0.1,
    head_cls randn*0.5, and the 1-D RoPE (cos, sin) bf16 [1, S, 128] of positions 0..S-1
    (theta 5e5, the config's sparse_rope_theta)."""
    g = torch.Generator("cpu").manual_seed(seed)
    hs = torch.randn(1, S, hidden, generator=g).bfloat16()
    wq = (torch.randn(D, hidden, generator=g) / math.sqrt(hidden)).bfloat16()
    wk = (torch.randn(D, hidden, generator=g) / math.sqrt(hidden)).bfloat16()
    nq = torch.randn(D, generator=g) * 0.1
    nk = torch.randn(D, generator=g) * 0.1
    hc = torch.randn(D, generator=g) * 0.5
    inv = 1.0 / 5.0e5 ** (torch.arange(0, D, 2).float() / D)
    ang = torch.arange(S).float()[:, None] * inv[None]
    emb = torch.cat([ang, ang], -1)[None]
    out = dict(hs=hs, wq=wq, wk=wk, nq=nq, nk=nk, hc=hc, cos=emb.cos().bfloat16(),
               sin=emb.sin().bfloat16())
    return {k: v.to(device) for k, v in out.items()}
