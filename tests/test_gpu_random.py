"""GPU parity on randomly drawn configurations: each seed draws the shape and the
parameters of one prefill (batch, heads, length, block size, window, routed slots,
dense threshold, packed documents), one decode step (sequence lengths, block size,
window, K, topm, paged or contiguous cache, fused or two-launch path) or one prefill
backward, and the result is compared with the oracle (the backward: with the fp32
autograd reference of the same attention) on the same inputs.  The fixed cases elsewhere pin known
edges; these cover the combinations between them.  Tolerances are the path's: routing
bit for bit on identical fp32 scores, outputs within 2e-2 abs / 1e-2 rel and 1.5 % of
the output scale.
"""

import math

import pytest
import torch

from ananta_ocr_amd import ops, pipeline
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2
SCALE = 1 / math.sqrt(128)


def _close(out, ref, what, tight=1.5e-2):
    out = out.float().cpu()
    ref = ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= ATOL + RTOL * ref.abs()), f"{what}: max err {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, \
        f"{what}: max err {err.max().item():.3e}"


def _pick(g, options):
    return options[int(torch.randint(len(options), (1,), generator=g))]


def _routed_slots(g, L, bs, lw, K):
    """Random routed slots of one sequence as routing returns them: remote block ids
    (distinct per row), some invalid or -1 slots, random biases."""
    t = torch.arange(L)
    lb = (lw + bs - 1) // bs
    hi = (t // bs - lb).clamp(min=0)
    idx = (torch.rand(L, K, generator=g) * (hi[:, None] + 1)).floor().long()
    valid = (torch.rand(L, K, generator=g) < 0.85) & (t // bs - lb >= 0)[:, None]
    for j in range(1, K):
        valid[:, j] &= ~(idx[:, j:j + 1] == idx[:, :j]).any(-1)
    idx = torch.where(torch.rand(L, K, generator=g) < 0.05, torch.full_like(idx, -1), idx)
    bias = torch.randn(L, K, generator=g) * 2
    return idx, bias, valid


@pytest.mark.parametrize("seed", range(60))
def test_prefill_random_configuration(seed):
    g = torch.Generator("cpu").manual_seed(7000 + seed)
    bs = _pick(g, [32, 64, 128])
    K = _pick(g, [0, 1, 3, 8, 16] + ([24, 40] if bs <= 64 else []))
    lw = int(torch.randint(1, 1100, (1,), generator=g))
    H = int(torch.randint(1, 4, (1,), generator=g))
    thr = _pick(g, [0, 1, 24, 129])
    packed = bool(torch.rand(1, generator=g) < 0.35)
    if packed:
        ndoc = int(torch.randint(2, 6, (1,), generator=g))
        lens = [int(torch.randint(1, 900, (1,), generator=g)) for _ in range(ndoc)]
        B, cu = 1, [0]
        for L in lens:
            cu.append(cu[-1] + L)
        S = cu[-1]
    else:
        B = int(torch.randint(1, 3, (1,), generator=g))
        S = int(torch.randint(1, 2000, (1,), generator=g))
        cu = None
    qs = _pick(g, [0.5, 1.0, 3.0])
    what = (f"seed {seed}: B={B} H={H} S={S} bs={bs} lw={lw} K={K} thr={thr} "
            f"docs={None if cu is None else len(cu) - 1}")
    print(what, flush=True)
    q = (torch.randn(B, H, S, 128, generator=g) * qs * 0.3).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.3).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    spans = [(cu[i], cu[i + 1]) for i in range(len(cu) - 1)] if cu else [(0, S)]
    Kd = max(K, 1)
    idx = torch.zeros(B, S, Kd, dtype=torch.long)
    bias = torch.zeros(B, S, Kd)
    valid = torch.zeros(B, S, Kd, dtype=torch.bool)
    for b in range(B):
        for s0, s1 in spans:
            i, bi, va = _routed_slots(g, s1 - s0, bs, lw, Kd)
            idx[b, s0:s1], bias[b, s0:s1], valid[b, s0:s1] = i, bi, va
    idx, bias, valid = idx[..., :K], bias[..., :K], valid[..., :K]
    kw = dict(dense_threshold=thr)
    if cu is not None:
        kw["cu_seqlens"] = torch.tensor(cu, dtype=torch.int32).to(DEV)
        out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx[0].to(DEV),
                               bias[0].to(DEV), valid[0].to(DEV), bs, lw, SCALE, **kw)
    else:
        out = ops.attn_prefill(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), bias.to(DEV),
                               valid.to(DEV), bs, lw, SCALE, **kw)
    for s0, s1 in spans:
        ref = O.dense_attend(q[:, :, s0:s1], k[:, :, s0:s1], v[:, :, s0:s1], idx[:, s0:s1],
                             bias[:, s0:s1], valid[:, s0:s1], bs, lw, SCALE)
        _close(out[:, :, s0:s1], ref, f"{what}, rows {s0}..{s1}")


@pytest.mark.parametrize("seed", range(40))
def test_decode_step_random_configuration(seed):
    g = torch.Generator("cpu").manual_seed(8000 + seed)
    bs = _pick(g, [32, 64, 128])
    lb = int(torch.randint(1, 9, (1,), generator=g))
    K = int(torch.randint(1, 17, (1,), generator=g))
    topm = int(torch.randint(K, 17, (1,), generator=g))
    B = int(torch.randint(1, 7, (1,), generator=g))
    H = int(torch.randint(1, 5, (1,), generator=g))
    paged = bool(torch.rand(1, generator=g) < 0.5)
    fused = bool(torch.rand(1, generator=g) < 0.7)
    lens = [int(torch.randint(1, 6000, (1,), generator=g)) for _ in range(B)]
    hc_scale = _pick(g, [0.0, 0.3])
    idx_scale = _pick(g, [128.0 / math.sqrt(128), 30.0])
    what = (f"seed {seed}: B={B} H={H} bs={bs} lb={lb} K={K} topm={topm} paged={paged} "
            f"fused={fused} lens={lens}")
    print(what, flush=True)
    lw, d, S = lb * bs, 128, max(lens)
    k = (torch.randn(B, H, S, 128, generator=g) * 0.3).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    q = (torch.randn(B, H, 128, generator=g) * 0.6).bfloat16()
    ik = torch.randn(B, S, d, generator=g)
    iq = torch.randn(B, d, generator=g)
    hc = torch.randn(d, generator=g) * hc_scale
    lens_t = torch.tensor(lens, dtype=torch.int32)
    kw = dict(seq_lens=lens_t.to(DEV))
    nblk = (S + bs - 1) // bs
    if paged:
        npg = [(L + bs - 1) // bs for L in lens]
        perm = torch.randperm(sum(npg), generator=g)
        table = torch.zeros(B, max(npg), dtype=torch.int32)
        kp = torch.zeros(sum(npg), bs, H, 128, dtype=torch.bfloat16)
        vp = torch.zeros_like(kp)
        ikp = torch.zeros(sum(npg), bs, d)
        o = 0
        for b in range(B):
            for pg in range(npg[b]):
                phys = int(perm[o + pg])
                table[b, pg] = phys
                seg = slice(pg * bs, min((pg + 1) * bs, lens[b]))
                n = seg.stop - seg.start
                kp[phys, :n] = k[b, :, seg].transpose(0, 1)
                vp[phys, :n] = v[b, :, seg].transpose(0, 1)
                ikp[phys, :n] = ik[b, seg]
            o += npg[b]
        kd, vd, ikd = kp.to(DEV), vp.to(DEV), ikp.to(DEV)
        kw.update(block_table=table.to(DEV), page_size=bs)
        nblk = max(npg)
    else:
        kd, vd, ikd = k.to(DEV), v.to(DEV), ik.to(DEV)
    st = pipeline.init_decode_state(ikd, hc.to(DEV), bs, nblk, **kw)
    out, (ti, bi, va), z = pipeline.decode_step(
        st, q.to(DEV), kd, vd, iq.to(DEV), ikd, hc.to(DEV), bs, lb, idx_scale, 1e-4, 1.0, K,
        topm, SCALE, return_routing=True, fused=fused, return_scores=True, **kw)
    out, ti, bi, va, z = out.cpu(), ti.cpu().long(), bi.cpu(), va.cpu(), z.cpu()
    kbar = st.kbar.cpu()
    Kp = ti.shape[-1]
    for b, L in enumerate(lens):
        kb_r, cv = O.kbar_headcls(ik[b:b + 1, :L], hc, bs)
        nb = kb_r.shape[1]
        torch.testing.assert_close(kbar[b:b + 1, :nb], kb_r, atol=1e-5, rtol=1e-5)
        z_r = O.block_scores_headcls(iq[b:b + 1, None], kb_r, cv, torch.tensor([[L - 1]]), bs,
                                     lb)
        zb = z[b:b + 1, None, :nb]
        sent = z_r < -5e8
        assert torch.equal(zb < -5e8, sent), f"{what}, sequence {b}: sentinel pattern"
        torch.testing.assert_close(zb[~sent], z_r[~sent], atol=2e-5, rtol=2e-5)
        # routing of the GPU's own scores, bit for bit
        t_r, b_r, v_r = O.infer_route_select(zb, None, idx_scale, 1e-4, 1.0, K, topm)
        kp_ = t_r.shape[-1]
        assert torch.equal(ti[b:b + 1, :, :kp_], t_r), f"{what}, sequence {b}: routed ids"
        assert torch.equal(va[b:b + 1, :, :kp_], v_r), f"{what}, sequence {b}: validity"
        torch.testing.assert_close(bi[b:b + 1, :, :kp_], b_r, atol=2e-5, rtol=1e-5)
        assert bool((ti[b, :, kp_:Kp] == -1).all())
        ref = O.decode_attend(q[b:b + 1, :, None].float(), k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                              t_r, b_r, v_r, torch.tensor([[L - 1]]), bs, lw, SCALE)
        _close(out[b:b + 1], ref[:, :, 0], f"{what}, sequence {b} ({L} tokens)")


@pytest.mark.parametrize("seed", range(24))
def test_backward_random_configuration(seed):
    """The prefill backward (dq, dk, dv and the routed slots' bias gradient) on drawn
    shapes against the fp32 autograd reference of the same attention."""
    from test_gpu_backward import _case, _close_grad, _ref
    g = torch.Generator("cpu").manual_seed(9000 + seed)
    bs = _pick(g, [32, 64, 96, 128])
    K = _pick(g, [1, 4, 12, 16] + ([24, 40, 64] if bs <= 64 else []))
    lw = int(torch.randint(1, 1000, (1,), generator=g))
    B = int(torch.randint(1, 3, (1,), generator=g))
    H = int(torch.randint(1, 4, (1,), generator=g))
    S = int(torch.randint(1, 1400, (1,), generator=g))
    what = f"seed {seed}: B={B} H={H} S={S} bs={bs} lw={lw} K={K}"
    print(what, flush=True)
    q, k, v, topi, bias, valid, dout = _case(9500 + seed, B, H, S, bs, lw, K)
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    br = bias.clone().requires_grad_()
    out_r = _ref(qr, kr, vr, topi, br, valid, bs, lw, SCALE)
    out_r.backward(dout.float())
    args = [t.to(DEV) for t in (q, k, v)]
    out, lse = ops.attn_prefill(*args, topi.to(DEV), bias.to(DEV), valid.to(DEV), bs, lw, SCALE,
                                return_lse=True)
    dq, dk, dv, db = ops.attn_prefill_backward(*args, out, lse, dout.to(DEV), topi.to(DEV),
                                               bias.to(DEV), valid.to(DEV), bs, lw, SCALE)
    torch.cuda.synchronize()
    _close_grad(out, out_r.detach(), f"{what}: out")
    _close_grad(dq, qr.grad, f"{what}: dq")
    _close_grad(dk, kr.grad, f"{what}: dk")
    _close_grad(dv, vr.grad, f"{what}: dv")
    _close_grad(db, br.grad, f"{what}: dbias")
    assert bool((db.cpu()[br.grad == 0] == 0).all()), f"{what}: gradient on a non-first slot"
