"""Extend (chunked / prefix-cached) prefill over a paged cache (pipeline.extend_prefill) on
the GPU against the oracle's per-request semantics: for request b, whose cache holds
seq_lens[b] tokens of which the first context_lens[b] were there before the step, the
query rows are the positions context_lens[b] .. seq_lens[b] - 1, and each must equal the
oracle's inference prefill of the whole sequence at that row (block summaries of the
sequence, block scores at the row's position, routing, attention over the window and the
routed blocks).  Routing ids and validity exact (ties to the lower block id), outputs to
2e-2 abs / 1e-2 rel and 1.5 % of the output scale.  A request stepped chunk by chunk
through the same page pool must equal its one-step result."""

import math

import pytest
import torch

from ananta_ocr_amd import pipeline
from oracle import dash_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _close(out, ref, what, tight=1.5e-2):
    out, ref = out.float().cpu(), ref.float().cpu()
    err = (out - ref).abs()
    assert torch.all(err <= 2e-2 + 1e-2 * ref.abs()), f"{what}: {err.max().item()}"
    assert err.max().item() <= tight * ref.abs().max().item() + 1e-6, f"{what}: {err.max().item()}"


def _paged(x, lens, table, bs, num_pages):
    """x [B, S, ...] -> pages [num_pages, bs, ...] through the block table."""
    B = x.shape[0]
    out = torch.zeros((num_pages, bs) + tuple(x.shape[2:]), dtype=x.dtype)
    for b in range(B):
        for c in range((lens[b] + bs - 1) // bs):
            n = min(bs, lens[b] - c * bs)
            out[table[b, c], :n] = x[b, c * bs:c * bs + n]
    return out


def _case(seed, seqs, ctxs, H, bs, lb, K, topm, scale_q=1.0):
    g = torch.Generator().manual_seed(seed)
    B, S = len(seqs), max(seqs)
    q = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    iq = torch.randn(B, S, 128, generator=g) * scale_q
    ik = torch.randn(B, S, 128, generator=g)
    hc = torch.randn(128, generator=g) * 0.3
    P = (S + bs - 1) // bs
    num_pages = B * P + 5
    table = torch.randperm(num_pages, generator=g)[:B * P].view(B, P).to(torch.int32)
    return q, k, v, iq, ik, hc, table, num_pages


def _oracle_rows(q, k, v, iq, ik, hc, b, seq, ctx, bs, lb, K, topm, idx_scale, scale):
    """The oracle's inference prefill of request b's whole sequence, rows ctx .. seq - 1."""
    kb, cv = O.kbar_headcls(ik[b:b + 1, :seq], hc, bs)
    pos = torch.arange(ctx, seq)[None]
    z = O.block_scores_headcls(iq[b:b + 1, ctx:seq], kb, cv, pos, bs, lb)
    ti, bi, va = O.infer_route_select(z, None, idx_scale, 1e-4, 1.0, K, topm)
    Kp = ti.shape[-1]
    full_t = torch.zeros(1, seq, Kp, dtype=torch.long)
    full_b = torch.zeros(1, seq, Kp)
    full_v = torch.zeros(1, seq, Kp, dtype=torch.bool)
    full_t[:, ctx:], full_b[:, ctx:], full_v[:, ctx:] = ti, bi, va
    out = O.dense_attend(q[b:b + 1, :, :seq], k[b:b + 1, :, :seq], v[b:b + 1, :, :seq], full_t,
                         full_b, full_v, bs, bs * lb, scale, rows=(ctx, seq))
    return out[0], ti[0], va[0]


@pytest.mark.parametrize("seqs,ctxs,H,bs,lb,K,topm", [
    ([900, 2400, 3000, 70], [0, 1500, 2700, 13], 2, 64, 8, 8, 8),
    ([1000, 1777], [640, 1], 2, 32, 4, 12, 16),      # the checkpoint's router geometry
])
def test_extend_prefill_matches_per_request_oracle(seqs, ctxs, H, bs, lb, K, topm):
    q, k, v, iq, ik, hc, table, num_pages = _case(len(seqs) + bs, seqs, ctxs, H, bs, lb, K, topm)
    B = len(seqs)
    idx_scale = 128.0 / math.sqrt(128)
    scale = 1.0 / math.sqrt(128)
    kc = _paged(k.transpose(1, 2), seqs, table, bs, num_pages)        # [pages, bs, H, D]
    vc = _paged(v.transpose(1, 2), seqs, table, bs, num_pages)
    ikc = _paged(ik, seqs, table, bs, num_pages)                      # [pages, bs, d]
    qrows = torch.cat([q[b, :, ctxs[b]:seqs[b]].transpose(0, 1) for b in range(B)])
    iqrows = torch.cat([iq[b, ctxs[b]:seqs[b]] for b in range(B)])
    qlens = [s - c for s, c in zip(seqs, ctxs)]
    cu = torch.tensor([0] + qlens).cumsum(0).to(torch.int32)
    state = pipeline.KBarPageCache(num_pages, 128, DEV)
    # the summaries the earlier steps left: every block of the cached context (the
    # boundary block over the tokens it held then)
    ctx_d = torch.tensor(ctxs, device=DEV)
    state.refresh_from(ikc.to(DEV), hc.to(DEV), bs, table.to(DEV), ctx_d, torch.zeros_like(ctx_d))
    out, (gi, gb, gv), qpos = pipeline.extend_prefill(
        state, qrows.to(DEV), kc.to(DEV), vc.to(DEV), iqrows.to(DEV), ikc.to(DEV), hc.to(DEV),
        bs, lb, idx_scale, 1e-4, 1.0, K, topm, table.to(DEV), torch.tensor(seqs).to(DEV),
        torch.tensor(ctxs).to(DEV), cu.to(DEV), max_query_len=max(qlens), return_routing=True)
    out = out.cpu()
    for b in range(B):
        r0, r1 = int(cu[b]), int(cu[b + 1])
        assert qpos[r0:r1].cpu().tolist() == list(range(ctxs[b], seqs[b]))
        ref, ti, va = _oracle_rows(q, k, v, iq, ik, hc, b, seqs[b], ctxs[b], bs, lb, K, topm,
                                   idx_scale, scale)
        kp = ti.shape[-1]
        assert torch.equal(gv[r0:r1, :kp].cpu(), va), b
        assert torch.equal(torch.where(va, gi[r0:r1, :kp].cpu().long(), -1),
                           torch.where(va, ti, -1)), b
        assert not gv[r0:r1, kp:].any()
        _close(out[r0:r1].transpose(0, 1), ref, f"request {b}")
    # the pool holds every used page's summary of the sequences as they now stand
    for b in range(B):
        kb, _ = O.kbar_headcls(ik[b:b + 1, :seqs[b]], hc, bs)
        nb = (seqs[b] + bs - 1) // bs
        got = state.kbar[table[b, :nb].long().to(DEV)].cpu()
        torch.testing.assert_close(got, kb[0], atol=2e-5, rtol=2e-5)


def test_extend_prefill_in_chunks_equals_one_step():
    """One request stepped through the cache in chunks (each step writes its tokens and
    extends the sequence) gives the rows of a single step over the whole prompt."""
    seqs, H, bs, lb, K, topm = [2600], 2, 64, 4, 8, 8
    q, k, v, iq, ik, hc, table, num_pages = _case(5, seqs, [0], H, bs, lb, K, topm)
    idx_scale = 128.0 / math.sqrt(128)
    S = seqs[0]
    kc = _paged(k.transpose(1, 2), seqs, table, bs, num_pages).to(DEV)
    vc = _paged(v.transpose(1, 2), seqs, table, bs, num_pages).to(DEV)
    ikc = _paged(ik, seqs, table, bs, num_pages).to(DEV)
    args = (hc.to(DEV), bs, lb, idx_scale, 1e-4, 1.0, K, topm, table.to(DEV))

    def step(state, c0, c1):
        cu = torch.tensor([0, c1 - c0], dtype=torch.int32, device=DEV)
        return pipeline.extend_prefill(
            state, q[0, :, c0:c1].transpose(0, 1).contiguous().to(DEV), kc, vc,
            iq[0, c0:c1].to(DEV), ikc, *args, torch.tensor([c1], device=DEV),
            torch.tensor([c0], device=DEV), cu, max_query_len=c1 - c0)

    one = step(pipeline.KBarPageCache(num_pages, 128, DEV), 0, S)
    st = pipeline.KBarPageCache(num_pages, 128, DEV)
    parts = [step(st, c0, min(c0 + 700, S)) for c0 in range(0, S, 700)]
    torch.testing.assert_close(torch.cat(parts).cpu(), one.cpu(), atol=0, rtol=0)
