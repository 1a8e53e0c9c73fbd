"""The allocation-free decode step (dash_decode_step_noalloc: the partials in the
library's fixed per-GPU scratch array) against the workspace entry point
(dash_decode_step) on the same inputs: identical routing, scores and outputs, on two
calls in a row, the second with a smaller input than the first (the array keeps the
first call's contents)."""

import ctypes
import math

import pytest
import torch

from ananta_ocr_amd import _lib, ops

DEV = "cuda"


def _inputs(B, H, S, bs, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, 128, generator=g) * 2).bfloat16()
    k = (torch.randn(B, H, S, 128, generator=g) / math.sqrt(128)).bfloat16()
    v = torch.randn(B, H, S, 128, generator=g).bfloat16()
    iq = torch.randn(B, 128, generator=g)
    ik = torch.randn(B, S, 128, generator=g)
    hc = torch.randn(128, generator=g) * 0.2
    lens = torch.randint(max(1, S // 3), S + 1, (B,), generator=g).to(torch.int32)
    return [t.to(DEV) for t in (q, k, v, iq, ik, hc, lens)]


@pytest.mark.gpu
def test_noalloc_decode_step_matches_workspace_entry_point():
    torch.cuda.set_device(0)
    for B, H, S, bs, lb, K, seed in [(8, 10, 6000, 64, 16, 16, 1), (3, 4, 1500, 32, 4, 12, 2)]:
        q, k, v, iq, ik, hc, lens = _inputs(B, H, S, bs, seed)
        nblk = (S + bs - 1) // bs
        kb0 = ops.kbar(ik, hc, bs, seq_lens=lens, nblk_cap=nblk)
        kb_ws, kb_na = kb0.clone(), kb0.clone()
        args = (bs, lb, 128.0 / math.sqrt(128), 1e-4, 1.0, K, 16, 1 / math.sqrt(128))
        ref = ops.decode_step_fused(q, k, v, iq, ik, hc, kb_ws, *args, seq_lens=lens,
                                    width=K, return_scores=True)
        got = ops.decode_step_fused(q, k, v, iq, ik, hc, kb_na, *args, seq_lens=lens,
                                    width=K, return_scores=True, no_alloc=True)
        torch.cuda.synchronize()
        (o_r, (i_r, b_r, v_r), z_r), (o_g, (i_g, b_g, v_g), z_g) = ref, got
        assert torch.equal(i_g, i_r) and torch.equal(v_g, v_r), (B, S)
        assert torch.equal(b_g, b_r), (B, S)
        for b in range(B):          # scores are written for the sequence's own blocks
            nb = (int(lens[b]) + bs - 1) // bs
            assert torch.equal(z_g[b, :nb], z_r[b, :nb]), (B, S, b)
        assert torch.equal(kb_na, kb_ws), (B, S)
        assert bool(v_g.any()), (B, S)
        assert torch.equal(o_g, o_r), (B, S)


def test_noalloc_refuses_sizes_beyond_its_scratch():
    """Refused on the host before any device call: the workspace these sizes need
    exceeds the fixed array."""
    if torch.cuda.is_available():
        # the placeholder pointers must never reach a launch on a real device
        pytest.skip("argument checks are exercised where no device is present")
    lib = _lib.load()
    cap = lib.dash_decode_step_scratch_bytes()
    assert cap == 64 << 20
    need = ctypes.c_int64(0)
    B, H, D, bs, lw = 4096, 32, 128, 64, 1024
    assert lib.dash_decode_step_workspace_size(B, H, D, bs, lw, need) == 0
    assert need.value > cap
    fake = ctypes.c_void_p(1 << 20)
    st = lib.dash_decode_step_noalloc(
        fake, 128, fake, 0, 128, 0, None, 0, 0, None, None, 1000, fake, 1, fake, 16 * 128,
        16, None, 0, None, None, 0, 128, 16, 1.0, 1e-4, 1.0, 16, 16, 16, fake, fake, fake, fake,
        16,
        fake, H * D, D, fake, 0, 0, 0, 0, fake, 0, 0, 0, 0, fake, 0, H * D, D, None, 0, 0,
        B, H, D, bs, lw, 0.1, None)
    assert st == -5
    assert b"scratch" in lib.dash_status_string(-5)
