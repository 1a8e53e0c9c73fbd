"""The C-ABI library loads and exports every entry point include/dash_hip.h
declares, with the ctypes signatures the Python layer uses.  No GPU calls."""

import os
import re

import pytest

from ananta_ocr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ERR_UNSUPPORTED = -2             # kErrUnsupported, a shape or stride the kernels do not take
ERR_INVALID = -3                 # kErrInvalid, inconsistent arguments


def _declared():
    text = open(os.path.join(ROOT, "include", "dash_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dash_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    declared = _declared()
    assert declared, "no entry points found in include/dash_hip.h"
    assert sorted(_lib.SIGNATURES) == declared


def test_header_argument_counts_match_binding():
    text = open(os.path.join(ROOT, "include", "dash_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\((.*?)\);", text, flags=re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), (name, len(params), len(args))


def test_library_loads_and_exports_every_symbol():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libdash_hip.so is not built (run __graft_entry__.build())")
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.dash_abi_version() == 1
    assert lib.dash_status_string(-2) == b"unsupported shape or parameter"


def test_cached_workspace_grows_and_is_released():
    """The host-side workspace cache: reused when large enough, replaced by a larger
    buffer, and dropped by release_workspaces (host memory here; the same code path
    serves device buffers)."""
    from ananta_ocr_amd import ops
    ops.release_workspaces()
    a = ops.cached_workspace("t", 1000, "cpu")
    assert a.numel() >= 1000 and ops.cached_workspace("t", 500, "cpu") is a
    b = ops.cached_workspace("t", 10 * a.numel(), "cpu")
    assert b.numel() >= 10 * a.numel() and ops.cached_workspace_bytes() == b.numel()
    ops.release_workspaces("cpu")
    assert ops.cached_workspace_bytes() == 0


def _call(name, **kw):
    """Calls entry point `name` with every pointer set to an aligned placeholder address
    and every integer or float from `kw` (name -> value, in header order), for argument
    checks that return before any device call."""
    lib = _lib.load()
    text = open(os.path.join(ROOT, "include", "dash_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    m = re.search(rf"\b{name}\s*\((.*?)\);", text, flags=re.S)
    params = [p.strip() for p in m.group(1).split(",")]
    args = []
    for p in params:
        pname = re.findall(r"\w+", p)[-1]
        if "*" in p:
            args.append(None if kw.get(pname, 1) is None else 0x100000)
        else:
            args.append(kw[pname])
    return getattr(lib, name)(*args)


def test_argument_checks_return_before_any_device_call():
    """Sizes that the kernels would read past are refused on the host: a prefill
    (forward or backward) whose total_rows is not B * S without cu_seqlens, and a decode
    router whose k_bar cache holds fewer blocks than S needs."""
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libdash_hip.so is not built (run __graft_entry__.build())")
    import torch
    if torch.cuda.is_available():
        # the placeholder pointers must never reach a launch on a real device
        pytest.skip("argument checks are exercised where no device is present")
    common = dict(q_sb=0, q_sh=0, q_st=128, k_sb=0, k_sh=0, k_st=128, v_sb=0, v_sh=0, v_st=128,
                  K=16, cu_seqlens=None, kmin=None, valid=None, B=2, H=10, S=1000, D=128,
                  block_size=64, local_window=512, scale=0.088)
    strides_o = dict(o_sb=0, o_sh=0, o_st=128)
    fwd = dict(common, **strides_o, lse_row=10, lse_sh=1, dense_threshold=32,
               workspace_bytes=1 << 40, stream=None)
    assert _call("dash_attn_prefill", **fwd, total_rows=1999) == ERR_INVALID
    bwd = dict(common, **strides_o, lse_row=10, lse_sh=1, do_sb=0, do_sh=0, do_st=128,
               dq_sb=0, dq_sh=0, dq_st=128, dk_sb=0, dk_sh=0, dk_st=128, dv_sb=0, dv_sh=0,
               dv_st=128, workspace_bytes=1 << 40, stream=None)
    assert _call("dash_attn_prefill_backward", **bwd, total_rows=1999) == ERR_INVALID
    # a K/V token stride whose 64-row stage offsets would not fit 32 bits
    big = (1 << 25) - 56
    for kv in (dict(k_st=big), dict(v_st=big)):
        assert _call("dash_attn_prefill", **dict(fwd, **kv), total_rows=2000) == ERR_UNSUPPORTED
        assert _call("dash_attn_prefill_backward", **dict(bwd, **kv),
                     total_rows=2000) == ERR_UNSUPPORTED
    dec = dict(iq_sb=128, ik_sb=0, ik_st=128, ik_sp=0, block_table=None, table_stride=0,
               page_size=0, seq_lens=None, q_pos=None, head_cls=1, refresh_tail=1, kb_sb=0,
               kb_table=None, kb_ts=0, bounds=None, cand=None, cand_stride=0, B=2, d=128,
               block_size=64, local_blocks=8, idx_scale=11.3, floor_p=1e-4, sigma=1.0, K=16,
               topm=16, Kout=16, valid=None, z_stride=16, stream=None)
    # 1,000 tokens need 16 blocks of 64
    assert _call("dash_decode_route", **dec, S=1000, nblk_cap=15) == ERR_INVALID
