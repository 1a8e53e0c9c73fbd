"""The C-ABI library loads and exports every entry point include/dash_hip.h
declares, with the ctypes signatures the Python layer uses.  No GPU calls."""

import os
import re

import pytest

from ananta_ocr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


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
