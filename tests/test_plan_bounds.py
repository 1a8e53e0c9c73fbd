"""Bounds rules of the library's host-side argument checks and plan arithmetic,
exercised on the CPU (no device pointer is ever dereferenced: every call here
returns before a launch).

* The prefill scatter kernel stores a sparse pair only where its chunk record and
  partial position fall inside the workspace (``dash_prefill_plan_target`` is the
  same rule, compiled for the host); malformed counts are refused.
* The workspace holds every chunk that consistent counts can produce: for any split
  of a sequence's routed pairs over its blocks, sum ceil(count / 256) fits.
* The decode router refuses a k_bar cache with fewer than ceil(S / block_size) rows.
* Split tiles ask for a workspace only where the library splits them.
"""

import ctypes
import random

import numpy as np
import pytest

from ananta_ocr_amd import _lib

KPFCH = 256           # sparse pairs per chunk record (dash_prefill.hip kPfCH)


def _lib_or_skip():
    try:
        return _lib.load()
    except ImportError:
        pytest.fail("libdash_hip.so is not built (run __graft_entry__.build())")


def _target(lib, chunk_cap, ppos, pos0, bch, q):
    rc, pp = ctypes.c_int64(0), ctypes.c_int64(0)
    st = lib.dash_prefill_plan_target(chunk_cap, ppos, pos0, bch, q, rc, pp)
    return st, rc.value, pp.value


def test_plan_target_in_bounds():
    lib = _lib_or_skip()
    st, rc, pp = _target(lib, 10, 10 * KPFCH, 0, 3, 300)
    assert st == 0 and rc == 3 + 300 // KPFCH and pp == 3 * KPFCH + 300
    st, rc, pp = _target(lib, 10, 20 * KPFCH, 5 * KPFCH, 9, KPFCH - 1)
    assert st == 0 and rc == 9 and pp == 5 * KPFCH + 9 * KPFCH + KPFCH - 1


@pytest.mark.parametrize("bch,q,why", [
    (9, KPFCH, "chunk record past chunk_cap"),
    (10, 0, "first chunk past chunk_cap"),
    (-1, 0, "negative chunk (garbage counter)"),
    (0, -5, "negative pair index"),
    (2, 2 ** 40, "count far past any capacity"),
])
def test_plan_target_refuses_malformed_counts(bch, q, why):
    lib = _lib_or_skip()
    st, _, _ = _target(lib, 10, 1 << 40, 0, bch, q)
    assert st == -3, why


def test_plan_target_refuses_partial_past_positions():
    lib = _lib_or_skip()
    # the record fits but the partial position runs past the positions of the workspace
    st, _, _ = _target(lib, 100, 4 * KPFCH, 2 * KPFCH, 1, KPFCH + 3)
    assert st == -3


def _ws_bytes(lib, B, H, S, rows, K, D, bs):
    n = ctypes.c_int64(0)
    assert lib.dash_attn_prefill_workspace_size(B, H, S, rows, K, D, bs, n) == 0
    return n.value


def test_workspace_holds_every_consistent_plan():
    """Brute force over random splits of the routed pairs: the chunks a sequence
    needs (sum over blocks of ceil(count/256)) never exceed the layout's per-sequence
    record capacity, and all sequences' pair positions fit the partials."""
    lib = _lib_or_skip()
    rng = random.Random(5)
    for _ in range(200):
        bs = rng.choice([32, 64])
        K = rng.randint(1, 16)
        B = rng.randint(1, 6)
        lens = [rng.randint(1, 3000) for _ in range(B)]
        S = max(lens)
        rows = sum(lens)
        chunk_cap = S * K // KPFCH + (S + bs - 1) // bs + 1
        ppos = (rows * K // KPFCH + rows // bs + B + 2) * KPFCH
        total_chunks = 0
        for L in lens:
            nblk = (L + bs - 1) // bs
            pairs = L * K                     # upper bound: every slot sparse
            # adversarial split: many blocks with one pair over a chunk boundary
            counts = np.random.default_rng(rng.randrange(1 << 30)).multinomial(
                pairs, [1.0 / nblk] * nblk).tolist()
            if rng.random() < 0.5:            # or a skewed split
                counts = [0] * nblk
                for i in range(nblk):
                    counts[i] = KPFCH + 1 if i < pairs // (KPFCH + 1) else 0
                counts[-1] += pairs - sum(counts)
            ch = sum((c + KPFCH - 1) // KPFCH for c in counts)
            assert ch <= chunk_cap, (L, K, bs, ch, chunk_cap)
            total_chunks += ch
        assert total_chunks * KPFCH <= ppos
        # the library's layout is at least this large: a partial row per (position,
        # head) of 128 byte-coded dims and its (log-sum-exp, scale) pair
        assert _ws_bytes(lib, B, 10, S, rows, K, 128, bs) >= ppos * 10 * (128 + 8)


def test_error_word_inside_cleared_counters():
    lib = _lib_or_skip()
    off = ctypes.c_int64(0)
    assert lib.dash_attn_prefill_error_offset(1, 10, 27300, 27300, 16, 128, 64, off) == 0
    nblk = (27300 + 63) // 64
    # block counters [B, nblk], then the arrival counter, then the error word
    assert off.value == nblk * 4 + 4
    assert off.value < _ws_bytes(lib, 1, 10, 27300, 27300, 16, 128, 64)


def _decode_route_status(lib, S, nblk_cap, bs=64, B=2, d=128):
    fake = ctypes.c_void_p(1 << 20)            # aligned, never dereferenced
    return lib.dash_decode_route(fake, d, fake, S * d, d, 0, None, 0, 0, None, None, S, fake, 1,
                                 fake, nblk_cap * d, nblk_cap, None, 0, None, None, 0, B, d, bs,
                                 2,
                                 1.0, 1e-4, 1.0, 4, 4, 4, fake, fake, fake, fake, nblk_cap,
                                 None)


def test_decode_router_refuses_undersized_kbar_cache():
    lib = _lib_or_skip()
    # 1,000 keys in 64-key blocks need 16 rows
    assert _decode_route_status(lib, 1000, 15) == -3
    assert _decode_route_status(lib, 1025, 16) == -3
    assert _decode_route_status(lib, -1, 16) == -3


def _split_bytes(lib, B, H, S, D=128):
    n = ctypes.c_int64(-1)
    assert lib.dash_attn_prefill_split_workspace_size(B, H, S, D, n) == 0
    return n.value


def test_split_tile_workspace():
    """Split tiles (every routed block with its tile) need a workspace only for a grid
    of fewer than 512 tiles over sequences of at most 64 tiles: 8 partial slots per
    tile, each 128 rows of bf16 output and an fp32 log-sum-exp."""
    lib = _lib_or_skip()
    tiles = 22 * 10                                   # 2,730 tokens, 10 heads
    assert _split_bytes(lib, 1, 10, 2730) >= tiles * 8 * 128 * (128 * 2 + 4)
    assert _split_bytes(lib, 1, 10, 27300) == 0       # 2,140 tiles fill the chip
    assert _split_bytes(lib, 1, 1, 60000) == 0        # 469 tiles, but 469 in one sequence
    assert _split_bytes(lib, 3, 2, 8192) > 0          # 64 tiles per sequence, 384 in all
    assert _split_bytes(lib, 3, 2, 8193) == 0         # 65 tiles per sequence
    assert _split_bytes(lib, 0, 2, 100) == 0
    # the prefill workspace covers either use
    full = ctypes.c_int64(0)
    assert lib.dash_attn_prefill_workspace_size(1, 10, 2730, 2730, 8, 128, 64, full) == 0
    assert full.value >= _split_bytes(lib, 1, 10, 2730)
