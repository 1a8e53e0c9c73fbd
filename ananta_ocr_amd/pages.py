"""Page-aware routing candidates on the HIP kernels (csrc/dash_pages.hip).

An OCR prompt holds the image tokens of every page, each page opened by a
``<PAGE>`` marker (or, without markers, a fixed number of image tokens per page).
Routing restricts a query's remote blocks to the image blocks of its own page.
Counterparts of the reference's functions, with their names and arguments:

* ``build_page_aware_ids``       -- _build_page_aware_ids (_sparse_base_impl.py:2189-2259)
* ``build_flat_image_token_mask`` -- _build_flat_image_token_mask (:2363-2380)
* ``build_kl_candidate_mask``    -- _build_kl_candidate_mask (:2457-2484) with
                                    _build_page_aware_image_block_mask (:2436-2455)
* ``_dash_page_ids`` / ``_dash_block_cand`` -- modeling_deepseekv2.py:87-110
* ``_uocr_dash_decode_allow``    -- modeling_anantaocr.py:450-496

``block_cand`` is the one-call form the prefill uses: [B, S, nblk] candidates for
every query in one launch (plus two small ones), without the reference's query
chunking and without host synchronisation.  The reference-named functions keep
its ``None`` returns, which need one synchronisation to decide.
"""

import ctypes
import os

import torch

from . import _lib
from .ops import _need_gpu, _ptr, _stream

PER_PAGE_IMAGE_TOKENS = 273
# Whether prompt tokens carry their page as queries (the reference's _PAGE_SCOPE_PREFILL,
# _sparse_base_impl.py:36: environment PAGE_SCOPE_PREFILL, switched on by
# configure_dash_inference(page_scope_prefill=True)).
PAGE_SCOPE = {"prefill": os.environ.get("PAGE_SCOPE_PREFILL", "0") == "1"}


def _workspace(B, L, device):
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().dash_pages_workspace_size(B, L, n), "dash_pages_workspace_size")
    return torch.empty((n.value + 15) // 16 * 4, dtype=torch.int32, device=device)


def _ids(source_input_ids, key_length):
    ids = source_input_ids[..., :key_length]
    if ids.shape[-1] < key_length:
        ids = torch.nn.functional.pad(ids, (0, key_length - ids.shape[-1]), value=-1)
    return ids.to(torch.int64).contiguous()


def page_ids(source_input_ids, image_token_id, page_token_id, key_length,
             per_page_image_tokens=PER_PAGE_IMAGE_TOKENS, page_scope_prefill=False):
    """(image_token_mask bool, image_token_page_ids int32, query_token_page_ids int32,
    enabled int32 [B, 2]) for token ids [B, L], padded with -1 or cut to key_length.
    enabled[b] = (row b has an image token, row b has a query page)."""
    _need_gpu(source_input_ids)
    lib = _lib.load()
    ids = _ids(source_input_ids, key_length)
    B, L = ids.shape
    dev = ids.device
    img = torch.empty(B, L, dtype=torch.uint8, device=dev)
    ipi = torch.empty(B, L, dtype=torch.int32, device=dev)
    qpi = torch.empty(B, L, dtype=torch.int32, device=dev)
    en = torch.empty(B, 2, dtype=torch.int32, device=dev)
    pt = -(1 << 62) if page_token_id is None else int(page_token_id)
    ws = _workspace(B, L, dev)
    st = lib.dash_page_ids(_ptr(ids), ids.stride(0), B, L, int(image_token_id), pt,
                           int(per_page_image_tokens), int(bool(page_scope_prefill)), _ptr(img),
                           _ptr(ipi), _ptr(qpi), _ptr(en), _ptr(ws), ws.numel() * 4, _stream())
    _lib.check(st, "dash_page_ids")
    return img.view(torch.bool), ipi, qpi, en


def build_page_aware_ids(source_input_ids, img_context_token_id, page_token_id, key_length,
                         per_page_image_tokens=PER_PAGE_IMAGE_TOKENS, page_scope_prefill=False):
    """(image_token_mask, image_token_page_ids, query_token_page_ids) [B, key_length]
    (ids as int64, as the reference returns them), or (None, None, None) when an id is
    missing, the ids are not [B, L], or the batch has no image token or no query page."""
    if source_input_ids is None or img_context_token_id is None or page_token_id is None:
        return None, None, None
    if source_input_ids.ndim != 2:
        return None, None, None
    img, ipi, qpi, en = page_ids(source_input_ids, img_context_token_id, page_token_id,
                                 key_length, per_page_image_tokens, page_scope_prefill)
    if not bool(en.any(0).all()):
        return None, None, None
    return img, ipi.long(), qpi.long()


def build_flat_image_token_mask(source_input_ids, img_context_token_id, key_length):
    """[B, key_length] bool image-token mask over all pages, or None without image tokens."""
    if source_input_ids is None or img_context_token_id is None:
        return None
    if source_input_ids.ndim != 2:
        return None
    mask = _ids(source_input_ids, key_length) == img_context_token_id
    if not bool(mask.any()):
        return None
    return mask


def block_pages(image_page_ids, num_key_blocks, block_size):
    """(bmin, bmax, bits) [B, nblk] of the image pages of every key block."""
    _need_gpu(image_page_ids)
    lib = _lib.load()
    ipi = image_page_ids.to(torch.int32).contiguous()
    B, L = ipi.shape
    dev = ipi.device
    bmin = torch.empty(B, num_key_blocks, dtype=torch.int32, device=dev)
    bmax = torch.empty_like(bmin)
    bits = torch.empty(B, num_key_blocks, dtype=torch.int64, device=dev)
    st = lib.dash_block_pages(_ptr(ipi), ipi.stride(0), B, L, int(block_size),
                              int(num_key_blocks), _ptr(bmin), _ptr(bmax), _ptr(bits), _stream())
    _lib.check(st, "dash_block_pages")
    return bmin, bmax, bits


def block_cand(pos_ids, num_key_blocks, block_size, image_token_mask=None,
               image_token_page_ids=None, query_token_page_ids=None,
               image_bucket_constraint=True, out=None):
    """[B, Lq, nblk] bool routing candidates of the queries at pos_ids [B, Lq]: the image
    blocks of the query's page (image_bucket_constraint with page ids), every image block
    (page ids missing, or no bucket constraint), or every block (no image mask); a row
    without a candidate allows every block."""
    _need_gpu(pos_ids)
    lib = _lib.load()
    pos = pos_ids.to(torch.int32).contiguous()
    B, Lq = pos.shape
    nblk = int(num_key_blocks)
    dev = pos.device
    if out is None:
        out = torch.empty(B, Lq, nblk, dtype=torch.bool, device=dev)
    o8 = out.view(torch.uint8)
    if image_bucket_constraint and image_token_page_ids is not None \
            and query_token_page_ids is not None:
        mode = 0
        ipi = image_token_page_ids.to(torch.int32).contiguous()
        qpi = query_token_page_ids.to(torch.int32).contiguous()
    elif image_token_mask is not None:
        mode = 1
        ipi = torch.where(image_token_mask.bool(), 0, -1).to(torch.int32).contiguous()
        qpi = None
    else:
        mode = 2
        ipi = qpi = None
    bmin = bmax = bits = None
    if mode != 2:
        bmin, bmax, bits = block_pages(ipi, nblk, block_size)
    st = lib.dash_block_cand(
        _ptr(qpi), 0 if qpi is None else qpi.stride(0), 0 if qpi is None else qpi.shape[1],
        _ptr(pos), pos.stride(0), Lq, _ptr(ipi), 0 if ipi is None else ipi.stride(0),
        0 if ipi is None else ipi.shape[1], _ptr(bmin), _ptr(bmax), _ptr(bits), nblk, mode, B,
        int(block_size), _ptr(o8), o8.stride(0), o8.stride(1), _stream())
    _lib.check(st, "dash_block_cand")
    return out


def build_kl_candidate_mask(pos_chunk, num_key_blocks, image_token_mask, batch, cq, block_size,
                            image_token_page_ids=None, query_token_page_ids=None,
                            image_bucket_constraint=True):
    """[B, 1, cq, nblk] bool candidates of a chunk of queries (the reference's shape)."""
    c = block_cand(pos_chunk, num_key_blocks, block_size, image_token_mask,
                   image_token_page_ids, query_token_page_ids, image_bucket_constraint)
    return c[:, None]


# ----------------------------------------------------------------------------- overlay

def _dash_page_ids(self, idx, src_ids, key_length):
    """(itm, ipi, qpi) for the layer's prompt (modeling_deepseekv2.py:87-95): page-aware
    ids with the indexer's bucket constraint, else the flat image mask."""
    if idx.image_bucket_constraint:
        return build_page_aware_ids(src_ids, idx.image_token_id, idx.page_token_id, key_length,
                                    getattr(idx, "per_page_image_tokens", PER_PAGE_IMAGE_TOKENS),
                                    getattr(idx, "page_scope_prefill", PAGE_SCOPE["prefill"]))
    itm = build_flat_image_token_mask(src_ids, idx.image_token_id, key_length)
    return itm, None, None


def _dash_block_cand(self, idx, router, pos_ids, itm, ipi, qpi, nblk, bsz, q_len):
    """[B, S, nblk] per-query candidate domain (modeling_deepseekv2.py:96-110), or None
    without image tokens and page ids.  One launch for every query (the reference
    builds it in query chunks to bound a [B, S, nblk, block_size] intermediate that the
    kernel never forms)."""
    if itm is None and (ipi is None or qpi is None):
        return None
    return block_cand(pos_ids, nblk, idx.block_size, itm, ipi, qpi,
                      image_bucket_constraint=idx.image_bucket_constraint)


class DecodePageState:
    """Page state of a decode batch (modeling_anantaocr.py:465-479): per key block of the
    prompt the smallest and largest image page it holds, the prompt page count and the
    running <PAGE> marker count, on the device."""

    def __init__(self, input_ids, image_token_id, page_token_id, block_size,
                 per_page_image_tokens=PER_PAGE_IMAGE_TOKENS):
        _need_gpu(input_ids)
        lib = _lib.load()
        ids = input_ids.to(torch.int64).contiguous()
        B, L = ids.shape
        self.bs = int(block_size)
        self.page_token_id = int(page_token_id)
        nblk = (L + self.bs - 1) // self.bs
        dev = ids.device
        self.bmin = torch.empty(B, nblk, dtype=torch.int32, device=dev)
        self.bmax = torch.empty_like(self.bmin)
        self.pp = torch.empty(B, dtype=torch.int32, device=dev)
        self.markers = torch.empty(B, dtype=torch.int32, device=dev)
        ws = _workspace(B, L, dev)
        st = lib.dash_decode_page_state(_ptr(ids), ids.stride(0), B, L, int(image_token_id),
                                        self.page_token_id, int(per_page_image_tokens), self.bs,
                                        nblk, _ptr(self.bmin), _ptr(self.bmax), _ptr(self.pp),
                                        _ptr(self.markers), _ptr(ws), ws.numel() * 4, _stream())
        _lib.check(st, "dash_decode_page_state")

    def allow(self, new_ids, total_len, out=None):
        """[B, ceil(total_len / block_size)] bool allow row of the step whose token is
        new_ids [B] (or [B, L], last column); updates the marker count."""
        lib = _lib.load()
        nid = new_ids if new_ids.dim() == 1 else new_ids[:, -1]
        nid = nid.to(torch.int64)
        B = nid.shape[0]
        nblk = (int(total_len) + self.bs - 1) // self.bs
        if out is None:
            out = torch.empty(B, nblk, dtype=torch.bool, device=nid.device)
        o8 = out.view(torch.uint8)
        st = lib.dash_decode_allow(_ptr(nid), nid.stride(0), B, self.page_token_id,
                                   _ptr(self.bmin), _ptr(self.bmax), self.bmin.shape[1],
                                   _ptr(self.pp), _ptr(self.markers), nblk, _ptr(o8),
                                   o8.stride(0), _stream())
        _lib.check(st, "dash_decode_allow")
        return out


def _uocr_dash_decode_allow(indexer, input_ids, cache):
    """The decode query's page-aware remote candidates (modeling_anantaocr.py:450-496):
    a prefill call (L > 1) records the page state on ``cache`` and returns None; a
    decode call returns the [B, nblk] allow row."""
    img_id, pg_id = indexer.image_token_id, indexer.page_token_id
    if img_id is None or pg_id is None:
        return None
    B, L = input_ids.shape
    if L > 1:
        cache._dash_pg = DecodePageState(input_ids, img_id, pg_id, indexer.block_size,
                                         getattr(indexer, "per_page_image_tokens",
                                                 PER_PAGE_IMAGE_TOKENS))
        return None
    st = getattr(cache, "_dash_pg", None)
    if st is None:
        return None
    return st.allow(input_ids, int(cache.get_seq_length()) + L)


def win_bounds_decode(allow, seq_lens, max_block, block_size, local_blocks, tile=128,
                      q_pos=None, out=None):
    """Window bounds of decode rows, as the serving router computes them
    (win_bounds_decode, whl:sglang/srt/layers/attention/unlimited_dash_ops/
    route_triton.py:466-526, one decode query per sequence): the span [lo, hi) of the
    allowed remote blocks of each row, the live remote width when none is allowed, and
    whether the span fits `tile` blocks.  allow [B, W] bool/u8 (the decode allow rows);
    returns (bounds int32 [B, 2], fit bool [B]); `out` = (bounds, fit) to write in place
    (fixed buffers for graph capture)."""
    _need_gpu(allow, seq_lens)
    lib = _lib.load()
    a = allow.view(torch.uint8) if allow.dtype == torch.bool else allow
    if a.dtype != torch.uint8:
        a = a.to(torch.uint8)
    if a.stride(-1) != 1:
        a = a.contiguous()
    B = a.shape[0]
    if out is None:
        bounds = torch.empty(B, 2, dtype=torch.int32, device=a.device)
        fit = torch.empty(B, dtype=torch.uint8, device=a.device)
    else:
        bounds, fit = out
    lens = seq_lens.to(device=a.device, dtype=torch.int32).contiguous()
    qp = None if q_pos is None else q_pos.to(device=a.device, dtype=torch.int32).contiguous()
    S = int(max_block) * int(block_size)
    st = lib.dash_decode_win_bounds(_ptr(a), a.stride(0), a.shape[1], _ptr(lens), _ptr(qp), B, S,
                                    int(max_block), int(block_size), int(local_blocks), int(tile),
                                    _ptr(bounds), _ptr(fit), _stream())
    _lib.check(st, "dash_decode_win_bounds")
    return bounds, fit.view(torch.bool) if fit.dtype == torch.uint8 else fit
