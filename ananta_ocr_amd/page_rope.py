"""Page2D RoPE state of an OCR prompt on the HIP kernels, without host synchronisation.

The two-axis RoPE gives every token a (token, page) coordinate: the page is the
<PAGE>-marker count (image pages of the prompt, then response pages counted again from
the prompt's instruction), the token coordinate the running count inside that page.
Counterparts of the reference (_sparse_base_impl.py):

* ``build_page_rope_pos``  -- _build_page_rope_pos + _page_rope_offsets (:2269-2362), as
  device tensors: coordinates, per-page prefill counts, the batch's page count and the
  "use 2-D" flag the reference decides on the host (dash_page_rope_pos)
* ``_build_page_rope_pos`` -- the same with the reference's signature and return value
  ((tok, page) or None; the None decision reads the flag once, as the reference's own
  checks do), setting ``_page_rope_meta`` on the indexer
* ``PageRope2D`` (= ``DeepseekV2IndexerRotary2D``) -- the cos/sin of the two axes
  (:1814-1891; dash_rope2d_cos_sin)
* ``main_rope_coords``     -- _main_rope_coords (:1356-1390): prefill coordinates and the
  per-step decode advance (dash_page_rope_advance), state kept on ``past_kv``
* ``page2d_cos_sin``       -- coordinates straight to cos/sin, with the 1-D fallback chosen
  on the device, for the router front end (no host read at all)
"""

import ctypes
from dataclasses import dataclass

import torch
import torch.nn as nn

from . import _lib
from .ops import _need_gpu, _ptr, _stream
from .pages import _ids


@dataclass
class PageRopePos:
    """Device results of dash_page_rope_pos for B rows of L tokens."""
    tok: torch.Tensor        # [B, L] int64
    page: torch.Tensor       # [B, L] int64
    pf_cnt: torch.Tensor     # [B, L + 1] int64, tokens of page p up to the last image token
    meta: torch.Tensor       # [2] int64: 1 + the largest page id, 1 if 2-D applies

    @property
    def n_pg(self):
        return self.meta[0]

    @property
    def ok(self):
        return self.meta[1] != 0


def build_page_rope_pos(source_input_ids, key_length, image_token_id, page_token_id,
                        page_span=0):
    """Page2D coordinates of [B, key_length] prompt ids (cut or padded with -1 to
    key_length, as _build_page_rope_pos does) on the GPU, with no host read."""
    _need_gpu(source_input_ids)
    lib = _lib.load()
    ids = _ids(source_input_ids, key_length)
    B, L = ids.shape
    dev = ids.device
    tok = torch.empty(B, L, dtype=torch.int64, device=dev)
    page = torch.empty(B, L, dtype=torch.int64, device=dev)
    pf = torch.empty(B, L + 1, dtype=torch.int64, device=dev)
    meta = torch.empty(2, dtype=torch.int64, device=dev)
    nbytes = ctypes.c_int64(0)
    _lib.check(lib.dash_page_rope_workspace_size(B, L, nbytes), "workspace")
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=dev)
    st = lib.dash_page_rope_pos(_ptr(ids), ids.stride(0), B, L, int(image_token_id),
                                int(page_token_id), int(page_span), _ptr(tok), _ptr(page),
                                _ptr(pf), pf.stride(0), _ptr(meta), _ptr(ws), ws.numel(),
                                _stream())
    _lib.check(st, "dash_page_rope_pos")
    return PageRopePos(tok, page, pf, meta)


def _build_page_rope_pos(idx, source_input_ids, key_length):
    """(tok_pos, page_pos) [B, key_length] int64, or None where the reference falls back
    to 1-D (_sparse_base_impl.py:2269-2312), for the indexer ``idx`` (its
    image_token_id, page_token_id, rope_page_span); sets ``idx._page_rope_meta`` =
    {'pf_cnt', 'n_pg'} (pf_cnt [B, key_length + 1], n_pg a device scalar)."""
    if source_input_ids is None or getattr(source_input_ids, "ndim", 0) != 2:
        return None
    if getattr(idx, "image_token_id", None) is None or getattr(idx, "page_token_id", None) is None:
        return None
    dev = idx.q_proj.weight.device if hasattr(idx, "q_proj") else source_input_ids.device
    pos = build_page_rope_pos(source_input_ids.to(dev), key_length, idx.image_token_id,
                              idx.page_token_id, int(getattr(idx, "rope_page_span", 0) or 0))
    if not bool(pos.ok):
        return None
    idx._page_rope_meta = {"pf_cnt": pos.pf_cnt, "n_pg": pos.n_pg}
    return pos.tok, pos.page


def rotary2d_inv_freq(dim, base_tok, base_page, page_pairs, tok_freq_mode="resample"):
    """Inverse frequencies of the token and page pairs (_sparse_base_impl.py:1848-1873),
    computed on the host as the reference's buffers are."""
    half = dim // 2
    page_pairs = int(page_pairs)
    if not (0 < page_pairs < half):
        raise ValueError(f"[IndexerRotary2D] page_pairs={page_pairs} must be in (0, {half}); "
                         f"dim={dim}")
    n_tok = half - page_pairs
    ar = torch.arange(0, n_tok, dtype=torch.int64).float()
    if str(tok_freq_mode).lower() == "truncate":
        inv_tok = 1.0 / (base_tok ** (ar * 2 / dim))
    else:
        inv_tok = 1.0 / (base_tok ** (ar / n_tok))
    inv_page = 1.0 / (base_page ** (torch.arange(0, page_pairs, dtype=torch.int64).float()
                                    / page_pairs))
    return inv_tok, inv_page


class PageRope2D(nn.Module):
    """Two-axis RoPE over (tok_pos, page_pos), DeepseekV2IndexerRotary2D
    (_sparse_base_impl.py:1814-1891): frequency pairs [0, n_tok) turn with the token
    coordinate, pairs [n_tok, dim/2) with the page coordinate (folded mod page_mod when
    page_mod > 0); cos/sin [B, S, dim] in x's dtype."""

    def __init__(self, dim, base_tok, base_page, page_pairs, tok_freq_mode="resample",
                 page_mod=0):
        super().__init__()
        inv_tok, inv_page = rotary2d_inv_freq(dim, base_tok, base_page, page_pairs,
                                              tok_freq_mode)
        self.register_buffer("inv_tok", inv_tok, persistent=False)
        self.register_buffer("inv_page", inv_page, persistent=False)
        self.dim = dim
        self.n_tok = inv_tok.numel()
        self.page_pairs = inv_page.numel()
        self.base_tok = base_tok
        self.base_page = base_page
        self.tok_freq_mode = str(tok_freq_mode).lower()
        self.page_mod = int(page_mod or 0)

    @torch.no_grad()
    def forward(self, x, tok_pos, page_pos):
        """tok_pos / page_pos [B, S] int -> (cos, sin) [B, S, dim] in x.dtype."""
        _need_gpu(x)
        dt = torch.bfloat16 if x.dtype == torch.bfloat16 else torch.float32
        cos, sin = rope2d_cos_sin(tok_pos.to(x.device), page_pos.to(x.device),
                                  self.inv_tok.to(x.device), self.inv_page.to(x.device),
                                  self.page_mod, dt)
        return cos.to(x.dtype), sin.to(x.dtype)


DeepseekV2IndexerRotary2D = PageRope2D


def rope2d_cos_sin(tok_pos, page_pos, inv_tok, inv_page, page_mod, dtype):
    """dash_rope2d_cos_sin: cos/sin [B, S, 2 (n_tok + page_pairs)] (bf16 or fp32)."""
    _need_gpu(tok_pos, page_pos)
    lib = _lib.load()
    tok = tok_pos.to(torch.int64)
    page = page_pos.to(torch.int64)
    if tok.shape != page.shape:
        page = page.expand(tok.shape)
    tok = tok.contiguous()
    page = page.contiguous()
    B, S = tok.shape
    it = inv_tok.float().contiguous()
    ip = inv_page.float().contiguous()
    dim = 2 * (it.numel() + ip.numel())
    cos = torch.empty(B, S, dim, dtype=dtype, device=tok.device)
    sin = torch.empty_like(cos)
    st = lib.dash_rope2d_cos_sin(_ptr(tok), _ptr(page), tok.stride(0), B, S, _ptr(it), it.numel(),
                                 _ptr(ip), ip.numel(), int(page_mod), _ptr(cos), _ptr(sin),
                                 int(dtype == torch.bfloat16), cos.stride(0), cos.stride(1),
                                 _stream())
    _lib.check(st, "dash_rope2d_cos_sin")
    return cos, sin


def page2d_cos_sin(pos, rope2d, fallback, dtype):
    """cos/sin of prompt coordinates ``pos`` (build_page_rope_pos) through ``rope2d``, or,
    where the reference would fall back to 1-D, the ``fallback`` (cos, sin) -- chosen on
    the device, so that nothing reads the flag on the host."""
    c2, s2 = rope2d_cos_sin(pos.tok, pos.page, rope2d.inv_tok.to(pos.tok.device),
                            rope2d.inv_page.to(pos.tok.device), rope2d.page_mod, dtype)
    c1, s1 = fallback
    return torch.where(pos.ok, c2, c1.to(dtype)), torch.where(pos.ok, s2, s1.to(dtype))


@dataclass
class PageRopeState:
    """Per-layer decode state of the page coordinates (the reference's
    past_kv._page_rope_state[layer] entry), all on the device."""
    page: torch.Tensor       # [B] int64, page of the last token
    tok: torch.Tensor        # [B] int64, token coordinate of the last token
    pf_cnt: torch.Tensor     # [B, >= n_pg] int64
    n_pg: torch.Tensor       # device scalar

    def __getitem__(self, k):            # the reference's dict keys
        return getattr(self, k)


def page_rope_advance(state, new_ids, page_token_id):
    """One generated token per row: the state (a PageRopeState, or the reference's dict
    with 'page', 'tok', 'pf_cnt', 'n_pg') moves in place (dash_page_rope_advance); returns
    the new (tok [B, 1], page [B, 1])."""
    lib = _lib.load()
    page, tok, pf = state["page"], state["tok"], state["pf_cnt"]
    _need_gpu(new_ids, page, tok, pf)
    dev = page.device
    for key, t in (("page", page), ("tok", tok)):
        if t.dtype != torch.int64 or not t.is_contiguous():
            t = t.to(torch.int64).contiguous()
            if isinstance(state, dict):
                state[key] = t
            else:
                setattr(state, key, t)
    page, tok = state["page"], state["tok"]
    n_pg = state["n_pg"]
    if not torch.is_tensor(n_pg) or n_pg.dtype != torch.int64 or n_pg.device != dev:
        n_pg = torch.as_tensor(n_pg, dtype=torch.int64, device=dev)
    n_pg = n_pg.reshape(1).contiguous()
    pf = pf.to(torch.int64)
    if pf.stride(-1) != 1:
        pf = pf.contiguous()
    B = page.shape[0]
    ids = new_ids.reshape(B, -1)[:, -1].to(device=dev, dtype=torch.int64).contiguous()
    out_t = torch.empty(B, dtype=torch.int64, device=dev)
    out_p = torch.empty(B, dtype=torch.int64, device=dev)
    st = lib.dash_page_rope_advance(_ptr(ids), 1, B, int(page_token_id), _ptr(page), _ptr(tok),
                                    _ptr(pf), pf.stride(0), _ptr(n_pg), _ptr(out_t), _ptr(out_p),
                                    _stream())
    _lib.check(st, "dash_page_rope_advance")
    return out_t[:, None], out_p[:, None]


def main_rope_coords(layer, q_len, past_kv):
    """_main_rope_coords (_sparse_base_impl.py:1356-1390) for an attention ``layer`` with
    ``indexer`` (image_token_id, page_token_id, rope_page_span), ``_main_rope_pos_2d``,
    ``_sparse_source_input_ids`` and ``layer_idx``.  Prefill (q_len > 1): the prompt's
    coordinates, and the decode state kept on ``past_kv._page_rope_state[layer_idx]``;
    decode: the state advanced by the newest token id.  None where the reference falls
    back to 1-D."""
    idx = getattr(layer, "indexer", None)
    if idx is None:
        return None
    if q_len > 1:
        coords = getattr(layer, "_main_rope_pos_2d", None)
        if coords is None:
            src = getattr(layer, "_sparse_source_input_ids", None)
            coords = _build_page_rope_pos(idx, src, q_len)
            layer._main_rope_pos_2d = coords
        if coords is None or coords[0].shape[-1] != q_len:
            return None
        if past_kv is not None:
            meta = getattr(idx, "_page_rope_meta", None)
            if meta is not None:
                st = getattr(past_kv, "_page_rope_state", None)
                if st is None:
                    st = {}
                    past_kv._page_rope_state = st
                st[layer.layer_idx] = PageRopeState(
                    page=coords[1][:, -1].clone(), tok=coords[0][:, -1].clone(),
                    pf_cnt=meta["pf_cnt"], n_pg=meta["n_pg"])
        return coords
    st = getattr(past_kv, "_page_rope_state", None) if past_kv is not None else None
    st = st.get(layer.layer_idx) if st else None
    ids = getattr(layer, "_sparse_source_input_ids", None)
    if st is None or ids is None or ids.shape[-1] < 1:
        return None
    return page_rope_advance(st, ids[:, -1], idx.page_token_id)
