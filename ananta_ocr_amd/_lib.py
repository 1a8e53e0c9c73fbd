"""ctypes binding of libdash_hip.so (the C ABI declared in include/dash_hip.h).

The library is built in-tree by ``ananta_ocr_amd.build``.  There is no CPU or
eager-PyTorch fallback: if the library is missing, every GPU entry point raises.
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdash_hip.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_f = ctypes.c_float

# name -> (restype, argtypes); mirrors include/dash_hip.h
SIGNATURES = {
    "dash_abi_version": (_i, []),
    "dash_status_string": (ctypes.c_char_p, [_i]),
    "dash_kbar": (_i, [_p, _l, _l, _l, _p, _p, _p, _l, _i, _p, _i, _i, _i, _i, _i, _p, _l, _i, _p]),
    "dash_block_scores": (_i, [_p, _l, _l, _p, _i, _p, _p, _l, _i, _p, _p, _i, _i, _i, _i, _i,
                               _p, _l, _p]),
    "dash_block_max_score": (_i, [_p, _l, _l, _i, _p, _p, _l, _p, _l, _l, _i, _i, _i, _i, _i,
                                  _i, _i, _p, _l, _l, _p]),
    "dash_router_qk_norm": (_i, [_p, _i, _l, _l, _i, _i, _p, _p, _f, _p, _p, _i, _l, _l, _p, _p,
                                 _p]),
    "dash_router_front": (_i, [_p, _l, _l, _i, _i, _i, _p, _p, _p, _p, _p, _f, _p, _p, _i, _l, _l,
                               _p, _i, _f, _p, _l, _p, _l, _p, _l, _i, _p]),
    "dash_router_front_pack_weights": (_i, [_p, _p, _i, _p, _p]),
    "dash_route": (_i, [_p, _l, _i, _i, _p, _p, _l, _f, _f, _f, _i, _i, _i, _p, _p, _p, _p]),
    "dash_train_route": (_i, [_p, _l, _i, _i, _p, _p, _l, _f, _f, _f, _i, _i, _p, _p, _p, _p,
                              _p, _p]),
    "dash_train_route_backward": (_i, [_p, _l, _i, _i, _p, _p, _l, _f, _f, _f, _i, _p, _p, _p,
                                       _p, _p, _p, _l, _p]),
    "dash_attn_prefill": (_i, [_p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l,
                               _p, _l, _l, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f,
                               _i, _l, _p, _l, _p]),
    "dash_attn_prefill_workspace_size": (_i, [_i, _i, _i, _l, _i, _i, _i, ctypes.POINTER(_l)]),
    "dash_attn_prefill_split_workspace_size": (_i, [_i, _i, _i, _i, ctypes.POINTER(_l)]),
    "dash_attn_prefill_backward_workspace_size": (_i, [_i, _i, _i, _l, _i, _i, _i,
                                                       ctypes.POINTER(_l)]),
    "dash_attn_prefill_backward": (_i, [_p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l,
                                        _p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l,
                                        _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f,
                                        _p, _l, _l, _l, _p, _l, _l, _l, _p, _l, _l, _l,
                                        _p, _l, _p, _l, _p]),
    "dash_attn_prefill_error_offset": (_i, [_i, _i, _i, _l, _i, _i, _i, ctypes.POINTER(_l)]),
    "dash_prefill_plan_target": (_i, [_l, _l, _l, _l, _l, ctypes.POINTER(_l), ctypes.POINTER(_l)]),
    "dash_decode_route": (_i, [_p, _l, _p, _l, _l, _l, _p, _l, _i, _p, _p, _i, _p, _i, _p, _l, _i,
                               _p, _l, _p,
                               _p, _l, _i, _i, _i, _i, _f, _f, _f, _i, _i, _i, _p, _p, _p, _p,
                               _l, _p]),
    "dash_attn_decode_workspace_size": (_i, [_i, _i, _i, _i, ctypes.POINTER(_l)]),
    "dash_attn_decode": (_i, [_p, _l, _l, _p, _l, _l, _l, _l, _p, _l, _l, _l, _l, _p, _l, _i,
                              _p, _p, _p, _p, _p, _i, _p, _i, _l, _l, _p, _l, _l, _i, _i, _i,
                              _i, _i, _i, _f, _i, _p, _l, _p]),
    "dash_decode_step_workspace_size": (_i, [_i, _i, _i, _i, _i, ctypes.POINTER(_l)]),
    "dash_decode_step": (_i, [_p, _l, _p, _l, _l, _l, _p, _l, _i, _p, _p, _i, _p, _i, _p, _l, _i,
                              _p, _l, _p,
                              _p, _l, _i, _i, _f, _f, _f, _i, _i, _i, _p, _p, _p, _p, _l,
                              _p, _l, _l, _p, _l, _l, _l, _l, _p, _l, _l, _l, _l,
                              _p, _i, _l, _l, _p, _l, _l, _i, _i, _i, _i, _i, _f, _p, _l, _p]),
    "dash_decode_step_noalloc": (_i, [_p, _l, _p, _l, _l, _l, _p, _l, _i, _p, _p, _i, _p, _i, _p,
                                      _l, _i, _p, _l, _p,
                                      _p, _l, _i, _i, _f, _f, _f, _i, _i, _i, _p, _p, _p,
                                      _p, _l, _p, _l, _l, _p, _l, _l, _l, _l, _p, _l, _l, _l,
                                      _l, _p, _i, _l, _l, _p, _l, _l, _i, _i, _i, _i, _i, _f,
                                      _p]),
    "dash_decode_step_scratch_bytes": (_l, []),
    "dash_decode_win_bounds": (_i, [_p, _l, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p]),
    "dash_page_ids": (_i, [_p, _l, _i, _i, _l, _l, _i, _i, _p, _p, _p, _p, _p, _l, _p]),
    "dash_pages_workspace_size": (_i, [_i, _i, ctypes.POINTER(_l)]),
    "dash_block_pages": (_i, [_p, _l, _i, _i, _i, _i, _p, _p, _p, _p]),
    "dash_block_cand": (_i, [_p, _l, _i, _p, _l, _i, _p, _l, _i, _p, _p, _p, _i, _i, _i, _i,
                             _p, _l, _l, _p]),
    "dash_decode_page_state": (_i, [_p, _l, _i, _i, _l, _l, _i, _i, _i, _p, _p, _p, _p, _p, _l,
                                    _p]),
    "dash_decode_allow": (_i, [_p, _l, _i, _l, _p, _p, _i, _p, _p, _i, _p, _l, _p]),
    "dash_page_rope_workspace_size": (_i, [_i, _i, ctypes.POINTER(_l)]),
    "dash_page_rope_pos": (_i, [_p, _l, _i, _i, _l, _l, _i, _p, _p, _p, _l, _p, _p, _l, _p]),
    "dash_rope2d_cos_sin": (_i, [_p, _p, _l, _i, _i, _p, _i, _p, _i, _i, _p, _p, _i, _l, _l,
                                 _p]),
    "dash_page_rope_advance": (_i, [_p, _l, _i, _l, _p, _p, _p, _l, _p, _p, _p, _p]),
}

_LIB = None


class DashError(RuntimeError):
    pass


def load(path=LIB_PATH):
    """Load (once) and return the library with argtypes set."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is missing: build it with `python -m ananta_ocr_amd.build` "
            f"(hipcc --offload-arch=gfx950).  There is no CPU fallback.")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def check(status, what):
    """Map a status code to an exception."""
    if status == 0:
        return
    msg = load().dash_status_string(status).decode()
    if status == -2:
        raise NotImplementedError(f"{what}: {msg}")
    raise DashError(f"{what}: {msg} (status {status})")
