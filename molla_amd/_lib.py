"""Loads libmolla_mi.so (the HIP/gfx950 kernels behind include/molla_mi.h).

There is no fallback: if the library is missing or fails to load, every
entry point raises.  Build it with `make -C molla_amd/csrc` or
`__graft_entry__.build()`.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmolla_mi.so")

P, I32, I64, F, SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t


class MiWeight(ctypes.Structure):
    _fields_ = [("data", P), ("kind", I32), ("rows", I32), ("cols", I32), ("row_bytes", I64)]


class MiLayerDesc(ctypes.Structure):
    _fields_ = [("width", I32), ("hidden", I32), ("heads", I32), ("kv_heads", I32), ("head_dim", I32),
                ("rope_dim", I32), ("neox", I32), ("eps", F), ("attn_scale", F), ("attn_norm", P),
                ("ffn_norm", P), ("rope_steps", P)] + \
               [(n, MiWeight) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] + \
               [("rope_factors", P), ("cache_form", I32)] + \
               [(n, P) for n in ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "attn_post_norm",
                                 "ffn_post_norm")] + \
               [("ungated", I32), ("act", I32), ("next_norm", P), ("prenormed", I32)]


# Every symbol include/molla_mi.h declares, with its C signature.
SIGNATURES = {
    "mi_version": (ctypes.c_int, []),
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_sync": (ctypes.c_int, [P]),
    "mi_block_elements": (ctypes.c_int, [ctypes.c_int]),
    "mi_block_bytes": (ctypes.c_int, [ctypes.c_int]),
    "mi_row_bytes": (I64, [ctypes.c_int, I32]),
    "mi_dequant": (ctypes.c_int, [P, ctypes.c_int, P, I64, P]),
    "mi_matvec_workspace": (SZ, [I32, I32]),
    "mi_matmul_workspace": (SZ, [I32, I32, I32]),
    "mi_matvec": (ctypes.c_int, [P, ctypes.c_int, P, I64, I32, I32, P, I32, P, I32, P, P, SZ]),
    "mi_matvec_noalloc": (ctypes.c_int, [P, ctypes.c_int, P, I64, I32, I32, P, I32, P, I32, P]),
    "mi_quantize": (ctypes.c_int, [P, P, I32, I32, P]),
    "mi_matvec_xq": (ctypes.c_int, [P, ctypes.c_int, P, I64, I32, I32, P, I32, P, I32, P]),
    "mi_rms_norm": (ctypes.c_int, [P, P, P, I32, I32, F, P, P]),
    "mi_rope_steps": (None, [P, I32, F]),
    "mi_rope": (ctypes.c_int, [P, P, I32, I32, I32, I32, P, P, I32, I64]),
    "mi_store_kv": (ctypes.c_int, [P, P, P, I32, P, P, I32]),
    "mi_attend_workspace": (SZ, [I32, I32, I32]),
    "mi_attend": (ctypes.c_int, [P, P, P, P, I32, I32, I32, F, I32, P, P, SZ]),
    "mi_cache_row": (I32, [I32, I32]),
    "mi_store_kv_form": (ctypes.c_int, [P, I32, P, P, I32, P, P, I32]),
    "mi_attend_form": (ctypes.c_int, [P, I32, P, P, P, I32, I32, I32, F, I32, P, P, SZ]),
    "mi_argmax": (ctypes.c_int, [P, P, I32, I32, P]),
    "mi_argmax_workspace": (SZ, [I32, I32]),
    "mi_matvec_route": (ctypes.c_int, [ctypes.c_int, I32, I32, I32, SZ, P]),
    "mi_argmax_ws": (ctypes.c_int, [P, P, I32, I32, P, P, SZ, P, P]),
    "mi_embed": (ctypes.c_int, [P, P, I32, I32, P, I32, P]),
    "mi_layer_workspace": (SZ, [ctypes.POINTER(MiLayerDesc), I32, I32]),
    "mi_decoder_layer": (ctypes.c_int, [P, ctypes.POINTER(MiLayerDesc), P, P, P, I64, P, I32, I32, P, SZ]),
    "mi_decoder_layer_paged": (ctypes.c_int, [P, ctypes.POINTER(MiLayerDesc), P, P, P, P, I64, P, I32, I32, P,
                                              SZ]),
}

_lib = None


class MiError(RuntimeError):
    """A refusal or device error reported by the library (mi_last_error)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"molla_mi error {code}: {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C molla_amd/csrc` "
                               "(there is no CPU fallback for the device kernels)")
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise MiError(rc, lib().mi_last_error().decode(errors="replace"))
