"""The C-ABI library loads, exports every symbol include/molla_mi.h declares,
and refuses bad arguments before touching a device (no GPU needed: every
call here returns from the argument checks in shim.cpp / layer.cpp)."""

import ctypes
import os
import re

import numpy as np
import pytest

import oracle
from molla_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "molla_mi.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_geometry_matches_reference_table():
    lib = _lib.lib()
    for kind in (2, 3, 6, 7, 8, 12, 13, 14):
        assert lib.mi_block_elements(kind) == oracle.block_elements(kind)
        assert lib.mi_block_bytes(kind) == oracle.block_bytes(kind)
    assert lib.mi_row_bytes(12, 4096) == 2304
    assert lib.mi_row_bytes(14, 4096) == 3360
    assert lib.mi_row_bytes(8, 896) == 952
    assert lib.mi_row_bytes(12, 300) == -1


def test_cache_rows():
    # tests/test_repack.mojo:561-600: an f16 row is the width; a q8_0 row is a
    # byte a value plus a half a 32-block, rounded up to 8 halves, under 5/8 of
    # the f16 row; a width of partial blocks has no q8 row.
    lib = _lib.lib()
    assert lib.mi_cache_row(0, 1024) == 1024
    assert lib.mi_cache_row(1, 1024) == 544
    for heads in range(1, 17):
        w = heads * 128
        row = lib.mi_cache_row(1, w)
        assert row % 8 == 0 and row * 8 < lib.mi_cache_row(0, w) * 5
    assert lib.mi_cache_row(1, 48) == -1 and lib.mi_cache_row(2, 64) == -1 and lib.mi_cache_row(0, 0) == -1


def test_rope_steps_match_oracle():
    lib = _lib.lib()
    for dim, base in ((128, 500000.0), (64, 10000.0), (8, 10000.0)):
        got = np.zeros(dim // 2, np.float32)
        lib.mi_rope_steps(got.ctypes.data_as(ctypes.c_void_p), dim, base)
        assert (got == oracle.rope_steps(dim, base)).all()


def _err(rc):
    return rc, _lib.lib().mi_last_error().decode()


def test_refusals_before_launch():
    lib = _lib.lib()
    fake = 0x100000  # never dereferenced: every case below is refused first
    # unknown kind
    rc, msg = _err(lib.mi_matvec_xq(None, 19, fake, 100, 4, 256, fake, 1, fake, 0, None))
    assert rc == -2 and "19" in msg
    # row_bytes mismatch
    rc, msg = _err(lib.mi_matvec_xq(None, 12, fake, 2300, 4, 4096, fake, 1, fake, 0, None))
    assert rc == -3 and "row_bytes" in msg
    # columns not whole superblocks
    rc, _ = _err(lib.mi_matvec_xq(None, 12, fake, 144, 4, 300, fake, 1, fake, 0, None))
    assert rc == -3
    # misaligned q4_k weight
    rc, _ = _err(lib.mi_matvec_xq(None, 12, fake + 4, 2304, 4, 4096, fake, 1, fake, 0, None))
    assert rc == -6
    # tokens out of range
    rc, _ = _err(lib.mi_matvec_xq(None, 12, fake, 2304, 4, 4096, fake, 9, fake, 0, None))
    assert rc == -1
    # GLU without aux
    rc, _ = _err(lib.mi_matvec_xq(None, 12, fake, 2304, 4, 4096, fake, 1, fake, 4, None))
    assert rc == -1
    # workspace too small
    rc, msg = _err(lib.mi_matvec(None, 12, fake, 2304, 4, 4096, fake, 1, fake, 0, None, fake, 16))
    assert rc == -4 and "workspace" in msg
    # dequant of a partial block
    rc, _ = _err(lib.mi_dequant(None, 14, fake, 300, fake))
    assert rc == -3
    # attention with no keys
    rc, msg = _err(lib.mi_attend(None, fake, fake, fake, 32, 8, 128, 0.1, 0, fake, fake, 1 << 20))
    assert rc == -3 and "at least one key" in msg
    # GQA group that is not 1/2/4/8
    rc, _ = _err(lib.mi_attend(None, fake, fake, fake, 12, 4, 128, 0.1, 5, fake, fake, 1 << 20))
    assert rc == -3


def test_layer_refuses_wrong_projection_shape():
    lib = _lib.lib()
    d = _lib.MiLayerDesc()
    d.width, d.hidden, d.heads, d.kv_heads, d.head_dim, d.rope_dim = 256, 512, 4, 2, 64, 64
    d.eps, d.attn_scale = 1e-5, 0.125
    d.attn_norm = d.ffn_norm = d.rope_steps = 0x100000
    shapes = {"wq": (256, 256), "wk": (128, 256), "wv": (128, 256), "wo": (256, 256),
              "gate": (512, 256), "up": (512, 256), "down": (256, 512)}
    for n, (r, c) in shapes.items():
        setattr(d, n, _lib.MiWeight(0x100000, 12, r, c, c // 256 * 144))
    d.wk = _lib.MiWeight(0x100000, 12, 256, 256, 144)  # wrong rows
    rc = lib.mi_decoder_layer(None, ctypes.byref(d), 0x100000, 0x100000, 0x100000, 0, 0x100000, 8, 1,
                              0x100000, 1 << 24)
    assert rc == -3 and "wk" in lib.mi_last_error().decode()


def test_mojo_binding_covers_the_header():
    """mojo/molla_mi.mojo binds every symbol include/molla_mi.h declares
    (one external_call each) and lays out mi_layer_desc at the C offsets."""
    import ctypes
    import re
    with open(os.path.join(ROOT, "mojo", "molla_mi.mojo")) as f:
        text = f.read()
    bound = set(re.findall(r'external_call\["(mi_[a-z0-9_]+)"', text))
    missing = [n for n in declared_symbols() if n not in bound]
    assert not missing, missing
    D = _lib.MiLayerDesc
    offsets = {"WEIGHTS": D.wq.offset, "ROPE_FACTORS": D.rope_factors.offset, "CACHE_FORM": D.cache_form.offset,
               "Q_BIAS": D.q_bias.offset, "K_BIAS": D.k_bias.offset, "V_BIAS": D.v_bias.offset,
               "Q_NORM": D.q_norm.offset, "K_NORM": D.k_norm.offset, "ATTN_POST_NORM": D.attn_post_norm.offset,
               "FFN_POST_NORM": D.ffn_post_norm.offset, "UNGATED": D.ungated.offset, "ACT": D.act.offset,
               "NEXT_NORM": D.next_norm.offset, "PRENORMED": D.prenormed.offset, "SIZE": ctypes.sizeof(D)}
    for name, want in offsets.items():
        m = re.search(rf"comptime {name} = (\d+)", text)
        assert m and int(m.group(1)) == want, (name, want)
    assert ctypes.sizeof(_lib.MiWeight) == 32
