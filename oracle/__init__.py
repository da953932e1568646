"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates molla's host path (src/molla/nn/quant.mojo, kernel.mojo,
rope.mojo, attention.mojo, block.mojo, model.mojo) in plain C
(`molla_oracle.c`) and wraps it with ctypes and numpy.  It is the checker the
HIP kernels are compared against and the CPU baseline bench.py times.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it;
the product path (molla_amd) never does.

Parity status per function (how each is pinned, not merely re-typed):
  dequant (all kinds)  -- reference known-answer blocks (tests/test_quant.mojo),
                          closed forms, an independent numpy decoder.
  row_dot / matvec     -- reference invariant |fused - dequant.dot| <=
                          1e-4*sum|w x| + 1e-6 (tests/test_kernel.mojo:437),
                          the 2x3 hand matvec, float64 brute force.
  rms_norm             -- mean-square-7.5 case (tests/test_kernel.mojo:280).
  softmax/silu/gelu    -- scalar cases (tests/test_kernel.mojo:161-278).
  rope                 -- ggml values at position 3 (tests/test_rope.mojo:93-190).
  attend               -- paper cases (tests/test_attention.mojo:150-236).
  layer                -- identity-weight hand case (tests/test_block.mojo:246)
                          and an independent numpy float64 layer.
  The last-ulp bits of Mojo's own exp/cos/sin are not reproducible without
  Mojo; they are "parity unpinned" at the ulp level and covered by tolerance.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmolla_oracle.so")

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = _declare(ctypes.CDLL(_LIB_PATH))
    return _lib


class Weight(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("kind", ctypes.c_int32), ("rows", ctypes.c_int32),
                ("cols", ctypes.c_int32), ("row_bytes", ctypes.c_int64)]


class Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("width", "hidden", "heads", "kv_heads", "head_dim", "rope_dim", "neox")] + \
               [(n, ctypes.c_float) for n in ("eps", "rope_base", "attn_scale")] + \
               [("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p)] + \
               [(n, Weight) for n in ("wq", "wk", "wv", "wo", "gate", "up", "down")] + \
               [("rope_factors", ctypes.c_void_p)] + \
               [(n, ctypes.c_void_p) for n in ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "attn_post_norm",
                                               "ffn_post_norm")] + \
               [("ungated", ctypes.c_int32), ("act", ctypes.c_int32)]

# block.mojo optional layer parts: f32 vectors the layer may carry
OPTIONAL_VECTORS = ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "attn_post_norm", "ffn_post_norm")


def _declare(l):
    P, I32, I64, F, U64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_uint64
    sig = {
        "or_block_elements": (ctypes.c_int, [ctypes.c_int]),
        "or_block_bytes": (ctypes.c_int, [ctypes.c_int]),
        "or_f16": (F, [ctypes.c_uint16]),
        "or_f32_to_f16": (ctypes.c_uint16, [F]),
        "or_dequant_run": (ctypes.c_int, [ctypes.c_int, P, I64, P]),
        "or_row_dot": (ctypes.c_int, [ctypes.c_int, P, P, I64, P]),
        "or_matvec": (ctypes.c_int, [ctypes.c_int, P, I64, I32, I32, P, P, I32]),
        "or_rms_norm": (None, [P, P, P, I32, F]),
        "or_softmax": (None, [P, I32]),
        "or_silu": (F, [F]),
        "or_gelu": (F, [F]),
        "or_swiglu": (None, [P, P, I32]),
        "or_argmax": (I32, [P, I32]),
        "or_rope_steps": (None, [P, I32, F]),
        "or_rope_angle": (None, [I32, F, I32, I32, P, P]),
        "or_rotate_run": (None, [P, I32, I32, I32, F, I32, I32]),
        "or_rotate_run_scaled": (None, [P, I32, I32, I32, F, I32, I32, P]),
        "or_q8_cache_round": (None, [P, I32]),
        "or_attend": (None, [I32, I32, I32, F, P, P, P, I32, P, P]),
        "or_layer_step": (ctypes.c_int, [ctypes.POINTER(Layer), P, P, P, I32, I32, I32, I32]),
        "or_layer_part": (ctypes.c_int, [ctypes.POINTER(Layer), P, P, P, I32, I32, I32, I32, I32]),
        "or_forward": (ctypes.c_int, [ctypes.POINTER(Layer), I32, P, I32, P, ctypes.POINTER(Weight),
                                      I32, I32, I32, P, P, I32, P, I32]),
        "or_xorshift_next": (U64, [ctypes.POINTER(U64)]),
        "or_test_blocks": (None, [ctypes.c_int, I32, U64, P]),
        "or_test_units": (None, [U64, I32, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    return l


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def block_elements(kind: int) -> int:
    return lib().or_block_elements(kind)


def block_bytes(kind: int) -> int:
    return lib().or_block_bytes(kind)


def row_bytes(kind: int, cols: int) -> int:
    return cols // block_elements(kind) * block_bytes(kind)


def f16(bits: int) -> float:
    return lib().or_f16(bits)


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    return np.array([lib().or_f32_to_f16(float(v)) for v in a], dtype=np.uint16)


def dequant(kind: int, blob: np.ndarray, count: int) -> np.ndarray:
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    out = np.zeros(count, dtype=np.float32)
    rc = lib().or_dequant_run(kind, _p(blob), count, _p(out))
    if rc != 0:
        raise ValueError(f"dequant refused kind {kind} count {count} (rc {rc})")
    return out


def row_dot(kind: int, blob: np.ndarray, x: np.ndarray) -> float:
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(1, dtype=np.float32)
    rc = lib().or_row_dot(kind, _p(blob), _p(x), x.size, _p(out))
    if rc != 0:
        raise ValueError(f"row_dot refused kind {kind} (rc {rc})")
    return float(out[0])


def matvec(kind: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 1) -> np.ndarray:
    """y = W x for `x` of shape (cols,) or (tokens, cols); batched calls loop."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    xs = x.reshape(-1, cols)
    y = np.zeros((xs.shape[0], rows), dtype=np.float32)
    for t in range(xs.shape[0]):
        xt = np.ascontiguousarray(xs[t])
        yt = np.zeros(rows, dtype=np.float32)
        rc = lib().or_matvec(kind, _p(w), row_bytes(kind, cols), rows, cols, _p(xt), _p(yt), threads)
        if rc != 0:
            raise ValueError(f"matvec refused (rc {rc})")
        y[t] = yt
    return y.reshape(x.shape[:-1] + (rows,)) if x.ndim > 1 else y[0]


def rms_norm(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    gain = np.ascontiguousarray(gain, dtype=np.float32)
    out = np.zeros_like(x)
    lib().or_rms_norm(_p(out), _p(x), _p(gain), x.size, eps)
    return out


def softmax(x: np.ndarray) -> np.ndarray:
    x = np.array(x, dtype=np.float32)
    lib().or_softmax(_p(x), x.size)
    return x


def silu(v: float) -> float:
    return lib().or_silu(v)


def gelu(v: float) -> float:
    return lib().or_gelu(v)


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return int(lib().or_argmax(_p(x), x.size))


def rope_steps(dim: int, base: float) -> np.ndarray:
    out = np.zeros(dim // 2, dtype=np.float32)
    lib().or_rope_steps(_p(out), dim, base)
    return out


def rope_angle(dim: int, base: float, pos: int, pair: int):
    c = np.zeros(1, dtype=np.float32)
    s = np.zeros(1, dtype=np.float32)
    lib().or_rope_angle(dim, base, pos, pair, _p(c), _p(s))
    return float(c[0]), float(s[0])


def rotate(x: np.ndarray, heads: int, head_dim: int, dim: int, base: float, neox: bool, pos: int,
           factors=None) -> np.ndarray:
    """rope.mojo:294 rotate_scaled; factors: one per pair (rope_freqs.weight) or None."""
    x = np.array(x, dtype=np.float32)
    if factors is None:
        lib().or_rotate_run(_p(x), heads, head_dim, dim, base, int(neox), pos)
    else:
        f = np.ascontiguousarray(factors, dtype=np.float32)
        if f.size < dim // 2:
            raise ValueError(f"rope wants {dim // 2} frequency factors but got {f.size}")
        if (f == 0).any():
            raise ValueError("a rope frequency factor of zero has no angle")
        lib().or_rotate_run_scaled(_p(x), heads, head_dim, dim, base, int(neox), pos, _p(f))
    return x


def attend(heads, kv_heads, head_dim, scale, q, keys, values, count) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    keys = np.ascontiguousarray(keys, dtype=np.float32)
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.zeros(heads * head_dim, dtype=np.float32)
    scores = np.zeros(count, dtype=np.float32)
    lib().or_attend(heads, kv_heads, head_dim, scale, _p(q), _p(keys), _p(values), count, _p(out), _p(scores))
    return out


def make_layer(spec: dict, weights: dict, keep: list) -> Layer:
    """spec: width, hidden, heads, kv_heads, head_dim, rope_dim, neox, eps, rope_base, attn_scale,
    optionally ungated (1: act(up) MLP) and act (0 silu, 1 gelu).
    weights: attn_norm, ffn_norm (f32 arrays); wq..down as (kind, rows, cols, bytes) (gate may be
    absent when ungated); optionally rope_factors (f32, rope_dim / 2) and the OPTIONAL_VECTORS."""
    L = Layer()
    for k in ("width", "hidden", "heads", "kv_heads", "head_dim", "rope_dim", "neox"):
        setattr(L, k, int(spec[k]))
    for k in ("eps", "rope_base", "attn_scale"):
        setattr(L, k, float(spec[k]))
    for k in ("attn_norm", "ffn_norm"):
        a = np.ascontiguousarray(weights[k], dtype=np.float32)
        keep.append(a)
        setattr(L, k, a.ctypes.data)
    for k in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
        if k not in weights:
            continue
        kind, rows, cols, blob = weights[k]
        blob = np.ascontiguousarray(blob, dtype=np.uint8)
        keep.append(blob)
        setattr(L, k, Weight(blob.ctypes.data, kind, rows, cols, row_bytes(kind, cols)))
    for k in OPTIONAL_VECTORS:
        v = weights.get(k)
        if v is not None:
            v = np.ascontiguousarray(v, dtype=np.float32)
            keep.append(v)
            setattr(L, k, v.ctypes.data)
    L.ungated = int(spec.get("ungated", 0))
    L.act = int(spec.get("act", 0))
    f = weights.get("rope_factors")  # rope_freqs.weight, one per pair, or absent
    if f is not None:
        f = np.ascontiguousarray(f, dtype=np.float32)
        keep.append(f)
        L.rope_factors = f.ctypes.data
    return L


def q8_cache_round(v: np.ndarray) -> np.ndarray:
    """The values a q8_0 KV cache row holding v reads back (whole 32-blocks)."""
    v = np.array(v, dtype=np.float32)
    lib().or_q8_cache_round(_p(v), v.size)
    return v


def _store_form(f16_store, q8_store) -> int:
    return 2 if q8_store else int(bool(f16_store))


def layer_step(L: Layer, x: np.ndarray, keys: np.ndarray, values: np.ndarray, slot: int, pos: int,
               f16_store: bool = False, threads: int = 1, q8_store: bool = False, parts: int = 3) -> None:
    """In place on x, keys[slot], values[slot] (f32 caches).  f16_store /
    q8_store: the new key and value go through what an f16 / q8_0 device cache
    holds before they are attended over.  parts: 1 the attention sublayer
    only (block.mojo:319), 2 the mlp sublayer only (:429), 3 the layer."""
    for a in (x, keys, values):
        assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    rc = lib().or_layer_part(ctypes.byref(L), _p(x), _p(keys), _p(values), slot, pos,
                             _store_form(f16_store, q8_store), threads, parts)
    if rc != 0:
        raise ValueError(f"layer refused (rc {rc})")


def forward(layers: list, embedding: np.ndarray, output_norm: np.ndarray, output: tuple, token: int,
            pos: int, slot: int, keys: list, values: list, f16_store: bool = False,
            threads: int = 1, q8_store: bool = False) -> np.ndarray:
    n = len(layers)
    arr = (Layer * n)(*layers)
    kind, rows, cols, blob = output
    blob = np.ascontiguousarray(blob, dtype=np.uint8)
    wout = Weight(blob.ctypes.data, kind, rows, cols, row_bytes(kind, cols))
    kp = (ctypes.c_void_p * n)(*[k.ctypes.data for k in keys])
    vp = (ctypes.c_void_p * n)(*[v.ctypes.data for v in values])
    logits = np.zeros(rows, dtype=np.float32)
    emb = np.ascontiguousarray(embedding, dtype=np.float32)
    onorm = np.ascontiguousarray(output_norm, dtype=np.float32)
    rc = lib().or_forward(arr, n, _p(emb), emb.shape[0], _p(onorm), ctypes.byref(wout), token, pos, slot,
                          ctypes.cast(kp, ctypes.c_void_p), ctypes.cast(vp, ctypes.c_void_p),
                          _store_form(f16_store, q8_store),
                          _p(logits), threads)
    if rc != 0:
        raise ValueError(f"forward refused (rc {rc})")
    return logits


def test_blocks(kind: int, count: int, seed: int) -> np.ndarray:
    out = np.zeros(count * block_bytes(kind), dtype=np.uint8)
    lib().or_test_blocks(kind, count, seed & 0xFFFFFFFFFFFFFFFF, _p(out))
    return out


def test_units(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().or_test_units(seed & 0xFFFFFFFFFFFFFFFF, n, _p(out))
    return out
