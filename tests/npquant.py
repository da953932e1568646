"""An independent numpy decoder for the GGUF block formats, and block builders.

Written from the byte layouts (ggml's block_q* structs as documented in
src/molla/nn/quant.mojo:19-28), vectorised over whole tensors, with float16
widening done by numpy rather than by bit manipulation.  It shares no code with
oracle/molla_oracle.c, so agreement between the two pins both.  The affine
forms are evaluated with the same float32 rounding points as quant.mojo
((d*sc)*q - dmin*m for q4_k, (d*sc)*q for q6_k), which numpy honours because
it never fuses a multiply into an add.
"""

from __future__ import annotations

import numpy as np

BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
         12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}


def _h(b: np.ndarray) -> np.ndarray:
    """Two little-endian bytes per row -> float32 via numpy's float16."""
    return np.ascontiguousarray(b).view("<f2").astype(np.float32).reshape(-1)


def _kscales(s: np.ndarray):
    """s: (n, 12) uint8 -> (sc, m): (n, 8) int, ggml get_scale_min_k4."""
    s = s.astype(np.int32)
    sc = np.empty((s.shape[0], 8), np.int32)
    m = np.empty((s.shape[0], 8), np.int32)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant(kind: int, blob: np.ndarray, count: int) -> np.ndarray:
    per, nb = BLOCK[kind]
    n = count // per
    b = np.ascontiguousarray(blob[: n * nb], dtype=np.uint8).reshape(n, nb)
    f32 = np.float32
    if kind == 0:
        return b.view("<f4").reshape(-1).astype(f32)
    if kind == 1:
        return _h(b)
    if kind == 30:
        return (b.astype(np.uint32)[:, 0] << 16 | b.astype(np.uint32)[:, 1] << 24).view(f32)
    if kind == 8:
        d = _h(b[:, 0:2])[:, None]
        return (b[:, 2:].view(np.int8).astype(f32) * d).reshape(-1)
    if kind == 2:
        d = _h(b[:, 0:2])[:, None]
        q = b[:, 2:18].astype(np.int32)
        v = np.concatenate([(q & 0xF) - 8, (q >> 4) - 8], axis=1).astype(f32)
        return (v * d).reshape(-1)
    if kind == 3:
        d = _h(b[:, 0:2])[:, None]
        m = _h(b[:, 2:4])[:, None]
        q = b[:, 4:20].astype(np.int32)
        v = np.concatenate([q & 0xF, q >> 4], axis=1).astype(f32)
        return (v * d + m).reshape(-1)
    if kind in (6, 7):
        off = 2 if kind == 6 else 4
        d = _h(b[:, 0:2])[:, None]
        qh = b[:, off:off + 4].copy().view("<u4").astype(np.int64).reshape(-1, 1)
        q = b[:, off + 4:off + 20].astype(np.int64)
        l = np.arange(16)
        lo = (q & 0xF) | (((qh >> l) & 1) << 4)
        hi = (q >> 4) | (((qh >> (l + 16)) & 1) << 4)
        v = np.concatenate([lo, hi], axis=1)
        if kind == 6:
            return ((v - 16).astype(f32) * d).reshape(-1)
        m = _h(b[:, 2:4])[:, None]
        return (v.astype(f32) * d + m).reshape(-1)
    if kind in (12, 13):
        d = _h(b[:, 0:2])
        dmin = _h(b[:, 2:4])
        sc, m = _kscales(b[:, 4:16])
        qs = b[:, 16:144] if kind == 12 else b[:, 48:176]
        qs = qs.astype(np.int32).reshape(n, 4, 32)
        vals = np.empty((n, 8, 32), np.int32)
        vals[:, 0::2, :] = qs & 0xF
        vals[:, 1::2, :] = qs >> 4
        if kind == 13:
            qh = b[:, 16:48].astype(np.int32)  # (n, 32)
            for g in range(8):
                vals[:, g, :] += ((qh >> g) & 1) * 16
        dsc = (d[:, None] * sc.astype(f32))[:, :, None]
        mm = (dmin[:, None] * m.astype(f32))[:, :, None]
        return (dsc * vals.astype(f32) - mm).reshape(-1)
    if kind == 14:
        ql = b[:, 0:128].astype(np.int32).reshape(n, 2, 64)
        qh = b[:, 128:192].astype(np.int32).reshape(n, 2, 32)
        sc = b[:, 192:208].view(np.int8).astype(f32).reshape(n, 2, 8)
        d = _h(b[:, 208:210])
        q = np.empty((n, 2, 4, 32), np.int32)
        q[:, :, 0] = (ql[:, :, :32] & 0xF) | ((qh & 3) << 4)
        q[:, :, 1] = (ql[:, :, 32:] & 0xF) | (((qh >> 2) & 3) << 4)
        q[:, :, 2] = (ql[:, :, :32] >> 4) | (((qh >> 4) & 3) << 4)
        q[:, :, 3] = (ql[:, :, 32:] >> 4) | (((qh >> 6) & 3) << 4)
        q = (q - 32).astype(f32).reshape(n, 2, 4, 2, 16)  # [n, half, quarter, g, 16]
        s = sc.reshape(n, 2, 4, 2)  # sc[8n + g + 2k] -> index k*2+g
        out = (d[:, None, None, None, None] * s[..., None]) * q
        return out.reshape(-1)
    raise ValueError(f"no decoder for kind {kind}")


def pack_kscales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of get_scale_min_k4: (n, 8) six-bit values -> (n, 12) bytes."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return out
