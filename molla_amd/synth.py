"""Seeded synthetic GGUF tensors and activations for the benchmark configs.

Each generator returns raw GGUF block bytes (a uint8 torch tensor, rows back to
back) exactly as a model file would hold them, on the requested device, from
a torch.Generator seeded per tensor.  The distributions follow the benchmark
configurations:
  Q8_0: d = f16(|N(0,1)| * 0.02), 32 int8 values uniform in [-127, 127].
  Q4_0: d = f16(|N(0,1)| * 0.01), nibbles uniform.
  Q4_K: d, dmin = f16(|N(0,1)| * 0.01), eight six-bit scales and mins uniform
        in 0..63 packed as ggml's get_scale_min_k4 reads them, nibbles uniform.
  Q6_K: ql / qh bytes uniform, sixteen int8 scales uniform in [-64, 63],
        d = f16(|N(0,1)| * 0.005).
  Q4_1, Q5_1: d = f16(|N(0,1)| * 0.01), m = f16(-|N(0,1)| * 0.08), the
        nibbles and fifth bits uniform.
  Q5_0: d = f16(|N(0,1)| * 0.01), nibbles and fifth bits uniform.
  Q5_K: as Q4_K, with the fifth-bit plane uniform.
Float16 fields are rounded to nearest even from float32.
"""

from __future__ import annotations

import torch

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 6, 7, 8, 12, 13, 14
BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24), Q8_0: (32, 34), Q4_K: (256, 144),
         Q5_K: (256, 176), Q6_K: (256, 210)}


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed & 0x7FFFFFFFFFFFFFFF)
    return g


def _rand_bytes(n: int, g, device) -> torch.Tensor:
    return torch.randint(0, 256, (n,), generator=g, device=device, dtype=torch.int32).to(torch.uint8)


def _half_bytes(v: torch.Tensor) -> torch.Tensor:
    """float32 (n,) -> (n, 2) little-endian float16 bytes."""
    return v.to(torch.float16).view(torch.int16).view(torch.uint8).reshape(-1, 2)


def _abs_normal(n: int, scale: float, g, device) -> torch.Tensor:
    return torch.randn(n, generator=g, device=device, dtype=torch.float32).abs() * scale


def pack_kscales(sc: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """(n, 8) six-bit scales and mins -> (n, 12) bytes; inverse of quant.mojo:161 _k_scale."""
    sc = sc.to(torch.int32)
    m = m.to(torch.int32)
    out = torch.empty((sc.shape[0], 12), dtype=torch.int32, device=sc.device)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return out.to(torch.uint8)


def quant_tensor(kind: int, rows: int, cols: int, seed: int, device="cpu") -> torch.Tensor:
    per, nb = BLOCK[kind]
    if cols % per:
        raise ValueError(f"{cols} columns is not a whole number of {per}-value blocks")
    n = rows * cols // per
    g = _gen(seed, device)
    b = _rand_bytes(n * nb, g, device).reshape(n, nb)
    if kind == Q8_0:
        b[:, 0:2] = _half_bytes(_abs_normal(n, 0.02, g, device))
        q = torch.randint(-127, 128, (n, 32), generator=g, device=device, dtype=torch.int32)
        b[:, 2:34] = q.to(torch.int8).view(torch.uint8)
    elif kind == Q4_0:
        b[:, 0:2] = _half_bytes(_abs_normal(n, 0.01, g, device))
    elif kind in (Q4_1, Q5_1):
        b[:, 0:2] = _half_bytes(_abs_normal(n, 0.01, g, device))
        b[:, 2:4] = _half_bytes(-_abs_normal(n, 0.08, g, device))
    elif kind == Q5_0:
        b[:, 0:2] = _half_bytes(_abs_normal(n, 0.01, g, device))
    elif kind in (Q4_K, Q5_K):
        b[:, 0:2] = _half_bytes(_abs_normal(n, 0.01, g, device))
        b[:, 2:4] = _half_bytes(_abs_normal(n, 0.01, g, device))
        sc = torch.randint(0, 64, (n, 8), generator=g, device=device, dtype=torch.int32)
        m = torch.randint(0, 64, (n, 8), generator=g, device=device, dtype=torch.int32)
        b[:, 4:16] = pack_kscales(sc, m)
    elif kind == Q6_K:
        s = torch.randint(-64, 64, (n, 16), generator=g, device=device, dtype=torch.int32)
        b[:, 192:208] = s.to(torch.int8).view(torch.uint8)
        b[:, 208:210] = _half_bytes(_abs_normal(n, 0.005, g, device))
    else:
        raise ValueError(f"no generator for ggml type {kind}")
    return b.reshape(-1)


def normal(n: int, seed: int, device="cpu", mean: float = 0.0, std: float = 1.0) -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn(n, generator=g, device=device, dtype=torch.float32) * std + mean


def tokens(n: int, vocab: int, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randint(0, vocab, (n,), generator=g, device=device, dtype=torch.int32)
