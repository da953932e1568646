"""Host-side mirror of molla's device entry points, over the C ABI.

Mirrors src/molla/nn/gpu.mojo (device_matvec_into :2148, device_matmul_into
:2945, device_matvec :3112), src/molla/nn/gpu_ops.mojo (rms_norm, rope,
store_kv, attend, argmax) and src/molla/nn/tensor.mojo (the Tensor view):
same names, same argument meaning, same refusals raised before anything is
queued.  Device memory and streams come from PyTorch (ROCm); the arithmetic is
all in libmolla_mi.so.  There is no CPU fallback: without the library or a
GPU every call raises.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import MiError, MiLayerDesc, MiWeight, check, lib

# ggml type numbers, src/molla/nn/quant.mojo:47-57
Q_F32, Q_F16, Q_Q4_0, Q_Q4_1, Q_Q5_0, Q_Q5_1, Q_Q8_0, Q_Q4_K, Q_Q5_K, Q_Q6_K = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14
KIND_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K",
              14: "Q6_K"}
# epilogues, src/molla/nn/gpu.mojo:781-803
EPI_NONE, EPI_BIAS, EPI_ADD, EPI_GLU, ACT_BIT = 0, 1, 2, 4, 8

WHERE_DEVICE = 2


def block_elements(kind: int) -> int:
    return lib().mi_block_elements(kind)


def block_bytes(kind: int) -> int:
    return lib().mi_block_bytes(kind)


class Tensor:
    """A view of a packed weight that owns nothing (tensor.mojo:66-121).

    `cols` is the fast axis (ggml order, tensor.mojo:15-19): a (rows x cols)
    matrix of `kind` blocks, rows back to back.  `address` is a device
    pointer; `keep` holds whatever owns the memory (a torch tensor).
    """

    def __init__(self, address: int, kind: int, cols: int, rows: int, keep=None):
        self.address = int(address)
        self.kind = kind
        self.cols = cols
        self.rows = rows
        self.place = WHERE_DEVICE
        self.keep = keep

    @staticmethod
    def from_bytes(blob, kind: int, cols: int, rows: int, device="cuda") -> "Tensor":
        """Upload raw GGUF bytes (numpy uint8 or a torch uint8 tensor) to the device."""
        t = torch.as_tensor(blob, dtype=torch.uint8) if not isinstance(blob, torch.Tensor) else blob
        t = t.to(device).contiguous()
        want = rows * row_bytes(kind, cols)
        if t.numel() != want:
            raise ValueError(f"{rows} rows of {cols} type-{kind} values take {want} bytes, got {t.numel()}")
        return Tensor(t.data_ptr(), kind, cols, rows, keep=t)

    def row_bytes(self) -> int:
        return row_bytes(self.kind, self.cols)

    def elements(self) -> int:
        return self.rows * self.cols

    def weight(self) -> MiWeight:
        return MiWeight(self.address, self.kind, self.rows, self.cols, self.row_bytes())


def row_bytes(kind: int, cols: int) -> int:
    rb = lib().mi_row_bytes(kind, cols)
    if rb < 0:
        raise ValueError(f"{cols} values is not a whole number of type-{kind} blocks")
    return rb


class DeviceContext:
    """One device and one stream, like MAX's DeviceContext in the reference
    (one per process, tests/main.mojo:52-60).  Holds the workspace the
    library draws scratch from; it grows on demand and is reused."""

    def __init__(self, device: int = 0, stream: torch.cuda.Stream | None = None):
        if not torch.cuda.is_available():
            raise RuntimeError("no GPU: the molla_amd kernels run only on a ROCm device")
        self.device = torch.device("cuda", device)
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        self._work = None
        lib()  # fail now, not at the first launch, if the library is missing

    @property
    def handle(self) -> int:
        return self.stream.cuda_stream

    def workspace(self, nbytes: int) -> torch.Tensor:
        nbytes = max(int(nbytes), 256)
        if self._work is None or self._work.numel() < nbytes:
            self._work = torch.empty(nbytes + 256, dtype=torch.uint8, device=self.device)
        return self._work

    def synchronize(self) -> None:
        check(lib().mi_sync(self.handle))


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _f32(t: torch.Tensor, name: str) -> None:
    if not (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()):
        raise ValueError(f"{name} has to be a contiguous float32 device tensor")


def check_matvec_shapes(w: Tensor, x_elements: int, out_elements: int, tokens: int = 1) -> None:
    """gpu.mojo:2070 check_matvec_shapes, before anything is launched."""
    if w.place != WHERE_DEVICE:
        raise ValueError("the weight is not resident on the device")
    if x_elements < tokens * w.cols:
        raise ValueError(f"matvec wants an input of {tokens * w.cols} but got {x_elements}")
    if out_elements < tokens * w.rows:
        raise ValueError(f"matvec wants an output of {tokens * w.rows} but got {out_elements}")


def device_matvec_into(ctx: DeviceContext, w: Tensor, x: torch.Tensor, out: torch.Tensor, at: int = 0,
                       epi: int = EPI_NONE, aux: torch.Tensor | None = None) -> None:
    """out[at + r] = epilogue(dot(row r of w, x)); queued, not synchronized (gpu.mojo:2148)."""
    device_matmul_into(ctx, w, x, out, 1, at, epi, aux)


def device_matmul_into(ctx: DeviceContext, w: Tensor, x: torch.Tensor, out: torch.Tensor, tokens: int,
                       at: int = 0, epi: int = EPI_NONE, aux: torch.Tensor | None = None) -> None:
    """out[at + t*rows + r] = dot(row r of w, x[t]) for t < tokens (gpu.mojo:2945)."""
    if tokens <= 0:
        raise ValueError("a batched matmul needs at least one token")
    if at < 0:
        raise ValueError("a matvec cannot write at a negative offset")
    _f32(x, "x")
    _f32(out, "out")
    check_matvec_shapes(w, x.numel(), out.numel() - at, tokens)
    if aux is not None:
        _f32(aux, "aux")
    # with room for split-K partial sums when the chunk is a prefill one
    need = lib().mi_matmul_workspace(w.rows, w.cols, tokens)
    work = ctx.workspace(need)
    y = out.data_ptr() + 4 * at
    # aux defaults to the output when the epilogue does not read it (gpu.mojo:2217)
    a = aux.data_ptr() if (aux is not None and epi & (EPI_BIAS | EPI_GLU)) else y
    check(lib().mi_matvec(ctx.handle, w.kind, w.address, w.row_bytes(), w.rows, w.cols, x.data_ptr(), tokens,
                          y, epi, a, work.data_ptr(), work.numel()))


def device_matvec(ctx: DeviceContext, w: Tensor, x: np.ndarray, out: np.ndarray) -> None:
    """Host vectors either side: upload, launch, synchronize, download (gpu.mojo:3112)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    check_matvec_shapes(w, x.size, out.size)
    d_x = torch.from_numpy(x).to(ctx.device)
    d_o = torch.empty(w.rows, dtype=torch.float32, device=ctx.device)
    device_matvec_into(ctx, w, d_x, d_o)
    ctx.synchronize()
    out[:] = d_o.cpu().numpy()


def device_dequant(ctx: DeviceContext, w: Tensor, count: int | None = None) -> torch.Tensor:
    """The whole tensor (or its first `count` values) as float32, bit-exact to quant.mojo:412."""
    n = w.elements() if count is None else count
    out = torch.empty(n, dtype=torch.float32, device=ctx.device)
    check(lib().mi_dequant(ctx.handle, w.kind, w.address, n, out.data_ptr()))
    return out


def device_rms_norm(ctx: DeviceContext, out: torch.Tensor, x: torch.Tensor, gain: torch.Tensor, eps: float,
                    tokens: int = 1) -> None:
    """gpu_ops.mojo rms_norm: out = x * rsqrt(mean(x^2) + eps) * gain, per token row."""
    for t, n in ((out, "out"), (x, "x"), (gain, "gain")):
        _f32(t, n)
    n = gain.numel()
    if x.numel() != n * tokens or out.numel() != n * tokens:
        raise ValueError("rms_norm wants the input and the output the same size as the gain")
    check(lib().mi_rms_norm(ctx.handle, x.data_ptr(), gain.data_ptr(), n, tokens, eps, out.data_ptr(), None))


def rope_steps(dim: int, base: float) -> np.ndarray:
    """rope.mojo:230 step_table, computed on the host in float64."""
    out = np.zeros(dim // 2, dtype=np.float32)
    lib().mi_rope_steps(out.ctypes.data_as(ctypes.c_void_p), dim, base)
    return out


def device_rope(ctx: DeviceContext, x: torch.Tensor, heads: int, head_dim: int, dim: int, neox: bool,
                steps: torch.Tensor, pos: torch.Tensor, tokens: int = 1, row_stride: int | None = None) -> None:
    """Rotate heads in place at positions pos[t] (device int32)."""
    _f32(x, "x")
    stride = heads * head_dim if row_stride is None else row_stride
    check(lib().mi_rope(ctx.handle, x.data_ptr(), heads, head_dim, dim, int(neox), steps.data_ptr(),
                        pos.data_ptr(), tokens, stride))


CACHE_F16, CACHE_Q8 = 0, 1  # repack.mojo:174-181


def cache_row(form: int, kv_width: int) -> int:
    """repack.mojo:221 cache_row: halves one cached position occupies."""
    row = lib().mi_cache_row(form, kv_width)
    if row < 0:
        raise ValueError(f"cache form {form} has no row of width {kv_width}")
    return row


def device_store_kv(ctx: DeviceContext, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor, slot: int, form: int = CACHE_F16) -> None:
    """gpu_ops.mojo:1582 device_store_kv: f32 rows -> the cache at `slot`, f16
    or q8_0 (the caches are torch halves either way, cache_row per slot)."""
    kvw = k.numel()
    if v.numel() != kvw:
        raise ValueError("store_kv wants k and v the same width")
    row = cache_row(form, kvw)
    if k_cache.numel() < (slot + 1) * row or v_cache.numel() < (slot + 1) * row:
        raise ValueError(f"the cache has no room for slot {slot}")
    check(lib().mi_store_kv_form(ctx.handle, form, k.data_ptr(), v.data_ptr(), kvw, k_cache.data_ptr(),
                                 v_cache.data_ptr(), slot))


def device_attend(ctx: DeviceContext, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  heads: int, kv_heads: int, head_dim: int, scale: float, count: int,
                  out: torch.Tensor, form: int = CACHE_F16) -> None:
    """attention.mojo:144 attend over `count` cached positions (f16 or q8_0 cache)."""
    if count <= 0:
        raise ValueError("attention needs at least one key to look at")
    if k_cache.numel() < count * cache_row(form, kv_heads * head_dim):
        raise ValueError("attention wants more keys than the cache holds")
    need = lib().mi_attend_workspace(heads, head_dim, count)
    work = ctx.workspace(need)
    check(lib().mi_attend_form(ctx.handle, form, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), heads,
                               kv_heads, head_dim, scale, count, out.data_ptr(), work.data_ptr(), work.numel()))


def device_argmax(ctx: DeviceContext, x: torch.Tensor, n: int, tokens: int = 1) -> torch.Tensor:
    """kernel.mojo:571 argmax per token row, ties to the lower index."""
    out = torch.empty(tokens, dtype=torch.int32, device=ctx.device)
    check(lib().mi_argmax(ctx.handle, x.data_ptr(), n, tokens, out.data_ptr()))
    return out


def device_argmax_ws(ctx: DeviceContext, x: torch.Tensor, n: int, tokens: int = 1, next_ids=None,
                     next_pos=None) -> torch.Tensor:
    """device_argmax spread over 64 parts a row (mi_argmax_ws); next_ids /
    next_pos (device int32[tokens]) get the pick and pos + 1 when given."""
    L = lib()
    out = torch.empty(tokens, dtype=torch.int32, device=ctx.device)
    work = torch.empty(L.mi_argmax_workspace(n, tokens), dtype=torch.uint8, device=ctx.device)
    check(L.mi_argmax_ws(ctx.handle, x.data_ptr(), n, tokens, out.data_ptr(), work.data_ptr(), work.numel(),
                         None if next_ids is None else next_ids.data_ptr(),
                         None if next_pos is None else next_pos.data_ptr()))
    return out


def device_embed(ctx: DeviceContext, embedding: torch.Tensor, ids: torch.Tensor, out: torch.Tensor) -> None:
    """model.mojo:102 embed for an f32 table, one row per token id (device int32)."""
    vocab, width = embedding.shape
    check(lib().mi_embed(ctx.handle, embedding.data_ptr(), vocab, width, ids.data_ptr(), ids.numel(),
                         out.data_ptr()))


__all__ = [n for n in dir() if not n.startswith("_")] + ["MiError"]
