"""GGUF model file -> device-resident Llama stack (the upload half of
src/molla/model/load.mojo and the GGUF-layout bind of
src/molla/engine/device.mojo:988-1066, for the decode path this library
runs).

    g = gguf.Gguf(path)
    plan = read_llama(g)            # host only: hyperparameters, tensor map, checks
    model = upload(ctx, g, plan)    # one device pool, GGUF bytes as they lie

The weights keep the file's layout: every quantized tensor is copied into
one device allocation (each at a 256-byte aligned offset) and the kernels
read the GGUF blocks there, so nothing is repacked.  The f32 norms are
copied the same way; a quantized token embedding is dequantized once on the
device (mi_dequant) into the f32 table the embedding lookup reads, and with
no output.weight the head reads the embedding's quantized blocks (tied
embeddings).  Llama 3.1's rope_freqs.weight, when present, becomes every
layer's rope frequency factors.

Names and keys follow llama.cpp's GGUF conventions, which molla reads too:
    token_embd.weight, output_norm.weight, output.weight, rope_freqs.weight,
    blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output, ffn_norm,
           ffn_gate, ffn_up, ffn_down}.weight
    <arch>.{embedding_length, feed_forward_length, block_count,
            attention.head_count, attention.head_count_kv,
            attention.layer_norm_rms_epsilon, attention.key_length,
            rope.freq_base, rope.dimension_count}
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .gguf import Gguf, GgufError, TensorInfo, ggml_type_name

QUANT_KINDS = (2, 3, 6, 7, 8, 12, 13, 14)  # Q4_0 Q4_1 Q5_0 Q5_1 Q8_0 Q4_K Q5_K Q6_K
F32, F16, BF16 = 0, 1, 30
LAYER_TENSORS = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "gate": "ffn_gate",
                 "up": "ffn_up", "down": "ffn_down"}
ARCHITECTURES = ("llama",)


@dataclass
class LlamaPlan:
    """What read_llama found: the layer geometry and every tensor to upload."""

    arch: str
    width: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    rope_dim: int
    rope_base: float
    eps: float
    n_layers: int
    vocab: int
    context: int
    embedding: TensorInfo
    output_norm: TensorInfo
    output: TensorInfo           # output.weight, or token_embd.weight when tied
    tied: bool
    rope_factors: TensorInfo | None
    layers: list = field(default_factory=list)  # per layer: {name: TensorInfo}, names as DeviceLayer + norms


def _matrix(t: TensorInfo, rows: int, cols: int, what: str) -> None:
    if t.n_dims != 2 or t.dims[0] != cols or t.dims[1] != rows:
        raise GgufError(f"{t.name}: {what} wants {rows} x {cols} (ne = [{cols}, {rows}]), file has ne = {list(t.dims)}")
    if t.kind not in QUANT_KINDS:
        raise GgufError(f"{t.name}: type {ggml_type_name(t.kind)} has no device matvec (block-quantized kinds only)")


def _vector(t: TensorInfo, n: int) -> None:
    if t.elements() != n:
        raise GgufError(f"{t.name}: wants {n} values, file has {t.elements()}")
    if t.kind not in (F32, F16, BF16):
        raise GgufError(f"{t.name}: type {ggml_type_name(t.kind)} for a vector (F32, F16 or BF16 expected)")


def read_llama(g: Gguf) -> LlamaPlan:
    """Hyperparameters and the tensor map of a Llama GGUF, checked against
    each other; raises GgufError naming the first thing that does not fit."""
    arch = g.architecture()
    if arch not in ARCHITECTURES:
        raise GgufError(f"architecture {arch!r}: this loader reads {', '.join(ARCHITECTURES)}")
    k = arch + "."
    width = g.uint_or(k + "embedding_length", 0)
    hidden = g.uint_or(k + "feed_forward_length", 0)
    n_layers = g.uint_or(k + "block_count", 0)
    heads = g.uint_or(k + "attention.head_count", 0)
    if width <= 0 or hidden <= 0 or n_layers <= 0 or heads <= 0:
        raise GgufError("missing embedding_length, feed_forward_length, block_count or attention.head_count")
    kv_heads = g.uint_or(k + "attention.head_count_kv", heads)
    head_dim = g.uint_or(k + "attention.key_length", width // heads)
    rope_dim = g.uint_or(k + "rope.dimension_count", head_dim)
    rope_base = g.float_or(k + "rope.freq_base", 10000.0)
    eps = g.float_or(k + "attention.layer_norm_rms_epsilon", 1e-5)

    def need(name: str) -> TensorInfo:
        i = g.tensor_index(name)
        if i < 0:
            raise GgufError(f"missing tensor {name}")
        return g.tensors[i]

    emb = need("token_embd.weight")
    if emb.n_dims != 2 or emb.dims[0] != width:
        raise GgufError(f"token_embd.weight: ne = {list(emb.dims)}, width {width}")
    vocab = emb.dims[1]
    if emb.kind not in QUANT_KINDS + (F32, F16, BF16):
        raise GgufError(f"token_embd.weight: type {ggml_type_name(emb.kind)} is not decodable here")
    onorm = need("output_norm.weight")
    _vector(onorm, width)
    tied = g.tensor_index("output.weight") < 0
    out = emb if tied else need("output.weight")
    _matrix(out, vocab, width, "the output head")
    factors = None
    if g.tensor_index("rope_freqs.weight") >= 0:
        factors = need("rope_freqs.weight")
        _vector(factors, rope_dim // 2)
    plan = LlamaPlan(arch, width, hidden, heads, kv_heads, head_dim, rope_dim, rope_base, eps, n_layers, vocab,
                     g.context_length(), emb, onorm, out, tied, factors)
    qw, kvw = heads * head_dim, kv_heads * head_dim
    shapes = {"wq": (qw, width), "wk": (kvw, width), "wv": (kvw, width), "wo": (width, qw),
              "gate": (hidden, width), "up": (hidden, width), "down": (width, hidden)}
    for i in range(n_layers):
        lt = {}
        for n, short in LAYER_TENSORS.items():
            t = need(f"blk.{i}.{short}.weight")
            _matrix(t, *shapes[n], n)
            lt[n] = t
        for n in ("attn_norm", "ffn_norm"):
            t = need(f"blk.{i}.{n}.weight")
            _vector(t, width)
            lt[n] = t
        if g.tensor_index(f"blk.{i}.attn_q.bias") >= 0:
            raise GgufError("q/k/v biases (Qwen 2) are not in this layer")
        plan.layers.append(lt)
    return plan


def _host_f32(g: Gguf, t: TensorInfo) -> np.ndarray:
    raw = np.frombuffer(g.tensor_data(t), dtype=np.uint8)
    if t.kind == F32:
        return raw.view(np.float32).copy()
    if t.kind == F16:
        return raw.view(np.float16).astype(np.float32)
    return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)  # BF16


def upload(ctx, g: Gguf, plan: LlamaPlan):
    """The plan's tensors on ctx's device, as a block.DeviceModel."""
    import torch

    from . import block, gpu

    dev = ctx.device
    quant = [plan.output] + [lt[n] for lt in plan.layers for n in LAYER_TENSORS]
    if plan.embedding.kind in QUANT_KINDS and plan.embedding is not plan.output:
        quant.append(plan.embedding)
    # one device pool for every quantized tensor, 256-byte aligned offsets
    offsets, total = {}, 0
    for t in quant:
        if t.name not in offsets:
            offsets[t.name] = total
            total += (t.nbytes() + 255) // 256 * 256
    pool = torch.empty(max(total, 256), dtype=torch.uint8, device=dev)
    for t in quant:
        off = offsets[t.name]
        src = torch.from_numpy(np.frombuffer(g.tensor_data(t), dtype=np.uint8).copy())
        pool[off:off + src.numel()].copy_(src)

    def qtensor(t: TensorInfo) -> gpu.Tensor:
        return gpu.Tensor(pool.data_ptr() + offsets[t.name], t.kind, t.dims[0], t.dims[1], keep=pool)

    def vec(t: TensorInfo) -> torch.Tensor:
        return torch.from_numpy(_host_f32(g, t)).to(dev)

    spec = block.BlockSpec(width=plan.width, hidden=plan.hidden, heads=plan.heads, kv_heads=plan.kv_heads,
                           head_dim=plan.head_dim, rope_dim=plan.rope_dim, rope_base=plan.rope_base, neox=False,
                           eps=plan.eps)
    steps = torch.from_numpy(gpu.rope_steps(plan.rope_dim, plan.rope_base)).to(dev)
    factors = vec(plan.rope_factors) if plan.rope_factors is not None else None
    layers = []
    for lt in plan.layers:
        ws = {n: qtensor(lt[n]) for n in LAYER_TENSORS}
        layers.append(block.DeviceLayer(spec, vec(lt["attn_norm"]), vec(lt["ffn_norm"]), ws, steps, factors))
    # the f32 table the embedding lookup reads
    e = plan.embedding
    if e.kind in QUANT_KINDS:
        emb = gpu.device_dequant(ctx, qtensor(e)).view(plan.vocab, plan.width)
    else:
        emb = vec(e).view(plan.vocab, plan.width)
    model = block.DeviceModel(spec, emb, layers, vec(plan.output_norm), qtensor(plan.output))
    model.pool = pool
    return model


def load_llama(ctx, path: str):
    """read_llama + upload for a file path; returns (plan, DeviceModel)."""
    with Gguf(path) as g:
        plan = read_llama(g)
        model = upload(ctx, g, plan)
    return plan, model
