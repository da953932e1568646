"""Host-side mirror of molla's device decoder layer and decode step.

Mirrors src/molla/nn/gpu_block.mojo: DeviceLayer (:301), device_layer (:899),
device_forward (:1644) and the engine's DeviceSession.step / generate
(src/molla/engine/device.mojo:859 / :922) for a Llama stack with an f32
embedding and a quantized head.  Every launch is one call into
libmolla_mi.so; nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from . import gpu
from ._lib import MiLayerDesc, check, lib


@dataclass
class BlockSpec:
    """block.mojo:61 BlockSpec for a gated-silu Llama layer."""

    width: int = 4096
    hidden: int = 14336
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    rope_dim: int = 128
    rope_base: float = 500000.0
    neox: bool = False  # Llama pairs adjacent elements (arch.mojo:146-152)
    eps: float = 1e-5
    ungated: bool = False  # block.mojo:80 gated: False computes act(up(x))
    act: int = 0  # block.mojo:83: 0 silu, gpu.ACT_BIT (8) gelu

    @property
    def attn_scale(self) -> float:
        # attention.mojo:112: f32(1 / sqrt(f64(head_dim)))
        return float(torch.tensor(1.0 / math.sqrt(self.head_dim), dtype=torch.float32))

    def q_width(self) -> int:
        return self.heads * self.head_dim

    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim


class DeviceLayer:
    """One layer's device-resident weights (gpu_block.mojo:301)."""

    NAMES = ("wq", "wk", "wv", "wo", "gate", "up", "down")

    OPTIONAL = ("q_bias", "k_bias", "v_bias", "q_norm", "k_norm", "attn_post_norm", "ffn_post_norm")

    def __init__(self, spec: BlockSpec, attn_norm: torch.Tensor, ffn_norm: torch.Tensor, weights: dict,
                 rope_steps: torch.Tensor, rope_factors: torch.Tensor | None = None, extras: dict | None = None):
        self.spec = spec
        self.attn_norm = attn_norm
        self.ffn_norm = ffn_norm
        self.weights = weights  # name -> gpu.Tensor
        self.rope_steps = rope_steps
        # rope_freqs.weight of a Llama 3.1 file, one factor per pair, or None
        self.rope_factors = rope_factors
        d = MiLayerDesc()
        d.width, d.hidden = spec.width, spec.hidden
        d.heads, d.kv_heads, d.head_dim = spec.heads, spec.kv_heads, spec.head_dim
        d.rope_dim, d.neox = spec.rope_dim, int(spec.neox)
        d.eps, d.attn_scale = spec.eps, spec.attn_scale
        d.attn_norm, d.ffn_norm, d.rope_steps = attn_norm.data_ptr(), ffn_norm.data_ptr(), rope_steps.data_ptr()
        for n in self.NAMES:
            if n == "gate" and spec.ungated and n not in weights:
                continue
            setattr(d, n, weights[n].weight())
        # block.mojo:116 LayerWeights' optional parts (device f32 vectors)
        self.extras = dict(extras or {})
        for n, t in self.extras.items():
            if n not in self.OPTIONAL:
                raise ValueError(f"unknown optional layer part {n!r}")
            if t.dtype != torch.float32 or not t.is_cuda:
                raise ValueError(f"{n} must be a device float32 tensor")
            setattr(d, n, t.data_ptr())
        d.ungated, d.act = int(spec.ungated), int(spec.act)
        if rope_factors is not None:
            if rope_factors.dtype != torch.float32 or rope_factors.numel() < spec.rope_dim // 2:
                raise ValueError(f"rope wants {spec.rope_dim // 2} f32 frequency factors")
            d.rope_factors = rope_factors.data_ptr()
        self.desc = d

    def weight_bytes(self) -> int:
        return sum(w.rows * w.row_bytes() for w in self.weights.values())


def layer_workspace(layer: DeviceLayer, max_count: int, tokens: int) -> int:
    return lib().mi_layer_workspace(ctypes.byref(layer.desc), max_count, tokens)


def with_cache_form(desc: MiLayerDesc, form: int) -> MiLayerDesc:
    """A copy of a layer descriptor reading and writing a cache of this form."""
    d = MiLayerDesc.from_buffer_copy(desc)
    d.cache_form = form
    return d


def chain_layers(descs: list) -> None:
    """Link consecutive layer descriptors (run in order on one workspace):
    layer i norms its output with layer i + 1's attn_norm, and layer i + 1
    starts from that instead of norming its input itself."""
    for a, b in zip(descs, descs[1:]):
        a.next_norm = b.attn_norm
        b.prenormed = 1


def device_layer(ctx: gpu.DeviceContext, layer: DeviceLayer, x: torch.Tensor, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, cache_stride: int, pos: torch.Tensor, max_count: int, tokens: int = 1,
                 work: torch.Tensor | None = None, form: int = gpu.CACHE_F16) -> None:
    """gpu_block.mojo:899 device_layer, in place on x ([tokens, width] f32).

    pos: device int32[tokens], the position (= cache slot) of each sequence's
    token; max_count bounds pos + 1.  form: the caches' form (gpu.CACHE_F16 or
    CACHE_Q8); cache_stride counts halves (sequences * cache_row apart)."""
    need = layer_workspace(layer, max_count, tokens)
    if work is None:
        work = ctx.workspace(need)
    desc = layer.desc if form == gpu.CACHE_F16 else with_cache_form(layer.desc, form)
    check(lib().mi_decoder_layer(ctx.handle, ctypes.byref(desc), x.data_ptr(), k_cache.data_ptr(),
                                 v_cache.data_ptr(), cache_stride, pos.data_ptr(), max_count, tokens,
                                 work.data_ptr(), work.numel()))


def device_layer_paged(ctx: gpu.DeviceContext, layer: DeviceLayer, x: torch.Tensor, k_pool: torch.Tensor,
                       v_pool: torch.Tensor, kv_index: torch.Tensor, index_stride: int, pos: torch.Tensor,
                       max_count: int, tokens: int = 1, work: torch.Tensor | None = None,
                       form: int = gpu.CACHE_F16) -> None:
    """device_layer over a paged pool (gpu.mojo:571 DevicePaging): kv_index is
    a device int32 [tokens, index_stride] of pool cells, one per position of
    each sequence (negative: not held), the new position's cell set before
    the call."""
    need = layer_workspace(layer, max_count, tokens)
    if work is None:
        work = ctx.workspace(need)
    desc = layer.desc if form == gpu.CACHE_F16 else with_cache_form(layer.desc, form)
    check(lib().mi_decoder_layer_paged(ctx.handle, ctypes.byref(desc), x.data_ptr(), k_pool.data_ptr(),
                                       v_pool.data_ptr(), kv_index.data_ptr(), index_stride, pos.data_ptr(),
                                       max_count, tokens, work.data_ptr(), work.numel()))


class DeviceModel:
    """A Llama stack on the device: f32 embedding, layers, final norm, head."""

    def __init__(self, spec: BlockSpec, embedding: torch.Tensor, layers: list, output_norm: torch.Tensor,
                 output: gpu.Tensor):
        self.spec = spec
        self.embedding = embedding
        self.layers = layers
        self.output_norm = output_norm
        self.output = output

    @property
    def vocab(self) -> int:
        return self.output.rows

    def weight_bytes(self) -> int:
        return sum(l.weight_bytes() for l in self.layers) + self.output.rows * self.output.row_bytes()


LAYER_SHAPES = ("wq", "wk", "wv", "wo", "gate", "up", "down")


def synthetic_model(spec: BlockSpec, n_layers: int, vocab: int, kind: int = gpu.Q_Q4_K, head_kind: int = gpu.Q_Q6_K,
                    seed: int = 1000, device="cuda") -> DeviceModel:
    """The seeded synthetic Llama of the benchmark's decode config: every
    projection of `kind` (synth.quant_tensor: the config's block
    distributions), gains N(1, 0.1), an f32 N(0, 1) embedding and a
    `head_kind` output head.  Tensors are generated on `device` from
    per-tensor seeds, so the same call gives the same bytes every time."""
    from . import synth

    steps = torch.from_numpy(gpu.rope_steps(spec.rope_dim, spec.rope_base)).to(device)
    qw, kvw = spec.q_width(), spec.kv_width()
    shapes = {"wq": (qw, spec.width), "wk": (kvw, spec.width), "wv": (kvw, spec.width), "wo": (spec.width, qw),
              "gate": (spec.hidden, spec.width), "up": (spec.hidden, spec.width), "down": (spec.width, spec.hidden)}
    layers = []
    for _ in range(n_layers):
        ws = {}
        for n, (r, c) in shapes.items():
            seed += 1
            ws[n] = gpu.Tensor.from_bytes(synth.quant_tensor(kind, r, c, seed, device=device), kind, c, r)
        an = synth.normal(spec.width, seed + 7, device=device, mean=1.0, std=0.1)
        fn = synth.normal(spec.width, seed + 8, device=device, mean=1.0, std=0.1)
        layers.append(DeviceLayer(spec, an, fn, ws, steps))
    emb = synth.normal(vocab * spec.width, 77, device=device).view(vocab, spec.width)
    onorm = synth.normal(spec.width, 78, device=device, mean=1.0, std=0.1)
    head = gpu.Tensor.from_bytes(synth.quant_tensor(head_kind, vocab, spec.width, 79, device=device), head_kind,
                                 spec.width, vocab)
    return DeviceModel(spec, emb, layers, onorm, head)


class DeviceSession:
    """KV caches and scratch for `batch` sequences decoding together
    (engine/device.mojo:194 DeviceKvCache + :809 DeviceSession)."""

    def __init__(self, ctx: gpu.DeviceContext, model: DeviceModel, batch: int, context: int,
                 cache_form: int = gpu.CACHE_F16):
        self.ctx, self.model, self.batch, self.context = ctx, model, batch, context
        s = model.spec
        kvw = s.kv_width()
        # f16 or q8_0 caches (repack.mojo:174-218), held as halves either way
        self.cache_form = cache_form
        self.cache_stride = context * gpu.cache_row(cache_form, kvw)
        self.descs = [with_cache_form(l.desc, cache_form) for l in model.layers]
        # at 2..8 tokens each layer also norms its output for the next one
        # (mi_layer_desc next_norm / prenormed; ignored at 1 token and above 8)
        chain_layers(self.descs)
        dev = ctx.device
        self.k = [torch.empty(batch * self.cache_stride, dtype=torch.float16, device=dev) for _ in model.layers]
        self.v = [torch.empty(batch * self.cache_stride, dtype=torch.float16, device=dev) for _ in model.layers]
        self.x = torch.empty(batch * s.width, dtype=torch.float32, device=dev)
        self.logits = torch.empty(batch * model.vocab, dtype=torch.float32, device=dev)
        self.pos = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.ids = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.picks = torch.zeros(batch, dtype=torch.int32, device=dev)
        need = max(layer_workspace(l, context, batch) for l in model.layers)
        need = max(need, lib().mi_matvec_workspace(s.width, batch))
        self.work = torch.empty(need + 256, dtype=torch.uint8, device=dev)
        self.amax_work = torch.empty(lib().mi_argmax_workspace(model.vocab, batch), dtype=torch.uint8, device=dev)

    def step(self, advance: bool = False) -> None:
        """One token for every sequence: embed ids, every layer at pos, final
        norm, head, argmax into picks (engine/device.mojo:859 step + :917 pick).
        advance=True also does advance()'s ids <- picks, pos += 1 inside the
        argmax launch.  Queued, not synchronized; reads ids and pos from
        device memory."""
        m, s, c = self.model, self.model.spec, self.ctx
        L = lib()
        check(L.mi_embed(c.handle, m.embedding.data_ptr(), m.embedding.shape[0], s.width, self.ids.data_ptr(),
                         self.batch, self.x.data_ptr()))
        for i, layer in enumerate(m.layers):
            check(L.mi_decoder_layer(c.handle, ctypes.byref(self.descs[i]), self.x.data_ptr(), self.k[i].data_ptr(),
                                     self.v[i].data_ptr(), self.cache_stride, self.pos.data_ptr(), self.context,
                                     self.batch, self.work.data_ptr(), self.work.numel()))
        xq = self.work.data_ptr()
        check(L.mi_rms_norm(c.handle, self.x.data_ptr(), m.output_norm.data_ptr(), s.width, self.batch, s.eps,
                            None, xq))
        check(L.mi_matvec_xq(c.handle, m.output.kind, m.output.address, m.output.row_bytes(), m.output.rows,
                             m.output.cols, xq, self.batch, self.logits.data_ptr(), gpu.EPI_NONE, None))
        self._pick(self.ids.data_ptr() if advance else None, self.pos.data_ptr() if advance else None)

    def _pick(self, next_ids, next_pos) -> None:
        check(lib().mi_argmax_ws(self.ctx.handle, self.logits.data_ptr(), self.model.vocab, self.batch,
                                 self.picks.data_ptr(), self.amax_work.data_ptr(), self.amax_work.numel(),
                                 next_ids, next_pos))

    def prefill(self, ids: torch.Tensor, seq: int = 0, start: int = 0, chunk: int = 256) -> None:
        """Feed a prompt to sequence `seq` from position `start` in chunks of
        `chunk` tokens (gpu_block.mojo:1654 forward over a chunk, chunk
        gpu.mojo:1695 PREFILL_CHUNK): embed the chunk, then every layer over
        it at once (mi_decoder_layer above 8 tokens runs the prefill matmul;
        the chunk's tokens are one sequence: cache stride 0 on that
        sequence's cache).  The prompt's last hidden row lands in x[seq], pos[seq]
        becomes start + len(ids) and ids[seq] the prompt's last id; finish()
        then picks every sequence's next token.  ids: device int32.  Queued,
        not synchronized."""
        m, s, c = self.model, self.model.spec, self.ctx
        L = lib()
        n_all = int(ids.numel())
        if n_all < 1 or start + n_all > self.context:
            raise ValueError(f"prompt of {n_all} at {start} does not fit a context of {self.context}")
        chunk = max(1, min(chunk, n_all))
        need = max(layer_workspace(l, self.context, chunk) for l in m.layers)
        if getattr(self, "_pwork", None) is None or self._pwork.numel() < need + 256:
            self._pwork = torch.empty(need + 256, dtype=torch.uint8, device=c.device)
            self._px = torch.empty(chunk * s.width, dtype=torch.float32, device=c.device)
        if self._px.numel() < chunk * s.width:
            self._px = torch.empty(chunk * s.width, dtype=torch.float32, device=c.device)
        halves = 2  # the caches are float16 tensors: offsets count halves
        for c0 in range(0, n_all, chunk):
            n = min(chunk, n_all - c0)
            pos = torch.arange(start + c0, start + c0 + n, dtype=torch.int32, device=c.device)
            check(L.mi_embed(c.handle, m.embedding.data_ptr(), m.embedding.shape[0], s.width,
                             ids[c0:c0 + n].data_ptr(), n, self._px.data_ptr()))
            for i in range(len(m.layers)):
                k = self.k[i].data_ptr() + halves * seq * self.cache_stride
                v = self.v[i].data_ptr() + halves * seq * self.cache_stride
                check(L.mi_decoder_layer(c.handle, ctypes.byref(self.descs[i]), self._px.data_ptr(), k, v, 0,
                                         pos.data_ptr(), self.context, n, self._pwork.data_ptr(),
                                         self._pwork.numel()))
        last = (n_all - 1) % chunk  # the last token's row in the last chunk
        self.x[seq * s.width:(seq + 1) * s.width].copy_(self._px[last * s.width:(last + 1) * s.width])
        self.pos[seq:seq + 1].fill_(start + n_all)
        self.ids[seq:seq + 1].copy_(ids[n_all - 1:n_all])

    def finish(self) -> None:
        """Norm, head and argmax over every sequence's hidden row in x (after
        prefill) into picks."""
        m, s, c = self.model, self.model.spec, self.ctx
        L = lib()
        xq = self.work.data_ptr()
        check(L.mi_rms_norm(c.handle, self.x.data_ptr(), m.output_norm.data_ptr(), s.width, self.batch, s.eps,
                            None, xq))
        check(L.mi_matvec_xq(c.handle, m.output.kind, m.output.address, m.output.row_bytes(), m.output.rows,
                             m.output.cols, xq, self.batch, self.logits.data_ptr(), gpu.EPI_NONE, None))
        self._pick(None, None)

    def advance(self) -> None:
        """Greedy decode bookkeeping on the device: next ids = picks, pos += 1."""
        self.ids.copy_(self.picks)
        self.pos.add_(1)

    def capture(self, advance: bool = True) -> "torch.cuda.CUDAGraph":
        """Record one step() followed by advance() (or, advance=False, only
        pos += 1, for feeding a prompt whose ids the caller writes) as one HIP
        graph on the session's stream, so a decode loop costs one launch per
        token instead of ~10 per layer from the host.  Every kernel of the step
        reads ids and pos from device memory and sizes its grid by the
        session's context, so one graph serves every position.  The stream has
        to be a created one (graphs cannot be captured on the null stream) and
        every kernel must have run once eagerly before (module loading is not
        capturable): run step() once first."""
        if self.ctx.stream == torch.cuda.default_stream(self.ctx.device):
            raise RuntimeError("capture: the session's DeviceContext needs its own stream")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.ctx.stream):
            if advance:
                self.step(advance=True)
            else:
                self.step()
                self.pos.add_(1)
        return g
