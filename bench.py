"""Benchmark: Q4_K matvec HBM GB/s on MI355X (+ the 8B Q4_K decode step).

Workload: Q4_K 14336 x 4096 matvec at batch 1 on
synthetic GGUF blocks (seeded), x fp32 ~ N(0,1).  A "step" is one matvec:
quantize x into the kernels' activation form, then the fused
dequantize-and-dot over the 33,030,144 weight bytes.  Weights are rotated over
enough distinct copies (>= 2 GiB) that every step reads cold HBM, past the
256 MB Infinity Cache.  Timing: HIP events on the launch stream around exactly
K steps after W warmup steps, bracketed by synchronize.

`value` = algorithmic bytes (weights + x + y) per step / wall time per step.
`roofline` = the matvec kernel alone: bytes / its average duration, timed
with HIP events on the launch stream around K back-to-back launches (the
quantize hoisted out).  `cpu_baseline` = the CPU
oracle (a C restatement of molla's serial host matvec, kernel.mojo:316) on the
same bytes, single thread, over a bounded number of repetitions.

"decode" (skipped with --no-decode) is config 5: a synthetic 8B model (32 Q4_K
layers, Q6_K head, f32 embedding, random weights), a 2048-token prompt
prefilled in 256-token chunks (`prefill_tokens_per_s`), then greedy decode of
256 tokens at batch 1 and 4 (and at
batch 1 over a q8_0 KV cache, `batch_1_q8_cache`), each
step replayed from one captured HIP graph; tokens/s, ms per step, the eager
(host-launched) ms per step and the weight-streaming fraction of 8 TB/s.

"head" (with the batched lines): config 3, the Q6_K 128256 x 4096 output
head at batch 1 and 8 and the argmax after it.

"prefill" (skipped with --no-prefill): the prefill matmul at a 256-token
chunk on each matrix of an 8B Q4_K_M layer (TFLOP/s, matrix-core fraction)
and the matmul-only tokens/s of an 8B prefill.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

ROWS, COLS = 14336, 4096
PEAK_GBS = 8000.0


def _algo_bytes(rows, cols, tokens, wbytes):
    return wbytes + 4 * tokens * (cols + rows)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-decode", action="store_true", help="skip the synthetic 8B decode step")
    ap.add_argument("--decode-tokens", type=int, default=256)
    ap.add_argument("--decode-batch", type=int, nargs="+", default=[1, 4, 8])
    ap.add_argument("--decode-q8", type=int, nargs="*", default=[1],
                    help="decode batch sizes also run over a q8_0 KV cache")
    ap.add_argument("--prompt", type=int, default=2048)
    ap.add_argument("--prefill-chunk", type=int, default=256, help="prompt tokens per prefill pass (PREFILL_CHUNK)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-batched", action="store_true", help="skip the batch-4/8 matrix-core tile lines")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 256-token prefill matmul lines")
    ap.add_argument("--no-configs", action="store_true", help="skip the BASELINE configs[0] and configs[3] lines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from molla_amd import gpu, synth
    from molla_amd._lib import check, lib

    torch.cuda.init()
    ctx = gpu.DeviceContext(0)
    L = lib()
    kind = gpu.Q_Q4_K
    rb = gpu.row_bytes(kind, COLS)
    wbytes = ROWS * rb
    copies = max(2, int((2 << 30) // wbytes) + 1)
    base = synth.quant_tensor(kind, ROWS, COLS, 20240101, device="cuda")
    ws = [base] + [base.clone() for _ in range(copies - 1)]
    x = synth.normal(COLS, 7, device="cuda")
    y = torch.empty(ROWS, dtype=torch.float32, device="cuda")
    xq = torch.empty(L.mi_matvec_workspace(COLS, 1), dtype=torch.uint8, device="cuda")
    h = ctx.handle

    def step(i):
        w = ws[i % copies]
        check(L.mi_quantize(h, x.data_ptr(), COLS, 1, xq.data_ptr()))
        check(L.mi_matvec_xq(h, kind, w.data_ptr(), rb, ROWS, COLS, xq.data_ptr(), 1, y.data_ptr(), 0, None))

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    e0.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    algo = _algo_bytes(ROWS, COLS, 1, wbytes)
    value = algo / (ms_per_step * 1e-3) / 1e9

    # dominant kernel alone: the same launches back to back with the quantize
    # hoisted out, HIP events on the launch stream around all of them (an
    # event pair around every launch would time the event records too)
    check(L.mi_quantize(h, x.data_ptr(), COLS, 1, xq.data_ptr()))
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(args.steps):
        w = ws[(args.warmup + i) % copies]
        check(L.mi_matvec_xq(h, kind, w.data_ptr(), rb, ROWS, COLS, xq.data_ptr(), 1, y.data_ptr(), 0, None))
    e1.record(stream)
    torch.cuda.synchronize()
    k_avg_ms = e0.elapsed_time(e1) / args.steps
    achieved = algo / (k_avg_ms * 1e-3) / 1e9

    line = {
        "metric": "Q4_K matvec HBM GB/s (% of peak); 8B Q4_K decode tokens/sec at batch 1",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k x int8-limb activations, int32/fp32 accumulate",
        "data": "synthetic (seeded GGUF Q4_K blocks, x ~ N(0,1)), weights rotated over "
                f"{copies} copies ({copies * wbytes / 2**30:.1f} GiB) so every step reads cold HBM",
        "config": {"workload": "Q4_K matvec 14336x4096, batch 1 (BASELINE configs[1], ffn gate/up)",
                   "rows": ROWS, "cols": COLS, "tokens": 1, "weight_bytes": wbytes,
                   "algorithmic_bytes_per_step": algo, "parallelism": "single GPU"},
        "pct_of_hbm_peak": round(100 * value / PEAK_GBS, 1),
        "roofline": {"bound": "hbm", "kernel": "rows_kernel<Q4_K, 4, 1> (matvec_rows.h)",
                     "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": _traffic_from_profile(),
                     "kernel_avg_us": round(k_avg_ms * 1e3, 3)},
    }

    if not args.no_batched:
        line["batched"] = _batched(L, h, kind, ws, copies, rb, stream)
        line["kinds"] = _kinds(L, h, stream)
        line["head"] = _head(L, h, stream)
        line["layer_kinds"] = _layer_kinds(L, h, stream)
    if not args.no_configs:
        line["config1"] = _config1(L, h, stream, cpu=not args.no_cpu)
        line["config4"] = _config4(L)
    peak = _stream_peak(stream)
    line["roofline"]["stream_peak"] = peak
    line["roofline"]["frac_of_stream_33MB"] = round(achieved / peak["read_33MB"]["GB_s"], 4)
    del ws
    torch.cuda.empty_cache()
    model = None
    if not args.no_decode or not args.no_cpu:
        from molla_amd import block
        model = block.synthetic_model(block.BlockSpec(), 32, 128256, device="cuda")
    if not args.no_cpu:
        line["cpu_baseline"] = _cpu_baseline(base, kind, rb, x, model)
    if not args.no_prefill:
        line["prefill"] = _prefill(L, h, stream)
    if not args.no_decode:
        line["decode"] = _decode(ctx, args, model)
    print(json.dumps(line), flush=True)


# An 8B Llama layer's matrices at one prompt chunk (gpu.mojo:1695
# PREFILL_CHUNK = 256 tokens), Q4_K_M kinds: (name, rows, cols, kind, count
# per layer).  attn_v and ffn_down are Q6_K in half of a Q4_K_M file's layers.
_PREFILL_SHAPES = [("attn_q", 4096, 4096, 12, 1), ("attn_k", 1024, 4096, 12, 1), ("attn_v", 1024, 4096, 14, 1),
                   ("attn_output", 4096, 4096, 12, 1), ("ffn_gate", 14336, 4096, 12, 1),
                   ("ffn_up", 14336, 4096, 12, 1), ("ffn_down", 4096, 14336, 14, 1)]


def _prefill(L, h, stream, tokens=256, reps=20):
    """The prefill matmul (mi_matvec at 256 tokens: prefill.hip) on each of
    an 8B layer's matrices, timed over `reps` back-to-back calls (activation
    halves + matrix-core tile + split-K reduce, all inside).  TFLOP/s counts
    the useful 2 rows cols tokens; the tile issues 2 half-precision MFMA
    products per useful one (3 for Q6_K), so `mfma_frac` is that work over
    the 2.5 PFLOP/s dense f16 peak.  `layer_us` sums one layer (attn_v and
    ffn_down as Q6_K); `matmul_tokens_per_s` = tokens / (32 layers x
    layer_us): the matmuls of an 8B prefill chunk, attention and the rest of
    the layer not included."""
    import torch

    from molla_amd import gpu, synth
    from molla_amd._lib import check

    ctx = gpu.DeviceContext(0)
    out, layer_us = {}, 0.0
    for name, rows, cols, kind, count in _PREFILL_SHAPES:
        blob = synth.quant_tensor(kind, rows, cols, 31, device="cuda")
        w = gpu.Tensor.from_bytes(blob, kind, cols, rows)
        x = synth.normal(tokens * cols, 32, device="cuda")
        y = torch.empty(tokens * rows, dtype=torch.float32, device="cuda")
        need = L.mi_matmul_workspace(rows, cols, tokens)
        work = torch.empty(need + 256, dtype=torch.uint8, device="cuda")

        def call():
            check(L.mi_matvec(h, kind, w.address, w.row_bytes(), rows, cols, x.data_ptr(), tokens, y.data_ptr(), 0,
                              None, work.data_ptr(), need))
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        tf = 2.0 * rows * cols * tokens / us / 1e6
        products = 3 if kind == 14 else 2
        out[name] = {"rows": rows, "cols": cols, "kind": gpu.KIND_NAMES.get(kind, kind), "us": round(us, 1),
                     "TFLOP_s": round(tf, 1), "mfma_frac": round(tf * products / 2500.0, 3)}
        layer_us += us * count
        del w, blob, work
    out["tokens"] = tokens
    out["layer_us"] = round(layer_us, 1)
    out["matmul_tokens_per_s"] = round(tokens / (32 * layer_us * 1e-6), 0)
    return out


def _batched(L, h, kind, ws, copies, rb, stream, reps=100):
    """Batch 4 and 8: the same weights against 4 / 8
    tokens on the f16 matrix-core tile (matvec_htile.hip; mi_quantize writes
    the activations' hx form it reads).  Weights are still read once per
    launch, so GB/s is over the same algorithmic bytes (plus the larger x and
    y); MFMA utilisation = useful f16 flops (2 rows cols tokens, times the
    two halves of each activation) over the 2.5 PFLOP/s dense f16 peak."""
    import torch

    from molla_amd import synth
    from molla_amd._lib import check

    out = {}
    for tokens in (4, 8):
        x = synth.normal(tokens * COLS, 11 + tokens, device="cuda")
        xq = torch.empty(L.mi_matvec_workspace(COLS, tokens), dtype=torch.uint8, device="cuda")
        y = torch.empty(tokens * ROWS, dtype=torch.float32, device="cuda")
        check(L.mi_quantize(h, x.data_ptr(), COLS, tokens, xq.data_ptr()))
        for i in range(10):
            check(L.mi_matvec_xq(h, kind, ws[i % copies].data_ptr(), rb, ROWS, COLS, xq.data_ptr(), tokens,
                                 y.data_ptr(), 0, None))
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(reps):
            check(L.mi_matvec_xq(h, kind, ws[i % copies].data_ptr(), rb, ROWS, COLS, xq.data_ptr(), tokens,
                                 y.data_ptr(), 0, None))
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        algo = _algo_bytes(ROWS, COLS, tokens, ROWS * rb)
        flops = 2.0 * ROWS * COLS * tokens * 2
        out[f"tokens_{tokens}"] = {"kernel": "htile_kernel<T, Q4_K> (v_mfma_f32_16x16x32_f16)",
                                   "us_per_launch": round(us, 3),
                                   "GB_s": round(algo / us / 1e3, 1),
                                   "frac_hbm_peak": round(algo / us / 1e3 / PEAK_GBS, 4),
                                   "mfma_f16_TFLOPs": round(flops / us / 1e6, 2),
                                   "mfma_util_of_2500TFLOPs": round(flops / us / 1e6 / 2500.0, 5)}
    return out


def _head(L, h, stream, reps=20):
    """Config 3: the Q6_K output head, 128256 x 4096, at batch 1 and 8, then
    argmax.  The weights (431 MB) are larger than the 256 MB Infinity Cache,
    so every launch streams them from HBM."""
    import torch

    from molla_amd import gpu, synth
    from molla_amd._lib import check

    rows, cols, kind = 128256, 4096, gpu.Q_Q6_K
    rb = gpu.row_bytes(kind, cols)
    w = synth.quant_tensor(kind, rows, cols, 79, device="cuda")
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    out = {}
    for tokens in (1, 8):
        x = synth.normal(tokens * cols, 23 + tokens, device="cuda")
        xq = torch.empty(L.mi_matvec_workspace(cols, tokens), dtype=torch.uint8, device="cuda")
        y = torch.empty(tokens * rows, dtype=torch.float32, device="cuda")
        picks = torch.empty(tokens, dtype=torch.int32, device="cuda")
        check(L.mi_quantize(h, x.data_ptr(), cols, tokens, xq.data_ptr()))

        def timed(fn):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / reps

        us = timed(lambda: check(L.mi_matvec_xq(h, kind, w.data_ptr(), rb, rows, cols, xq.data_ptr(), tokens,
                                                y.data_ptr(), 0, None)))
        am1 = timed(lambda: check(L.mi_argmax(h, y.data_ptr(), rows, tokens, picks.data_ptr())))
        aw = torch.empty(L.mi_argmax_workspace(rows, tokens), dtype=torch.uint8, device="cuda")
        am = timed(lambda: check(L.mi_argmax_ws(h, y.data_ptr(), rows, tokens, picks.data_ptr(), aw.data_ptr(),
                                                aw.numel(), None, None)))
        gbs = rows * rb / us / 1e3
        out[f"tokens_{tokens}"] = {"logits_us": round(us, 2), "GB_s": round(gbs, 1),
                                   "frac_hbm_peak": round(gbs / PEAK_GBS, 4), "argmax_us": round(am, 2),
                                   "argmax_one_block_us": round(am1, 2)}
    return out


def _layer_kinds(L, h, stream, reps=30):
    """One 8B-shaped decoder layer (config 4's shape) at context 2049, at 1
    and 4 tokens, with every projection Q4_K and with a Q4_K_M file's kinds
    (Q6_K attn_v and ffn_down): microseconds a layer call, eager."""
    import ctypes

    import torch

    from molla_amd import block, gpu, synth
    from molla_amd._lib import check

    spec = block.BlockSpec()
    qw, kvw = spec.q_width(), spec.kv_width()
    shapes = {"wq": (qw, spec.width), "wk": (kvw, spec.width), "wv": (kvw, spec.width), "wo": (spec.width, qw),
              "gate": (spec.hidden, spec.width), "up": (spec.hidden, spec.width), "down": (spec.width, spec.hidden)}
    steps = torch.from_numpy(gpu.rope_steps(spec.rope_dim, spec.rope_base)).cuda()
    ctx = gpu.DeviceContext(0, stream=stream)
    out = {}
    for name, q6 in (("all_q4_k", ()), ("q4_k_m", ("wv", "down"))):
        ws = {}
        for i, (n, (r, c)) in enumerate(shapes.items()):
            kind = gpu.Q_Q6_K if n in q6 else gpu.Q_Q4_K
            ws[n] = gpu.Tensor.from_bytes(synth.quant_tensor(kind, r, c, 500 + i, device="cuda"), kind, c, r)
        an = synth.normal(spec.width, 510, device="cuda", mean=1.0, std=0.1)
        fn = synth.normal(spec.width, 511, device="cuda", mean=1.0, std=0.1)
        layer = block.DeviceLayer(spec, an, fn, ws, steps)
        for tokens in (1, 4):
            count = 2049
            stride = count * kvw
            k = synth.normal(tokens * stride, 40, device="cuda").half()
            v = synth.normal(tokens * stride, 41, device="cuda").half()
            x = synth.normal(tokens * spec.width, 42, device="cuda")
            pos = torch.full((tokens,), count - 1, dtype=torch.int32, device="cuda")
            need = block.layer_workspace(layer, count, tokens)
            work = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
            d = layer.desc

            def call():
                check(L.mi_decoder_layer(ctx.handle, ctypes.byref(d), x.data_ptr(), k.data_ptr(), v.data_ptr(),
                                         stride, pos.data_ptr(), count, tokens, work.data_ptr(), work.numel()))
            with torch.cuda.stream(stream):
                for _ in range(3):
                    call()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    call()
                e1.record(stream)
                torch.cuda.synchronize()
            out[f"{name}_tokens_{tokens}_us"] = round(e0.elapsed_time(e1) * 1e3 / reps, 2)
        del ws, layer
        torch.cuda.empty_cache()
    return out


def _config1(L, h, stream, cpu=True, reps=400):
    """one Q8_0 4864x896 matvec at batch 1 (the
    reference's CPU-path config).  GPU: mi_matvec_xq on weights rotated over
    copies worth 1 GiB (cold), K back-to-back launches between HIP events;
    the activation's quantize is one more launch per call and is timed with
    it as `step_us`.  CPU: the oracle's matvec (kernel.mojo:316) on the same
    bytes, one thread and every usable one."""
    import numpy as np
    import torch

    import oracle
    from molla_amd import gpu, synth
    from molla_amd._lib import check

    rows, cols, kind = 4864, 896, gpu.Q_Q8_0
    rb = gpu.row_bytes(kind, cols)
    wbytes = rows * rb
    n = max(2, (1 << 30) // wbytes + 1)
    base = synth.quant_tensor(kind, rows, cols, 4864, device="cuda")
    ws = base.repeat(n)
    x = synth.normal(cols, 896, device="cuda")
    xq = torch.empty(L.mi_matvec_workspace(cols, 1), dtype=torch.uint8, device="cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    algo = _algo_bytes(rows, cols, 1, wbytes)

    def run(count, with_quant):
        for i in range(count):
            if with_quant:
                check(L.mi_quantize(h, x.data_ptr(), cols, 1, xq.data_ptr()))
            check(L.mi_matvec_xq(h, kind, ws.data_ptr() + (i % n) * wbytes, rb, rows, cols, xq.data_ptr(), 1,
                                 y.data_ptr(), 0, None))
    out = {"workload": "Q8_0 matvec 4864x896, batch 1 (BASELINE configs[0])", "weight_bytes": wbytes,
           "algorithmic_bytes": algo}
    check(L.mi_quantize(h, x.data_ptr(), cols, 1, xq.data_ptr()))
    for with_quant, key in ((False, "kernel_us"), (True, "step_us")):
        run(10, with_quant)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run(reps, with_quant)
        e1.record(stream)
        torch.cuda.synchronize()
        out[key] = round(e0.elapsed_time(e1) * 1e3 / reps, 3)
    out["GB_s"] = round(algo / out["kernel_us"] / 1e3, 1)
    out["frac_hbm_peak"] = round(algo / out["kernel_us"] / 1e3 / PEAK_GBS, 4)
    if cpu:
        blob = base.cpu().numpy()
        xh = x.cpu().numpy()
        threads = max(1, min(16, _host_facts()["usable_cpus"] or 1))
        t1, r1 = _timed(lambda: oracle.matvec(kind, blob, rows, cols, xh, threads=1), 2.0, 2000)
        tn, rn = _timed(lambda: oracle.matvec(kind, blob, rows, cols, xh, threads=threads), 1.0, 2000)
        out["cpu"] = {"us_1_thread": round(t1 * 1e6, 1), "GB_s_1_thread": round(algo / t1 / 1e9, 3), "reps_1": r1,
                      "threads": threads, f"us_{threads}_threads": round(tn * 1e6, 1),
                      f"GB_s_{threads}_threads": round(algo / tn / 1e9, 3), f"reps_{threads}": rn}
    del ws, base
    torch.cuda.empty_cache()
    return out


def _config4(L, copies=16, reps=8):
    """one 8B Llama layer (4096 wide, 32 query / 8 key
    heads of 128, MLP 14336, Q4_K, RMSNorm gains N(1, 0.1)) at batch 1 over an
    f16 cache pre-filled with N(0, 1) to 4096 positions, the token at
    position 4096.  `copies` distinct layers, each with its own cache
    (2.2 GB in all, past the 256 MB Infinity Cache), run in turn from one
    captured HIP graph, so each call streams cold weights and a cold cache;
    us per layer = graph time / copies.  The roofline is the layer's
    algorithmic bytes (weights + the 4097 cached keys and values) at 8 TB/s."""
    import ctypes

    import torch

    from molla_amd import block, gpu, synth
    from molla_amd._lib import check

    spec = block.BlockSpec()
    qw, kvw = spec.q_width(), spec.kv_width()
    shapes = {"wq": (qw, spec.width), "wk": (kvw, spec.width), "wv": (kvw, spec.width), "wo": (spec.width, qw),
              "gate": (spec.hidden, spec.width), "up": (spec.hidden, spec.width), "down": (spec.width, spec.hidden)}
    steps = torch.from_numpy(gpu.rope_steps(spec.rope_dim, spec.rope_base)).cuda()
    stream = torch.cuda.Stream()  # graphs are captured on a created stream
    ctx = gpu.DeviceContext(0, stream=stream)
    pos_v, count = 4096, 4097
    stride = count * kvw
    layers, caches = [], []
    for c in range(copies):
        ws = {n: gpu.Tensor.from_bytes(synth.quant_tensor(gpu.Q_Q4_K, r, cc, 700 + 10 * c + i, device="cuda"),
                                       gpu.Q_Q4_K, cc, r) for i, (n, (r, cc)) in enumerate(shapes.items())}
        an = synth.normal(spec.width, 780 + c, device="cuda", mean=1.0, std=0.1)
        fn = synth.normal(spec.width, 880 + c, device="cuda", mean=1.0, std=0.1)
        layers.append(block.DeviceLayer(spec, an, fn, ws, steps))
        caches.append((synth.normal(stride, 40 + c, device="cuda").half(),
                       synth.normal(stride, 140 + c, device="cuda").half()))
    x = synth.normal(spec.width, 42, device="cuda")
    pos = torch.full((1,), pos_v, dtype=torch.int32, device="cuda")
    need = block.layer_workspace(layers[0], count, 1)
    work = torch.empty(need + 256, dtype=torch.uint8, device="cuda")
    descs = [l.desc for l in layers]

    def all_layers():
        for d, (k, v) in zip(descs, caches):
            check(L.mi_decoder_layer(ctx.handle, ctypes.byref(d), x.data_ptr(), k.data_ptr(), v.data_ptr(), stride,
                                     pos.data_ptr(), count, 1, work.data_ptr(), work.numel()))
    with torch.cuda.stream(stream):
        all_layers()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            all_layers()
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * copies)
    wbytes = layers[0].weight_bytes()
    algo = wbytes + 2 * 2 * count * kvw
    del g, layers, caches, work
    torch.cuda.empty_cache()
    return {"workload": "8B Llama layer, Q4_K, batch 1, token at position 4096 over an f16 cache (BASELINE configs[3])",
            "us_per_layer": round(us, 2), "weight_bytes": wbytes, "algorithmic_bytes": algo,
            "GB_s": round(algo / us / 1e3, 1), "frac_hbm_peak": round(algo / us / 1e3 / PEAK_GBS, 4),
            "roofline_us": round(algo / PEAK_GBS / 1e3, 2), "copies": copies}


def _kinds(L, h, stream, reps=100):
    """Every other block-quantized kind at the same 14336x4096 batch-1 shape
    (and batch 4 on the same launch path a decode step uses): weights rotated
    over copies worth > 512 MB, twice the Infinity Cache, so reads are cold."""
    import torch

    from molla_amd import gpu, synth
    from molla_amd._lib import check

    x = synth.normal(4 * COLS, 21, device="cuda")
    xq = torch.empty(L.mi_matvec_workspace(COLS, 4), dtype=torch.uint8, device="cuda")
    y = torch.empty(4 * ROWS, dtype=torch.float32, device="cuda")
    check(L.mi_quantize(h, x.data_ptr(), COLS, 4, xq.data_ptr()))
    names = {gpu.Q_Q4_0: "q4_0", gpu.Q_Q4_1: "q4_1", gpu.Q_Q5_0: "q5_0", gpu.Q_Q5_1: "q5_1", gpu.Q_Q8_0: "q8_0",
             gpu.Q_Q5_K: "q5_k", gpu.Q_Q6_K: "q6_k"}
    out = {}
    for kind, name in names.items():
        rb = gpu.row_bytes(kind, COLS)
        wbytes = ROWS * rb
        n = max(2, (512 << 20) // wbytes + 1)
        base = synth.quant_tensor(kind, ROWS, COLS, 31 + kind, device="cuda")
        ws = [base] + [base.clone() for _ in range(n - 1)]
        row = {}
        for tokens in (1, 4):
            for i in range(5):
                check(L.mi_matvec_xq(h, kind, ws[i % n].data_ptr(), rb, ROWS, COLS, xq.data_ptr(), tokens,
                                     y.data_ptr(), 0, None))
            torch.cuda.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(reps):
                check(L.mi_matvec_xq(h, kind, ws[i % n].data_ptr(), rb, ROWS, COLS, xq.data_ptr(), tokens,
                                     y.data_ptr(), 0, None))
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / reps
            algo = _algo_bytes(ROWS, COLS, tokens, wbytes)
            row[f"tokens_{tokens}"] = {"us": round(us, 3), "GB_s": round(algo / us / 1e3, 1),
                                       "frac_hbm_peak": round(algo / us / 1e3 / PEAK_GBS, 4)}
        out[name] = row
        del ws, base
    torch.cuda.empty_cache()
    return out


def _traffic_from_profile():
    """HBM bytes per launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel's reading), or None."""
    p = os.path.join(ROOT, "profiles", "q4k_matvec_14336x4096_traffic.json")
    if os.path.exists(p):
        with open(p) as f:
            return json.load(f).get("bytes_per_launch")
    return None


def _host_facts():
    """The host the CPU baseline ran on: logical CPUs, the ones this process
    may use, and the CPU model from /proc/cpuinfo."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"nproc": os.cpu_count(), "usable_cpus": usable, "cpu_model": model}


def _timed(fn, budget_s, max_reps):
    t0 = time.perf_counter()
    reps = 0
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el > budget_s or reps >= max_reps:
            return el / reps, reps


def _cpu_baseline(w_dev, kind, rb, x_dev, model=None):
    """The CPU oracle (a C restatement of molla's host path) on the GPU box's
    host, bounded to roughly 15-25 s of work:
      * the config-2 matvec (kernel.mojo:316, the same bytes as the GPU
        line), serial as the reference's host path is -- this is `value` --
        and row-parallel over `threads` cores with OpenMP (the courtesy
        variant of the reference's own baseline);
      * one config-4 decoder layer (block.mojo:466: hidden 4096, 32/8 heads
        of 128, MLP 14336, Q4_K, a cache of 4096 positions, the token at
        4096), serial and threaded;
      * one token of the synthetic 8B model (model.mojo:178 forward at
        position 0 over the decode line's weights), serial and threaded."""
    import numpy as np

    import oracle
    from molla_amd import synth

    facts = _host_facts()
    threads = max(1, min(16, facts["usable_cpus"] or 1))
    blob = w_dev.cpu().numpy()
    x = x_dev.cpu().numpy()
    algo = _algo_bytes(ROWS, COLS, 1, ROWS * rb)
    per1, reps1 = _timed(lambda: oracle.matvec(kind, blob, ROWS, COLS, x, threads=1), 6.0, 200)
    pern, repsn = _timed(lambda: oracle.matvec(kind, blob, ROWS, COLS, x, threads=threads), 2.0, 400)
    out = {"value": round(algo / per1 / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{reps1} full Q4_K 14336x4096 matvecs (same bytes), {per1 * 1e3:.1f} ms each, one thread",
           "host": facts,
           "matvec_threads": {"threads": threads, "GB_s": round(algo / pern / 1e9, 3), "ms": round(pern * 1e3, 3),
                              "reps": repsn}}

    # config 4: one layer at position 4096
    spec = dict(width=4096, hidden=14336, heads=32, kv_heads=8, head_dim=128, rope_dim=128, neox=0, eps=1e-5,
                rope_base=500000.0, attn_scale=float(np.float32(1 / np.sqrt(128.0))))
    shapes = {"wq": (4096, 4096), "wk": (1024, 4096), "wv": (1024, 4096), "wo": (4096, 4096),
              "gate": (14336, 4096), "up": (14336, 4096), "down": (4096, 14336)}
    host = {n: (kind, r, c, synth.quant_tensor(kind, r, c, 500 + i).numpy()) for i, (n, (r, c)) in
            enumerate(shapes.items())}
    host["attn_norm"] = synth.normal(4096, 510, mean=1.0, std=0.1).numpy()
    host["ffn_norm"] = synth.normal(4096, 511, mean=1.0, std=0.1).numpy()
    keep = []
    L = oracle.make_layer(spec, host, keep)
    pos = 4096
    keys0 = synth.normal((pos + 1) * 1024, 512).half().float().numpy()
    vals0 = synth.normal((pos + 1) * 1024, 513).half().float().numpy()
    xl = synth.normal(4096, 514).numpy()

    def layer(t):
        oracle.layer_step(L, xl.copy(), keys0.copy(), vals0.copy(), pos, pos, f16_store=True, threads=t)
    l1, lr1 = _timed(lambda: layer(1), 3.0, 50)
    ln, lrn = _timed(lambda: layer(threads), 1.5, 100)
    lbytes = sum(host[n][3].nbytes for n in shapes) + 2 * 2 * (pos + 1) * 1024
    out["layer_config4"] = {"bytes": lbytes, "ms_1_thread": round(l1 * 1e3, 2), "reps_1": lr1,
                            f"ms_{threads}_threads": round(ln * 1e3, 2), f"reps_{threads}": lrn}
    del host, keep, L, keys0, vals0

    if model is not None:
        s = model.spec
        ospec = dict(width=s.width, hidden=s.hidden, heads=s.heads, kv_heads=s.kv_heads, head_dim=s.head_dim,
                     rope_dim=s.rope_dim, neox=int(s.neox), eps=s.eps, rope_base=s.rope_base,
                     attn_scale=s.attn_scale)
        keep = []
        layers = []
        for lay in model.layers:
            w = {n: (t.kind, t.rows, t.cols, t.keep.cpu().numpy()) for n, t in lay.weights.items()}
            w["attn_norm"] = lay.attn_norm.cpu().numpy()
            w["ffn_norm"] = lay.ffn_norm.cpu().numpy()
            layers.append(oracle.make_layer(ospec, w, keep))
        head = (model.output.kind, model.output.rows, model.output.cols, model.output.keep.cpu().numpy())
        emb = model.embedding.cpu().numpy()
        onorm = model.output_norm.cpu().numpy()
        kvw = s.kv_width()

        def token(t):
            ks = [np.zeros(kvw, np.float32) for _ in layers]
            vs = [np.zeros(kvw, np.float32) for _ in layers]
            oracle.forward(layers, emb, onorm, head, 17, 0, 0, ks, vs, f16_store=True, threads=t)
        t1, _ = _timed(lambda: token(1), 0.0, 1)
        tn, trn = _timed(lambda: token(threads), 1.0, 5)
        out["token_8b"] = {"weight_bytes": model.weight_bytes(), "s_1_thread": round(t1, 3),
                           "tokens_per_s_1_thread": round(1 / t1, 3), f"s_{threads}_threads": round(tn, 3),
                           f"tokens_per_s_{threads}_threads": round(1 / tn, 2), f"reps_{threads}": trn}
        del layers, keep, head, emb
    return out


def _stream_peak(stream, reps=200):
    """The read ceiling measured on this box: plain streaming reads
    (libmolla_probe.so probe_read, every loaded byte folded into the result)
    of buffers the size of the decode step's matrices (wo 9.4 MB, q|k|v
    14.2 MB, one 33 MB Q4_K matrix, gate+up 66 MB), each rotated over 2 GiB
    so every launch reads cold HBM and timed like the roofline (K
    back-to-back launches between HIP events), and of a 1 GiB buffer; the
    best over two access shapes (grid-stride, contiguous chunk per wave with
    8 or 16 loads in flight) and four grid sizes."""
    import ctypes

    import torch

    plib = ctypes.CDLL(os.path.join(ROOT, "molla_amd", "libmolla_probe.so"))
    plib.probe_read.restype = ctypes.c_int
    plib.probe_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                ctypes.c_int32]
    size = ROWS * (COLS // 256) * 144
    sizes = (("read_9MB", 9437184, reps), ("read_14MB", 14155776, reps), ("read_33MB", size, reps),
             ("read_66MB", 2 * size, reps // 2), ("read_1GiB", 1 << 30, 10))
    span = 2 << 30
    big = torch.empty(span + (1 << 30), dtype=torch.uint8, device="cuda")
    big.view(torch.float32).zero_()
    sink = torch.zeros(1, device="cuda")
    h = stream.cuda_stream
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def run(nbytes, count, blocks, variant):
        slot = (nbytes + 4095) // 4096 * 4096
        n = max(1, span // slot) if nbytes < span else 1
        for i in range(count):
            off = (i % n) * slot
            if plib.probe_read(h, big.data_ptr() + off, nbytes, blocks, sink.data_ptr(), variant) != 0:
                raise RuntimeError("probe_read launch failed")

    out = {}
    for name, nbytes, count in sizes:
        best = None
        for variant in (0, 1, 2):
            for blocks in (1024, 2048, 4096, 8192):
                run(nbytes, 5, blocks, variant)
                torch.cuda.synchronize()
                e0.record(stream)
                run(nbytes, count, blocks, variant)
                e1.record(stream)
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / count
                if best is None or us < best[0]:
                    best = (us, blocks, variant)
        out[name] = {"bytes": nbytes, "us": round(best[0], 3), "GB_s": round(nbytes / best[0] / 1e3, 1),
                     "blocks": best[1], "shape": ("grid-stride", "chunk x8", "chunk x16")[best[2]]}
    del big
    torch.cuda.empty_cache()
    return out


def _decode(ctx, args, model=None):
    """Config 5: synthetic 8B (32 layers, Q4_K, Q6_K head, f32 embedding);
    a prompt of uniform random ids prefilled in 256-token chunks through the
    prefill layer (gpu_block.mojo:1654 forward over a chunk; each sequence of
    a batch on its own), then greedy decode at each batch size asked for
    (independent sequences, one token each per step).  Reported per batch:
    decode tokens/s over all sequences, ms per step, and the prefill's time
    and prompt tokens/s (HIP events around all of it, head included)."""
    import torch

    from molla_amd import block, gpu, synth

    spec = block.BlockSpec()
    vocab = 128256
    dev = "cuda"
    if model is None:
        model = block.synthetic_model(spec, 32, vocab, device=dev)
    wb = model.weight_bytes()
    out = {"metric": "8B Q4_K decode tokens/sec", "prompt": args.prompt, "generated": args.decode_tokens,
           "weight_bytes_per_step": wb}
    # the session's own stream: the step is captured as one HIP graph
    # (DeviceSession.capture), which removes the host's ~10 launches per layer
    stream = torch.cuda.Stream()
    dctx = gpu.DeviceContext(0, stream=stream)
    eager_n = 16
    runs = [(b, gpu.CACHE_F16) for b in args.decode_batch] + [(b, gpu.CACHE_Q8) for b in args.decode_q8]
    for batch, form in runs:
        ctxlen = args.prompt + args.decode_tokens + eager_n + 1
        with torch.cuda.stream(stream):
            sess = block.DeviceSession(dctx, model, batch=batch, context=ctxlen, cache_form=form)
            prompt = synth.tokens(args.prompt * batch, vocab, 5 + batch, device=dev).view(args.prompt, batch)
            sess.pos.zero_()
            # the prompt in 256-token chunks through the prefill layer, each
            # sequence on its own (DeviceSession.prefill), then the head over
            # every sequence's last row; a first small chunk loads the kernels
            warm = prompt[:16, 0].contiguous()
            sess.prefill(warm, seq=0, start=0, chunk=16)
            stream.synchronize()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for b in range(batch):
                sess.prefill(prompt[:, b].contiguous(), seq=b, start=0, chunk=args.prefill_chunk)
            sess.finish()
            e1.record(stream)
            stream.synchronize()
            prefill_ms = e0.elapsed_time(e1)
            sess.ids.copy_(sess.picks)
            # a few eager steps, for the host-launch cost the graph removes
            e0.record(stream)
            for _ in range(eager_n):
                sess.step()
                sess.advance()
            e1.record(stream)
            stream.synchronize()
            eager_ms = e0.elapsed_time(e1) / eager_n
            gd = sess.capture(advance=True)
            e0.record(stream)
            for _ in range(args.decode_tokens):
                gd.replay()
            e1.record(stream)
            stream.synchronize()
        ms_step = e0.elapsed_time(e1) / args.decode_tokens
        gbs = wb / (ms_step * 1e-3) / 1e9
        out[f"batch_{batch}" + ("_q8_cache" if form == gpu.CACHE_Q8 else "")] = {"tokens_per_s": round(1000 * batch / ms_step, 2), "ms_per_step": round(ms_step, 3),
                                 "weight_stream_gbs": round(gbs, 1), "frac_of_weight_roofline": round(gbs / PEAK_GBS, 4),
                                 "eager_ms_per_step": round(eager_ms, 3),
                                 "prefill_ms": round(prefill_ms, 2),
                                 "prefill_tokens_per_s": round(batch * args.prompt / (prefill_ms * 1e-3), 1)}
        del gd
        del sess
        torch.cuda.empty_cache()
    return out


if __name__ == "__main__":
    main()
