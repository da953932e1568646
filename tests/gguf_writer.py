"""A small GGUF v3 writer for the tests: builds files for molla_amd.gguf and
molla_amd.load to read back (the format as the GGUF specification lays it
out; see molla_amd/gguf.py for the layout).

    write_gguf(path, kvs, tensors, alignment=32)
      kvs:     [(key, value_type, value)]; value_type a GGUF_* code, and for
               GGUF_ARRAY value = (element_type, [elements])
      tensors: [(name, dims, ggml_type, bytes)], dims fastest first
"""

from __future__ import annotations

import struct

import numpy as np

import oracle
from molla_amd import synth

from molla_amd.gguf import (GGUF_ARRAY, GGUF_BOOL, GGUF_FLOAT32, GGUF_FLOAT64, GGUF_INT8, GGUF_INT16,
                            GGUF_INT32, GGUF_INT64, GGUF_STRING, GGUF_UINT8, GGUF_UINT16, GGUF_UINT32,
                            GGUF_UINT64)

_FMT = {GGUF_UINT8: "<B", GGUF_INT8: "<b", GGUF_UINT16: "<H", GGUF_INT16: "<h", GGUF_UINT32: "<I",
        GGUF_INT32: "<i", GGUF_FLOAT32: "<f", GGUF_BOOL: "<B", GGUF_UINT64: "<Q", GGUF_INT64: "<q",
        GGUF_FLOAT64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(kind: int, value) -> bytes:
    if kind == GGUF_STRING:
        return _string(value)
    if kind == GGUF_ARRAY:
        element, items = value
        out = struct.pack("<IQ", element, len(items))
        return out + b"".join(_value(element, v) for v in items)
    return struct.pack(_FMT[kind], value)


def header_bytes(kvs, tensors, alignment: int = 32, version: int = 3) -> tuple[bytes, list]:
    """The bytes before the data section and each tensor's data offset."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for key, kind, value in kvs:
        out += _string(key) + struct.pack("<I", kind) + _value(kind, value)
    offsets, at = [], 0
    for _, _, _, data in tensors:
        offsets.append(at)
        at += len(data)
        at += (-at) % alignment
    for (name, dims, kind, _), off in zip(tensors, offsets):
        out += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", kind, off)
    out += b"\0" * ((-len(out)) % alignment)
    return bytes(out), offsets


def write_gguf(path: str, kvs, tensors, alignment: int = 32, version: int = 3) -> None:
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in kvs):
        kvs = list(kvs) + [("general.alignment", GGUF_UINT32, alignment)]
    head, offsets = header_bytes(kvs, tensors, alignment, version)
    with open(path, "wb") as f:
        f.write(head)
        at = 0
        for (_, _, _, data), off in zip(tensors, offsets):
            f.write(b"\0" * (off - at))
            f.write(bytes(data))
            at = off + len(data)


def llama_file(path, width=256, hidden=512, heads=4, kv_heads=2, layers=2, vocab=300, kinds=None, tied=False,
               factors=True, seed=1):
    """A Llama GGUF with synthetic weights; returns the host tensors by name."""
    kinds = kinds or {}
    head_dim = width // heads
    kvs = [("general.architecture", GGUF_STRING, "llama"),
           ("llama.embedding_length", GGUF_UINT32, width), ("llama.feed_forward_length", GGUF_UINT32, hidden),
           ("llama.block_count", GGUF_UINT32, layers), ("llama.attention.head_count", GGUF_UINT32, heads),
           ("llama.attention.head_count_kv", GGUF_UINT32, kv_heads),
           ("llama.attention.layer_norm_rms_epsilon", GGUF_FLOAT32, 1e-5),
           ("llama.rope.freq_base", GGUF_FLOAT32, 500000.0), ("llama.context_length", GGUF_UINT32, 8192)]
    ts, host = [], {}
    s = seed * 1000

    def add(name, dims, kind, data):
        ts.append((name, dims, kind, data))
        host[name] = (kind, data)

    def quant(name, rows, cols, kind):
        nonlocal s
        s += 1
        add(name, (cols, rows), kind, synth.quant_tensor(kind, rows, cols, s).numpy().tobytes())

    def vec(name, n, mean=1.0, std=0.1):
        nonlocal s
        s += 1
        add(name, (n,), 0, synth.normal(n, s, mean=mean, std=std).numpy().tobytes())

    quant("token_embd.weight", vocab, width, kinds.get("embd", oracle.Q8_0))
    vec("output_norm.weight", width)
    if not tied:
        quant("output.weight", vocab, width, kinds.get("output", oracle.Q6_K))
    if factors:
        pairs = head_dim // 2
        f = np.concatenate([np.ones(pairs - pairs // 2), np.linspace(1.5, 8.0, pairs // 2)]).astype(np.float32)
        add("rope_freqs.weight", (pairs,), 0, f.tobytes())
    qw, kvw = heads * head_dim, kv_heads * head_dim
    for i in range(layers):
        vec(f"blk.{i}.attn_norm.weight", width)
        vec(f"blk.{i}.ffn_norm.weight", width)
        quant(f"blk.{i}.attn_q.weight", qw, width, kinds.get("attn", oracle.Q4_K))
        quant(f"blk.{i}.attn_k.weight", kvw, width, kinds.get("attn", oracle.Q4_K))
        quant(f"blk.{i}.attn_v.weight", kvw, width, kinds.get("attn_v", oracle.Q6_K))
        quant(f"blk.{i}.attn_output.weight", width, qw, kinds.get("attn", oracle.Q4_K))
        quant(f"blk.{i}.ffn_gate.weight", hidden, width, kinds.get("ffn", oracle.Q4_K))
        quant(f"blk.{i}.ffn_up.weight", hidden, width, kinds.get("ffn", oracle.Q4_K))
        quant(f"blk.{i}.ffn_down.weight", width, hidden, kinds.get("down", oracle.Q6_K))
    write_gguf(path, kvs, ts)
    return host
