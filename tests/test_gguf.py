"""GGUF reader and Llama plan (molla_amd.gguf, molla_amd.load.read_llama) on
files written by tests/gguf_writer.py, following the reference's reader tests
(tests/test_gguf.mojo: typed keys, arrays counted without decoding, the
fallback getters, alignment, and the refusals of a malformed file)."""

import struct

import numpy as np
import pytest

import oracle
from molla_amd import gguf, load, synth
from molla_amd.gguf import (GGUF_ARRAY, GGUF_BOOL, GGUF_FLOAT32, GGUF_FLOAT64, GGUF_INT8, GGUF_INT16,
                            GGUF_INT32, GGUF_INT64, GGUF_STRING, GGUF_UINT8, GGUF_UINT16, GGUF_UINT32,
                            GGUF_UINT64, Gguf, GgufError)
from tests.gguf_writer import header_bytes, llama_file, write_gguf

KVS = [
    ("general.architecture", GGUF_STRING, "llama"),
    ("general.name", GGUF_STRING, "tiny"),
    ("a.u8", GGUF_UINT8, 200), ("a.i8", GGUF_INT8, -5), ("a.u16", GGUF_UINT16, 60000),
    ("a.i16", GGUF_INT16, -300), ("a.u32", GGUF_UINT32, 4000000000), ("a.i32", GGUF_INT32, -7),
    ("a.u64", GGUF_UINT64, 1 << 40), ("a.i64", GGUF_INT64, -(1 << 40)),
    ("a.f32", GGUF_FLOAT32, 0.5), ("a.f64", GGUF_FLOAT64, 1e-300), ("a.bool", GGUF_BOOL, 1),
    ("llama.rope.freq_base", GGUF_UINT32, 10000),  # an integer where a float is expected
    ("tokenizer.ggml.tokens", GGUF_ARRAY, (GGUF_STRING, ["<s>", "a", "bé"])),
    ("tokenizer.ggml.scores", GGUF_ARRAY, (GGUF_FLOAT32, [0.0, -1.5, 2.25])),
]


def tensors_small():
    q = synth.quant_tensor(oracle.Q4_K, 3, 512, 5).numpy().tobytes()
    f = np.arange(7, dtype=np.float32).tobytes()
    return [("w.q4k", (512, 3), 12, q), ("v.f32", (7,), 0, f)]


def test_round_trip_metadata_and_tensors(tmp_path):
    p = str(tmp_path / "a.gguf")
    ts = tensors_small()
    write_gguf(p, KVS, ts)
    with Gguf(p) as g:
        assert g.version == 3 and g.kv_count == len(KVS) and g.tensor_count == 2
        assert g.alignment == 32 and g.data_start % 32 == 0
        for key, kind, value in KVS:
            i = g.find(key)
            assert i >= 0 and g.key_name(i) == key and g.kvs[i].kind == kind
        assert g.string(g.find("general.name")) == "tiny"
        assert g.uint(g.find("a.u8")) == 200 and g.uint(g.find("a.i8")) == -5
        assert g.uint(g.find("a.u64")) == 1 << 40 and g.uint(g.find("a.i64")) == -(1 << 40)
        assert g.flt(g.find("a.f32")) == 0.5 and g.flt(g.find("a.f64")) == 1e-300
        assert g.value("a.bool") is True and g.value("missing") is None
        # arrays are counted from the directory; elements decode on request
        assert g.array_count("tokenizer.ggml.tokens") == 3 and g.array_count("a.u8") == 0
        assert g.value("tokenizer.ggml.tokens") == ["<s>", "a", "bé"]
        assert g.value("tokenizer.ggml.scores") == [0.0, -1.5, 2.25]
        # fallbacks: absent key, wrong type
        assert g.string_or("nope", "x") == "x" and g.string_or("a.u8", "x") == "x"
        assert g.uint_or("nope", 9) == 9 and g.uint_or("general.name", 9) == 9
        assert g.float_or("llama.rope.freq_base", 1.0) == 10000.0  # an int accepted as a float
        assert g.float_or("general.name", 2.0) == 2.0
        assert g.bool_or("a.bool", False) is True and g.bool_or("nope", True) is True
        with pytest.raises(GgufError):
            g.uint(g.find("general.name"))
        with pytest.raises(GgufError):
            g.string(g.find("a.u8"))
        with pytest.raises(GgufError):
            g.flt(g.find("a.u8"))
        assert g.architecture() == "llama" and g.has("a.f32") and not g.has("a.f16")
        # tensors
        assert g.tensor_index("v.f32") == 1 and g.tensor_index("nope") == -1
        assert g.tensor_prefixed("w.") and not g.tensor_prefixed("x.")
        t = g.tensor("w.q4k")
        assert t.dims == (512, 3) and t.kind == 12 and t.elements() == 1536 and t.nbytes() == 3 * 288
        for (name, _, _, data) in ts:
            ti = g.tensor(name)
            assert ti.offset % 32 == 0
            assert bytes(g.tensor_data(ti)) == data
        assert gguf.ggml_type_name(12) == "Q4_K" and gguf.value_type_name(GGUF_ARRAY) == "arr"


def test_custom_alignment(tmp_path):
    p = str(tmp_path / "b.gguf")
    write_gguf(p, KVS[:2], tensors_small(), alignment=64)
    with Gguf(p) as g:
        assert g.alignment == 64 and g.data_start % 64 == 0
        assert all(t.offset % 64 == 0 for t in g.tensors)
        assert bytes(g.tensor_data(g.tensor("v.f32"))) == np.arange(7, dtype=np.float32).tobytes()


def _expect_refusal(tmp_path, blob, what):
    p = str(tmp_path / "bad.gguf")
    with open(p, "wb") as f:
        f.write(blob)
    with pytest.raises(GgufError, match=what):
        Gguf(p)


def test_refusals(tmp_path):
    good, _ = header_bytes(KVS[:2], [])
    _expect_refusal(tmp_path, b"GGML" + good[4:], "bad magic")
    _expect_refusal(tmp_path, b"GG", "bad magic")
    _expect_refusal(tmp_path, good[:4] + struct.pack("<I", 1) + good[8:], "version")
    _expect_refusal(tmp_path, good[:30], "truncated")
    nested, _ = header_bytes([("x", GGUF_ARRAY, (GGUF_UINT8, []))], [])
    nested = nested.replace(struct.pack("<II", GGUF_ARRAY, GGUF_UINT8), struct.pack("<II", GGUF_ARRAY, GGUF_ARRAY))
    _expect_refusal(tmp_path, nested, "nested")
    five, _ = header_bytes([], [("t", (1, 1, 1, 1), 0, b"\0" * 4)])
    five = five.replace(struct.pack("<I", 4) + struct.pack("<Q", 1) * 4,
                        struct.pack("<I", 5) + struct.pack("<Q", 1) * 4)
    _expect_refusal(tmp_path, five, "dimensions")
    odd, _ = header_bytes([("general.alignment", GGUF_UINT32, 48)], [])
    _expect_refusal(tmp_path, odd, "power of two")


def test_tensor_past_the_end(tmp_path):
    p = str(tmp_path / "c.gguf")
    write_gguf(p, KVS[:1], tensors_small())
    with open(p, "r+b") as f:  # cut the last tensor short
        f.truncate(f.seek(0, 2) - 8)
    with Gguf(p) as g:
        with pytest.raises(GgufError, match="past the end"):
            g.tensor_data(g.tensor("v.f32"))


# ---- a tiny Llama file (tests/gguf_writer.py llama_file) -------------------------


def test_read_llama_plan(tmp_path):
    p = str(tmp_path / "m.gguf")
    llama_file(p)
    with Gguf(p) as g:
        plan = load.read_llama(g)
    assert (plan.width, plan.hidden, plan.heads, plan.kv_heads, plan.head_dim) == (256, 512, 4, 2, 64)
    assert (plan.rope_dim, plan.rope_base, plan.n_layers, plan.vocab, plan.context) == (64, 500000.0, 2, 300, 8192)
    assert abs(plan.eps - 1e-5) < 1e-12 and not plan.tied and plan.rope_factors is not None
    assert plan.output.name == "output.weight" and len(plan.layers) == 2
    assert plan.layers[1]["down"].name == "blk.1.ffn_down.weight" and plan.layers[1]["down"].kind == oracle.Q6_K


def test_read_llama_tied_head(tmp_path):
    p = str(tmp_path / "t.gguf")
    llama_file(p, tied=True, factors=False)
    with Gguf(p) as g:
        plan = load.read_llama(g)
    assert plan.tied and plan.output is plan.embedding and plan.rope_factors is None


def test_read_llama_refusals(tmp_path):
    p = str(tmp_path / "r.gguf")
    llama_file(p, layers=1)
    with Gguf(p) as g:
        plan = load.read_llama(g)
    assert plan.n_layers == 1
    # a projection stored unquantized has no device matvec
    q = str(tmp_path / "f32.gguf")
    host = llama_file(q, layers=1)
    with Gguf(q) as g:
        kvs = [(kv.key, kv.kind, g.value(kv.key)) for kv in g.kvs]
        ts = [(t.name, t.dims, t.kind, bytes(g.tensor_data(t))) for t in g.tensors]
    ts = [(n, d, 0, b"\0" * (d[0] * d[1] * 4)) if n == "blk.0.attn_q.weight" else (n, d, k, b)
          for (n, d, k, b) in ts]
    write_gguf(q, kvs, ts)
    with Gguf(q) as g:
        with pytest.raises(GgufError, match="no device matvec"):
            load.read_llama(g)
    # a missing tensor is named (the file otherwise as written)
    with Gguf(p) as g:
        ts = [(t.name, t.dims, t.kind, bytes(g.tensor_data(t))) for t in g.tensors]
    ts2 = [t for t in ts if t[0] != "blk.0.ffn_up.weight"]
    write_gguf(q, kvs, ts2)
    with Gguf(q) as g:
        with pytest.raises(GgufError, match="blk.0.ffn_up.weight"):
            load.read_llama(g)
    assert host  # the writer returned the host tensors
