"""GGUF reader: header, metadata and tensor directory, read in place from a
memory map (the host side of src/molla/model/gguf.mojo, whose accessor names
and refusals this mirrors: `Gguf.find`, `uint`, `string`, `flt`, the `*_or`
fallbacks, `array_count`, `tensor_index`, `architecture`, ...).

Layout (GGUF v2/v3, little endian):
    "GGUF"  u32 version  u64 tensor_count  u64 kv_count
    kv_count x (string key, u32 type, value)
    tensor_count x (string name, u32 n_dims, n_dims x u64 ne, u32 ggml type, u64 offset)
    padding to general.alignment (32 when absent), then tensor data;
    a tensor's bytes start at data_start + offset.
A string is u64 length + bytes; an array is u32 element type + u64 count +
elements.  ne[0] is the fastest dimension: a [rows x cols] weight matrix has
ne = (cols, rows), its rows back to back in GGUF blocks.

Every read is bounds checked against the file, and array elements are only
skipped over, so the directory of a model file costs a few KB no matter how
large its vocabulary is.  Values are decoded on request from the recorded
offset.
"""

from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass

GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32 = 0, 1, 2, 3, 4, 5
GGUF_FLOAT32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY, GGUF_UINT64, GGUF_INT64, GGUF_FLOAT64 = 6, 7, 8, 9, 10, 11, 12
GGUF_MAX_DIMS = 4
DEFAULT_ALIGNMENT = 32

# fixed-size scalar types: struct format and size
_SCALAR = {GGUF_UINT8: "<B", GGUF_INT8: "<b", GGUF_UINT16: "<H", GGUF_INT16: "<h", GGUF_UINT32: "<I",
           GGUF_INT32: "<i", GGUF_FLOAT32: "<f", GGUF_BOOL: "<B", GGUF_UINT64: "<Q", GGUF_INT64: "<q",
           GGUF_FLOAT64: "<d"}
_INTS = (GGUF_UINT8, GGUF_INT8, GGUF_UINT16, GGUF_INT16, GGUF_UINT32, GGUF_INT32, GGUF_UINT64, GGUF_INT64,
         GGUF_BOOL)

# ggml type -> (values per block, bytes per block), quant.mojo block_elements / block_bytes
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
              12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}
GGML_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0", 9: "Q8_1",
              10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 16: "IQ2_XXS",
              17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S",
              23: "IQ4_XS", 24: "I8", 25: "I16", 26: "I32", 27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16"}
VALUE_NAMES = {GGUF_UINT8: "u8", GGUF_INT8: "i8", GGUF_UINT16: "u16", GGUF_INT16: "i16", GGUF_UINT32: "u32",
               GGUF_INT32: "i32", GGUF_FLOAT32: "f32", GGUF_BOOL: "bool", GGUF_STRING: "str",
               GGUF_ARRAY: "arr", GGUF_UINT64: "u64", GGUF_INT64: "i64", GGUF_FLOAT64: "f64"}


class GgufError(ValueError):
    """A malformed or unsupported GGUF file."""


def ggml_type_name(kind: int) -> str:
    return GGML_NAMES.get(kind, f"type{kind}")


def value_type_name(kind: int) -> str:
    return VALUE_NAMES.get(kind, f"type{kind}")


@dataclass(frozen=True)
class KeyValue:
    key: str
    kind: int      # GGUF value type
    payload: int   # file offset of the value (of the first element, for an array)
    element: int   # element type of an array, -1 otherwise
    count: int     # elements of an array, 1 otherwise


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dims: tuple    # ne[0..n_dims), fastest first
    kind: int      # ggml type
    offset: int    # from the start of the data section

    @property
    def n_dims(self) -> int:
        return len(self.dims)

    def dim(self, i: int) -> int:
        return self.dims[i] if i < len(self.dims) else 1

    def elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def nbytes(self) -> int:
        """Bytes of the tensor's data: whole blocks along ne[0]."""
        if self.kind not in GGML_BLOCK:
            raise GgufError(f"tensor {self.name}: ggml type {ggml_type_name(self.kind)} has no block geometry here")
        per, nb = GGML_BLOCK[self.kind]
        if self.dims[0] % per:
            raise GgufError(f"tensor {self.name}: {self.dims[0]} values is not a whole number of {per}-value blocks")
        return self.elements() // per * nb


class _Cursor:
    def __init__(self, buf, length: int):
        self.buf, self.length, self.at = buf, length, 0

    def need(self, n: int) -> None:
        if n < 0 or self.at + n > self.length:
            raise GgufError(f"gguf truncated: {n} bytes wanted at offset {self.at} of {self.length}")

    def scalar(self, kind: int):
        fmt = _SCALAR[kind]
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.buf, self.at)[0]
        self.at += n
        return v

    def u32(self) -> int:
        return self.scalar(GGUF_UINT32)

    def u64(self) -> int:
        return self.scalar(GGUF_UINT64)

    def skip(self, n: int) -> None:
        self.need(n)
        self.at += n

    def string(self) -> str:
        n = self.u64()
        self.need(n)
        s = bytes(self.buf[self.at:self.at + n]).decode("utf-8", errors="replace")
        self.at += n
        return s


class Gguf:
    """A parsed GGUF file, mapped read-only (src/molla/model/gguf.mojo Gguf)."""

    def __init__(self, path: str):
        self.path = path
        self._file = open(path, "rb")
        size = os.fstat(self._file.fileno()).st_size
        if size == 0:
            self._file.close()
            raise GgufError("not a gguf file: empty")
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        self.length = size
        self.version = 0
        self.kvs: list[KeyValue] = []
        self.tensors: list[TensorInfo] = []
        self.alignment = DEFAULT_ALIGNMENT
        self.data_start = 0
        self._keys: dict[str, int] = {}
        self._names: dict[str, int] = {}
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    # ---- parsing -------------------------------------------------------------
    def _parse(self) -> None:
        cur = _Cursor(self._map, self.length)
        if self.length < 4 or bytes(self._map[0:4]) != b"GGUF":
            raise GgufError("not a gguf file: bad magic")
        cur.skip(4)
        self.version = cur.u32()
        if self.version not in (2, 3):
            raise GgufError(f"unsupported gguf version {self.version}")
        tensor_count, kv_count = cur.u64(), cur.u64()
        # every entry takes at least a few bytes: bounds the counts by the file
        if tensor_count > self.length or kv_count > self.length:
            raise GgufError("gguf counts exceed the file")
        for _ in range(kv_count):
            key = cur.string()
            kind = cur.u32()
            element, count, payload = -1, 1, cur.at
            if kind == GGUF_ARRAY:
                element, count = cur.u32(), cur.u64()
                payload = cur.at
                if element == GGUF_STRING:
                    for _ in range(count):
                        cur.skip(cur.u64())
                elif element == GGUF_ARRAY:
                    raise GgufError("gguf nested arrays are not in the format")
                elif element in _SCALAR:
                    cur.skip(struct.calcsize(_SCALAR[element]) * count)
                else:
                    raise GgufError(f"gguf array of unknown type {element}")
            elif kind == GGUF_STRING:
                cur.skip(cur.u64())
            elif kind in _SCALAR:
                cur.skip(struct.calcsize(_SCALAR[kind]))
            else:
                raise GgufError(f"gguf value of unknown type {kind} for key {key}")
            self._keys.setdefault(key, len(self.kvs))
            self.kvs.append(KeyValue(key, kind, payload, element, count))
        for _ in range(tensor_count):
            name = cur.string()
            n_dims = cur.u32()
            if n_dims < 1 or n_dims > GGUF_MAX_DIMS:
                raise GgufError(f"gguf tensor {name} has {n_dims} dimensions")
            dims = tuple(cur.u64() for _ in range(n_dims))
            kind = cur.u32()
            offset = cur.u64()
            self._names.setdefault(name, len(self.tensors))
            self.tensors.append(TensorInfo(name, dims, kind, offset))
        i = self.find("general.alignment")
        if i >= 0:
            self.alignment = self.uint(i)
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GgufError(f"gguf alignment {self.alignment} is not a power of two")
        self.data_start = cur.at + (-cur.at) % self.alignment
        if self.data_start > self.length:
            raise GgufError("gguf header runs past the end of the file")

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:  # a tensor_data view is still alive: unmapped when it goes
                pass
            self._map = None
        if getattr(self, "_file", None) is not None:
            self._file.close()
            self._file = None

    def __enter__(self) -> "Gguf":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    @property
    def tensor_count(self) -> int:
        return len(self.tensors)

    @property
    def kv_count(self) -> int:
        return len(self.kvs)

    # ---- metadata --------------------------------------------------------------
    def find(self, key: str) -> int:
        """Index of a key, or -1."""
        return self._keys.get(key, -1)

    def key_name(self, i: int) -> str:
        return self.kvs[i].key

    def _scalar_at(self, kind: int, at: int):
        return struct.unpack_from(_SCALAR[kind], self._map, at)[0]

    def uint(self, i: int) -> int:
        """An integer (or bool) value; the reference's `uint` widening."""
        kv = self.kvs[i]
        if kv.kind not in _INTS:
            raise GgufError(f"gguf key {kv.key} is not an integer")
        return int(self._scalar_at(kv.kind, kv.payload))

    def string(self, i: int) -> str:
        kv = self.kvs[i]
        if kv.kind != GGUF_STRING:
            raise GgufError(f"gguf key {kv.key} is not a string")
        cur = _Cursor(self._map, self.length)
        cur.at = kv.payload
        return cur.string()

    def flt(self, i: int) -> float:
        kv = self.kvs[i]
        if kv.kind not in (GGUF_FLOAT32, GGUF_FLOAT64):
            raise GgufError(f"gguf key {kv.key} is not a float")
        return float(self._scalar_at(kv.kind, kv.payload))

    def array(self, i: int) -> list:
        """Every element of an array key (decoded on request)."""
        kv = self.kvs[i]
        if kv.kind != GGUF_ARRAY:
            raise GgufError(f"gguf key {kv.key} is not an array")
        cur = _Cursor(self._map, self.length)
        cur.at = kv.payload
        if kv.element == GGUF_STRING:
            return [cur.string() for _ in range(kv.count)]
        return [cur.scalar(kv.element) for _ in range(kv.count)]

    def value(self, key: str):
        """A key's value as a Python object (int, float, bool, str, list), or None."""
        i = self.find(key)
        if i < 0:
            return None
        kv = self.kvs[i]
        if kv.kind == GGUF_ARRAY:
            return self.array(i)
        if kv.kind == GGUF_STRING:
            return self.string(i)
        if kv.kind == GGUF_BOOL:
            return self.uint(i) != 0
        if kv.kind in (GGUF_FLOAT32, GGUF_FLOAT64):
            return self.flt(i)
        return self.uint(i)

    def string_or(self, key: str, fallback: str) -> str:
        i = self.find(key)
        try:
            return self.string(i) if i >= 0 else fallback
        except GgufError:
            return fallback

    def uint_or(self, key: str, fallback: int) -> int:
        i = self.find(key)
        try:
            return self.uint(i) if i >= 0 else fallback
        except GgufError:
            return fallback

    def float_or(self, key: str, fallback: float) -> float:
        """A float, or an integer where a float was expected (writers emit
        rope.freq_base as 10000), or the fallback."""
        i = self.find(key)
        if i < 0:
            return fallback
        for get in (self.flt, self.uint):
            try:
                return float(get(i))
            except GgufError:
                pass
        return fallback

    def bool_or(self, key: str, fallback: bool) -> bool:
        i = self.find(key)
        try:
            return self.uint(i) != 0 if i >= 0 else fallback
        except GgufError:
            return fallback

    def has(self, key: str) -> bool:
        return self.find(key) >= 0

    def array_count(self, key: str) -> int:
        i = self.find(key)
        if i < 0 or self.kvs[i].kind != GGUF_ARRAY:
            return 0
        return self.kvs[i].count

    # ---- tensors -------------------------------------------------------------------
    def tensor_index(self, name: str) -> int:
        return self._names.get(name, -1)

    def tensor_prefixed(self, prefix: str) -> bool:
        return any(t.name.startswith(prefix) for t in self.tensors)

    def tensor(self, name: str) -> TensorInfo:
        i = self.tensor_index(name)
        if i < 0:
            raise GgufError(f"gguf has no tensor {name}")
        return self.tensors[i]

    def tensor_data(self, t: TensorInfo) -> memoryview:
        """The tensor's bytes in the mapping (no copy), bounds checked."""
        start = self.data_start + t.offset
        n = t.nbytes()
        if t.offset % self.alignment:
            raise GgufError(f"tensor {t.name}: offset {t.offset} breaks the file's {self.alignment}-byte alignment")
        if start + n > self.length:
            raise GgufError(f"tensor {t.name}: {n} bytes at {start} run past the end of the file")
        return memoryview(self._map)[start:start + n]

    # ---- model facts ---------------------------------------------------------------
    def architecture(self) -> str:
        return self.string_or("general.architecture", "unknown")

    def context_length(self) -> int:
        return self.uint_or(self.architecture() + ".context_length", 0)

    def block_count(self) -> int:
        return self.uint_or(self.architecture() + ".block_count", 0)

    def embedding_length(self) -> int:
        return self.uint_or(self.architecture() + ".embedding_length", 0)
