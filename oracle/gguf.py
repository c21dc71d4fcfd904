"""GGUF v3 restatement for tests (test infrastructure: only tests/, smoke() and bench.py's CPU
baseline use this package; the product path never does).

* ``GgufBuilder`` restates ferrum_gguf's writer (ferrum_gguf/src/io/writer.rs:58-115): header,
  metadata, tensor directory, alignment padding after the header and after every tensor. The
  reader tests build their hostile inputs from it exactly as the reference's tests do.
* ``parse`` restates the reader (ferrum_gguf/src/io/reader.rs:172-247) in plain Python, without
  the hostile-input checks; it is the independent second reading of well-formed files the native
  parser is compared with.

Values are ``V(tag, v)`` pairs (any object with ``tag`` and ``v`` attributes works); arrays hold a
list of such pairs. Tags: U8 0, I8 1, U16 2, I16 3, U32 4, I32 5, F32 6, BOOL 7, STR 8, ARR 9,
U64 10, I64 11, F64 12 (reader.rs:125-157).
"""
from __future__ import annotations

import struct
from collections import namedtuple

import numpy as np

MAGIC = 0x46554747
DEFAULT_ALIGNMENT = 32
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0 = 0, 1, 2, 8

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "?", U64: "Q",
        I64: "q", F64: "d"}

V = namedtuple("V", "tag v")


def _put_str(out: bytearray, s: str) -> None:
    b = s.encode("utf-8")
    out += struct.pack("<Q", len(b)) + b


def _put_value(out: bytearray, val) -> None:
    """writer.rs:37-56. An array's element tag is its first element's (U32 when empty)."""
    tag, v = val.tag, val.v
    if tag == STR:
        _put_str(out, v)
    elif tag == ARR:
        out += struct.pack("<IQ", v[0].tag if v else U32, len(v))
        for e in v:
            _put_value(out, e)
    elif tag == F32:
        out += struct.pack("<f", v)
    else:
        out += struct.pack("<" + _FMT[tag], v)


class GgufBuilder:
    """writer.rs:7-115: accumulate metadata and tensors, then serialise one GGUF v3 file."""

    def __init__(self):
        self.kv = []
        self.tensors = []

    def meta(self, key: str, val) -> None:
        self.kv.append((key, val))

    def tensor_f32(self, name: str, dims, data) -> None:
        self.tensor_raw(name, dims, GGML_F32, np.asarray(data, dtype="<f4").tobytes())

    def tensor_raw(self, name: str, dims, ggml_type: int, data: bytes) -> None:
        self.tensors.append((name, [int(d) for d in dims], ggml_type, bytes(data)))

    def into_bytes(self) -> bytes:
        head = bytearray(struct.pack("<IIQQ", MAGIC, 3, len(self.tensors), len(self.kv)))
        alignment = DEFAULT_ALIGNMENT
        for key, val in self.kv:
            _put_str(head, key)
            head += struct.pack("<I", val.tag)
            _put_value(head, val)
            if key == "general.alignment" and val.tag == U32:
                alignment = max(int(val.v), 1)
        data, offset = bytearray(), 0
        for name, dims, ty, raw in self.tensors:
            _put_str(head, name)
            head += struct.pack("<I", len(dims))
            for d in dims:
                head += struct.pack("<Q", d)
            head += struct.pack("<IQ", ty, offset)
            padded = -(-len(raw) // alignment) * alignment
            data += raw + bytes(padded - len(raw))
            offset += padded
        head += bytes(-(-len(head) // alignment) * alignment - len(head))
        return bytes(head + data)


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.o = data, 0

    def take(self, fmt: str):
        v = struct.unpack_from("<" + fmt, self.d, self.o)
        self.o += struct.calcsize("<" + fmt)
        return v[0] if len(v) == 1 else v

    def string(self) -> str:
        n = self.take("Q")
        s = self.d[self.o:self.o + n].decode("utf-8")
        self.o += n
        return s

    def value(self, tag: int) -> V:
        if tag == STR:
            return V(STR, self.string())
        if tag == ARR:
            et, cnt = self.take("I"), self.take("Q")
            return V(ARR, [self.value(et) for _ in range(cnt)])
        return V(tag, self.take(_FMT[tag]))


def parse(data: bytes):
    """reader.rs:172-247 for well-formed files: (kv list, tensor list, data start). Tensors are
    dicts with name, dims, type, offset."""
    r = _Reader(data)
    magic, version = r.take("I"), r.take("I")
    if magic != MAGIC or version != 3:
        raise ValueError("not a GGUF v3 file")
    n_tensors, n_kv = r.take("Q"), r.take("Q")
    kv = []
    for _ in range(n_kv):
        key = r.string()
        kv.append((key, r.value(r.take("I"))))
    tensors = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.take("I")
        dims = [r.take("Q") for _ in range(nd)]
        ty, off = r.take("I"), r.take("Q")
        tensors.append({"name": name, "dims": dims, "type": ty, "offset": off})
    align = next((int(v.v) for k, v in kv if k == "general.alignment"), DEFAULT_ALIGNMENT)
    return kv, tensors, -(-r.o // align) * align
