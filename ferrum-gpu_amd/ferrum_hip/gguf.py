"""Python mirror of ferrum_gguf's reader (ferrum_gguf/src/io/reader.rs) over libferrum_hip's GGUF
v3 parser (the fh_gguf_* entry points of include/ferrum_hip.h).

`Gguf.parse`, `Gguf.parse_prefix`, `get`, `uint`, `float`, `string`, `tensor`, `tensor_bytes`,
`data_offset` keep the reference's names, argument meanings and error texts (GgufError messages
start with "gguf: "). Parsing, bounds checks and tensor directory live in the native library;
this module only converts what it hands out into Python values. Tensors go to the device without
a host decode: `upload_qweight` keeps a Q8_0/Q4_0 tensor's stored bytes as a resident weight,
`tensor_f32` decodes on the device.
"""
from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import Gpu, GpuBuf, QWeight, lib

MAGIC = 0x46554747
DEFAULT_ALIGNMENT = 32

# ggml tensor type ids (ferrum_gguf/src/lib.rs:24-55)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1 = 0, 1, 2, 3
GGML_Q5_0, GGML_Q5_1, GGML_Q8_0, GGML_Q8_1 = 6, 7, 8, 9
GGML_Q2_K, GGML_Q3_K, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 10, 11, 12, 13, 14
GGML_I16, GGML_I32, GGML_MXFP4 = 25, 26, 39

# metadata value tags (reader.rs:125-157)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "?", U64: "Q",
        I64: "q", F64: "d"}
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32,
       F32: np.float32, BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}


class GgufError(ValueError):
    """ferrum_gguf::GgufError; str() is the reference's Display text ("gguf: ...")."""


def _check(status: int) -> None:
    if status != 0:
        raise GgufError(lib().fh_last_error().decode("utf-8", "replace"))


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_void_p), ("name_len", ctypes.c_size_t), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.c_uint64 * 4), ("ggml_type", ctypes.c_uint32), ("offset", ctypes.c_uint64),
                ("elements", ctypes.c_uint64), ("nbytes", ctypes.c_uint64)]


@dataclass(frozen=True)
class Value:
    """reader.rs:26-54: a metadata value and its tag. Arrays hold a list of Values."""
    tag: int
    v: object

    def __eq__(self, other):  # derive(PartialEq): same tag and equal payload (NaN != NaN)
        return isinstance(other, Value) and self.tag == other.tag and self.v == other.v


@dataclass(frozen=True)
class TensorInfo:
    """reader.rs:58-80: one tensor's directory entry (dims innermost first)."""
    name: str
    dims: tuple
    ggml_type: int
    offset: int
    n_elements: int
    nbytes: int

    def elements(self) -> int:
        return self.n_elements


def nbytes(ggml_type: int, n: int) -> int:
    """quant::nbytes (ferrum_gguf/src/codec/quant.rs:17-47)."""
    out = ctypes.c_uint64()
    _check(lib().fh_ggml_nbytes(ggml_type, n, ctypes.byref(out)))
    return out.value


class Gguf:
    """ferrum_gguf::Gguf (reader.rs:82-322): a parsed file that keeps its bytes."""

    def __init__(self, handle: ctypes.c_void_p):
        self._h = handle
        self._kv: Optional[list] = None
        self._tensors: Optional[list] = None

    # ---- construction ----
    @classmethod
    def parse(cls, data: bytes) -> "Gguf":
        """Gguf::parse (reader.rs:165-170)."""
        buf = bytes(data)
        h = ctypes.c_void_p()
        _check(lib().fh_gguf_parse(buf, len(buf), ctypes.byref(h)))
        return cls(h)

    @classmethod
    def parse_prefix(cls, data: bytes, total: int) -> "Gguf":
        """Gguf::parse_prefix (reader.rs:172-247): header of a longer file."""
        buf = bytes(data)
        h = ctypes.c_void_p()
        _check(lib().fh_gguf_parse_prefix(buf, len(buf), total, ctypes.byref(h)))
        return cls(h)

    @classmethod
    def open(cls, path: str) -> "Gguf":
        """Parse a file through a read-only mapping (nothing is read until used)."""
        h = ctypes.c_void_p()
        _check(lib().fh_gguf_open(path.encode(), ctypes.byref(h)))
        return cls(h)

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            lib().fh_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __repr__(self) -> str:
        buf = ctypes.create_string_buffer(128)
        lib().fh_gguf_describe(self._h, buf, 128)
        return buf.value.decode()

    # ---- metadata ----
    def _value(self, i: int) -> Value:
        L = lib()
        ty, data, n = ctypes.c_uint32(), ctypes.c_void_p(), ctypes.c_size_t()
        _check(L.fh_gguf_kv_value(self._h, i, ctypes.byref(ty), ctypes.byref(data), ctypes.byref(n)))
        raw = ctypes.string_at(data.value, n.value) if n.value else b""
        t = ty.value
        if t == STR:
            return Value(STR, raw.decode("utf-8"))
        if t != ARR:
            return Value(t, struct.unpack("<" + _FMT[t], raw)[0])
        et, cnt = ctypes.c_uint32(), ctypes.c_uint64()
        _check(L.fh_gguf_kv_array(self._h, i, ctypes.byref(et), ctypes.byref(cnt)))
        if et.value == STR:
            s, sl, out = ctypes.c_void_p(), ctypes.c_size_t(), []
            for j in range(cnt.value):
                _check(L.fh_gguf_kv_array_string(self._h, i, j, ctypes.byref(s), ctypes.byref(sl)))
                out.append(Value(STR, ctypes.string_at(s.value, sl.value).decode("utf-8") if sl.value else ""))
            return Value(ARR, out)
        if cnt.value == 0:
            return Value(ARR, [])
        vals = np.frombuffer(raw, dtype=np.dtype(_NP[et.value]).newbyteorder("<"), count=cnt.value)
        conv = bool if et.value == BOOL else (float if et.value in (F32, F64) else int)
        return Value(ARR, [Value(et.value, conv(v)) for v in vals])

    @property
    def kv(self) -> list:
        """Metadata in file order: [(key, Value)]."""
        if self._kv is None:
            L, out = lib(), []
            k, kl = ctypes.c_void_p(), ctypes.c_size_t()
            for i in range(L.fh_gguf_kv_count(self._h)):
                _check(L.fh_gguf_kv_key(self._h, i, ctypes.byref(k), ctypes.byref(kl)))
                out.append((ctypes.string_at(k.value, kl.value).decode("utf-8") if kl.value else "",
                            self._value(i)))
            self._kv = out
        return self._kv

    def get(self, key: str) -> Optional[Value]:
        """Gguf::get (reader.rs:249-252): the first entry with this key."""
        i = ctypes.c_size_t()
        if lib().fh_gguf_find_key(self._h, key.encode(), ctypes.byref(i)) != 0:
            return None
        return self._value(i.value)

    def uint(self, key: str) -> int:
        """reader.rs:254-268: any non-negative integer width."""
        out = ctypes.c_uint64()
        _check(lib().fh_gguf_get_uint(self._h, key.encode(), ctypes.byref(out)))
        return out.value

    def float(self, key: str) -> float:
        """reader.rs:270-277: an f32 value."""
        out = ctypes.c_float()
        _check(lib().fh_gguf_get_float(self._h, key.encode(), ctypes.byref(out)))
        return out.value

    def string(self, key: str) -> str:
        """reader.rs:279-286."""
        s, n = ctypes.c_void_p(), ctypes.c_size_t()
        _check(lib().fh_gguf_get_string(self._h, key.encode(), ctypes.byref(s), ctypes.byref(n)))
        return ctypes.string_at(s.value, n.value).decode("utf-8") if n.value else ""

    # ---- tensors ----
    @property
    def tensors(self) -> list:
        """The tensor directory in file order."""
        if self._tensors is None:
            L, out, t = lib(), [], _Tensor()
            for i in range(L.fh_gguf_tensor_count(self._h)):
                _check(L.fh_gguf_tensor_info(self._h, i, ctypes.byref(t)))
                out.append(TensorInfo(ctypes.string_at(t.name, t.name_len).decode("utf-8") if t.name_len else "",
                                      tuple(t.dims[:t.n_dims]), t.ggml_type, t.offset, t.elements, t.nbytes))
            self._tensors = out
        return self._tensors

    def tensor(self, name: str) -> Optional[TensorInfo]:
        """Gguf::tensor (reader.rs:289-291)."""
        i = ctypes.c_size_t()
        if lib().fh_gguf_find_tensor(self._h, name.encode(), ctypes.byref(i)) != 0:
            return None
        return self.tensors[i.value]

    def tensor_bytes(self, name: str) -> bytes:
        """Gguf::tensor_bytes (reader.rs:294-305): the stored bytes, undecoded."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _check(lib().fh_gguf_tensor_bytes(self._h, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value) if n.value else b""

    def data_offset(self) -> int:
        """reader.rs:308-310."""
        return lib().fh_gguf_data_offset(self._h)

    # ---- device ----
    def tensor_f32(self, gpu: Gpu, name: str) -> GpuBuf:
        """Gguf::tensor_f32 (reader.rs:313-318) decoded on the device into a new f32 buffer."""
        h = ctypes.c_void_p()
        _check(lib().fh_gguf_upload_f32(gpu.handle, self._h, name.encode(), ctypes.byref(h)))
        return GpuBuf(gpu, h)

    def upload_qweight(self, gpu: Gpu, name: str) -> QWeight:
        """A Q8_0/Q4_0 tensor of dims [k, n] as a resident weight, straight from its bytes."""
        h = ctypes.c_void_p()
        _check(lib().fh_gguf_upload_qweight(gpu.handle, self._h, name.encode(), ctypes.byref(h)))
        return QWeight(gpu, h)


class GgufBuilder:
    """ferrum_gguf's GgufBuilder (ferrum_gguf/src/io/writer.rs:7-115): metadata and tensors in,
    one GGUF v3 file out (header, metadata, tensor directory, padding to the alignment after the
    header and after every tensor). Values are `Value(tag, v)`; arrays hold Values."""

    def __init__(self):
        self._kv: list = []
        self._tensors: list = []

    def meta(self, key: str, val: Value) -> None:
        self._kv.append((key, val))

    def tensor_f32(self, name: str, dims, data) -> None:
        self.tensor_raw(name, dims, GGML_F32, np.ascontiguousarray(data, dtype="<f4").tobytes())

    def tensor_raw(self, name: str, dims, ggml_type: int, data) -> None:
        self._tensors.append((name, [int(d) for d in dims], int(ggml_type), bytes(data)))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    @classmethod
    def _value(cls, val: Value) -> bytes:
        if val.tag == STR:
            return cls._str(val.v)
        if val.tag == ARR:
            head = struct.pack("<IQ", val.v[0].tag if val.v else U32, len(val.v))
            return head + b"".join(cls._value(e) for e in val.v)
        return struct.pack("<" + _FMT[val.tag], val.v)

    def into_bytes(self) -> bytes:
        parts = [struct.pack("<IIQQ", MAGIC, 3, len(self._tensors), len(self._kv))]
        alignment = DEFAULT_ALIGNMENT
        for key, val in self._kv:
            parts += [self._str(key), struct.pack("<I", val.tag), self._value(val)]
            if key == "general.alignment" and val.tag == U32:
                alignment = max(int(val.v), 1)
        data, offset = [], 0
        for name, dims, ty, raw in self._tensors:
            parts += [self._str(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                      struct.pack("<IQ", ty, offset)]
            pad = -len(raw) % alignment
            data += [raw, bytes(pad)]
            offset += len(raw) + pad
        head = b"".join(parts)
        return head + bytes(-len(head) % alignment) + b"".join(data)
