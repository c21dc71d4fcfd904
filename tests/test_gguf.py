"""GGUF v3 reader through the C ABI (CPU only: parsing touches no device).

The cases restate the reference reader's own tests (ferrum_gguf/src/io/reader.rs:324-610) on
files built by oracle/gguf.py's restatement of the reference writer, and read the reference's
fixture model.gguf (tests/golden/model.gguf, a GPT-2 written by another encoder) with both the
native parser and oracle/gguf.py's independent reader.
"""
import hashlib
import os
import struct

import numpy as np
import pytest

from ferrum_hip import gguf as G
from ferrum_hip.gguf import Gguf, GgufError, Value
from oracle import gguf as og

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODEL = os.path.join(GOLDEN, "model.gguf")


def sample() -> bytes:
    """reader.rs:330-344"""
    b = og.GgufBuilder()
    b.meta("general.architecture", Value(G.STR, "gpt2"))
    b.meta("gpt2.block_count", Value(G.U32, 2))
    b.meta("x.eps", Value(G.F32, np.float32(1e-5).item()))
    b.meta("x.list", Value(G.ARR, [Value(G.STR, "a"), Value(G.STR, "bc")]))
    b.tensor_f32("w", [3, 2], [1.0, 2.0, 3.0, 4.0, 5.0, 6.0])
    b.tensor_f32("b", [2], [0.5, -0.5])
    return b.into_bytes()


def err(f) -> str:
    with pytest.raises(GgufError) as e:
        f()
    return str(e.value)


def f32s(raw: bytes) -> list:
    return np.frombuffer(raw, "<f4").tolist()


def test_a_header_only_parse_checks_extents_against_the_file_length():
    """reader.rs:346-365"""
    b = og.GgufBuilder()
    b.meta("general.architecture", Value(G.STR, "x"))
    b.tensor_f32("w", [100], [1.0] * 100)
    data = b.into_bytes()
    head = data[:len(data) - 400]
    g = Gguf.parse_prefix(head, len(data))
    assert g.tensor("w").dims == (100,)
    assert g.data_offset() <= len(head) and g.data_offset() % 32 == 0
    assert "header-only" in err(lambda: g.tensor_bytes("w"))
    assert "extends past" in err(lambda: Gguf.parse_prefix(head, g.data_offset() + 399))
    assert "longer than the file" in err(lambda: Gguf.parse_prefix(head, len(head) - 1))


def test_raw_bytes_are_the_stored_encoding():
    """reader.rs:392-407"""
    g = Gguf.parse(sample())
    assert g.tensor_bytes("b") == struct.pack("<ff", 0.5, -0.5)
    assert len(g.tensor_bytes("w")) == 24
    assert "missing tensor" in err(lambda: g.tensor_bytes("nope"))


def test_round_trips_metadata_and_tensors():
    """reader.rs:409-431 (tensor_f32 of F32 tensors is their stored bytes; the device decode is
    covered by the GPU tests)."""
    g = Gguf.parse(sample())
    assert g.string("general.architecture") == "gpt2"
    assert g.uint("gpt2.block_count") == 2
    assert g.float("x.eps") == np.float32(1e-5)
    assert g.get("x.list") == Value(G.ARR, [Value(G.STR, "a"), Value(G.STR, "bc")])
    assert g.tensor("w").dims == (3, 2)
    assert g.tensor("w").ggml_type == G.GGML_F32
    assert f32s(g.tensor_bytes("w")) == [1.0, 2.0, 3.0, 4.0, 5.0, 6.0]
    assert f32s(g.tensor_bytes("b")) == [0.5, -0.5]
    assert [k for k, _ in g.kv] == ["general.architecture", "gpt2.block_count", "x.eps", "x.list"]
    assert [t.name for t in g.tensors] == ["w", "b"]
    assert g.tensor("w").elements() == 6 and g.tensor("w").nbytes == 24


def test_typed_getters_report_what_is_wrong():
    """reader.rs:433-459"""
    g = Gguf.parse(sample())
    assert "missing key" in err(lambda: g.uint("missing"))
    assert "non-negative integer" in err(lambda: g.uint("general.architecture"))
    assert "is not an f32" in err(lambda: g.float("gpt2.block_count"))
    assert "is not a string" in err(lambda: g.string("gpt2.block_count"))
    assert "missing key" in err(lambda: g.float("missing"))
    assert "missing key" in err(lambda: g.string("missing"))
    assert g.tensor("nope") is None
    assert g.get("nope") is None


def test_rejects_bad_headers():
    """reader.rs:461-476"""
    good = sample()
    bad_magic = b"X" + good[1:]
    assert "magic" in err(lambda: Gguf.parse(bad_magic))
    v2 = good[:4] + b"\x02" + good[5:]
    assert "version" in err(lambda: Gguf.parse(v2))
    err(lambda: Gguf.parse(b""))
    err(lambda: Gguf.parse(good[:10]))


def test_every_truncation_is_an_error_not_a_panic():
    """reader.rs:478-486: the last tensor holds 8 real bytes and 24 of alignment padding, so
    cutting only padding leaves a valid file."""
    good = sample()
    for cut in range(len(good) - 24):
        with pytest.raises(GgufError):
            Gguf.parse(good[:cut])
    Gguf.parse(good[:len(good) - 24])


def test_hostile_counts_do_not_allocate_or_panic():
    """reader.rs:488-500"""
    s = sample()
    huge_kv = s[:16] + struct.pack("<Q", 2**64 - 1) + s[24:]
    assert "exceed" in err(lambda: Gguf.parse(huge_kv))
    huge_tensors = s[:8] + struct.pack("<Q", 2**64 - 1) + s[16:]
    err(lambda: Gguf.parse(huge_tensors))


def test_hostile_array_and_tensor_sizes_are_rejected():
    """reader.rs:502-527"""
    b = og.GgufBuilder()
    b.meta("a", Value(G.ARR, [Value(G.U8, 1)]))
    data = bytearray(b.into_bytes())
    at = 24 + 9 + 4 + 4  # header, key, value tag, element tag
    data[at:at + 8] = struct.pack("<Q", 1 << 60)
    assert "array length" in err(lambda: Gguf.parse(bytes(data)))

    t = og.GgufBuilder()
    t.tensor_raw("w", [1 << 40, 1 << 40], G.GGML_F32, bytes(4))
    assert "overflows" in err(lambda: Gguf.parse(t.into_bytes()))
    t = og.GgufBuilder()
    t.tensor_raw("w", [1000], G.GGML_F32, bytes(4))
    assert "past the end" in err(lambda: Gguf.parse(t.into_bytes()))


def test_duplicate_names_and_bad_dims_are_rejected():
    """reader.rs:529-545"""
    b = og.GgufBuilder()
    b.tensor_f32("w", [1], [1.0])
    b.tensor_f32("w", [1], [2.0])
    assert "duplicate" in err(lambda: Gguf.parse(b.into_bytes()))
    z = og.GgufBuilder()
    z.tensor_raw("w", [], G.GGML_F32, b"")
    assert "dims" in err(lambda: Gguf.parse(z.into_bytes()))
    five = og.GgufBuilder()
    five.tensor_raw("w", [1, 1, 1, 1, 1], G.GGML_F32, bytes(4))
    assert "has 5 dims" in err(lambda: Gguf.parse(five.into_bytes()))


def test_custom_alignment_is_honoured():
    """reader.rs:547-557"""
    b = og.GgufBuilder()
    b.meta("general.alignment", Value(G.U32, 64))
    b.tensor_f32("w", [2], [7.0, 8.0])
    g = Gguf.parse(b.into_bytes())
    assert f32s(g.tensor_bytes("w")) == [7.0, 8.0]
    assert g.data_offset() % 64 == 0 and g.data_offset() > 32
    bad = og.GgufBuilder()
    bad.meta("general.alignment", Value(G.U32, 0))
    assert "alignment" in err(lambda: Gguf.parse(bad.into_bytes()))
    wrong_type = og.GgufBuilder()
    wrong_type.meta("general.alignment", Value(G.U64, 64))
    assert "alignment" in err(lambda: Gguf.parse(wrong_type.into_bytes()))


def test_debug_output_summarises_without_dumping_bytes():
    """reader.rs:559-565"""
    s = repr(Gguf.parse(sample()))
    assert "4 keys" in s and "2 tensors" in s, s
    assert len(s) < 100


def test_nested_arrays_and_unknown_value_types_are_rejected():
    """reader.rs:567-585"""
    b = og.GgufBuilder()
    b.meta("a", Value(G.ARR, [Value(G.ARR, [Value(G.U8, 1)])]))
    assert "nested arrays" in err(lambda: Gguf.parse(b.into_bytes()))
    b = og.GgufBuilder()
    b.meta("a", Value(G.U8, 1))
    data = bytearray(b.into_bytes())
    data[33:37] = struct.pack("<I", 99)  # the value tag follows the header and the key
    assert "unknown metadata value type 99" in err(lambda: Gguf.parse(bytes(data)))


def test_uint_accepts_every_integer_width_and_rejects_negatives():
    """reader.rs:587-605"""
    b = og.GgufBuilder()
    for k, v in [("u8", Value(G.U8, 7)), ("u16", Value(G.U16, 300)), ("u32", Value(G.U32, 70_000)),
                 ("u64", Value(G.U64, 5_000_000_000)), ("i32", Value(G.I32, 12)), ("i64", Value(G.I64, 34)),
                 ("neg32", Value(G.I32, -1)), ("neg64", Value(G.I64, -1)), ("i8", Value(G.I8, 3)),
                 ("i16", Value(G.I16, 3))]:
        b.meta(k, v)
    g = Gguf.parse(b.into_bytes())
    for k, want in [("u8", 7), ("u16", 300), ("u32", 70_000), ("u64", 5_000_000_000), ("i32", 12), ("i64", 34)]:
        assert g.uint(k) == want, k
    for k in ("neg32", "neg64", "i8", "i16"):  # i8 and i16 are not among uint's widths
        assert "non-negative integer" in err(lambda: g.uint(k))


def test_element_count_overflow_is_an_error():
    """reader.rs:607-616 (the parse computes the element count of every tensor)."""
    t = og.GgufBuilder()
    t.tensor_raw("x", [2**64 - 1, 2], G.GGML_F32, b"")
    assert "element count overflows" in err(lambda: Gguf.parse(t.into_bytes()))


def test_every_value_type_round_trips():
    vals = [("u8", Value(G.U8, 255)), ("i8", Value(G.I8, -128)), ("u16", Value(G.U16, 65535)),
            ("i16", Value(G.I16, -32768)), ("u32", Value(G.U32, 2**32 - 1)), ("i32", Value(G.I32, -2**31)),
            ("f32", Value(G.F32, -1.5)), ("t", Value(G.BOOL, True)), ("f", Value(G.BOOL, False)),
            ("s", Value(G.STR, "héllo ✓")), ("empty", Value(G.STR, "")),
            ("u64", Value(G.U64, 2**64 - 1)), ("i64", Value(G.I64, -2**63)), ("f64", Value(G.F64, 1e300)),
            ("ai", Value(G.ARR, [Value(G.I32, -1), Value(G.I32, 7)])),
            ("af", Value(G.ARR, [Value(G.F32, 0.25), Value(G.F32, -2.0)])),
            ("none", Value(G.ARR, []))]
    b = og.GgufBuilder()
    for k, v in vals:
        b.meta(k, v)
    g = Gguf.parse(b.into_bytes())
    assert g.kv == vals
    assert g.string("s") == "héllo ✓" and g.string("empty") == ""


def test_invalid_utf8_is_rejected():
    def one_key(key: bytes) -> bytes:  # a file whose only entry is key = u8 1, padded to 32
        d = struct.pack("<IIQQ", og.MAGIC, 3, 0, 1) + struct.pack("<Q", len(key)) + key + struct.pack("<IB", 0, 1)
        return d + bytes(-len(d) % 32)

    for bad in (b"\xff", b"\xc0\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80", b"a\xe2\x82"):
        assert "UTF-8" in err(lambda: Gguf.parse(one_key(bad))), bad
    assert Gguf.parse(one_key("ŀ€𐍈".encode())).uint("ŀ€𐍈") == 1


def test_nbytes_matches_the_reference_table():
    """quant.rs:17-47 and blocks.rs:34-48."""
    per = {G.GGML_Q4_0: (18, 32), G.GGML_Q4_1: (20, 32), G.GGML_Q5_0: (22, 32), G.GGML_Q5_1: (24, 32),
           G.GGML_Q8_0: (34, 32), G.GGML_Q8_1: (36, 32), G.GGML_MXFP4: (17, 32), G.GGML_Q2_K: (84, 256),
           G.GGML_Q3_K: (110, 256), G.GGML_Q4_K: (144, 256), G.GGML_Q5_K: (176, 256), G.GGML_Q6_K: (210, 256)}
    for ty, (b, e) in per.items():
        assert G.nbytes(ty, 3 * e) == 3 * b
        assert "not a multiple of the block size" in err(lambda: G.nbytes(ty, e + 1))
    assert G.nbytes(G.GGML_F32, 5) == 20 and G.nbytes(G.GGML_I32, 5) == 20
    assert G.nbytes(G.GGML_F16, 5) == 10 and G.nbytes(G.GGML_I16, 5) == 10
    assert "unsupported ggml tensor type 4" in err(lambda: G.nbytes(4, 32))
    assert "overflows" in err(lambda: G.nbytes(G.GGML_F32, 2**63))


def test_reference_fixture_parses_like_the_independent_reader():
    """tests/golden/model.gguf (the reference's fixtures/bpe/model.gguf): every key, value, tensor
    entry and tensor byte agrees between the native parser and oracle/gguf.py's reader."""
    data = open(MODEL, "rb").read()
    assert hashlib.sha256(data).hexdigest() == "623af38b770ace7617725682bf84c0bb212d62ab78be1784e6b9775928af36ec"
    kv, tensors, base = og.parse(data)
    for g in (Gguf.parse(data), Gguf.open(MODEL)):
        assert g.data_offset() == base
        assert [(k, v.tag) for k, v in g.kv] == [(k, v.tag) for k, v in kv]
        for (k, got), (_, want) in zip(g.kv, kv):
            if want.tag == G.ARR:
                assert [(e.tag, e.v) for e in got.v] == [(e.tag, e.v) for e in want.v], k
            else:
                assert (got.tag, got.v) == (want.tag, want.v), k
        assert len(g.tensors) == len(tensors) == 29
        for t, w in zip(g.tensors, tensors):
            assert (t.name, list(t.dims), t.ggml_type, t.offset) == (w["name"], w["dims"], w["type"], w["offset"])
            n = int(np.prod(w["dims"]))
            nb = n * 4 if w["type"] == G.GGML_F32 else n // 32 * 34
            assert g.tensor_bytes(t.name) == data[base + w["offset"]: base + w["offset"] + nb]
        assert g.uint("gpt2.block_count") == 2 and g.uint("gpt2.embedding_length") == 64
        assert g.float("gpt2.attention.layer_norm_epsilon") == np.float32(1e-5)
        assert g.string("general.architecture") == "gpt2"
        assert len(g.get("tokenizer.ggml.tokens").v) == 320


def test_open_reports_a_missing_file():
    assert "cannot open" in err(lambda: Gguf.open(os.path.join(GOLDEN, "no_such_file.gguf")))


def test_hostile_mutations_of_the_fixture_never_crash():
    """Random byte flips and truncations of a real file: every outcome is a clean parse or a
    GgufError."""
    data = open(MODEL, "rb").read()
    head = data[:10000]  # header (9920 bytes) plus the start of the data
    rng = np.random.default_rng(5)
    for _ in range(3000):
        m = bytearray(head)
        for at in rng.integers(0, len(m), rng.integers(1, 4)):
            m[at] = int(rng.integers(0, 256))
        cut = int(rng.integers(0, len(m) + 1))
        try:
            Gguf.parse_prefix(bytes(m[:cut]), len(data))
        except GgufError:
            pass
