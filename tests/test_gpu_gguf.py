"""GPU tests of the GGUF container's device uploads: tensors go from the file (a memory mapping)
to resident weights and f32 buffers with no host decode, bit-exact against the oracle.

Pins: the reference's fixture model.gguf (GPT-2 written by another encoder); the oracle's codec
(itself pinned by the reference's known answers and this fixture); the exhaustive binary16 table
(every one of the 65,536 bit patterns, the oracle's f16_to_f32 being checked against numpy's
IEEE conversion in tests/test_oracle.py)."""
import os

import numpy as np
import pytest

from oracle import gguf as og

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODEL = os.path.join(GOLDEN, "model.gguf")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def fh():
    import ferrum_hip

    return ferrum_hip


@pytest.fixture(scope="module")
def G():
    from ferrum_hip import gguf

    return gguf


@pytest.fixture(scope="module")
def g(fh):
    gpu = fh.Gpu.open_for_test()
    if gpu is None:
        pytest.skip("no gfx950 device")
    yield gpu
    gpu.close()


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fixture_tensors_upload_without_a_round_trip(fh, G, g, orc):
    """Every Q8_0 matrix of model.gguf becomes a resident weight straight from the mapped file:
    the resident bytes are the stored bytes, which are also what the reference's load-time
    re-encode (decode then quantise_matrix) produces, and the product matches the CPU path."""
    gf = G.Gguf.open(MODEL)
    q8 = [t for t in gf.tensors if t.ggml_type == G.GGML_Q8_0]
    assert len(q8) == 10
    for t in q8:
        say("gguf upload", t.name, t.dims)
        k, n = t.dims[0], int(np.prod(t.dims[1:]))
        raw = np.frombuffer(gf.tensor_bytes(t.name), np.uint8)
        qw = gf.upload_qweight(g, t.name)
        assert (qw.kind(), qw.k(), qw.n()) == (fh.QKind.Q8_0, k, n)
        assert np.array_equal(qw.read_gguf(), raw)
        w_in_out = orc.dequantised_in_out(orc.Q8_0, raw, k, n)
        assert np.array_equal(orc.quantise_matrix(orc.Q8_0, w_in_out, k, n), raw), t.name
        x = orc.rand_vec(k, 11)
        y = g.zeros(n)
        fh.linear_q(g, g.upload(x), qw, y, 1)
        want = orc.matmul(x, w_in_out, 1, k, n)
        assert orc.max_rel_err(g.read(y), want) <= 1e-5, t.name


def test_fixture_tensor_f32_on_the_device(G, g, orc):
    """Gguf::tensor_f32 for every tensor of model.gguf: F32 tensors are their stored values,
    Q8_0 tensors decode exactly as the oracle's decode (GGUF order, dims[0] contiguous)."""
    gf = G.Gguf.open(MODEL)
    for t in gf.tensors:
        raw = np.frombuffer(gf.tensor_bytes(t.name), np.uint8)
        got = g.read(gf.tensor_f32(g, t.name))
        if t.ggml_type == G.GGML_F32:
            want = raw.view("<f4")
        else:
            want = orc.decode(orc.Q8_0, raw, t.elements())
        assert np.array_equal(bits(got), bits(want)), t.name


def test_f16_tensors_decode_every_bit_pattern_exactly(G, g, orc):
    b = og.GgufBuilder()
    patterns = np.arange(65536, dtype=np.uint16)
    b.tensor_raw("h", [256, 256], G.GGML_F16, patterns.astype("<u2").tobytes())
    gf = G.Gguf.parse(b.into_bytes())
    got = g.read(gf.tensor_f32(g, "h"))
    want = orc.f16_to_f32_array(patterns)
    assert np.array_equal(bits(got), bits(want))


def test_q4_0_tensor_uploads_and_multiplies(fh, G, g, orc):
    k, n = 896, 1152
    w = orc.rand_vec(k * n, 21) * np.float32(0.02)
    raw = orc.quantise_matrix(orc.Q4_0, w, k, n)
    b = og.GgufBuilder()
    b.meta("general.alignment", og.V(og.U32, 256))
    b.tensor_f32("bias", [n], np.zeros(n, np.float32))
    b.tensor_raw("w", [k, n], G.GGML_Q4_0, raw.tobytes())
    gf = G.Gguf.parse(b.into_bytes())
    qw = gf.upload_qweight(g, "w")
    assert (qw.kind(), qw.k(), qw.n()) == (fh.QKind.Q4_0, k, n)
    assert np.array_equal(qw.read_gguf(), raw)
    x = orc.rand_vec(k, 3)
    y = g.zeros(n)
    fh.linear_q(g, g.upload(x), qw, y, 1)
    want = orc.matmul(x, orc.dequantised_in_out(orc.Q4_0, raw, k, n), 1, k, n)
    assert orc.max_rel_err(g.read(y), want) <= 1e-5
    dq = g.read(gf.tensor_f32(g, "w"))
    assert np.array_equal(bits(dq), bits(orc.decode(orc.Q4_0, raw, k * n)))


def test_upload_errors(G, g):
    b = og.GgufBuilder()
    b.tensor_f32("f", [64], np.ones(64, np.float32))
    b.tensor_raw("q41", [32], G.GGML_Q4_1, bytes(20))
    b.tensor_raw("i", [4], G.GGML_I32, bytes(16))
    b.tensor_raw("q8", [32, 2], G.GGML_Q8_0, bytes(68))
    data = b.into_bytes()
    gf = G.Gguf.parse(data)
    for name, call, text in [("f", "upload_qweight", "not a weight format"), ("q41", "upload_qweight", "not a weight format"),
                             ("i", "tensor_f32", "integer tensors"), ("nope", "upload_qweight", "missing tensor"),
                             ("nope", "tensor_f32", "missing tensor")]:
        with pytest.raises(G.GgufError) as e:
            getattr(gf, call)(g, name)
        assert text in str(e.value), (name, call, str(e.value))
    assert not g.read(gf.tensor_f32(g, "q41")).any()  # a read-only block type decodes (all-zero block)
    head = G.Gguf.parse_prefix(data[:gf.data_offset()], len(data))
    with pytest.raises(G.GgufError) as e:
        head.upload_qweight(g, "q8")
    assert "header-only" in str(e.value)
