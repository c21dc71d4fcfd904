"""GPU parity tests for the device codec and the QAT snap (bit-exact against the oracle).
Mirrors ferrum_wgpu/src/ops/qat.rs:68-214 and adds the encode/decode kernels, including the
reference's golden GGUF fixture (fixtures/bpe/model.gguf's Q8_0 blocks) and large-size
round-trip properties."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def fh():
    import ferrum_hip

    return ferrum_hip


@pytest.fixture(scope="module")
def g(fh):
    gpu = fh.Gpu.open_for_test()
    if gpu is None:
        pytest.skip("no gfx950 device")
    yield gpu
    gpu.close()


def nasty(orc, n):
    """ferrum_wgpu/src/ops/qat.rs:68-80"""
    v = orc.rand_vec(n, 9) * np.float32(3.0)
    i = np.arange(n)
    sel = (i // 32) % 7
    v = np.where(sel == 0, v * np.float32(1e-6), v)
    v = np.where(sel == 1, np.float32(0), v)
    v = np.where(sel == 2, v * np.float32(1e4), v)
    v = np.where(sel == 3, (i % 9).astype(np.float32) - np.float32(4), v)
    return v.astype(np.float32)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- encode / decode ----

@pytest.mark.parametrize("n_blocks", [1, 7, 8, 127, 128, 129, 1000, 4096 + 3])
def test_encode_and_decode_rows_are_bit_exact(fh, g, orc, n_blocks):
    n = 32 * n_blocks
    x = nasty(orc, n)
    for kind in (fh.QKind.Q8_0, fh.QKind.Q4_0):
        say("codec", kind.label(), n_blocks)
        want = orc.encode(int(kind), x)
        got = g.read_bytes(fh.encode(g, kind, g.upload(x), n))
        assert np.array_equal(got, want), (kind, n_blocks)
        dec = g.read(fh.decode(g, kind, g.upload_bytes(want), n))
        assert np.array_equal(bits(dec), bits(orc.decode(int(kind), want, n)))


def test_codec_golden_fixture(fh, g):
    z = np.load(os.path.join(GOLDEN, "codec_nasty.npz"))
    x = z["x"]
    for kind, key, dkey in [(fh.QKind.Q8_0, "q8_0", "dq8_0"), (fh.QKind.Q4_0, "q4_0", "dq4_0")]:
        assert np.array_equal(g.read_bytes(fh.encode(g, kind, g.upload(x), x.size)), z[key])
        assert np.array_equal(bits(g.read(fh.decode(g, kind, g.upload_bytes(z[key]), x.size))), bits(z[dkey]))
    dst = g.zeros(x.size)
    fh.q8_snap_rows(g, g.upload(x), dst, 32)
    assert np.array_equal(bits(g.read(dst)), bits(z["snap_rows"]))
    dst = g.zeros(x.size)
    fh.q8_snap_cols(g, g.upload(x), dst, (64, 32))
    assert np.array_equal(bits(g.read(dst)), bits(z["snap_cols_64x32"]))


def test_reference_gguf_fixture_round_trips_on_the_device(fh, g, orc):
    """fixtures/bpe/model.gguf: decode -> encode on the device gives the file's bytes back, for
    all 4352 blocks, and the decoded values equal the oracle's."""
    info = json.load(open(os.path.join(GOLDEN, "model_gguf_q8_0.json")))
    blob = np.fromfile(os.path.join(GOLDEN, "model_gguf_q8_0.bin"), np.uint8)
    n = blob.size // 34 * 32
    vals = g.read(fh.decode(g, fh.QKind.Q8_0, g.upload_bytes(blob), n))
    assert np.array_equal(bits(vals), bits(orc.decode(orc.Q8_0, blob, n)))
    assert np.array_equal(g.read_bytes(fh.encode(g, fh.QKind.Q8_0, g.upload(vals), n)), blob)
    # and as resident weights: each tensor uploaded as GGUF rows reads back bit-exact
    for t in info["tensors"]:
        ne0, ne1 = t["dims"][0], int(np.prod(t["dims"][1:]))
        raw = blob[t["offset"]:t["offset"] + t["bytes"]]
        qw = fh.upload_qweight(g, fh.QKind.Q8_0, raw, ne0, ne1)
        assert np.array_equal(qw.read_gguf(), raw)
        want = orc.dequantised_in_out(orc.Q8_0, raw, ne0, ne1)
        assert np.array_equal(bits(qw.dequantised()), bits(want)), t["name"]


def test_large_codec_round_trip_properties(fh, g, orc):
    """At the 1.1B-Llama FFN size (2048 x 5632): encode is idempotent on decoded values and
    decode(encode(decode(b))) == decode(b), checked on the device only (size-independent)."""
    rng = np.random.default_rng(4)
    n = 2048 * 5632
    x = (rng.standard_normal(n) * 0.02).astype(np.float32)
    gx = g.upload(x)
    for kind in (fh.QKind.Q8_0, fh.QKind.Q4_0):
        b1 = fh.encode(g, kind, gx, n)
        d1 = fh.decode(g, kind, b1, n)
        b2 = fh.encode(g, kind, d1, n)
        d2 = fh.decode(g, kind, b2, n)
        assert np.array_equal(bits(g.read(d1)), bits(g.read(d2)))
        # spot-check against the oracle on a slice
        sl = slice(0, 32 * 4096)
        assert np.array_equal(g.read_bytes(b1)[: 4096 * kind.file_bytes()], orc.encode(int(kind), x[sl]))


# ---- snap (ops/qat.rs tests) ----

def test_values_that_round_to_zero_are_positive_zero_like_the_cpu(fh, g):
    blk = np.zeros(32, np.float32)
    blk[0], blk[1], blk[2] = 127.0, -0.3, -0.0
    src, dst = g.upload(blk), g.zeros(32)
    fh.q8_snap_rows(g, src, dst, 32)
    got = g.read(dst)
    assert bits(got)[1] == 0 and bits(got)[2] == 0


@pytest.mark.parametrize("n", [32, 96, 4096, 64 * 100, 32 * 100003])
def test_row_blocks_match_the_cpu_snap_bit_for_bit(fh, g, orc, n):
    data = nasty(orc, n)
    want = orc.snap_rows(data, 32)
    src, dst = g.upload(data), g.zeros(n)
    fh.q8_snap_rows(g, src, dst, 32)
    bad = int(np.sum(bits(g.read(dst)) != bits(want)))
    say(f"rows n={n}: {bad} of {n} differ")
    assert bad == 0


@pytest.mark.parametrize("rows_in,cols_out", [(32, 1), (32, 7), (64, 33), (96, 128), (256, 64), (2048, 300)])
def test_column_blocks_match_the_cpu_snap_bit_for_bit(fh, g, orc, rows_in, cols_out):
    data = nasty(orc, rows_in * cols_out)
    want = orc.snap_cols(data, rows_in, cols_out)
    src, dst = g.upload(data), g.zeros(data.size)
    fh.q8_snap_cols(g, src, dst, (rows_in, cols_out))
    assert int(np.sum(bits(g.read(dst)) != bits(want))) == 0


def test_ties_round_away_from_zero_and_the_scale_is_rounded_to_f16(fh, g, orc):
    blk = np.zeros(32, np.float32)
    blk[:5] = [127.0, 2.5, -2.5, 0.5, -0.49999997]
    dst = g.zeros(32)
    fh.q8_snap_rows(g, g.upload(blk), dst, 32)
    assert list(g.read(dst)[:5]) == [127.0, 3.0, -3.0, 1.0, 0.0]
    blk = np.zeros(32, np.float32)
    blk[0], blk[1] = np.float32(127.0) / np.float32(3.0), 1.0
    dst = g.zeros(32)
    fh.q8_snap_rows(g, g.upload(blk), dst, 32)
    assert np.array_equal(g.read(dst), orc.snap_rows(blk, 32))


def test_the_snap_is_idempotent_on_the_device(fh, g, orc):
    data = orc.rand_vec(64 * 4, 12)
    a, b, c = g.upload(data), g.zeros(256), g.zeros(256)
    fh.q8_snap_cols(g, a, b, (64, 4))
    fh.q8_snap_cols(g, b, c, (64, 4))
    assert np.array_equal(g.read(b), g.read(c))


def test_ineligible_shapes_are_copied_unchanged(fh, g, orc):
    data = orc.rand_vec(8 * 5, 13)
    dst = g.zeros(40)
    fh.q8_snap_cols(g, g.upload(data), dst, (8, 5))
    assert np.array_equal(g.read(dst), data)
    dst = g.zeros(40)
    fh.q8_snap_rows(g, g.upload(data), dst, 8)
    assert np.array_equal(g.read(dst), data)
    odd = orc.rand_vec(40, 14)
    dst = g.zeros(40)
    fh.q8_snap_rows(g, g.upload(odd), dst, 32)
    assert np.array_equal(g.read(dst), odd)


def test_shape_errors_and_faults_are_reported(fh, g):
    a, b = g.zeros(64), g.zeros(32)
    with pytest.raises(fh.GpuError, match="destination"):
        fh.q8_snap_rows(g, a, b, 32)
    with pytest.raises(fh.GpuError):
        fh.q8_snap_cols(g, a, b, (32, 2))
    c = g.zeros(64)
    with pytest.raises(fh.GpuError, match="is not 32 x 3"):
        fh.q8_snap_cols(g, a, c, (32, 3))
    assert g.sweep_faults(lambda: fh.q8_snap_cols(g, a, c, (32, 2))) == 1
    assert g.sweep_faults(lambda: fh.q8_snap_rows(g, a, c, 32)) == 1
    assert g.sweep_faults(lambda: fh.q8_snap_rows(g, a, c, 8)) == 1


# ---- grouped snap pass (fh_snap_plan_*, GpuTrainer::record_snap's loop in one launch) ----

def test_snap_plan_equals_the_single_calls_bit_for_bit(fh, g, orc):
    """Every mode and fallback in one plan: column snaps in the f32x4 form (cols a multiple of
    4) and the per-column form (7, 33 and 301 columns), row snaps, row snaps and column snaps whose
    shapes are not whole blocks (copied, as the single calls do), plain copies of odd lengths."""
    cases = [(fh.SNAP_COLS, (64, 32)), (fh.SNAP_COLS, (32, 7)), (fh.SNAP_COLS, (96, 33)), (fh.SNAP_COLS, (256, 300)),
             (fh.SNAP_COLS, (64, 301)), (fh.SNAP_ROWS, 32), (fh.SNAP_ROWS, 8), (fh.SNAP_COLS, (8, 5)),
             (fh.SNAP_COPY, None), (fh.SNAP_ROWS, 64), (fh.SNAP_COLS, (2048, 256))]
    sizes = [64 * 32, 32 * 7, 96 * 33, 256 * 300, 64 * 301, 32 * 1000, 8 * 13, 8 * 5, 1237, 64 * 77, 2048 * 256]
    probs, want = [], []
    for i, ((mode, shape), n) in enumerate(zip(cases, sizes)):
        data = nasty(orc, n) if n % 32 == 0 else (orc.rand_vec(n, 40 + i) * np.float32(3)).astype(np.float32)
        src, dst, one = g.upload(data), g.zeros(n), g.zeros(n)
        if mode == fh.SNAP_COLS:
            fh.q8_snap_cols(g, src, one, shape)
        elif mode == fh.SNAP_ROWS:
            fh.q8_snap_rows(g, src, one, shape)
        else:
            g.copy_f32(src, 0, one, 0, n)
        probs.append((mode, src, dst, shape))
        want.append((dst, g.read(one), data, mode, shape))
    plan = fh.SnapPlan(g, probs)
    assert plan.bytes() == 8 * sum(sizes)
    for rep in range(2):
        plan.run()
        for dst, single, data, mode, shape in want:
            got = g.read(dst)
            assert np.array_equal(bits(got), bits(single)), (mode, shape, rep)
            if mode == fh.SNAP_COLS and shape[0] % 32 == 0:
                assert np.array_equal(bits(got), bits(orc.snap_cols(data, *shape))), shape
            elif mode == fh.SNAP_ROWS and shape % 32 == 0 and data.size % 32 == 0:
                assert np.array_equal(bits(got), bits(orc.snap_rows(data, shape))), shape
            else:
                assert np.array_equal(bits(got), bits(data)), (mode, shape)
    plan.free()


def test_snap_plan_runs_the_tinyllama_qat_pass(fh, g, orc):
    """Config 5's QAT fake-quant pass as one launch: the column snap of two blocks' worth of
    TinyLlama-1.1B matrices (seven shapes each), bit-exact with the oracle's snap_cols."""
    rng = np.random.default_rng(12)
    shapes = [(2048, 2048), (2048, 256), (2048, 256), (2048, 2048), (2048, 5632), (2048, 5632), (5632, 2048)]
    probs, checks = [], []
    for a, b in shapes:
        w = (rng.standard_normal(a * b) * 0.02).astype(np.float32)
        want = orc.snap_cols(w, a, b)
        for _ in range(2):
            src, dst = g.upload(w), g.zeros(a * b)
            probs.append((fh.SNAP_COLS, src, dst, (a, b)))
            checks.append((dst, want))
    plan = fh.SnapPlan(g, probs)
    plan.run()
    for dst, want in checks:
        assert np.array_equal(g.read(dst).view(np.uint32), want.view(np.uint32))
    plan.free()


def test_snap_plan_refusals(fh, g):
    a, b = g.zeros(64), g.zeros(64)
    with pytest.raises(fh.GpuError, match="is not 32 x 3"):
        fh.SnapPlan(g, [(fh.SNAP_COLS, a, b, (32, 3))])
    with pytest.raises(fh.GpuError, match="has mode 7"):
        fh.SnapPlan(g, [(7, a, b, 0)])
    with pytest.raises(fh.GpuError, match="destination"):
        fh.SnapPlan(g, [(fh.SNAP_ROWS, a, g.zeros(32), 32)])
    fh.SnapPlan(g, [(fh.SNAP_ROWS, a, b, 32)]).run()  # the device still works
