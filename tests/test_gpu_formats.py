"""The weight formats beyond Q8_0 / Q4_0 on the device (F16, MXFP4, FP8 E4M3 / E5M2, Q2_K) and the
read-only GGUF block types, against the CPU oracle. Mirrors ferrum_wgpu/src/ops/quant/
ext_tests.rs (sizes and eligibility, bad shapes, requantisation, decode parity, every kernel
against the CPU matmul, the kernel choice, the GEMV's one-row rule, closeness to the f32
product), with this library's resident layout (the GGUF rows themselves, so the device bytes are
the file bytes) in place of the reference's repacked records.

Bars: encode, decode and dequantise bit-exact; the one-thread-per-output kernel bit-exact with
the CPU matmul on the decoded weights (same operation order); the GEMV and tiled kernels within
the reference's REDUCING 1e-5 (ferrum_wgpu/src/tolerance.rs:7)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu
REDUCING = 1e-5


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


def ext(fh):
    return [fh.QKind.Fp4, fh.QKind.Fp8E4M3, fh.QKind.Fp8E5M2, fh.QKind.Q2K, fh.QKind.F16]


def shapes(fh, kind):
    """ext_tests.rs:12-18"""
    if kind == fh.QKind.Q2K:
        return [(256, 1), (256, 5), (512, 17)]
    return [(32, 1), (32, 5), (64, 3), (96, 65)]


def weights(orc, n):
    """ext_tests.rs:20-31: rand_vec * 2 with blocks of 1e-5, 0 and 300 scale."""
    v = orc.rand_vec(n, 21) * np.float32(2.0)
    for i in range(n):
        m = i // 32 % 5
        if m == 0:
            v[i] *= np.float32(1e-5)
        elif m == 1:
            v[i] = 0.0
        elif m == 2:
            v[i] *= np.float32(300.0)
    return v


def oid(orc, kind):
    return int(kind)  # the oracle uses the same ids


def test_sizes_eligibility_and_the_layout(fh, g, orc):
    for kind in ext(fh):
        e = kind.elems()
        assert fh.nbytes(kind, 3 * e) == 3 * kind.file_bytes() == orc.nbytes(oid(orc, kind), 3 * e)
        with pytest.raises(fh.GpuError):
            fh.nbytes(kind, e + 1 if e == 256 else 33)
    assert (fh.QKind.Fp4.elems(), fh.QKind.Q2K.elems()) == (32, 256)
    assert fh.eligible_for(fh.QKind.Fp4, 96) and not fh.eligible_for(fh.QKind.Q2K, 96)
    assert fh.eligible_for(fh.QKind.Q2K, 768) and not fh.eligible_for(fh.QKind.Q2K, 0)
    assert fh.effective(fh.QKind.Q2K, 96) == fh.QKind.Q4_0 and fh.effective(fh.QKind.Q2K, 512) == fh.QKind.Q2K
    assert fh.QKind.Fp8E4M3.ggml() is None and fh.QKind.Fp4.ggml() == 39
    for kind in ext(fh):  # resident bytes are the GGUF bytes
        k = kind.elems() * 2
        qw = fh.upload_quantised(g, kind, orc.rand_vec(k * 8, 1), k, 8)
        assert qw.device_bytes() == 8 * 2 * kind.file_bytes()
        assert (qw.k(), qw.n(), qw.kind()) == (k, 8, kind)


def test_pack_and_quantise_refuse_bad_shapes(fh, g, orc):
    """ext_tests.rs:94-112"""
    for kind in ext(fh):
        k = kind.elems()
        with pytest.raises(fh.GpuError, match="whole"):
            fh.upload_qweight(g, kind, np.zeros(100, np.uint8), k + 1, 1)
        with pytest.raises(fh.GpuError, match="needs"):
            fh.upload_qweight(g, kind, np.zeros(3, np.uint8), k, 1)
        with pytest.raises(fh.GpuError):
            fh.upload_quantised(g, kind, np.zeros(k + 1), k + 1, 1)
        with pytest.raises(fh.GpuError):
            fh.upload_quantised(g, kind, np.zeros(2 * k - 1), k, 2)
    with pytest.raises(fh.GpuError):
        fh.upload_quantised(g, fh.QKind.Q2K, np.zeros(96), 96, 1)
    fh.upload_quantised(g, fh.QKind.Fp4, np.zeros(96), 96, 1)


def test_device_encode_is_bit_exact(fh, g, orc):
    """The device encoders against the oracle's restatement of the reference's, on the reference's
    awkward weights (blocks scaled by 1e-5, zero and 300) and wide random data (1287 Q2_K
    super-blocks: a partly filled last workgroup of sixteen)."""
    rng = np.random.default_rng(5)
    for kind in ext(fh):
        for data in (weights(orc, 4096), rng.standard_normal(8192).astype(np.float32) * np.float32(3.0),
                     orc.rand_vec(2048, 9), (rng.standard_normal(256 * 1287) * 0.02).astype(np.float32)):
            n = data.size
            want = orc.encode(oid(orc, kind), data)
            got = g.read_bytes(fh.encode(g, kind, g.upload(data), n))[: want.size]
            assert np.array_equal(got, want), (kind, n, np.flatnonzero(got != want)[:8])


def test_device_decode_is_bit_exact_for_every_block_type(fh, g, orc):
    """Random block bytes with finite f16 scales, for the weight formats and the read-only types
    (Q4_1, Q5_0, Q5_1, Q8_1, Q3_K, Q4_K, Q5_K, Q6_K)."""
    rng = np.random.default_rng(6)
    scale_at = {orc.Q4_1: (0, 2), orc.Q5_0: (0,), orc.Q5_1: (0, 2), orc.Q8_1: (0, 2), orc.Q2_K: (80, 82),
                orc.Q3_K: (108,), orc.Q4_K: (0, 2), orc.Q5_K: (0, 2), orc.Q6_K: (208,), orc.FP8_E4M3: (0,),
                orc.FP8_E5M2: (0,), orc.MXFP4: (), orc.F16: ()}
    for ty, offs in scale_at.items():
        nb, ne = orc.BLOCK_BYTES[ty], orc.BLOCK_ELEMS[ty]
        blocks = 67
        raw = rng.integers(0, 256, blocks * nb, dtype=np.uint8).reshape(blocks, nb)
        for o in offs:  # finite scales of modest size
            raw[:, o:o + 2] = np.frombuffer(rng.uniform(-2, 2, blocks).astype(np.float16).tobytes(),
                                            np.uint8).reshape(blocks, 2)
        if ty == orc.F16:
            raw = np.frombuffer(rng.standard_normal(blocks * 32).astype(np.float16).tobytes(), np.uint8)
        if ty == orc.MXFP4:
            raw[:, 0] = rng.integers(100, 150, blocks)
        raw = raw.reshape(-1)
        n = blocks * ne
        want = orc.decode(ty, raw, n)
        got = g.read(fh.decode(g, fh.QKind(ty) if ty in set(map(int, fh.QKind)) else ty, g.upload_bytes(raw), n))
        nan = np.isnan(want)  # the FP8 NaN codes: NaN on both sides (payload bits may differ)
        assert np.array_equal(np.isnan(got), nan), ty
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), \
            (ty, np.flatnonzero(got[~nan] != want[~nan])[:5])


def test_requantising_dequantised_weights_stays_close(fh, g, orc):
    """ext_tests.rs:115-139 (the device quantiser; MXFP4 requantises exactly)."""
    for kind in ext(fh):
        for k, n in shapes(fh, kind):
            qw = fh.upload_quantised(g, kind, weights(orc, k * n), k, n)
            rows = orc.decode(oid(orc, kind), qw.read_gguf(), k * n)
            again = fh.upload_quantised(g, kind, orc.transpose(rows, n, k), k, n)
            back = orc.decode(oid(orc, kind), again.read_gguf(), k * n)
            if kind in (fh.QKind.Fp4, fh.QKind.F16):
                assert np.array_equal(back, rows), (kind, k, n)
            else:
                assert np.abs(rows - back).max() <= 0.35 * np.abs(rows).max() + 1e-30, (kind, k, n)


def test_dequantised_values_match_the_cpu_decode(fh, g, orc):
    """ext_tests.rs:142-170: the identity product returns the decoded weights, and dequantise
    gives them too, bit for bit."""
    for kind in ext(fh):
        for k, n in shapes(fh, kind):
            b = orc.quantise_matrix(oid(orc, kind), weights(orc, k * n), k, n)
            rows = orc.decode(oid(orc, kind), b, k * n).reshape(n, k)
            w = fh.upload_qweight(g, kind, b, k, n)
            eye = np.eye(k, dtype=np.float32).reshape(-1)
            gy = g.zeros(k * n)
            fh.linear_q(g, g.upload(eye), w, gy, k)
            assert np.array_equal(g.read(gy).reshape(k, n), rows.T), (kind, k, n)
            assert np.array_equal(w.dequantised(), rows.T.reshape(-1)), (kind, k, n)
            assert np.array_equal(w.read_gguf(), b)


def test_every_kernel_matches_the_cpu_matmul(fh, g, orc):
    """ext_tests.rs:173-238: every path, rows 1, 3, 17, 33; the one-thread-per-output kernel
    bit-exact, the others within REDUCING."""
    for kind in ext(fh):
        for k, n in shapes(fh, kind):
            b = orc.quantise_matrix(oid(orc, kind), orc.rand_vec(k * n, 17), k, n)
            wd = orc.transpose(orc.decode(oid(orc, kind), b, k * n), n, k)
            qw = fh.upload_qweight(g, kind, b, k, n)
            for rows in (1, 3, 17, 33):
                x = orc.rand_vec(rows * k, 5)
                want = orc.matmul(x, wd, rows, k, n)
                gx = g.upload(x)
                paths = [fh.QPath.Naive, fh.QPath.Gemv, fh.QPath.Tiled, fh.QPath.Auto] if rows == 1 else \
                    [fh.QPath.Naive, fh.QPath.Tiled, fh.QPath.Auto]
                for path in paths:
                    gy = g.zeros(rows * n)
                    fh.linear_q_with(g, gx, qw, gy, rows, path)
                    got = g.read(gy)
                    if path == fh.QPath.Naive:
                        assert np.array_equal(got, want), (kind, k, n, rows)
                    else:
                        e = orc.max_rel_err(got, want)
                        assert e <= REDUCING, (kind, path, rows, k, n, e)


def test_kernel_choice_and_the_one_row_gemv(fh, g, orc):
    for kind in ext(fh):
        assert fh.choose(32, kind, 512, 1408) == fh.QPath.Tiled and fh.choose(1, kind, 512, 512) == fh.QPath.Gemv
    qw = fh.upload_quantised(g, fh.QKind.Fp4, orc.rand_vec(32 * 4, 2), 32, 4)
    with pytest.raises(fh.GpuError, match="one row"):
        fh.linear_q_with(g, g.upload(orc.rand_vec(64, 3)), qw, g.zeros(8), 2, fh.QPath.Gemv)
    with pytest.raises(fh.GpuError):
        fh.linear_q_with(g, g.upload(orc.rand_vec(64, 3)), qw, g.zeros(8), 2, fh.QPath.TiledFast)


def test_the_quantised_product_stays_near_the_f32_product(fh, g, orc):
    """ext_tests.rs:267-292: loose bounds that only a wrongly decoded format fails."""
    for kind, k, bound in ((fh.QKind.Fp4, 128, 0.35), (fh.QKind.Fp8E4M3, 128, 0.04), (fh.QKind.Fp8E5M2, 128, 0.08),
                           (fh.QKind.Q2K, 256, 0.9), (fh.QKind.F16, 128, 1e-3)):
        n, rows = 24, 5
        w, x = orc.rand_vec(k * n, 4), orc.rand_vec(rows * k, 6)
        want = orc.matmul(x, w, rows, k, n)
        qw = fh.upload_quantised(g, kind, w, k, n)
        gy = g.zeros(rows * n)
        fh.linear_q(g, g.upload(x), qw, gy, rows)
        assert np.abs(g.read(gy) - want).max() <= bound * np.abs(want).max(), kind


def test_larger_products_stay_within_reducing(fh, g, orc):
    """Wider shapes than the reference's tests (k up to 2048, several tiles each way)."""
    rng = np.random.default_rng(8)
    for kind in ext(fh):
        k, n, rows = 2048, 300, 70
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        b = orc.quantise_matrix(oid(orc, kind), w, k, n)
        wd = orc.transpose(orc.decode(oid(orc, kind), b, k * n), n, k)
        qw = fh.upload_qweight(g, kind, b, k, n)
        for r in (1, rows):
            x = rng.standard_normal(r * k).astype(np.float32)
            want = orc.matmul(x, wd, r, k, n)
            gy = g.zeros(r * n)
            fh.linear_q(g, g.upload(x), qw, gy, r)
            e = orc.max_rel_err(g.read(gy), want)
            say(f"{kind.label()} {r}x{k}x{n}: {e:.2e}")
            assert e <= REDUCING


def _close_or_same_special(got, want):
    """NaN where the CPU has NaN, the same infinity where it has one, REDUCING elsewhere."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    inf = np.isinf(want)
    assert np.array_equal(got[inf], want[inf])
    fin = np.isfinite(want)
    assert np.all(np.isfinite(got[fin]))
    e = orc_max_rel(got[fin], want[fin])
    assert e <= REDUCING, e


def orc_max_rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want) / np.maximum(np.abs(want), 1.0))) if got.size else 0.0


def _block_bytes(fh, kind, rows, k, fill):
    """GGUF rows of `kind` built byte by byte: fill(r, b) -> the bytes of block b of row r."""
    bb = kind.file_bytes()
    out = np.zeros((rows, k // kind.elems(), bb), np.uint8)
    for r in range(rows):
        for b in range(k // kind.elems()):
            out[r, b] = fill(r, b)
    return out.reshape(-1)


def test_gemv_decodes_every_code_like_the_cpu(fh, g, orc):
    """The one-row GEMV on hand-built blocks holding every code of each format (FP8 E4M3 / E5M2
    including NaN and infinity codes, every MXFP4 nibble pair under E8M0 scales down to the
    denormal ones, every finite F16 pattern), against the CPU matmul on the oracle's decode: NaN and
    infinities where the CPU has them, REDUCING elsewhere."""
    rng = np.random.default_rng(31)
    scales = np.float16([1.0, 0.5, 2.0, 1e-3, 3.0, -0.75, 2.0 ** -20, 0.25]).view(np.uint16)
    cases = []
    for kind in (fh.QKind.Fp8E4M3, fh.QKind.Fp8E5M2):
        bad = [0x7f, 0xff] if kind == fh.QKind.Fp8E4M3 else [0x7c, 0x7d, 0x7e, 0x7f, 0xfc, 0xfd, 0xfe, 0xff]
        k, rows = 512, 6

        top = 0x7e if kind == fh.QKind.Fp8E4M3 else 0x7c  # the largest finite E4M3 / E5M2's +infinity

        def fill(r, b, bad=bad, top=top):
            codes = (np.arange(32) + 32 * b + 7 * r) % 256
            if r != 1:  # row 1 keeps its NaN / infinity codes
                codes = np.where(np.isin(codes, bad), 0, codes)
            if r == 2 and b == 3:  # row 2 holds one +infinity (E5M2)
                codes[0] = top
            return np.concatenate([np.frombuffer(scales[(b + r) % 8].tobytes(), np.uint8), codes.astype(np.uint8)])

        cases.append((kind, k, rows, _block_bytes(fh, kind, rows, k, fill)))
    e8 = [0, 1, 2, 3, 125, 126, 127, 128, 129, 130, 120, 127, 131, 124, 127, 128]
    cases.append((fh.QKind.Fp4, 512, 4, _block_bytes(
        fh, fh.QKind.Fp4, 4, 512,
        lambda r, b: np.concatenate([[e8[(b + r) % 16]], (np.arange(16) + 16 * b + 37 * r) % 256]).astype(np.uint8))))
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = np.isfinite(pats.view(np.float16))
    pats = np.where(finite, pats, 0).astype(np.uint16)
    cases.append((fh.QKind.F16, 65536, 1, pats.view(np.uint8).copy()))
    for kind, k, rows, raw in cases:
        wd = orc.transpose(orc.decode(oid(orc, kind), raw, k * rows), rows, k)
        x = (rng.standard_normal(k) * (1e-3 if kind == fh.QKind.F16 else 1.0)).astype(np.float32)
        want = orc.matmul(x, wd, 1, k, rows)
        qw = fh.upload_qweight(g, kind, raw, k, rows)
        gy = g.zeros(rows)
        fh.linear_q_with(g, g.upload(x), qw, gy, 1, fh.QPath.Gemv)
        got = g.read(gy)
        say(f"{kind.label()}: {got} vs {want}")
        _close_or_same_special(got, want)
        qw.free()


def test_mfma_gemm_on_every_code(fh, g, orc):
    """The multi-row MFMA GEMM (F16, FP8 E4M3 / E5M2, MXFP4) decodes every code as the CPU does:
    with x the 512 x 512 identity the product is the decoded weight itself, compared bit for bit
    with the CPU matmul on the oracle's decode (every FP8 code under f16 scales down to a
    subnormal one, every MXFP4 nibble pair under E8M0 scales down to the denormal ones, random
    F16 patterns, random Q2_K super-blocks under varied d and dmin). A block holding an infinity or
    NaN makes its output column NaN, as the CPU's 0 x inf terms do."""
    rng = np.random.default_rng(34)
    scales = np.float16([1.0, 0.5, 2.0, 1e-3, 3.0, -0.75, 2.0 ** -20, 0.25]).view(np.uint16)
    k, n = 512, 70
    x = np.eye(k, dtype=np.float32).reshape(-1)
    for kind in (fh.QKind.Fp8E4M3, fh.QKind.Fp8E5M2, fh.QKind.Fp4, fh.QKind.F16, fh.QKind.Q2K):
        if kind == fh.QKind.Q2K:
            raw = rng.integers(0, 256, (n * k // 256, 84), dtype=np.uint8)
            dd = np.float16(rng.choice([0.01, 0.5, 3.0, 2.0 ** -18, 1e-3], (n * k // 256, 2)))
            raw[:, 80:84] = dd.view(np.uint8).reshape(-1, 4)
            raw = raw.reshape(-1)
        elif kind == fh.QKind.F16:
            pats = (rng.integers(0, 65536, k * n)).astype(np.uint16)
            finite = np.isfinite(pats.view(np.float16))
            keep = np.zeros(k * n, bool)
            keep[3 * k + 5] = keep[7 * k + 100] = True  # rows 3 and 7 hold one non-finite half each
            raw = np.where(finite | keep, pats, 0).astype(np.uint16).view(np.uint8).copy()
        elif kind == fh.QKind.Fp4:
            e8 = [0, 1, 2, 3, 125, 126, 127, 128, 129, 130, 120, 127, 131, 124, 127, 128]
            raw = _block_bytes(fh, kind, n, k, lambda r, b: np.concatenate(
                [[e8[(b + r) % 16]], (np.arange(16) + 16 * b + 37 * r) % 256]).astype(np.uint8))
        else:
            bad = [0x7f, 0xff] if kind == fh.QKind.Fp8E4M3 else [0x7c, 0x7d, 0x7e, 0x7f, 0xfc, 0xfd, 0xfe, 0xff]

            def fill(r, b, bad=bad):
                codes = (np.arange(32) + 32 * b + 7 * r) % 256
                if r not in (1, 9):  # rows 1 and 9 keep their non-finite codes
                    codes = np.where(np.isin(codes, bad), 0, codes)
                return np.concatenate([np.frombuffer(scales[(b + r) % 8].tobytes(), np.uint8),
                                       codes.astype(np.uint8)])

            raw = _block_bytes(fh, kind, n, k, fill)
        wd = orc.transpose(orc.decode(oid(orc, kind), raw, k * n), n, k)
        want = orc.matmul(x, wd, k, k, n)
        qw = fh.upload_qweight(g, kind, raw, k, n)
        gy = g.zeros(k * n)
        fh.linear_q_with(g, g.upload(x), qw, gy, k, fh.QPath.Tiled)
        got = g.read(gy)
        nan = np.isnan(want)
        say(f"{kind.label()}: {int(nan.sum())} NaN outputs, {int(np.isinf(want).sum())} infinite")
        assert np.array_equal(np.isnan(got), nan), kind
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), kind
        qw.free()


def test_gemv_takes_x_at_any_float_offset(fh, g, orc):
    """x handed over as a raw pointer 4, 8, 12 and 16 bytes into a buffer: the misaligned ones run
    the scalar-load GEMV, the aligned one the segment GEMV; all within REDUCING."""
    rng = np.random.default_rng(32)
    for kind in ext(fh):
        k, n = (512, 37) if kind == fh.QKind.Q2K else (96, 37)
        b = orc.quantise_matrix(oid(orc, kind), (rng.standard_normal(k * n) * 0.02).astype(np.float32), k, n)
        wd = orc.transpose(orc.decode(oid(orc, kind), b, k * n), n, k)
        qw = fh.upload_qweight(g, kind, b, k, n)
        x = rng.standard_normal(k + 4).astype(np.float32)
        gx = g.upload(x)
        for off in (1, 2, 3, 4):
            want = orc.matmul(x[off:off + k].copy(), wd, 1, k, n)
            gy = g.zeros(n)
            fh.linear_q_ptr(g, gx.device_ptr() + 4 * off, qw, gy.device_ptr(), 1, fh.QPath.Gemv)
            e = orc.max_rel_err(g.read(gy), want)
            assert e <= REDUCING, (kind, off, e)
        qw.free()


def test_gemv_launch_shapes_cover_every_row_grouping(fh, g, orc):
    """k = 2048 with 3001, 4101 and 16401 output rows (and 33001 for MXFP4), so the GEMV
    runs with groups of 8, 4, 2 and 1 rows and partial groups at the end, within REDUCING. Q2_K rows are random bytes under fixed
    super-block scales (any such bytes decode to finite values)."""
    rng = np.random.default_rng(33)
    k = 2048
    for kind in ext(fh):
        for n in (3001, 4101, 16401) + ((33001,) if kind == fh.QKind.Fp4 else ()):
            if kind == fh.QKind.Q2K:
                raw = rng.integers(0, 256, (n * k // 256, 84), dtype=np.uint8)
                raw[:, 80:84] = np.frombuffer(np.float16([0.001, 0.0004]).tobytes(), np.uint8)  # |w| ~ 0.02
                raw = raw.reshape(-1)
            else:
                raw = orc.quantise_matrix(oid(orc, kind), (rng.standard_normal(k * n) * 0.02).astype(np.float32), k, n)
            wd = orc.transpose(orc.decode(oid(orc, kind), raw, k * n), n, k)
            x = rng.standard_normal(k).astype(np.float32)
            want = orc.matmul(x, wd, 1, k, n)
            qw = fh.upload_qweight(g, kind, raw, k, n)
            gy = g.zeros(n)
            fh.linear_q_with(g, g.upload(x), qw, gy, 1, fh.QPath.Gemv)
            e = orc.max_rel_err(g.read(gy), want)
            say(f"{kind.label()} 1x{k}x{n}: {e:.2e}")
            assert e <= REDUCING, (kind, n, e)
            qw.free()


def test_gguf_uploads_of_the_new_formats(fh, g, orc):
    """A GGUF holding MXFP4, Q2_K and F16 matrices and read-only block tensors: the matrices
    upload as resident weights (bytes kept), every tensor decodes on the device as the oracle
    decodes it."""
    from oracle import gguf as og
    from ferrum_hip.gguf import Gguf

    rng = np.random.default_rng(9)
    b = og.GgufBuilder()
    b.meta("general.architecture", og.V(og.STR, "test"))
    tensors = {}
    for name, ty, k, n in (("w.mxfp4", orc.MXFP4, 64, 5), ("w.q2k", orc.Q2_K, 256, 3), ("w.f16", orc.F16, 32, 4)):
        raw = orc.encode(ty, rng.standard_normal(k * n).astype(np.float32))
        b.tensor_raw(name, [k, n], ty, raw.tobytes())
        tensors[name] = (ty, k, n, raw)
    for ty in (orc.Q4_1, orc.Q5_0, orc.Q5_1, orc.Q8_1, orc.Q3_K, orc.Q4_K, orc.Q5_K, orc.Q6_K):
        nb, ne = orc.BLOCK_BYTES[ty], orc.BLOCK_ELEMS[ty]
        raw = rng.integers(0, 256, 2 * nb, dtype=np.uint8).reshape(2, nb)
        raw[:, 0:2] = np.frombuffer(np.float16([0.5, -0.25]).tobytes(), np.uint8).reshape(2, 2)
        if ty in (orc.Q3_K,):
            raw[:, 108:110] = np.frombuffer(np.float16([0.5, -0.25]).tobytes(), np.uint8).reshape(2, 2)
        if ty in (orc.Q6_K,):
            raw[:, 208:210] = np.frombuffer(np.float16([0.5, -0.25]).tobytes(), np.uint8).reshape(2, 2)
        if ty in (orc.Q4_1, orc.Q5_1, orc.Q8_1, orc.Q4_K, orc.Q5_K):
            raw[:, 2:4] = np.frombuffer(np.float16([0.125, 1.0]).tobytes(), np.uint8).reshape(2, 2)
        raw = raw.reshape(-1)
        b.tensor_raw(f"t.{ty}", [2 * ne], ty, raw.tobytes())
        tensors[f"t.{ty}"] = (ty, 2 * ne, 1, raw)
    gg = Gguf.parse(b.into_bytes())
    for name, (ty, k, n, raw) in tensors.items():
        got = g.read(gg.tensor_f32(g, name))
        assert np.array_equal(got, orc.decode(ty, raw, k * n)), name
        if name.startswith("w."):
            qw = gg.upload_qweight(g, name)
            assert (qw.k(), qw.n(), int(qw.kind())) == (k, n, ty)
            assert np.array_equal(qw.read_gguf(), raw)
