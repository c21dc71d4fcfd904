"""the TinyLlama-1.1B layer products (d 2048, FFN 5632, 32 q / 4 kv heads: fused
QKV 2048 x 2560, attention output 2048 x 2048, fused gate/up 2048 x 11264, down 5632 x 2048), Q4_0
and Q8_0, activations ~ N(0, 1), weights ~ N(0, 0.02), M in {1, 8, 64, 512, 4096}, against the
CPU oracle (ferrum_ref's matmul on the dequantised weights, ferrum_ref/src/kernels/matmul.rs:49-107,
the tuned variant on 16 threads), plus the Q8_0 QAT fake-quant pass (q8_snap_cols over every matrix
shape, ferrum_ref/src/training/qat.rs:36-54) bit for bit.

Bars (written here):
  * the library's own path choice (AUTO: the GEMV at M = 1, the few-row kernel at 8 and 64, the
    precise MFMA GEMM at 512 and 4096): max_rel_err < 1e-5 against the CPU (REDUCING,
    ferrum_wgpu/src/tolerance.rs:7); where the CPU's own f32 product is itself 1e-5 or more from
    the float64 product (k = 5632), the device's distance from float64 may not exceed the CPU's;
  * the scoring GEMM (TiledFast) at M = 512 and 4096: every output within the MFMA-GEMM bound
    |g - w| <= 1e-3 + 2e-3 |w| of the CPU; the fraction of outputs outside it is printed (and must
    be 0);
  * M = 4096 compares the first 256 output columns of each product (the device computes them all);
  * the snap: bit-exact.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REDUCING = 1e-5
THREADS = 16
SHAPES = [(2048, 2560), (2048, 2048), (2048, 11264), (5632, 2048)]
COLS_AT_4096 = 256


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


@pytest.fixture(scope="module")
def weights(fh, orc):
    """Per (kind, shape): the GGUF bytes and the dequantised [k, n] weight."""
    rng = np.random.default_rng(55)
    out = {}
    for k, n in SHAPES:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        for kind in (fh.QKind.Q4_0, fh.QKind.Q8_0):
            b = orc.quantise_matrix(int(kind), w, k, n)
            out[(kind, k, n)] = (b, orc.dequantised_in_out(int(kind), b, k, n).reshape(k, n))
    return out


def run(fh, g, kind, b, x, m, k, n, path):
    qw = fh.upload_qweight(g, kind, b, k, n)
    gx, gy = g.upload(x), g.zeros(m * n)
    fh.linear_q_with(g, gx, qw, gy, m, path)
    got = g.read(gy).reshape(m, n)
    qw.free()
    return got


@pytest.mark.parametrize("kind_name", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("m", [1, 8, 64, 512, 4096])
def test_config5_products_through_the_librarys_choice(fh, g, orc, weights, kind_name, m):
    kind = fh.QKind[kind_name]
    rng = np.random.default_rng(100 + m)
    for k, n in SHAPES:
        b, wd = weights[(kind, k, n)]
        x = rng.standard_normal(m * k).astype(np.float32)
        path = fh.choose(m, kind, k, n)
        got = run(fh, g, kind, b, x, m, k, n, fh.QPath.Auto)
        cols = n if m < 4096 else COLS_AT_4096
        ws = np.ascontiguousarray(wd[:, :cols])
        want = orc.matmul_tuned(x, ws.reshape(-1), m, k, cols, THREADS).reshape(m, cols)
        got = np.ascontiguousarray(got[:, :cols])
        e = orc.max_rel_err(got.reshape(-1), want.reshape(-1))
        ex = x.reshape(m, k).astype(np.float64) @ ws.astype(np.float64)
        den = np.maximum(np.abs(ex), 1.0)
        e_dev = float(np.max(np.abs(got - ex) / den))
        e_cpu = float(np.max(np.abs(want - ex) / den))
        say(f"{kind_name} M={m} {k}x{n} ({path.name}): vs CPU {e:.2e}; vs float64 device {e_dev:.2e}, CPU {e_cpu:.2e}")
        assert e < REDUCING or e_dev <= e_cpu, (k, n, e, e_dev, e_cpu)


@pytest.mark.parametrize("kind_name", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("m", [512, 4096])
def test_config5_scoring_gemm_meets_the_per_output_bound(fh, g, orc, weights, kind_name, m):
    kind = fh.QKind[kind_name]
    rng = np.random.default_rng(200 + m)
    for k, n in SHAPES:
        b, wd = weights[(kind, k, n)]
        x = rng.standard_normal(m * k).astype(np.float32)
        got = run(fh, g, kind, b, x, m, k, n, fh.QPath.TiledFast)
        cols = n if m < 4096 else COLS_AT_4096
        ws = np.ascontiguousarray(wd[:, :cols])
        want = orc.matmul_tuned(x, ws.reshape(-1), m, k, cols, THREADS).reshape(m, cols)
        d = np.abs(got[:, :cols] - want)
        frac = float(np.mean(d > 1e-3 + 2e-3 * np.abs(want)))
        say(f"{kind_name} M={m} {k}x{n} TiledFast: worst {float(np.max(d / (1e-3 + 2e-3 * np.abs(want)))):.3f} of the "
            f"bound, outside it {frac:.2e}, max_rel_err {orc.max_rel_err(got[:, :cols].reshape(-1), want.reshape(-1)):.2e}")
        assert frac == 0.0


@pytest.mark.parametrize("rows_in,cols_out", [(2048, 2048), (2048, 256), (2048, 5632), (5632, 2048)])
def test_qat_fake_quant_pass_is_bit_exact_at_full_size(fh, g, orc, rows_in, cols_out):
    """Gpt2::fake_quantize's column snap (training/qat.rs:36-54) on every TinyLlama-1.1B matrix
    shape, [in, out] row-major, weights ~ N(0, 0.02)."""
    w = (np.random.default_rng(rows_in + cols_out).standard_normal(rows_in * cols_out) * 0.02).astype(np.float32)
    src, dst = g.upload(w), g.zeros(w.size)
    fh.q8_snap_cols(g, src, dst, (rows_in, cols_out))
    assert np.array_equal(g.read(dst).view(np.uint32), orc.snap_cols(w, rows_in, cols_out).view(np.uint32))
