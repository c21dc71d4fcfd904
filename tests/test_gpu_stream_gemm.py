"""The MFMA GEMMs' streaming 256 x 256 kernels (QPath.Tiled and QPath.TiledFast on products with
at least 128 such tiles): one CTA per CU working through its tiles stage by stage, K split up to 4
ways.

The reference path it replaces for these shapes is `linear_q` on many rows
(ferrum_wgpu/src/ops/quant.rs:326-381, qlinear_tiled.wgsl:93-128), whose tests hold every product
to REDUCING (1e-5, ferrum_wgpu/src/tolerance.rs:7) against ferrum_ref's CPU matmul on the
dequantised weights (kernels/matmul.rs:49-107). Bar (written here): max_rel_err < 1e-5 against the
CPU oracle's f32 product (16-thread matmul_tuned, bit-identical to matmul), or, where the CPU's own
f32 product is that far from the float64 product, no farther from float64 than the CPU. Every
output is compared: the kernel deals tiles to CTAs in an XCD-grouped order, so a mistake in that
order shows up in some column tile, not necessarily the first.

The scoring GEMM (TiledFast, no counterpart in the reference) is held to the MFMA-GEMM bound on
every output, |g - w| <= 1e-3 + 2e-3 |w| against the same CPU product (0 outputs outside it). It
takes the streaming kernel from 640 tiles on: the TinyLlama gate/up at M = 4096 (704 tiles), a
ragged product with an odd block count (2085 x 1120 x 20000, 711 tiles) and one with a 2-way K
split (2560 x 2048 x 16384, 640 tiles).

Cases: whole tiles with a 2-way K split (2048 x 2048 x 4096), ragged rows, columns and an odd block
count with a padding stage (2085 x 1120 x 4196), and the TinyLlama down product at M = 4096
(4096 x 5632 x 2048, 176 blocks, 2-way split)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

REDUCING = 1e-5
THREADS = 16


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


@pytest.mark.parametrize("kind_name", ["Q4_0", "Q8_0"])
@pytest.mark.parametrize("m,k,n", [(2048, 2048, 4096), (2085, 1120, 4196), (4096, 5632, 2048)])
def test_stream_precise_gemm_matches_the_cpu(fh, g, orc, kind_name, m, k, n):
    kind = fh.QKind[kind_name]
    rng = np.random.default_rng(m + k + n)
    w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    x = rng.standard_normal(m * k).astype(np.float32)
    say(f"stream GEMM {kind_name} {m}x{k}x{n}: uploading")
    qw = fh.upload_quantised(g, kind, w, k, n)
    b = qw.read_gguf()
    wd = orc.dequantised_in_out(int(kind), b, k, n)
    gx, gy = g.upload(x), g.zeros(m * n)
    fh.linear_q_with(g, gx, qw, gy, m, fh.QPath.Tiled)
    got = g.read(gy).reshape(m, n)
    again = g.zeros(m * n)
    fh.linear_q_with(g, gx, qw, again, m, fh.QPath.Tiled)
    assert np.array_equal(g.read(again).reshape(m, n).view(np.uint32), got.view(np.uint32)), "not deterministic"
    qw.free()
    want = orc.matmul_tuned(x, wd, m, k, n, THREADS).reshape(m, n)
    e = orc.max_rel_err(got.reshape(-1), want.reshape(-1))
    ex = x.reshape(m, k).astype(np.float64) @ wd.reshape(k, n).astype(np.float64)
    den = np.maximum(np.abs(ex), 1.0)
    e_dev = float(np.max(np.abs(got - ex) / den))
    e_cpu = float(np.max(np.abs(want - ex) / den))
    say(f"stream GEMM {kind_name} {m}x{k}x{n}: vs CPU {e:.2e}; vs float64 device {e_dev:.2e}, CPU {e_cpu:.2e}")
    assert np.all(np.isfinite(got))
    assert e < REDUCING or e_dev <= e_cpu, (e, e_dev, e_cpu)


@pytest.mark.parametrize("kind_name", ["Q4_0", "Q8_0"])
@pytest.mark.parametrize("m,k,n", [(4096, 2048, 11264), (2085, 1120, 20000), (2560, 2048, 16384)])
def test_stream_fast_gemm_meets_the_per_output_bound(fh, g, orc, kind_name, m, k, n):
    kind = fh.QKind[kind_name]
    rng = np.random.default_rng(m + k + n + 1)
    w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    x = rng.standard_normal(m * k).astype(np.float32)
    say(f"stream fast GEMM {kind_name} {m}x{k}x{n}: uploading")
    qw = fh.upload_quantised(g, kind, w, k, n)
    b = qw.read_gguf()
    wd = orc.dequantised_in_out(int(kind), b, k, n)
    gx, gy = g.upload(x), g.zeros(m * n)
    fh.linear_q_with(g, gx, qw, gy, m, fh.QPath.TiledFast)
    got = g.read(gy).reshape(m, n)
    again = g.zeros(m * n)
    fh.linear_q_with(g, gx, qw, again, m, fh.QPath.TiledFast)
    assert np.array_equal(g.read(again).reshape(m, n).view(np.uint32), got.view(np.uint32)), "not deterministic"
    qw.free()
    want = orc.matmul_tuned(x, wd, m, k, n, THREADS).reshape(m, n)
    r = np.abs(got - want) / (1e-3 + 2e-3 * np.abs(want))
    frac = float(np.mean(r > 1.0))
    say(f"stream fast GEMM {kind_name} {m}x{k}x{n}: worst {float(r.max()):.3f} of the bound, outside {frac:.2e}, "
        f"max_rel_err {orc.max_rel_err(got.reshape(-1), want.reshape(-1)):.2e}")
    assert np.all(np.isfinite(got))
    assert frac == 0.0
