"""fh_linear_q_noalloc (no counterpart in the reference): the product without any device
allocation, its scratch taken from the library's static per-GPU array. Called through the C ABI,
its output must equal fh_linear_q_ptr's bit for bit (the same kernels on the same inputs), on two
calls in a row of which the second is smaller (the array keeps the first call's contents), for
every kernel path; and both stay within the reference's 1e-5 of the CPU product
(ferrum_wgpu/src/tolerance.rs:7) where the path keeps it."""
import ctypes

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


def case(fh, g, orc, kind, rows, k, n, seed, cpu=True):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    x = rng.standard_normal(rows * k).astype(np.float32)
    b = orc.quantise_matrix(int(kind), w, k, n)
    qw = fh.upload_qweight(g, kind, b, k, n)
    want = orc.matmul_tuned(x, orc.dequantised_in_out(int(kind), b, k, n), rows, k, n, 8) if cpu else None
    return qw, g.upload(x), g.zeros(rows * n), g.zeros(rows * n), want


# (path, rows, k, n): a larger product, then a smaller one, per path
PATHS = [
    ("Gemv", [(1, 4864, 896), (1, 896, 1152)]),
    ("Auto", [(1, 2048, 5632), (1, 768, 2304)]),
    ("Tiled", [(64, 2048, 2048), (8, 896, 1152)]),
    ("Auto", [(512, 896, 1152), (64, 896, 896)]),
    ("TiledF16", [(256, 2048, 2048), (32, 896, 1152)]),
    ("TiledFast", [(128, 896, 4864), (96, 896, 1152)]),
    ("Naive", [(4, 256, 320), (2, 64, 96)]),
]


@pytest.mark.parametrize("kind_name", ["Q8_0", "Q4_0"])
@pytest.mark.parametrize("path_name,shapes", PATHS, ids=[f"{p}-{s[0][0]}" for p, s in PATHS])
def test_noalloc_equals_linear_q_on_two_calls_in_a_row(fh, g, orc, kind_name, path_name, shapes):
    kind, path = fh.QKind[kind_name], fh.QPath[path_name]
    cases = [case(fh, g, orc, kind, r, k, n, 40 + i) for i, (r, k, n) in enumerate(shapes)]
    if path == fh.QPath.TiledFast:
        for qw, gx, ya, _, _ in cases:  # an ordinary fast product builds the correction operand
            fh.linear_q_with(g, gx, qw, ya, len(gx) // qw.k(), path)
    for (r, k, n), (qw, gx, ya, _, _) in zip(shapes, cases):
        fh.linear_q_ptr(g, gx.device_ptr(), qw, ya.device_ptr(), r, path)
    for (r, k, n), (qw, gx, _, yb, _) in zip(shapes, cases):
        say(f"noalloc {kind_name} {path_name} rows {r} {k}x{n}")
        fh.linear_q_noalloc(g, gx.device_ptr(), qw, yb.device_ptr(), r, path)
    for (r, k, n), (qw, gx, ya, yb, want) in zip(shapes, cases):
        a, b = g.read(ya), g.read(yb)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (path_name, r, k, n)
        e = orc.max_rel_err(b, want)
        say(f"  rows {r} {k}x{n}: bit-identical to linear_q, max rel err {e:.2e}")
        if path not in (fh.QPath.TiledFast, fh.QPath.TiledF16):
            assert e < REDUCING, (path_name, r, k, n, e)
        else:  # the MFMA-GEMM bound in the max norm
            assert np.abs(b - want).max() <= 1e-3 + 2e-3 * np.abs(want).max()


def test_noalloc_refuses_what_it_cannot_do_without_allocating(fh, g, orc):
    # more scratch than the array holds: the split x of 4096 rows of 4096 is 64 MiB
    qw, gx, ya, yb, _ = case(fh, g, orc, fh.QKind.Q4_0, 4096, 4096, 256, 7, cpu=False)
    with pytest.raises(fh.GpuError) as err:
        fh.linear_q_noalloc(g, gx.device_ptr(), qw, yb.device_ptr(), 4096, fh.QPath.Tiled)
    assert "scratch" in str(err.value)
    # the fast GEMM before its correction operand exists
    with pytest.raises(fh.GpuError) as err:
        fh.linear_q_noalloc(g, gx.device_ptr(), qw, yb.device_ptr(), 4096, fh.QPath.TiledFast)
    assert "correction operand" in str(err.value)
    with pytest.raises(fh.GpuError, match="null pointer"):
        fh._check(fh.lib().fh_linear_q_noalloc(g.handle, None, qw.handle, ctypes.c_void_p(yb.device_ptr()), 1, 0))
    # the device still works, and a product that fits runs
    fh.linear_q_noalloc(g, gx.device_ptr(), qw, yb.device_ptr(), 16, fh.QPath.Tiled)
    fh.linear_q_ptr(g, gx.device_ptr(), qw, ya.device_ptr(), 16, fh.QPath.Tiled)
    assert np.array_equal(g.read(ya)[:16 * 256], g.read(yb)[:16 * 256])


def test_noalloc_calls_through_two_handles_of_one_gpu_do_not_race(fh, g, orc):
    """Two handles of one GPU (two streams) share its one scratch array: each noalloc call waits
    for the previous one's work on that GPU, so interleaved calls through both handles, issued
    without any synchronisation between them, still equal linear_q_ptr's results bit for bit."""
    ordinal = int(__import__("os").environ.get("FERRUM_HIP_DEVICE", "0"))
    g2 = fh.Gpu(ordinal)
    work = []
    try:
        kind = fh.QKind.Q4_0
        for i, h in enumerate((g, g2, g, g2)):
            rows, k, n = (256, 2048, 2048) if i % 2 == 0 else (192, 2048, 1024)
            qw, gx, ya, yb, _ = case(fh, h, orc, kind, rows, k, n, 60 + i, cpu=False)
            fh.linear_q_ptr(h, gx.device_ptr(), qw, ya.device_ptr(), rows, fh.QPath.Tiled)
            work.append((h, qw, gx, ya, yb, rows))
        g.sync()
        g2.sync()
        for rep in range(3):
            for h, qw, gx, _, yb, rows in work:
                fh.linear_q_noalloc(h, gx.device_ptr(), qw, yb.device_ptr(), rows, fh.QPath.Tiled)
        g.sync()
        g2.sync()
        for i, (h, qw, gx, ya, yb, rows) in enumerate(work):
            assert np.array_equal(h.read(ya).view(np.uint32), h.read(yb).view(np.uint32)), i
        say("noalloc through two handles of one GPU: 12 interleaved calls equal linear_q_ptr")
    finally:
        for h, qw, gx, ya, yb, rows in work:
            for b in (gx, ya, yb):
                b.free()
            qw.free()
        g2.close()


def test_noalloc_refuses_overlapping_x_and_y(fh, g, orc):
    qw, gx, ya, yb, _ = case(fh, g, orc, fh.QKind.Q8_0, 8, 256, 256, 9, cpu=False)
    with pytest.raises(fh.GpuError, match="overlap"):
        fh.linear_q_noalloc(g, gx.device_ptr(), qw, gx.device_ptr() + 4 * 256, 8, fh.QPath.Rows)
