"""CPU-only checks of the C-ABI library: it loads, exports every symbol the header declares,
and its host-side argument handling works without a GPU (no compute calls here)."""
import ctypes
import os
import re
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def fh():
    import ferrum_hip

    if not os.path.exists(ferrum_hip.LIB_PATH):
        pytest.fail(f"{ferrum_hip.LIB_PATH} missing: run __graft_entry__.build()")
    ferrum_hip.lib()
    return ferrum_hip


def test_library_exports_every_declared_symbol(fh):
    names = fh.exported_symbols()
    assert len(names) >= 40
    out = subprocess.run(["nm", "-D", "--defined-only", fh.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (fh_\w+)$", out, re.M))
    missing = [n for n in names if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    extra = sorted(exported - set(names))
    assert not extra, f"exported but not declared: {extra}"
    for n in names:
        assert getattr(fh.lib(), n) is not None


def test_library_is_built_for_gfx950_only(fh):
    """The offload bundle inside our own build names exactly one device target: gfx950."""
    data = open(fh.LIB_PATH, "rb").read()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", data))
    assert targets == {b"gfx950"}, targets


def test_abi_version_and_host_side_helpers(fh):
    L = fh.lib()
    assert L.fh_abi_version() == 1
    assert fh.nbytes(fh.QKind.Q8_0, 64) == 68
    assert fh.nbytes(fh.QKind.Q4_0, 64) == 36
    with pytest.raises(fh.GpuError, match="multiple"):
        fh.nbytes(fh.QKind.Q8_0, 33)
    assert L.fh_nbytes(15, 32) == 0 and b"unsupported" in L.fh_last_error()
    assert fh.eligible(32) and fh.eligible(96) and not fh.eligible(0) and not fh.eligible(33)


def test_choose_rules(fh):
    """The MI355X dispatch (replaces quant.rs:306-323, which was measured on MX330/Xe):
    one row -> the int8-MFMA GEMV while its 32-bit offsets cover a row (k <= 2^25); 2 to 16 rows
    -> the few-row kernel; 17 to 32 rows -> the few-row kernel while k <= 4864; 33 to 64 rows ->
    the few-row kernel only for n >= 2560 and k <= 2048; otherwise the precise MFMA GEMM. The
    boundary is measured (bench.py --choose-sweep, one linear_q per product at the config 2 and
    config 5 shapes)."""
    Q8, Q4 = fh.QKind.Q8_0, fh.QKind.Q4_0
    for kind in (Q8, Q4):
        assert fh.choose(1, kind, 768, 2304) == fh.QPath.Gemv
        assert fh.choose(1, kind, 4864, 896) == fh.QPath.Gemv
        assert fh.choose(1, kind, 8192, 64) == fh.QPath.Gemv
        assert fh.choose(1, kind, 8192 + 32, 64) == fh.QPath.Gemv
        assert fh.choose(1, kind, 2**25, 151936) == fh.QPath.Gemv
        assert fh.choose(1, kind, 2**25 + 32, 8) == fh.QPath.Tiled
        assert fh.choose(2, kind, 768, 2304) == fh.QPath.Rows
        assert fh.choose(8, kind, 5632, 2048) == fh.QPath.Rows
        assert fh.choose(64, kind, 2048, 11264) == fh.QPath.Rows
        assert fh.choose(16, kind, 5632, 2048) == fh.QPath.Rows
        assert fh.choose(24, kind, 5632, 2048) == fh.QPath.Tiled
        assert fh.choose(32, kind, 4864, 896) == fh.QPath.Rows
        assert fh.choose(48, kind, 4864, 896) == fh.QPath.Tiled
        assert fh.choose(48, kind, 2048, 2048) == fh.QPath.Tiled
        assert fh.choose(48, kind, 896, 1152) == fh.QPath.Tiled
        assert fh.choose(64, kind, 896, 4864) == fh.QPath.Rows
        assert fh.choose(64, kind, 2048, 2560) == fh.QPath.Rows
        assert fh.choose(65, kind, 2048, 2048) == fh.QPath.Tiled
        assert fh.choose(512, kind, 896, 4864) == fh.QPath.Tiled


def test_device_calls_without_a_device_fail_cleanly(fh):
    L = fh.lib()
    assert L.fh_device_sync(None) != 0
    assert b"no device" in L.fh_last_error()
    assert L.fh_linear_q(None, None, None, None, 1, 0) != 0
    h = ctypes.c_void_p()
    # Without a GPU, opening fails with a message rather than crashing; with one, it succeeds.
    st = L.fh_device_open(0, ctypes.byref(h))
    if st == 0:
        L.fh_device_close(h)
    else:
        assert L.fh_last_error()


def test_the_header_cites_the_reference_for_each_entry_point(fh):
    text = open(fh.HEADER).read()
    blocks = re.split(r"\n(?=FH_API )", text)
    # every section of declarations sits under a comment naming a reference file
    assert len(re.findall(r"\.rs:\d+", text)) >= 20
    assert "no counterpart in the reference" in text.lower()
    assert len(blocks) > 40
