"""Python host mirror of ferrum_wgpu's quantized-weight API over libferrum_hip (the C ABI in
include/ferrum_hip.h).

Names, argument meanings and error texts follow the reference's `ops_quant` / `ops_qat` modules
(ferrum_wgpu/src/ops/quant.rs, ferrum_wgpu/src/ops/qat.rs) and the slice of the device layer
they use (`Gpu`, `GpuBuf`; ferrum_wgpu/src/device/). Every call goes through the native
library; there is no fallback: if the library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes
import enum
import os
from typing import Callable, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libferrum_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(HERE)), "include", "ferrum_hip.h")

QK = 32
QK_K = 256


class GpuError(RuntimeError):
    """ferrum_wgpu::device::GpuError: a message tests match by substring."""


class QKind(enum.IntEnum):
    """ferrum_wgpu/src/ops/quant.rs:27-121, by ggml type id (FP8 has none: 1024 and 1025 are this
    library's ids). Q8_0 and Q4_0 run on the tiled planes and the MFMA kernels; F16, Fp4 (MXFP4),
    the FP8 formats and Q2K stay as GGUF rows and are decoded on the fly."""
    F16 = 1
    Q4_0 = 2
    Q8_0 = 8
    Q2K = 10
    Fp4 = 39
    Fp8E4M3 = 1024
    Fp8E5M2 = 1025

    def label(self) -> str:
        return {QKind.Q8_0: "Q8_0", QKind.Q4_0: "Q4_0", QKind.F16: "F16", QKind.Fp4: "MXFP4",
                QKind.Fp8E4M3: "FP8 E4M3", QKind.Fp8E5M2: "FP8 E5M2", QKind.Q2K: "Q2_K"}[self]

    def elems(self) -> int:
        """Elements per block along the input axis."""
        return QK_K if self == QKind.Q2K else QK

    def file_bytes(self) -> int:
        """Bytes of one block in a GGUF file (the FP8 formats use Q8_0's layout)."""
        return {QKind.Q8_0: 34, QKind.Q4_0: 18, QKind.F16: 64, QKind.Fp4: 17, QKind.Fp8E4M3: 34,
                QKind.Fp8E5M2: 34, QKind.Q2K: 84}[self]

    def ggml(self):
        """The GGUF tensor type, None for the FP8 formats (llama.cpp has none)."""
        return None if self in (QKind.Fp8E4M3, QKind.Fp8E5M2) else int(self)


class QPath(enum.IntEnum):
    """ferrum_wgpu/src/ops/quant.rs:292-305. Tiled is the MFMA dequant-GEMM here (within the
    reference's 1e-5); TiledFast (no counterpart in the reference) is the scoring GEMM with an fp8
    correction, within the MFMA-GEMM tolerance |g - w| <= 1e-3 + 2e-3 |w|; TiledF16 (no
    counterpart either) dequantises the weights to f16 and runs plain f16 MFMA: it rounds both
    operands to f16 and does not meet that tolerance on every output (measured: 5.4e-5 of Q4_0
    and 1.1e-4 of Q8_0 outputs outside it at M = 4096, the worst at twice the bound); Rows (no
    counterpart either) is the few-row kernel for 1 to 64 rows, within the reference's 1e-5."""
    Auto = 0
    Naive = 1
    Gemv = 2
    Tiled = 3
    TiledFast = 4
    TiledF16 = 5
    Rows = 6


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `make -C {os.path.dirname(HERE)}` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    L = ctypes.CDLL(LIB_PATH)
    P, S, I, U64, I64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64, ctypes.c_int64
    U32 = ctypes.c_uint32
    PP = ctypes.POINTER(ctypes.c_void_p)
    sigs = {
        "fh_last_error": (ctypes.c_char_p, []),
        "fh_abi_version": (I, []),
        "fh_device_open": (I, [I, PP]),
        "fh_device_close": (None, [P]),
        "fh_device_sync": (I, [P]),
        "fh_device_info": (I, [P, ctypes.c_char_p, S, ctypes.POINTER(I)]),
        "fh_device_stream": (P, [P]),
        "fh_debug_fail_after": (None, [P, I64]),
        "fh_debug_commands": (U64, [P]),
        "fh_buffer_zeros": (I, [P, S, PP]),
        "fh_buffer_upload": (I, [P, P, S, PP]),
        "fh_buffer_read": (I, [P, P, P, S]),
        "fh_buffer_write": (I, [P, P, P, S]),
        "fh_bytes_zeros": (I, [P, S, PP]),
        "fh_bytes_upload": (I, [P, P, S, PP]),
        "fh_bytes_read": (I, [P, P, P, S]),
        "fh_buffer_len": (S, [P]),
        "fh_buffer_nbytes": (S, [P]),
        "fh_buffer_device_ptr": (P, [P]),
        "fh_buffer_free": (None, [P]),
        "fh_copy_f32": (I, [P, P, S, P, S, S]),
        "fh_nbytes": (S, [I, S]),
        "fh_encode": (I, [P, I, P, S, P]),
        "fh_decode": (I, [P, I, P, S, P]),
        "fh_qweight_upload_gguf": (I, [P, I, P, S, S, S, PP]),
        "fh_qweight_upload_f32": (I, [P, I, P, S, S, PP]),
        "fh_qweight_quantise": (I, [P, I, P, S, S, PP]),
        "fh_qweight_free": (None, [P]),
        "fh_qweight_kind": (I, [P]),
        "fh_qweight_k": (S, [P]),
        "fh_qweight_n": (S, [P]),
        "fh_qweight_device_bytes": (U64, [P]),
        "fh_qweight_read_gguf": (I, [P, P, P, S]),
        "fh_qweight_dequantise": (I, [P, P, P]),
        "fh_choose": (I, [S, I, S, S]),
        "fh_linear_q": (I, [P, P, P, P, S, I]),
        "fh_linear_q_ptr": (I, [P, P, P, P, S, I]),
        "fh_linear_q_noalloc": (I, [P, P, P, P, S, I]),
        "fh_gemv_plan_create": (I, [P, P, S, PP]),
        "fh_gemv_plan_run": (I, [P, P]),
        "fh_gemv_plan_run_launch": (I, [P, P, S]),
        "fh_gemv_plan_launches": (S, [P]),
        "fh_gemv_plan_bytes": (U64, [P]),
        "fh_gemv_plan_free": (None, [P]),
        "fh_rows_plan_create": (I, [P, P, S, PP]),
        "fh_rows_plan_run": (I, [P, P]),
        "fh_rows_plan_launches": (S, [P]),
        "fh_rows_plan_bytes": (U64, [P]),
        "fh_rows_plan_free": (None, [P]),
        "fh_snap_plan_create": (I, [P, P, S, PP]),
        "fh_snap_plan_run": (I, [P, P]),
        "fh_snap_plan_bytes": (U64, [P]),
        "fh_snap_plan_free": (None, [P]),
        "fh_q8_snap_rows": (I, [P, P, P, S]),
        "fh_q8_snap_cols": (I, [P, P, P, S, S]),
        "fh_ggml_nbytes": (I, [U32, U64, ctypes.POINTER(U64)]),
        "fh_gguf_parse": (I, [P, S, PP]),
        "fh_gguf_parse_prefix": (I, [P, S, U64, PP]),
        "fh_gguf_open": (I, [ctypes.c_char_p, PP]),
        "fh_gguf_close": (None, [P]),
        "fh_gguf_describe": (S, [P, ctypes.c_char_p, S]),
        "fh_gguf_kv_count": (S, [P]),
        "fh_gguf_kv_key": (I, [P, S, PP, ctypes.POINTER(S)]),
        "fh_gguf_kv_value": (I, [P, S, ctypes.POINTER(U32), PP, ctypes.POINTER(S)]),
        "fh_gguf_kv_array": (I, [P, S, ctypes.POINTER(U32), ctypes.POINTER(U64)]),
        "fh_gguf_kv_array_string": (I, [P, S, U64, PP, ctypes.POINTER(S)]),
        "fh_gguf_find_key": (I, [P, ctypes.c_char_p, ctypes.POINTER(S)]),
        "fh_gguf_get_uint": (I, [P, ctypes.c_char_p, ctypes.POINTER(U64)]),
        "fh_gguf_get_float": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
        "fh_gguf_get_string": (I, [P, ctypes.c_char_p, PP, ctypes.POINTER(S)]),
        "fh_gguf_tensor_count": (S, [P]),
        "fh_gguf_tensor_info": (I, [P, S, P]),
        "fh_gguf_find_tensor": (I, [P, ctypes.c_char_p, ctypes.POINTER(S)]),
        "fh_gguf_tensor_bytes": (I, [P, ctypes.c_char_p, PP, ctypes.POINTER(S)]),
        "fh_gguf_data_offset": (U64, [P]),
        "fh_gguf_upload_qweight": (I, [P, P, ctypes.c_char_p, PP]),
        "fh_gguf_upload_f32": (I, [P, P, ctypes.c_char_p, PP]),
        "fh_gpt2_from_gguf": (I, [P, P, PP]),
        "fh_gpt2_free": (None, [P]),
        "fh_gpt2_config": (I, [P] + [ctypes.POINTER(S)] * 6),
        "fh_gpt2_kind": (I, [P]),
        "fh_gpt2_pos": (S, [P]),
        "fh_gpt2_reset": (None, [P]),
        "fh_gpt2_step_bytes": (U64, [P]),
        "fh_gpt2_step_launches": (S, [P]),
        "fh_gpt2_feed": (I, [P, P, S, P]),
        "fh_gpt2_generate": (I, [P, P, P, S, S, P]),
        "fh_llama_from_gguf": (I, [P, P, I, PP]),
        "fh_llama_free": (None, [P]),
        "fh_llama_config": (I, [P, P]),
        "fh_llama_weight_bytes": (U64, [P]),
        "fh_llama_device_bytes": (U64, [P]),
        "fh_llama_forward_all": (I, [P, P, P, S, P]),
        "fh_llama_score": (I, [P, P, P, S, P, P]),
        "fh_llama_score_device": (I, [P, P, P, S, P]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if L.fh_abi_version() != 1:
        raise RuntimeError("libferrum_hip ABI version mismatch")
    _lib = L
    return L


def exported_symbols() -> list[str]:
    """Names the header declares (every one must resolve in the library)."""
    import re
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^FH_API [^(]*?\b(fh_\w+)\(", text, re.M)))


def _check(status: int) -> None:
    if status != 0:
        raise GpuError(lib().fh_last_error().decode("utf-8", "replace"))


def _np(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class GpuBuf:
    """ferrum_wgpu::tensor::GpuBuf (f32 elements), or a byte buffer for packed blocks."""

    def __init__(self, gpu: "Gpu", handle: ctypes.c_void_p):
        self.gpu, self._h = gpu, handle

    @property
    def handle(self):
        return self._h

    def len(self) -> int:
        return lib().fh_buffer_len(self._h)

    def __len__(self) -> int:
        return self.len()

    def nbytes(self) -> int:
        return lib().fh_buffer_nbytes(self._h)

    def device_ptr(self) -> int:
        return lib().fh_buffer_device_ptr(self._h)

    def free(self) -> None:
        if self._h:
            lib().fh_buffer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    """ferrum_wgpu::device::Gpu, reduced to what the quantized path uses."""

    def __init__(self, ordinal: int = 0):
        h = ctypes.c_void_p()
        _check(lib().fh_device_open(ordinal, ctypes.byref(h)))
        self._h = h

    @staticmethod
    def open_for_test() -> Optional["Gpu"]:
        """device/mod.rs:192-201: a device, or None (with the reason printed) when there is none."""
        try:
            return Gpu(int(os.environ.get("FERRUM_HIP_DEVICE", "0")))
        except (GpuError, RuntimeError) as e:
            print(f"no GPU for this test: {e}")
            return None

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            lib().fh_device_close(self._h)
            self._h = None

    def info(self) -> tuple[str, int]:
        name = ctypes.create_string_buffer(256)
        cus = ctypes.c_int()
        _check(lib().fh_device_info(self._h, name, 256, ctypes.byref(cus)))
        return name.value.decode(), cus.value

    def stream(self) -> int:
        return lib().fh_device_stream(self._h)

    def sync(self) -> None:
        _check(lib().fh_device_sync(self._h))

    def zeros(self, n: int) -> GpuBuf:
        h = ctypes.c_void_p()
        _check(lib().fh_buffer_zeros(self._h, n, ctypes.byref(h)))
        return GpuBuf(self, h)

    def upload(self, data) -> GpuBuf:
        a = _np(data).reshape(-1)
        h = ctypes.c_void_p()
        _check(lib().fh_buffer_upload(self._h, _ptr(a), a.size, ctypes.byref(h)))
        return GpuBuf(self, h)

    def write(self, buf: GpuBuf, data) -> None:
        a = _np(data).reshape(-1)
        _check(lib().fh_buffer_write(self._h, buf.handle, _ptr(a), a.size))

    def read(self, buf: GpuBuf) -> np.ndarray:
        out = np.empty(buf.len(), np.float32)
        _check(lib().fh_buffer_read(self._h, buf.handle, _ptr(out), out.size))
        return out

    def bytes_zeros(self, nbytes: int) -> GpuBuf:
        h = ctypes.c_void_p()
        _check(lib().fh_bytes_zeros(self._h, nbytes, ctypes.byref(h)))
        return GpuBuf(self, h)

    def upload_bytes(self, data) -> GpuBuf:
        a = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        h = ctypes.c_void_p()
        _check(lib().fh_bytes_upload(self._h, _ptr(a), a.size, ctypes.byref(h)))
        return GpuBuf(self, h)

    def read_bytes(self, buf: GpuBuf) -> np.ndarray:
        out = np.empty(buf.nbytes(), np.uint8)
        _check(lib().fh_bytes_read(self._h, buf.handle, _ptr(out), out.size))
        return out

    def copy_f32(self, src: GpuBuf, src_off: int, dst: GpuBuf, dst_off: int, n: int) -> None:
        _check(lib().fh_copy_f32(self._h, src.handle, src_off, dst.handle, dst_off, n))

    # ---- test hooks (device/runtime.rs:218-256) ----
    def fail_after(self, n: Optional[int]) -> None:
        lib().fh_debug_fail_after(self._h, -1 if n is None else n)

    def commands(self) -> int:
        return lib().fh_debug_commands(self._h)

    def sweep_faults(self, f: Callable[[], None]) -> int:
        """Fail command 0, then 1, ... until `f` succeeds; every failure must be the injected
        fault. Returns how many commands `f` issues."""
        for k in range(100_000):
            self.fail_after(k)
            try:
                f()
            except GpuError as e:
                assert "injected fault" in str(e), f"command {k}: {e}"
                continue
            self.fail_after(None)
            return k
        raise AssertionError("the operation never succeeded")

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class QWeight:
    """ferrum_wgpu/src/ops/quant.rs:155-182: a resident quantized weight (GGUF rows)."""

    def __init__(self, gpu: Gpu, handle):
        self.gpu, self._h = gpu, handle

    @property
    def handle(self):
        return self._h

    def kind(self) -> QKind:
        return QKind(lib().fh_qweight_kind(self._h))

    def k(self) -> int:
        return lib().fh_qweight_k(self._h)

    def n(self) -> int:
        return lib().fh_qweight_n(self._h)

    def device_bytes(self) -> int:
        return lib().fh_qweight_device_bytes(self._h)

    def gguf_bytes(self) -> int:
        """Bytes of the weight's GGUF rows."""
        return nbytes(self.kind(), self.k() * self.n())

    def read_gguf(self) -> np.ndarray:
        out = np.empty(self.gguf_bytes(), np.uint8)
        _check(lib().fh_qweight_read_gguf(self.gpu.handle, self._h, _ptr(out), out.size))
        return out

    def dequantised(self) -> np.ndarray:
        """The [k, n] f32 weight the CPU path multiplies by, dequantised on the device."""
        out = self.gpu.zeros(self.k() * self.n())
        _check(lib().fh_qweight_dequantise(self.gpu.handle, self._h, out.handle))
        return self.gpu.read(out)

    def free(self) -> None:
        if self._h:
            lib().fh_qweight_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def eligible(k: int) -> bool:
    """quant.rs:125-129"""
    return k > 0 and k % QK == 0


def eligible_for(kind: QKind, k: int) -> bool:
    """quant.rs:131-134"""
    return k > 0 and k % QKind(kind).elems() == 0


def effective(kind: QKind, k: int) -> QKind:
    """quant.rs:136-145: Q2_K needs 256-wide blocks; a width of whole 32s uses Q4_0 instead."""
    if kind == QKind.Q2K and not eligible_for(kind, k) and eligible(k):
        return QKind.Q4_0
    return QKind(kind)


def nbytes(kind: QKind, n: int) -> int:
    """ferrum_gguf/src/codec/quant.rs:17-47"""
    r = lib().fh_nbytes(int(kind), n)
    if r == 0 and n != 0:
        raise GpuError(lib().fh_last_error().decode())
    return r


def upload_qweight(gpu: Gpu, kind: QKind, data, k: int, n: int) -> QWeight:
    """quant.rs:267-277: GGUF rows (n rows of k/elems blocks), resident bit-exact."""
    a = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    h = ctypes.c_void_p()
    _check(lib().fh_qweight_upload_gguf(gpu.handle, int(kind), _ptr(a), a.size, k, n, ctypes.byref(h)))
    return QWeight(gpu, h)


def upload_quantised(gpu: Gpu, kind: QKind, w, k: int, n: int) -> QWeight:
    """quant.rs:279-288: quantise an [in, out] f32 weight (on the device) and keep it resident."""
    a = _np(w).reshape(-1)
    if a.size != k * n:
        raise GpuError(f"cannot quantise {a.size} elements as a {k} x {n} weight in whole "
                       f"{QKind(kind).elems()}-blocks")
    h = ctypes.c_void_p()
    _check(lib().fh_qweight_upload_f32(gpu.handle, int(kind), _ptr(a), k, n, ctypes.byref(h)))
    return QWeight(gpu, h)


def quantise_matrix(gpu: Gpu, kind: QKind, w: GpuBuf, k: int, n: int) -> QWeight:
    """quant.rs:238-252 on the device, from a resident [k, n] f32 buffer."""
    h = ctypes.c_void_p()
    _check(lib().fh_qweight_quantise(gpu.handle, int(kind), w.handle, k, n, ctypes.byref(h)))
    return QWeight(gpu, h)


def encode(gpu: Gpu, kind: QKind, src: GpuBuf, n: int, dst: Optional[GpuBuf] = None) -> GpuBuf:
    """ferrum_gguf quant::encode on the device: n values -> GGUF blocks."""
    dst = dst or gpu.bytes_zeros(nbytes(kind, n))
    _check(lib().fh_encode(gpu.handle, int(kind), src.handle, n, dst.handle))
    return dst


def decode(gpu: Gpu, kind: QKind, src: GpuBuf, n: int, dst: Optional[GpuBuf] = None) -> GpuBuf:
    """ferrum_gguf quant::decode on the device: GGUF blocks -> n f32 values."""
    dst = dst or gpu.zeros(n)
    _check(lib().fh_decode(gpu.handle, int(kind), src.handle, n, dst.handle))
    return dst


def choose(rows: int, kind: QKind, k: int, n: int) -> QPath:
    """quant.rs:306-323, re-derived for MI355X."""
    return QPath(lib().fh_choose(rows, int(kind), k, n))


def linear_q(gpu: Gpu, x: GpuBuf, w: QWeight, y: GpuBuf, rows: int) -> None:
    """quant.rs:326-335: y[rows, n] = x[rows, k] * W (no bias)."""
    linear_q_with(gpu, x, w, y, rows, QPath.Auto)


def linear_q_with(gpu: Gpu, x: GpuBuf, w: QWeight, y: GpuBuf, rows: int, path: QPath) -> None:
    """quant.rs:337-381"""
    _check(lib().fh_linear_q(gpu.handle, x.handle, w.handle, y.handle, rows, int(path)))


def linear_q_ptr(gpu: Gpu, x_ptr: int, w: QWeight, y_ptr: int, rows: int, path: QPath = QPath.Auto) -> None:
    """linear_q on raw device pointers (e.g. torch tensors' data_ptr())."""
    _check(lib().fh_linear_q_ptr(gpu.handle, x_ptr, w.handle, y_ptr, rows, int(path)))


NOALLOC_SCRATCH_BYTES = 32 << 20  # FH_NOALLOC_SCRATCH_BYTES


def linear_q_noalloc(gpu: Gpu, x_ptr: int, w: QWeight, y_ptr: int, rows: int, path: QPath = QPath.Auto) -> None:
    """linear_q_ptr without any device allocation (no counterpart in the reference): scratch from
    the library's static per-GPU array; calls that overlap on one GPU race."""
    _check(lib().fh_linear_q_noalloc(gpu.handle, x_ptr, w.handle, y_ptr, rows, int(path)))


class _Problem(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p)]


class GemvPlan:
    """Many independent batch-1 products in one launch per (format, width class); no
    counterpart in the reference (which issues one linear_q per matrix)."""

    def __init__(self, gpu: Gpu, problems: Sequence[tuple[QWeight, int, int]]):
        arr = (_Problem * max(len(problems), 1))()
        for i, (w, xp, yp) in enumerate(problems):
            arr[i] = _Problem(w.handle.value if hasattr(w.handle, "value") else w.handle, xp, yp)
        self._keep = [p[0] for p in problems]
        self.gpu = gpu
        h = ctypes.c_void_p()
        _check(lib().fh_gemv_plan_create(gpu.handle, ctypes.cast(arr, ctypes.c_void_p), len(problems),
                                         ctypes.byref(h)))
        self._h = h

    def run(self) -> None:
        _check(lib().fh_gemv_plan_run(self.gpu.handle, self._h))

    def run_launch(self, i: int) -> None:
        """Launch i alone (launches must run in order: one may write the next one's prepared x)."""
        _check(lib().fh_gemv_plan_run_launch(self.gpu.handle, self._h, i))

    def launches(self) -> int:
        return lib().fh_gemv_plan_launches(self._h)

    def bytes(self) -> int:
        return lib().fh_gemv_plan_bytes(self._h)

    def free(self) -> None:
        if self._h:
            lib().fh_gemv_plan_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class _RowsProblem(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("x", ctypes.c_void_p), ("y", ctypes.c_void_p), ("rows", ctypes.c_size_t)]


class RowsPlan:
    """Many independent few-row products (1 to 64 rows each) in one launch pair per block format,
    on the QPath.Rows kernel; no counterpart in the reference (which issues one linear_q per
    matrix). problems: (weight, x device pointer, y device pointer, rows)."""

    def __init__(self, gpu: Gpu, problems: Sequence[tuple[QWeight, int, int, int]]):
        arr = (_RowsProblem * max(len(problems), 1))()
        for i, (w, xp, yp, rows) in enumerate(problems):
            arr[i] = _RowsProblem(w.handle.value if hasattr(w.handle, "value") else w.handle, xp, yp, rows)
        self._keep = [p[0] for p in problems]
        self.gpu = gpu
        h = ctypes.c_void_p()
        _check(lib().fh_rows_plan_create(gpu.handle, ctypes.cast(arr, ctypes.c_void_p), len(problems),
                                         ctypes.byref(h)))
        self._h = h

    def run(self) -> None:
        _check(lib().fh_rows_plan_run(self.gpu.handle, self._h))

    def launches(self) -> int:
        return lib().fh_rows_plan_launches(self._h)

    def bytes(self) -> int:
        return lib().fh_rows_plan_bytes(self._h)

    def free(self) -> None:
        if self._h:
            lib().fh_rows_plan_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


SNAP_ROWS, SNAP_COLS, SNAP_COPY = 0, 1, 2


class _SnapProblem(ctypes.Structure):
    _fields_ = [("src", ctypes.c_void_p), ("dst", ctypes.c_void_p), ("len", ctypes.c_size_t), ("a", ctypes.c_size_t),
                ("b", ctypes.c_size_t), ("mode", ctypes.c_int)]


class SnapPlan:
    """A whole QAT snap pass in one launch (GpuTrainer::record_snap's loop of q8_snap_rows /
    q8_snap_cols / copy calls, ferrum_wgpu/src/training/gpt2/qat.rs:58-72). problems: (mode,
    src, dst, shape), src and dst GpuBufs of one length; shape is ne0 for SNAP_ROWS,
    (rows_in, cols_out) for SNAP_COLS and ignored for SNAP_COPY; the single calls' fallbacks
    apply. No counterpart in the reference as one launch."""

    def __init__(self, gpu: Gpu, problems):
        arr = (_SnapProblem * max(len(problems), 1))()
        self._keep = []
        for i, (mode, src, dst, shape) in enumerate(problems):
            n = src.len()
            if dst.len() != n:
                raise GpuError(f"snap plan: problem {i}: source holds {n} elements but destination {dst.len()}")
            self._keep += [src, dst]
            if mode == SNAP_COLS:
                a, b = shape
            elif mode == SNAP_ROWS:
                a, b = shape, 0
            else:
                a, b = 0, 0
            arr[i] = _SnapProblem(src.device_ptr(), dst.device_ptr(), n, a, b, mode)
        self.gpu = gpu
        h = ctypes.c_void_p()
        _check(lib().fh_snap_plan_create(gpu.handle, ctypes.cast(arr, ctypes.c_void_p), len(problems), ctypes.byref(h)))
        self._h = h

    def run(self) -> None:
        _check(lib().fh_snap_plan_run(self.gpu.handle, self._h))

    def bytes(self) -> int:
        return lib().fh_snap_plan_bytes(self._h)

    def free(self) -> None:
        if self._h:
            lib().fh_snap_plan_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def q8_snap_rows(gpu: Gpu, src: GpuBuf, dst: GpuBuf, ne0: int) -> None:
    """ferrum_wgpu/src/ops/qat.rs:21-29"""
    _check(lib().fh_q8_snap_rows(gpu.handle, src.handle, dst.handle, ne0))


def q8_snap_cols(gpu: Gpu, src: GpuBuf, dst: GpuBuf, shape: tuple[int, int]) -> None:
    """ferrum_wgpu/src/ops/qat.rs:33-57"""
    rows_in, cols_out = shape
    _check(lib().fh_q8_snap_cols(gpu.handle, src.handle, dst.handle, rows_in, cols_out))
