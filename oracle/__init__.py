"""ctypes bindings for the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, always as the checker or the timed CPU baseline, never by
the product path. Build with ``make -C oracle``.

Each wrapper names the reference function it restates; see ``oracle.h`` for file:line.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, MXFP4 = 3, 6, 7, 9, 10, 11, 12, 13, 14, 39
FP8_E4M3, FP8_E5M2 = 1024, 1025  # no ggml type (ferrum_wgpu/src/ops/quant.rs:38-41); the oracle's own ids
QK, QK_K = 32, 256
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18, F16: 64, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_1: 36, Q2_K: 84, Q3_K: 110, Q4_K: 144,
               Q5_K: 176, Q6_K: 210, MXFP4: 17, FP8_E4M3: 34, FP8_E5M2: 34}
BLOCK_ELEMS = {t: (QK_K if t in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) else QK) for t in BLOCK_BYTES}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: run `make -C {HERE}`")
        L = ctypes.CDLL(LIB_PATH)
        P, S, U32, U64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64
        sig = {
            "fo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "fo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "fo_nbytes": (ctypes.c_int64, [U32, S]),
            "fo_decode": (ctypes.c_int, [U32, P, S, S, P]),
            "fo_encode": (ctypes.c_int, [U32, P, S, P]),
            "fo_transpose": (None, [P, S, S, P]),
            "fo_quantise_matrix": (ctypes.c_int, [U32, P, S, S, P]),
            "fo_snap_block": (None, [P, P]),
            "fo_snap_rows": (None, [P, S, S]),
            "fo_snap_cols": (None, [P, S, S]),
            "fo_matmul": (ctypes.c_int, [P, P, S, S, S, P]),
            "fo_matmul_threaded": (ctypes.c_int, [P, P, S, S, S, ctypes.c_int, P]),
            "fo_matmul_tuned": (ctypes.c_int, [P, P, S, S, S, ctypes.c_int, P]),
            "fo_gemv": (None, [P, P, P, S, S, P]),
            "fo_rand_vec": (None, [S, U64, P]),
            "fo_max_rel_err": (ctypes.c_float, [P, P, S]),
            "fo_gelu": (ctypes.c_float, [ctypes.c_float]),
            "fo_layernorm": (None, [P, P, P, S, P]),
            "fo_argmax": (S, [P, S]),
            "fo_gpt2_generate": (ctypes.c_int, [P, P, S, S, P]),
            "fo_gpt2_cache_new": (P, [P]),
            "fo_gpt2_cache_free": (None, [P, P]),
            "fo_gpt2_feed": (ctypes.c_int, [P, P, S, P]),
            "fo_layout": (ctypes.c_int, [U32, P, P]),
            "fo_dequant": (ctypes.c_int, [U32, P, S, P]),
            "fo_fp8_decode": (ctypes.c_float, [ctypes.c_int, ctypes.c_uint8]),
            "fo_fp8_encode": (ctypes.c_uint8, [ctypes.c_int, ctypes.c_float]),
            "fo_mxfp4_half_scale": (ctypes.c_float, [ctypes.c_uint8]),
            "fo_q2k_nearest_int": (ctypes.c_int32, [ctypes.c_float]),
            "fo_q2k_fit": (None, [P, P, P, P]),
            "fo_rope_tables": (None, [S, S, S, ctypes.c_float, P, ctypes.c_float, P, P]),
            "fo_rmsnorm": (None, [P, P, S, S, ctypes.c_float, P]),
            "fo_apply_rope": (None, [P, S, S, S, S, P, P, ctypes.c_int]),
            "fo_attend_row": (None, [P, P, P, S, S, S, S, P, P]),
            "fo_silu": (ctypes.c_float, [ctypes.c_float]),
            "fo_swiglu": (None, [P, P, S, P]),
            "fo_score": (None, [P, P, S, S, P, P]),
            "fo_llama_forward": (ctypes.c_int, [P, P, S, ctypes.c_int, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def f16_to_f32(h: int) -> float:
    """ferrum_gguf/src/codec/f16.rs:4-22"""
    return lib().fo_f16_to_f32(h)


def f32_to_f16(x: float) -> int:
    """ferrum_gguf/src/codec/f16.rs:25-53"""
    return lib().fo_f32_to_f16(x)


def f16_to_f32_array(h: np.ndarray) -> np.ndarray:
    """Element-wise :func:`f16_to_f32` (via the codec's F16 decode)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return decode(F16, h.view(np.uint8), h.size)


def f32_to_f16_array(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    return encode(F16, x).view(np.uint16)


def nbytes(ty: int, n: int) -> int:
    """ferrum_gguf/src/codec/quant.rs:17-47 (-1 for an error)."""
    return lib().fo_nbytes(ty, n)


def decode(ty: int, data: np.ndarray, n: int) -> np.ndarray:
    """ferrum_gguf/src/codec/quant.rs:50-88"""
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(n, np.float32)
    if lib().fo_decode(ty, _p(data), data.size, n, _p(out)) != 0:
        raise ValueError("tensor byte length does not match its type and element count")
    return out


def encode(ty: int, data) -> np.ndarray:
    """ferrum_gguf/src/codec/quant.rs:91-136 (q2k.rs, mxfp4.rs, fp8.rs for those formats)."""
    data = _f32(data)
    nb = nbytes(ty, data.size)
    if nb < 0:
        raise ValueError(f"{data.size} elements is not a multiple of the block size {BLOCK_ELEMS.get(ty, QK)}")
    out = np.empty(nb, np.uint8)
    rc = lib().fo_encode(ty, _p(data), data.size, _p(out))
    if rc == -2:
        raise ValueError(f"tensor type {ty} is read-only: it can be loaded but not written")
    if rc != 0:
        raise ValueError("encode failed")
    return out


def transpose(a, rows: int, cols: int) -> np.ndarray:
    """ferrum_ref/src/models/llama/params.rs:24-32"""
    a = _f32(a)
    out = np.empty(rows * cols, np.float32)
    lib().fo_transpose(_p(a), rows, cols, _p(out))
    return out


def quantise_matrix(ty: int, w, k: int, n: int) -> np.ndarray:
    """ferrum_wgpu/src/ops/quant.rs:238-252: [k, n] f32 -> GGUF rows [n][k/elems]."""
    w = _f32(w)
    e = BLOCK_ELEMS.get(ty, QK)
    if k == 0 or k % e or w.size != k * n:
        raise ValueError(f"cannot quantise {w.size} elements as a {k} x {n} weight in whole {e}-blocks")
    out = np.empty(n * (k // e) * BLOCK_BYTES[ty], np.uint8)
    if lib().fo_quantise_matrix(ty, _p(w), k, n, _p(out)) != 0:
        raise ValueError("quantise failed")
    return out


def dequantise_bytes(ty: int, data, n: int) -> np.ndarray:
    """ferrum_wgpu/src/ops/quant.rs:256-264"""
    return decode(ty, data, n)


def dequantised_in_out(ty: int, data, k: int, n: int) -> np.ndarray:
    """The [k, n] f32 weight the reference's CPU path multiplies by: transpose(decode(bytes))
    (ferrum_wgpu/src/models/llama/mod.rs:188-200; ops/quant/tests.rs:27-29,143)."""
    return transpose(decode(ty, data, k * n), n, k)


def snap_block(block) -> np.ndarray:
    """ferrum_ref/src/training/qat.rs:20-24"""
    block = _f32(block)
    out = np.empty(32, np.float32)
    lib().fo_snap_block(_p(block), _p(out))
    return out


def snap_rows(data, ne0: int) -> np.ndarray:
    """ferrum_ref/src/training/qat.rs:27-35 (returns a snapped copy)."""
    d = _f32(data).copy()
    lib().fo_snap_rows(_p(d), d.size, ne0)
    return d


def snap_cols(data, rows_in: int, cols_out: int) -> np.ndarray:
    """ferrum_ref/src/training/qat.rs:38-54 (returns a snapped copy)."""
    d = _f32(data).copy()
    lib().fo_snap_cols(_p(d), rows_in, cols_out)
    return d


def matmul(a, b, m: int, k: int, n: int) -> np.ndarray:
    """ferrum_ref/src/kernels/matmul.rs:62-69"""
    a, b = _f32(a), _f32(b)
    assert a.size == m * k and b.size == k * n
    out = np.empty(m * n, np.float32)
    lib().fo_matmul(_p(a), _p(b), m, k, n, _p(out))
    return out


def matmul_threaded(a, b, m: int, k: int, n: int, threads: int) -> np.ndarray:
    """ferrum_ref/src/kernels/matmul.rs:73-94"""
    a, b = _f32(a), _f32(b)
    out = np.empty(m * n, np.float32)
    lib().fo_matmul_threaded(_p(a), _p(b), m, k, n, threads, _p(out))
    return out


def matmul_tuned(a, b, m: int, k: int, n: int, threads: int) -> np.ndarray:
    """ferrum_ref/src/kernels/tuned.rs:99-134"""
    a, b = _f32(a), _f32(b)
    out = np.empty(m * n, np.float32)
    lib().fo_matmul_tuned(_p(a), _p(b), m, k, n, threads, _p(out))
    return out


def gemv(x, w, bias, k: int, n: int) -> np.ndarray:
    """ferrum_ref/src/models/gpt2/decode.rs:42-53 (w is [k, n])."""
    x, w = _f32(x), _f32(w)
    b = None if bias is None else _f32(bias)
    y = np.empty(n, np.float32)
    lib().fo_gemv(_p(x), _p(w), None if b is None else _p(b), k, n, _p(y))
    return y


def rand_vec(length: int, seed: int) -> np.ndarray:
    """ferrum_ref/src/kernels/matmul.rs:97-107"""
    out = np.empty(length, np.float32)
    lib().fo_rand_vec(length, seed, _p(out))
    return out


def max_rel_err(got, want) -> float:
    """ferrum_wgpu/src/tolerance.rs:14-26"""
    got, want = _f32(got), _f32(want)
    if got.size != want.size:
        return float("inf")
    return lib().fo_max_rel_err(_p(got), _p(want), got.size)


def gelu(x: float) -> float:
    """ferrum_ref/src/kernels/nn.rs:12-15"""
    return lib().fo_gelu(x)


def layernorm(x, g, b) -> np.ndarray:
    """ferrum_ref/src/kernels/nn.rs:31-44 (one row)."""
    x, g, b = _f32(x), _f32(g), _f32(b)
    y = np.empty_like(x)
    lib().fo_layernorm(_p(x), _p(g), _p(b), x.size, _p(y))
    return y


def argmax(v) -> int:
    """ferrum_model/src/sampling.rs:32-40"""
    v = _f32(v)
    return lib().fo_argmax(_p(v), v.size)


class _Gpt2(ctypes.Structure):
    _fields_ = [
        ("vocab", ctypes.c_size_t), ("ctx", ctypes.c_size_t), ("dim", ctypes.c_size_t),
        ("heads", ctypes.c_size_t), ("layers", ctypes.c_size_t), ("hidden", ctypes.c_size_t),
        ("tok", ctypes.c_void_p), ("pos", ctypes.c_void_p), ("blocks", ctypes.c_void_p),
        ("lnf_g", ctypes.c_void_p), ("lnf_b", ctypes.c_void_p), ("head", ctypes.c_void_p),
    ]


# Per-block tensor order of the reference (ferrum_ref/src/models/gpt2/mod.rs:57-90).
GPT2_BLOCK_NAMES = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                    "ln2_g", "ln2_b", "w1", "b1", "w2", "b2")


def _gpt2_struct(model: dict, keep: list):
    def ptr(a):
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data

    blocks = (ctypes.c_void_p * (model["layers"] * 16))()
    keep.append(blocks)
    for l, blk in enumerate(model["blocks"]):
        for i, name in enumerate(GPT2_BLOCK_NAMES):
            blocks[l * 16 + i] = ptr(blk[name])
    g = _Gpt2(model["vocab"], model["ctx"], model["dim"], model["heads"], model["layers"],
              model["hidden"], ptr(model["tok"]), ptr(model["pos"]),
              ctypes.cast(blocks, ctypes.c_void_p), ptr(model["lnf_g"]), ptr(model["lnf_b"]),
              ptr(model["head"]))
    keep.append(g)
    return g


class Gpt2Cpu:
    """Gpt2::feed with its Cache (ferrum_ref/src/models/gpt2/decode.rs:7-117): one token at a
    time, the next-token logits back."""

    def __init__(self, model: dict):
        self._keep = []
        self._g = _gpt2_struct(model, self._keep)
        self.vocab = model["vocab"]
        self._c = lib().fo_gpt2_cache_new(ctypes.byref(self._g))

    def feed(self, token: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        if lib().fo_gpt2_feed(ctypes.byref(self._g), self._c, int(token), _p(out)) != 0:
            raise ValueError("context full or token out of range")
        return out

    def __del__(self):
        try:
            lib().fo_gpt2_cache_free(ctypes.byref(self._g), self._c)
        except Exception:
            pass


def gpt2_generate(model: dict, prompt, n_new: int) -> list[int]:
    """Greedy cached decode (ferrum_ref/src/models/gpt2/decode.rs:57-117 per token).

    ``model`` holds cfg ints (vocab, ctx, dim, heads, layers, hidden) and f32 arrays ``tok``,
    ``pos``, ``blocks`` (list of dicts keyed by GPT2_BLOCK_NAMES), ``lnf_g``, ``lnf_b``, ``head``.
    """
    keep = []
    g = _gpt2_struct(model, keep)
    pr = np.ascontiguousarray(prompt, dtype=np.uint64)
    out = np.zeros(max(n_new, 1), np.uint64)
    rc = lib().fo_gpt2_generate(ctypes.byref(g), _p(pr), pr.size, n_new, _p(out))
    if rc != 0:
        raise ValueError("gpt2 generate failed (context full or token out of range)")
    return [int(t) for t in out[:n_new]]


# ---- Llama / Qwen2 (oracle/llama.c) ----

# Per-block tensor order of the reference (ferrum_ref/src/models/llama/mod.rs:99-128).
LLAMA_BLOCK_NAMES = ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "ffn_norm", "gate", "up", "down")


def rope_tables(start: int, n: int, rope_dim: int, base: float, freq_factors=None, linear_factor=1.0):
    """ferrum_ref/src/models/llama/ops.rs:78-101: (cos, sin), each [n, rope_dim/2]."""
    half = rope_dim // 2
    c, s = np.empty(n * half, np.float32), np.empty(n * half, np.float32)
    ff = None if freq_factors is None or len(freq_factors) == 0 else _f32(freq_factors)
    lib().fo_rope_tables(start, n, rope_dim, base, None if ff is None else _p(ff), linear_factor, _p(c), _p(s))
    return c, s


def rmsnorm(x, g, rows: int, cols: int, eps: float) -> np.ndarray:
    """ferrum_ref/src/models/llama/ops.rs:55-66"""
    x, g = _f32(x), _f32(g)
    y = np.empty(rows * cols, np.float32)
    lib().fo_rmsnorm(_p(x), _p(g), rows, cols, eps, _p(y))
    return y


def apply_rope(x, rows: int, heads: int, hd: int, rope_dim: int, cos, sin, neox: bool) -> np.ndarray:
    """ferrum_ref/src/models/llama/ops.rs:105-127 (returns a rotated copy)."""
    y = _f32(x).copy()
    c, s = _f32(cos), _f32(sin)
    lib().fo_apply_rope(_p(y), rows, heads, hd, rope_dim, _p(c), _p(s), int(bool(neox)))
    return y


def attend_row(q, k, v, length: int, heads: int, kv_heads: int, hd: int) -> np.ndarray:
    """ferrum_ref/src/models/llama/ops.rs:131-162"""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty(heads * hd, np.float32)
    scratch = np.empty(max(length, 1), np.float32)
    lib().fo_attend_row(_p(q), _p(k), _p(v), length, heads, kv_heads, hd, _p(scratch), _p(out))
    return out


def silu(x: float) -> float:
    """ferrum_ref/src/models/llama/ops.rs:69-71"""
    return lib().fo_silu(x)


def swiglu(gate, up) -> np.ndarray:
    """ferrum_ref/src/models/llama/ops.rs:74-76"""
    g, u = _f32(gate), _f32(up)
    out = np.empty(g.size, np.float32)
    lib().fo_swiglu(_p(g), _p(u), g.size, _p(out))
    return out


def score(logits, targets, vocab: int):
    """ferrum_ref/src/kernels/nn.rs:117-129: per row (log-probability of the target, whether the
    target is the first maximum), as two arrays."""
    lg = _f32(logits)
    tg = np.ascontiguousarray(targets, dtype=np.uint64)
    rows = tg.size
    assert lg.size == rows * vocab
    lp = np.empty(rows, np.float32)
    hit = np.empty(rows, np.uint8)
    lib().fo_score(_p(lg), _p(tg), rows, vocab, _p(lp), _p(hit))
    return lp, hit.astype(bool)


class _Llama(ctypes.Structure):
    _fields_ = [
        ("vocab", ctypes.c_size_t), ("ctx", ctypes.c_size_t), ("dim", ctypes.c_size_t),
        ("heads", ctypes.c_size_t), ("kv_heads", ctypes.c_size_t), ("head_dim", ctypes.c_size_t),
        ("layers", ctypes.c_size_t), ("hidden", ctypes.c_size_t), ("rope_dim", ctypes.c_size_t),
        ("rope_base", ctypes.c_float), ("eps", ctypes.c_float), ("neox", ctypes.c_int),
        ("freq_factors", ctypes.c_void_p), ("linear_factor", ctypes.c_float),
        ("tok", ctypes.c_void_p), ("blocks", ctypes.c_void_p), ("out_norm", ctypes.c_void_p),
        ("head", ctypes.c_void_p),
    ]


def _llama_struct(m: dict, keep: list):
    def ptr(a):
        if a is None or len(a) == 0:
            return None
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data

    n = len(LLAMA_BLOCK_NAMES)
    blocks = (ctypes.c_void_p * (m["layers"] * n))()
    keep.append(blocks)
    for l, blk in enumerate(m["blocks"]):
        for i, name in enumerate(LLAMA_BLOCK_NAMES):
            blocks[l * n + i] = ptr(blk[name])
    g = _Llama(m["vocab"], m["ctx"], m["dim"], m["heads"], m["kv_heads"], m["head_dim"], m["layers"],
               m["hidden"], m["rope_dim"], m["rope_base"], m["eps"], int(bool(m["neox"])),
               ptr(m.get("freq_factors")), m.get("linear_factor", 1.0), ptr(m["tok"]),
               ctypes.cast(blocks, ctypes.c_void_p), ptr(m["out_norm"]), ptr(m["head"]))
    keep.append(g)
    return g


def llama_forward(m: dict, ids, threads: int = 1) -> np.ndarray:
    """Llama::forward_logits (ferrum_ref/src/models/llama/mod.rs:166-175,202-259): every
    position's logits, [len(ids), vocab]; bit-identical for any thread count."""
    keep = []
    g = _llama_struct(m, keep)
    ids = np.ascontiguousarray(ids, dtype=np.uint64)
    out = np.empty(max(ids.size, 1) * m["vocab"], np.float32)
    rc = lib().fo_llama_forward(ctypes.byref(g), _p(ids), ids.size, threads, _p(out))
    if rc == -1:
        raise ValueError(f"sequence length {ids.size} must be in 1..={m['ctx']} with tokens below {m['vocab']}")
    if rc != 0:
        raise MemoryError("llama forward: out of memory")
    return out[: ids.size * m["vocab"]].reshape(ids.size, m["vocab"])


def llama_score(m: dict, ids, threads: int = 1):
    """GpuLlama::score's oracle (ferrum_wgpu/src/models/llama/forward.rs:76-88 over
    forward_logits and nn::score): for each i < len - 1, the log-probability of ids[i + 1] after
    ids[..=i] and whether it is the first argmax."""
    if len(ids) < 2:
        raise ValueError("scoring needs at least 2 tokens")
    logits = llama_forward(m, ids[:-1], threads)
    return score(logits, ids[1:], m["vocab"])


# ---- formats beyond Q8_0 / Q4_0 (oracle/formats.c) ----

def fp8_decode(e5m2: bool, code: int) -> float:
    """ferrum_gguf/src/codec/fp8.rs:34-63"""
    return lib().fo_fp8_decode(int(e5m2), code)


def fp8_encode(e5m2: bool, x: float) -> int:
    """ferrum_gguf/src/codec/fp8.rs:65-96"""
    return lib().fo_fp8_encode(int(e5m2), x)


def mxfp4_half_scale(e: int) -> float:
    """ferrum_gguf/src/codec/mxfp4.rs:26-33"""
    return lib().fo_mxfp4_half_scale(e)


def q2k_fit(x16) -> tuple:
    """ferrum_gguf/src/codec/q2k.rs:24-93: (scale, negated min, levels) of one 16-value sub-block."""
    x = _f32(x16)
    if x.size != 16:
        raise ValueError("a Q2_K sub-block has 16 values")
    lv = np.empty(16, np.uint8)
    sc, mn = ctypes.c_float(), ctypes.c_float()
    lib().fo_q2k_fit(_p(x), _p(lv), ctypes.byref(sc), ctypes.byref(mn))
    return sc.value, mn.value, lv


def q2k_nearest_int(x: float) -> int:
    """ferrum_gguf/src/codec/q2k.rs:16-19"""
    return lib().fo_q2k_nearest_int(x)
