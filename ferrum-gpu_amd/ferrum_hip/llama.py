"""Python mirror of the batched passes of ferrum_wgpu's GpuLlama (ferrum_wgpu/src/models/llama/
forward.rs:13-88: forward_all and score) over libferrum_hip's fh_llama_* entry points
(include/ferrum_hip.h).

`forward_all` and `score` keep the reference's names, return shapes and error texts ("sequence
length N must be in 1..=ctx", "token T is out of range for vocab V", "scoring needs at least 2
tokens"). The model is built from a `llama` or `qwen2` GGUF whose matrices stay packed (Q8_0 or
Q4_0) on the device. `random_gguf` writes such a file with synthetic weights for benchmarks.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import Gpu, GpuBuf, GpuError, QKind, QPath, _check, encode, lib
from .gguf import F32, STR, U32, Gguf, GgufBuilder, Value


class _Cfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("vocab", "ctx", "dim", "heads", "kv_heads", "head_dim", "layers",
                                                 "hidden", "rope_dim")] + \
               [("rope_base", ctypes.c_float), ("eps", ctypes.c_float), ("linear_factor", ctypes.c_float),
                ("neox", ctypes.c_int), ("tied", ctypes.c_int), ("kind", ctypes.c_int), ("path", ctypes.c_int)]


@dataclass(frozen=True)
class Config:
    """ferrum_ref/src/models/llama/mod.rs:24-51, plus how the model is stored."""
    vocab: int
    ctx: int
    dim: int
    heads: int
    kv_heads: int
    head_dim: int
    layers: int
    hidden: int
    rope_dim: int
    rope_base: float
    eps: float
    linear_factor: float
    neox: bool
    tied: bool
    kind: QKind
    path: QPath

    def q_dim(self) -> int:
        return self.heads * self.head_dim

    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


class GpuLlama:
    """A resident quantized Llama / Qwen2 for full-sequence passes (no KV cache)."""

    def __init__(self, gpu: Gpu, handle):
        self.gpu, self._h = gpu, handle
        c = _Cfg()
        _check(lib().fh_llama_config(self._h, ctypes.byref(c)))
        self._cfg = Config(c.vocab, c.ctx, c.dim, c.heads, c.kv_heads, c.head_dim, c.layers, c.hidden, c.rope_dim,
                           c.rope_base, c.eps, c.linear_factor, bool(c.neox), bool(c.tied), QKind(c.kind),
                           QPath(c.path))

    @classmethod
    def from_gguf(cls, gpu: Gpu, g: Gguf, path: QPath = QPath.Tiled) -> "GpuLlama":
        h = ctypes.c_void_p()
        _check(lib().fh_llama_from_gguf(gpu.handle, g.handle, int(path), ctypes.byref(h)))
        return cls(gpu, h)

    def config(self) -> Config:
        return self._cfg

    def weight_bytes(self) -> int:
        """Packed bytes of every block matrix and the head (what one forward reads)."""
        return lib().fh_llama_weight_bytes(self._h)

    def device_bytes(self) -> int:
        """Device memory the model holds (padded weight planes, the fast path's correction
        operands, vectors, tables and the activation arena)."""
        return lib().fh_llama_device_bytes(self._h)

    @staticmethod
    def _ids(ids) -> np.ndarray:
        a = np.asarray(ids)
        if a.size and (a.min() < 0 or a.max() > np.iinfo(np.int32).max):
            raise GpuError(f"token {int(a.min() if a.min() < 0 else a.max())} is out of range")
        return np.ascontiguousarray(a, dtype=np.int32)

    def forward_all(self, ids) -> np.ndarray:
        """GpuLlama::forward_all (forward.rs:13-15): every position's logits, [len(ids), vocab]."""
        a = self._ids(ids)
        out = np.empty((max(a.size, 1), self._cfg.vocab), np.float32)
        _check(lib().fh_llama_forward_all(self.gpu.handle, self._h, a.ctypes.data_as(ctypes.c_void_p), a.size,
                                          out.ctypes.data_as(ctypes.c_void_p)))
        return out[: a.size]

    def score_arrays(self, ids) -> tuple[np.ndarray, np.ndarray]:
        """score as two arrays: log-probabilities [len - 1] and first-argmax flags [len - 1]."""
        a = self._ids(ids)
        rows = max(a.size - 1, 1)
        lp, hit = np.empty(rows, np.float32), np.empty(rows, np.uint8)
        _check(lib().fh_llama_score(self.gpu.handle, self._h, a.ctypes.data_as(ctypes.c_void_p), a.size,
                                    lp.ctypes.data_as(ctypes.c_void_p), hit.ctypes.data_as(ctypes.c_void_p)))
        return lp[: a.size - 1], hit[: a.size - 1].astype(bool)

    def score(self, ids) -> list[tuple[float, bool]]:
        """GpuLlama::score (forward.rs:76-88): for each i < len - 1, (log p(ids[i + 1] | ids[..=i]),
        whether ids[i + 1] is the first argmax)."""
        lp, hit = self.score_arrays(ids)
        return [(float(a), bool(b)) for a, b in zip(lp, hit)]

    def score_device(self, ids: GpuBuf, n: int, out: GpuBuf) -> None:
        """The score pass on n device-resident int32 ids into out (2 (n - 1) floats), enqueued on
        the device stream without waiting."""
        _check(lib().fh_llama_score_device(self.gpu.handle, self._h, ids.handle, n, out.handle))

    def free(self) -> None:
        if self._h:
            lib().fh_llama_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


QWEN2_0_5B = {"vocab": 151936, "ctx": 32768, "dim": 896, "heads": 14, "kv_heads": 2, "head_dim": 64, "layers": 24,
              "hidden": 4864, "rope_dim": 64, "rope_base": 1e6, "eps": 1e-6, "neox": True}


def random_gguf(gpu: Gpu, cfg: dict, kind: QKind = QKind.Q4_0, seed: int = 0, biases: bool = True,
                tied: bool = True) -> bytes:
    """A `qwen2` (neox) or `llama` GGUF of synthetic weights, laid out as ferrum_model writes
    one (ferrum_model/src/gguf/llama/mod.rs:223-323), every matrix packed by the device encoder.
    The values follow the distributions of ferrum_ref's Llama::random (params.rs:38-93), drawn
    from numpy's PCG64 instead of its xorshift: matrices uniform in [-1, 1) times 0.5 (q and k
    0.5 sqrt(8 / dim), so attention scores stay O(1)), biases times 0.1, norm gains 1 + 0.1 u, the
    embedding times 1. Weights are drawn directly as GGUF rows ([out][in])."""
    arch = "qwen2" if cfg["neox"] else "llama"
    d, h, v = cfg["dim"], cfg["hidden"], cfg["vocab"]
    qd, kvd = cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(seed)
    b = GgufBuilder()
    b.meta("general.architecture", Value(STR, arch))
    for key, val in (("context_length", cfg["ctx"]), ("embedding_length", d), ("block_count", cfg["layers"]),
                     ("feed_forward_length", h), ("attention.head_count", cfg["heads"]),
                     ("attention.head_count_kv", cfg["kv_heads"]), ("attention.key_length", cfg["head_dim"]),
                     ("rope.dimension_count", cfg["rope_dim"])):
        b.meta(f"{arch}.{key}", Value(U32, int(val)))
    b.meta(f"{arch}.rope.freq_base", Value(F32, float(cfg["rope_base"])))
    b.meta(f"{arch}.attention.layer_norm_rms_epsilon", Value(F32, float(cfg["eps"])))

    def uni(n, scale):
        return (rng.random(n, dtype=np.float32) * np.float32(2.0) - np.float32(1.0)) * np.float32(scale)

    def rows(name, n_rows, ne0, scale):
        src = gpu.upload(uni(n_rows * ne0, scale))
        packed = encode(gpu, kind, src, n_rows * ne0)
        b.tensor_raw(name, [ne0, n_rows], int(kind), gpu.read_bytes(packed).tobytes())
        src.free()
        packed.free()

    def vec(name, data):
        b.tensor_f32(name, [len(data)], np.asarray(data, np.float32))

    gain = lambda n: np.float32(1.0) + np.float32(0.1) * uni(n, 1.0)
    qk = float(np.float32(0.5) * np.sqrt(np.float32(8.0) / np.float32(d)))
    rows("token_embd.weight", v, d, 1.0)
    for i in range(cfg["layers"]):
        n = f"blk.{i}."
        vec(n + "attn_norm.weight", gain(d))
        for stem, out, scale in (("attn_q", qd, qk), ("attn_k", kvd, qk), ("attn_v", kvd, 0.5)):
            rows(n + stem + ".weight", out, d, scale)
            if biases:
                vec(n + stem + ".bias", uni(out, 0.1))
        rows(n + "attn_output.weight", d, qd, 0.5)
        vec(n + "ffn_norm.weight", gain(d))
        rows(n + "ffn_gate.weight", h, d, 0.5)
        rows(n + "ffn_up.weight", h, d, 0.5)
        rows(n + "ffn_down.weight", d, h, 0.5)
    vec("output_norm.weight", gain(d))
    if not tied:
        rows("output.weight", v, d, 0.5)
    return b.into_bytes()


__all__ = ["Config", "GpuLlama", "GpuError", "QWEN2_0_5B", "random_gguf"]
