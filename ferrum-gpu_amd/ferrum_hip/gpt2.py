"""Python mirror of ferrum_wgpu's GpuGpt2 (ferrum_wgpu/src/models/gpt2.rs:52-265) over the
quantized decoder of libferrum_hip (the fh_gpt2_* entry points of include/ferrum_hip.h).

`feed`, `reset`, `pos` and `config` keep the reference's names and error texts ("context of N
tokens is full", "token T is out of range for vocab V"). The model is built from a `gpt2` GGUF
whose matrices stay packed (Q8_0 or Q4_0) on the device; `generate` runs greedy decoding with
the picks kept on the device.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import Gpu, GpuError, QKind, _check, encode, lib, upload_quantised
from .gguf import ARR, F32, GGML_F32, STR, U32, Gguf, GgufBuilder, Value


@dataclass(frozen=True)
class Config:
    """ferrum_ref/src/models/gpt2/mod.rs:16-31"""
    vocab: int
    ctx: int
    dim: int
    heads: int
    layers: int
    hidden: int

    def head_dim(self) -> int:
        return self.dim // self.heads


class GpuGpt2:
    """A resident quantized GPT-2 with its KV cache (one per model, ctx positions)."""

    def __init__(self, gpu: Gpu, handle):
        self.gpu, self._h = gpu, handle
        v = [ctypes.c_size_t() for _ in range(6)]
        _check(lib().fh_gpt2_config(self._h, *[ctypes.byref(x) for x in v]))
        self._cfg = Config(*[x.value for x in v])

    @classmethod
    def from_gguf(cls, gpu: Gpu, g: Gguf) -> "GpuGpt2":
        h = ctypes.c_void_p()
        _check(lib().fh_gpt2_from_gguf(gpu.handle, g.handle, ctypes.byref(h)))
        return cls(gpu, h)

    def config(self) -> Config:
        return self._cfg

    def kind(self) -> QKind:
        return QKind(lib().fh_gpt2_kind(self._h))

    def pos(self) -> int:
        """GpuGpt2::pos (gpt2.rs:205-208)"""
        return lib().fh_gpt2_pos(self._h)

    def reset(self) -> None:
        """GpuGpt2::reset (gpt2.rs:210-213)"""
        lib().fh_gpt2_reset(self._h)

    def step_bytes(self) -> int:
        return lib().fh_gpt2_step_bytes(self._h)

    def step_launches(self) -> int:
        """Kernel launches in one decode step (2 per layer + 3 on the fused step)."""
        return lib().fh_gpt2_step_launches(self._h)

    def feed(self, token: int, logits: bool = True):
        """GpuGpt2::feed (gpt2.rs:216-265): the next-token logits row (or None)."""
        out = np.empty(self._cfg.vocab, np.float32) if logits else None
        ptr = out.ctypes.data_as(ctypes.c_void_p) if logits else None
        _check(lib().fh_gpt2_feed(self.gpu.handle, self._h, int(token), ptr))
        return out

    def generate(self, prompt, n_new: int) -> list[int]:
        """Greedy decode from the current position: the n_new picked token ids."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(n_new, 1), np.int32)
        _check(lib().fh_gpt2_generate(self.gpu.handle, self._h, p.ctypes.data_as(ctypes.c_void_p), p.size, n_new,
                                      out.ctypes.data_as(ctypes.c_void_p)))
        return [int(t) for t in out[:n_new]]

    def free(self) -> None:
        if self._h:
            lib().fh_gpt2_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


BLOCK_NAMES = ("ln1_g", "ln1_b", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln2_g", "ln2_b", "w1",
               "b1", "w2", "b2")


def gpt2_init(cfg: dict, seed: int) -> dict:
    """Synthetic weights with GPT-2's initialisation (Radford et al. 2019, sec. 2.3, as the common
    GPT-2 implementations apply it): matrices, token and position embeddings N(0, 0.02), the two
    residual projections per block (attention output, FFN down) N(0, 0.02 / sqrt(2 layers)),
    biases 0, LayerNorm gains 1 and shifts 0, the head tied to the token embedding. f32, seeded
    (numpy's PCG64). Matrices are [in, out] row-major, as ferrum_ref's Gpt2 keeps them
    (ferrum_ref/src/models/gpt2/mod.rs:62-117); "head" is None for the tied head."""
    d, h, v, ctx, L = cfg["dim"], cfg["hidden"], cfg["vocab"], cfg["ctx"], cfg["layers"]
    rng = np.random.default_rng(seed)

    def normal(n, std):
        return (rng.standard_normal(n, dtype=np.float32) * np.float32(std)).astype(np.float32)

    zeros = lambda n: np.zeros(n, np.float32)
    ones = lambda n: np.ones(n, np.float32)
    proj = 0.02 / np.sqrt(2 * L)
    m = dict(cfg)
    m["tok"] = normal(v * d, 0.02)
    m["pos"] = normal(ctx * d, 0.02)
    m["blocks"] = [{"ln1_g": ones(d), "ln1_b": zeros(d), "wq": normal(d * d, 0.02), "bq": zeros(d),
                    "wk": normal(d * d, 0.02), "bk": zeros(d), "wv": normal(d * d, 0.02), "bv": zeros(d),
                    "wo": normal(d * d, proj), "bo": zeros(d), "ln2_g": ones(d), "ln2_b": zeros(d),
                    "w1": normal(d * h, 0.02), "b1": zeros(h), "w2": normal(h * d, proj), "b2": zeros(d)}
                   for _ in range(L)]
    m["lnf_g"], m["lnf_b"] = ones(d), zeros(d)
    m["head"] = None
    return m


def to_gguf(gpu: Gpu, m: dict, kind: QKind = QKind.Q8_0) -> bytes:
    """A `gpt2` GGUF laid out as ferrum_model writes it (ferrum_model/src/gguf/gpt2.rs:179-233:
    the same keys, tensor names, order and row layout), every matrix packed by the device
    encoder: the token embedding row by row (quant::encode), [in, out] matrices as GGUF rows
    (quantise_matrix), the fused QKV as the rows of Q, then K, then V. A head of None is tied
    (no output.weight)."""
    d, h, v, ctx = m["dim"], m["hidden"], m["vocab"], m["ctx"]
    b = GgufBuilder()
    b.meta("general.architecture", Value(STR, "gpt2"))
    b.meta("general.name", Value(STR, "ferrum-gpu Transformer"))
    b.meta("general.quantization_version", Value(U32, 2))
    for key, val in (("context_length", ctx), ("embedding_length", d), ("block_count", m["layers"]),
                     ("feed_forward_length", h), ("attention.head_count", m["heads"])):
        b.meta(f"gpt2.{key}", Value(U32, int(val)))
    b.meta("gpt2.attention.layer_norm_epsilon", Value(F32, float(np.float32(1e-5))))

    def rows_of(w, inp, out):  # [in, out] -> GGUF rows bytes
        return upload_quantised(gpu, kind, w, inp, out).read_gguf().tobytes()

    tok = gpu.upload(m["tok"])
    b.tensor_raw("token_embd.weight", [d, v], int(kind), gpu.read_bytes(encode(gpu, kind, tok, v * d)).tobytes())
    tok.free()
    b.tensor_f32("position_embd.weight", [d, ctx], m["pos"])
    for i, blk in enumerate(m["blocks"]):
        n = f"blk.{i}."
        b.tensor_f32(n + "attn_norm.weight", [d], blk["ln1_g"])
        b.tensor_f32(n + "attn_norm.bias", [d], blk["ln1_b"])
        qkv = b"".join(rows_of(blk[w], d, d) for w in ("wq", "wk", "wv"))
        b.tensor_raw(n + "attn_qkv.weight", [d, 3 * d], int(kind), qkv)
        b.tensor_f32(n + "attn_qkv.bias", [3 * d], np.concatenate([blk["bq"], blk["bk"], blk["bv"]]))
        b.tensor_raw(n + "attn_output.weight", [d, d], int(kind), rows_of(blk["wo"], d, d))
        b.tensor_f32(n + "attn_output.bias", [d], blk["bo"])
        b.tensor_f32(n + "ffn_norm.weight", [d], blk["ln2_g"])
        b.tensor_f32(n + "ffn_norm.bias", [d], blk["ln2_b"])
        b.tensor_raw(n + "ffn_up.weight", [d, h], int(kind), rows_of(blk["w1"], d, h))
        b.tensor_f32(n + "ffn_up.bias", [h], blk["b1"])
        b.tensor_raw(n + "ffn_down.weight", [h, d], int(kind), rows_of(blk["w2"], h, d))
        b.tensor_f32(n + "ffn_down.bias", [d], blk["b2"])
    b.tensor_f32("output_norm.weight", [d], m["lnf_g"])
    b.tensor_f32("output_norm.bias", [d], m["lnf_b"])
    if m.get("head") is not None:
        b.tensor_raw("output.weight", [d, v], int(kind), rows_of(m["head"], d, v))
    return b.into_bytes()


__all__ = ["BLOCK_NAMES", "Config", "GpuGpt2", "GpuError", "gpt2_init", "to_gguf"]
