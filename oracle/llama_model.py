"""Llama / Qwen2 model construction for tests (test infrastructure; see oracle/__init__.py).

* ``llama_random`` restates Llama::random (ferrum_ref/src/models/llama/params.rs:38-93): the
                   reference's seeded weights, drawn from its rand_vec in the same order.
* ``dequantised``  restates dequantised (ferrum_wgpu/src/models/llama/mod.rs:188-213): every
                   matrix whose input width is whole 32-blocks replaced by decode(encode(.)), the
                   head included; the embedding stays as it is.
* ``to_gguf``      restates the llama/qwen2 writer (ferrum_model/src/gguf/llama/mod.rs:223-323):
                   `llama` (NORM RoPE) or `qwen2` (NEOX RoPE) metadata, GGUF rows quantised when
                   their length is whole 32-blocks, F32 vectors, the head omitted when tied.
* ``from_gguf``    the f32 model such a file stores (ferrum_model/src/gguf/llama/mod.rs:107-209,
                   for the files to_gguf writes): decoded matrices back to [in, out], the head
                   the transposed embedding when `output.weight` is absent.

Models are dicts: vocab, ctx, dim, heads, kv_heads, head_dim, layers, hidden, rope_dim,
rope_base, neox, eps, freq_factors (None or rope_dim/2 floats), linear_factor, tok
[vocab*dim], blocks (dicts keyed by LLAMA_BLOCK_NAMES, matrices [in, out] row-major, biases None
when absent), out_norm, head [dim*vocab], tied.
"""
from __future__ import annotations

import numpy as np

from . import (BLOCK_BYTES, F32, LLAMA_BLOCK_NAMES, Q4_0, Q8_0, decode, dequantised_in_out, encode,
               quantise_matrix, rand_vec, transpose)
from . import gguf as og

CONFIG_KEYS = ("vocab", "ctx", "dim", "heads", "kv_heads", "head_dim", "layers", "hidden", "rope_dim",
               "rope_base", "neox", "eps")


def config(vocab, ctx, dim, heads, kv_heads, head_dim, layers, hidden, rope_dim=None, rope_base=10000.0,
           neox=False, eps=1e-5) -> dict:
    return {"vocab": vocab, "ctx": ctx, "dim": dim, "heads": heads, "kv_heads": kv_heads, "head_dim": head_dim,
            "layers": layers, "hidden": hidden, "rope_dim": head_dim if rope_dim is None else rope_dim,
            "rope_base": float(np.float32(rope_base)), "neox": bool(neox), "eps": float(np.float32(eps))}


def q_dim(c: dict) -> int:
    return c["heads"] * c["head_dim"]


def kv_dim(c: dict) -> int:
    return c["kv_heads"] * c["head_dim"]


def llama_random(cfg: dict, seed: int, biases: bool, tied: bool) -> dict:
    """Llama::random: s counts up from max(seed, 1) * 1000; per block attn_norm, wq, (bq), wk,
    (bk), wv, (bv), wo, ffn_norm, gate, up, down; then tok, the head (unless tied), out_norm."""
    d, h = cfg["dim"], cfg["hidden"]
    qd, kvd = q_dim(cfg), kv_dim(cfg)
    s = [max(seed, 1) * 1000]

    def draw(n):
        s[0] += 1
        return rand_vec(n, s[0])

    def mat(n, scale):
        return (draw(n) * np.float32(scale)).astype(np.float32)

    def gain(n):
        return (np.float32(1.0) + np.float32(0.1) * draw(n)).astype(np.float32)

    qk = np.float32(0.5) * np.sqrt(np.float32(8.0) / np.float32(d))
    blocks = []
    for _ in range(cfg["layers"]):
        b = {"attn_norm": gain(d)}
        b["wq"] = mat(d * qd, qk)
        b["bq"] = mat(qd, 0.1) if biases else None
        b["wk"] = mat(d * kvd, qk)
        b["bk"] = mat(kvd, 0.1) if biases else None
        b["wv"] = mat(d * kvd, 0.5)
        b["bv"] = mat(kvd, 0.1) if biases else None
        b["wo"] = mat(qd * d, 0.5)
        b["ffn_norm"] = gain(d)
        b["gate"] = mat(d * h, 0.5)
        b["up"] = mat(d * h, 0.5)
        b["down"] = mat(h * d, 0.5)
        blocks.append(b)
    m = dict(cfg)
    m["freq_factors"] = None
    m["linear_factor"] = 1.0
    m["blocks"] = blocks
    m["tok"] = mat(cfg["vocab"] * d, 1.0)
    m["head"] = transpose(m["tok"], cfg["vocab"], d) if tied else mat(d * cfg["vocab"], 0.5)
    m["out_norm"] = gain(d)
    m["tied"] = bool(tied)
    return m


def _matrices(c: dict):
    """(block key, input width, output width) of every block matrix."""
    d, h, qd, kvd = c["dim"], c["hidden"], q_dim(c), kv_dim(c)
    return (("wq", d, qd), ("wk", d, kvd), ("wv", d, kvd), ("wo", qd, d), ("gate", d, h), ("up", d, h),
            ("down", h, d))


def dequantised(m: dict, kind: int) -> dict:
    """dequantised(m, kind): the f32 model the device multiplies by when it stores `kind`."""
    def snap(w, k, n):
        if k % 32:
            return np.asarray(w, np.float32).copy()
        return dequantised_in_out(kind, quantise_matrix(kind, w, k, n), k, n)

    out = dict(m)
    out["blocks"] = []
    for b in m["blocks"]:
        nb = dict(b)
        for key, k, n in _matrices(m):
            nb[key] = snap(b[key], k, n)
        out["blocks"].append(nb)
    head = snap(m["head"], m["dim"], m["vocab"])
    out["tied"] = bool(m["tied"]) and np.array_equal(head, m["head"])
    out["head"] = head
    return out


def _arch(m: dict) -> str:
    return "qwen2" if m["neox"] else "llama"


def to_gguf(m: dict, kind: int = Q4_0) -> bytes:
    """The llama/qwen2 writer: metadata in file order, then token_embd, the blocks' tensors, the
    output norm, the head (untied only) and rope_freqs (when present)."""
    arch = _arch(m)
    d, h, qd, kvd = m["dim"], m["hidden"], q_dim(m), kv_dim(m)
    b = og.GgufBuilder()
    b.meta("general.architecture", og.V(og.STR, arch))
    for key, val in (("context_length", m["ctx"]), ("embedding_length", d), ("block_count", m["layers"]),
                     ("feed_forward_length", h), ("attention.head_count", m["heads"]),
                     ("attention.head_count_kv", m["kv_heads"]), ("attention.key_length", m["head_dim"]),
                     ("rope.dimension_count", m["rope_dim"])):
        b.meta(f"{arch}.{key}", og.V(og.U32, val))
    b.meta(f"{arch}.rope.freq_base", og.V(og.F32, m["rope_base"]))
    b.meta(f"{arch}.attention.layer_norm_rms_epsilon", og.V(og.F32, m["eps"]))
    if m.get("linear_factor", 1.0) != 1.0:
        b.meta(f"{arch}.rope.scaling.type", og.V(og.STR, "linear"))
        b.meta(f"{arch}.rope.scaling.factor", og.V(og.F32, m["linear_factor"]))

    def rows(name, data, n_rows, ne0):
        ty = kind if ne0 % 32 == 0 else F32
        raw = encode(ty, data) if ty != F32 else np.ascontiguousarray(data, np.float32).view(np.uint8)
        b.tensor_raw(name, [ne0, n_rows], ty, raw.tobytes())

    def matrix(name, w, inp, out):
        rows(name, transpose(w, inp, out), out, inp)

    def vec(name, v):
        b.tensor_f32(name, [len(v)], np.asarray(v, np.float32))

    rows("token_embd.weight", m["tok"], m["vocab"], d)
    for i, blk in enumerate(m["blocks"]):
        n = f"blk.{i}."
        vec(n + "attn_norm.weight", blk["attn_norm"])
        for key, bias, stem, k, o in (("wq", "bq", "attn_q", d, qd), ("wk", "bk", "attn_k", d, kvd),
                                      ("wv", "bv", "attn_v", d, kvd)):
            matrix(n + stem + ".weight", blk[key], k, o)
            if blk[bias] is not None and len(blk[bias]):
                vec(n + stem + ".bias", blk[bias])
        matrix(n + "attn_output.weight", blk["wo"], qd, d)
        vec(n + "ffn_norm.weight", blk["ffn_norm"])
        matrix(n + "ffn_gate.weight", blk["gate"], d, h)
        matrix(n + "ffn_up.weight", blk["up"], d, h)
        matrix(n + "ffn_down.weight", blk["down"], h, d)
    vec("output_norm.weight", m["out_norm"])
    if not m["tied"]:
        matrix("output.weight", m["head"], d, m["vocab"])
    if m.get("freq_factors") is not None and len(m["freq_factors"]):
        vec("rope_freqs.weight", m["freq_factors"])
    return b.into_bytes()


def from_gguf(data: bytes) -> dict:
    """The f32 model a llama/qwen2 GGUF of Q8_0/Q4_0/F32 tensors stores."""
    kv, tensors, base = og.parse(data)
    meta = {k: v.v for k, v in kv}
    by = {t["name"]: t for t in tensors}
    arch = meta["general.architecture"]
    assert arch in ("llama", "qwen2"), arch

    def f32(name):
        t = by[name]
        n = int(np.prod(t["dims"]))
        if t["type"] == F32:
            return np.frombuffer(data, np.float32, n, base + t["offset"]).copy()
        raw = np.frombuffer(data, np.uint8, n // 32 * BLOCK_BYTES[t["type"]], base + t["offset"])
        return decode(t["type"], raw, n)

    def matrix(name):  # GGUF rows [out][in] -> [in, out]
        ne0, n_rows = by[name]["dims"]
        return transpose(f32(name), n_rows, ne0)

    def opt(name):
        return f32(name) if name in by else None

    a = lambda k: meta[f"{arch}.{k}"]
    d, heads = a("embedding_length"), a("attention.head_count")
    hd = meta.get(f"{arch}.attention.key_length", d // heads)
    m = {"vocab": by["token_embd.weight"]["dims"][1], "ctx": meta.get(f"{arch}.context_length", 2048), "dim": d,
         "heads": heads, "kv_heads": meta.get(f"{arch}.attention.head_count_kv", heads), "head_dim": hd,
         "layers": a("block_count"), "hidden": a("feed_forward_length"),
         "rope_dim": meta.get(f"{arch}.rope.dimension_count", hd),
         "rope_base": meta.get(f"{arch}.rope.freq_base", 10000.0), "neox": arch == "qwen2",
         "eps": meta.get(f"{arch}.attention.layer_norm_rms_epsilon", 1e-5)}
    factor = meta.get(f"{arch}.rope.scaling.factor", meta.get(f"{arch}.rope.scale_linear"))
    m["linear_factor"] = 1.0 if not factor else factor
    m["freq_factors"] = opt("rope_freqs.weight")
    m["tok"] = f32("token_embd.weight")
    m["blocks"] = []
    for i in range(m["layers"]):
        n = f"blk.{i}."
        m["blocks"].append({
            "attn_norm": f32(n + "attn_norm.weight"),
            "wq": matrix(n + "attn_q.weight"), "bq": opt(n + "attn_q.bias"),
            "wk": matrix(n + "attn_k.weight"), "bk": opt(n + "attn_k.bias"),
            "wv": matrix(n + "attn_v.weight"), "bv": opt(n + "attn_v.bias"),
            "wo": matrix(n + "attn_output.weight"), "ffn_norm": f32(n + "ffn_norm.weight"),
            "gate": matrix(n + "ffn_gate.weight"), "up": matrix(n + "ffn_up.weight"),
            "down": matrix(n + "ffn_down.weight")})
    m["out_norm"] = f32("output_norm.weight")
    m["tied"] = "output.weight" not in by
    m["head"] = transpose(m["tok"], m["vocab"], d) if m["tied"] else matrix("output.weight")
    return m


__all__ = ["config", "llama_random", "dequantised", "to_gguf", "from_gguf", "q_dim", "kv_dim", "Q4_0", "Q8_0",
           "LLAMA_BLOCK_NAMES"]
