"""GPT-2 model construction for tests (test infrastructure; see oracle/__init__.py).

* ``gpt2_random``   restates Gpt2::random (ferrum_ref/src/models/gpt2/mod.rs:139-190): the
                    reference's seeded weights, drawn from its rand_vec in the same order.
* ``gpt2_init``     restates Gpt2::init (ferrum_ref/src/models/gpt2/params.rs:160-180): the
                    random draws rescaled to GPT-style magnitudes, gains 1, biases 0.
* ``fake_quantize`` restates Gpt2::fake_quantize (ferrum_ref/src/training/qat.rs:56-74): the f32
                    model a Q8_0 export stores, which the CPU decode runs on.
* ``to_gguf``       restates to_gguf (ferrum_model/src/gguf/gpt2.rs:179-233): GGUF rows of every
                    matrix (quantised per block format when the row is whole 32-blocks), F32
                    vectors, the head omitted when it is the transposed embedding.
* ``from_gguf``     the inverse for a file of Q8_0/Q4_0/F32 tensors: the f32 model whose matrices
                    are the decoded stored values (what the CPU path multiplies by).

Models are dicts: vocab, ctx, dim, heads, layers, hidden, tok [vocab*dim], pos [ctx*dim], blocks
(dicts keyed by GPT2_BLOCK_NAMES, matrices [in, out] row-major), lnf_g, lnf_b, head [dim*vocab].
"""
from __future__ import annotations

import numpy as np

from . import (BLOCK_BYTES, F32, GPT2_BLOCK_NAMES, Q4_0, Q8_0, decode, encode, rand_vec,
               snap_cols, snap_rows, transpose)
from . import gguf as og

LN_EPS = np.float32(1e-5)  # ferrum_ref/src/kernels/nn.rs:6


def gpt2_random(cfg: dict, seed: int) -> dict:
    """Gpt2::random: weights rand_vec(n, s) * scale (gains 1 + 0.1 * rand_vec) with s counting up
    from max(seed, 1) * 1000, in the order the reference draws them."""
    d, h, v, ctx = cfg["dim"], cfg["hidden"], cfg["vocab"], cfg["ctx"]
    s = [max(seed, 1) * 1000]

    def draw(n):
        s[0] += 1
        return rand_vec(n, s[0])

    def mat(n, scale):
        return (draw(n) * np.float32(scale)).astype(np.float32)

    def gain(n):
        return (np.float32(1.0) + np.float32(0.1) * draw(n)).astype(np.float32)

    blocks = []
    for _ in range(cfg["layers"]):
        b = {}
        b["ln1_g"] = gain(d)
        b["ln1_b"] = mat(d, 0.1)
        b["wq"] = mat(d * d, 0.5)
        b["bq"] = mat(d, 0.1)
        b["wk"] = mat(d * d, 0.5)
        b["bk"] = mat(d, 0.1)
        b["wv"] = mat(d * d, 0.5)
        b["bv"] = mat(d, 0.1)
        b["wo"] = mat(d * d, 0.5)
        b["bo"] = mat(d, 0.1)
        b["ln2_g"] = gain(d)
        b["ln2_b"] = mat(d, 0.1)
        b["w1"] = mat(d * h, 0.5)
        b["b1"] = mat(h, 0.1)
        b["w2"] = mat(h * d, 0.5)
        b["b2"] = mat(d, 0.1)
        blocks.append(b)
    m = dict(cfg)
    m["blocks"] = blocks
    m["tok"] = mat(v * d, 1.0)
    m["pos"] = mat(ctx * d, 0.5)
    m["lnf_g"] = gain(d)
    m["lnf_b"] = mat(d, 0.1)
    m["head"] = mat(d * v, 0.5)
    return m


def gpt2_init(cfg: dict, seed: int) -> dict:
    """Gpt2::init (ferrum_ref/src/models/gpt2/params.rs:160-180): Gpt2::random's draws, then every
    canonical parameter by kind: the token and position embeddings, the block matrices (canonical
    block indices 2, 4, 6, 8, 12, 14) and the head times 0.02 * sqrt(3) in f32 (rand_vec is uniform
    on [-1, 1), std 1 / sqrt(3)); LayerNorm gains (block indices 0, 10 and the final one) 1; block
    biases and LayerNorm shifts 0. The head stays untied (tie_head ties it)."""
    m = gpt2_random(cfg, seed)
    scale = np.float32(0.02) * np.sqrt(np.float32(3.0))
    weights = ("wq", "wk", "wv", "wo", "w1", "w2")
    gains = ("ln1_g", "ln2_g")
    for b in m["blocks"]:
        for k in GPT2_BLOCK_NAMES:
            if k in weights:
                b[k] = (b[k] * scale).astype(np.float32)
            elif k in gains:
                b[k] = np.ones_like(b[k])
            else:
                b[k] = np.zeros_like(b[k])
    for k in ("tok", "pos", "head"):
        m[k] = (m[k] * scale).astype(np.float32)
    m["lnf_g"], m["lnf_b"] = np.ones_like(m["lnf_g"]), np.zeros_like(m["lnf_b"])
    return m


def tie_head(m: dict) -> dict:
    """Gpt2::tie_head (mod.rs:119-123): head = tok transposed."""
    t = dict(m)
    t["head"] = transpose(m["tok"], m["vocab"], m["dim"])
    return t


def fake_quantize(m: dict) -> dict:
    """Gpt2::fake_quantize: the token embedding snapped along its rows, the block matrices and
    the head down their columns; vectors and position embeddings unchanged."""
    d, h, v = m["dim"], m["hidden"], m["vocab"]
    q = dict(m)
    q["tok"] = snap_rows(m["tok"], d)
    q["blocks"] = []
    for b in m["blocks"]:
        nb = dict(b)
        for k in ("wq", "wk", "wv", "wo"):
            nb[k] = snap_cols(b[k], d, d)
        nb["w1"] = snap_cols(b["w1"], d, h)
        nb["w2"] = snap_cols(b["w2"], h, d)
        q["blocks"].append(nb)
    q["head"] = snap_cols(m["head"], d, v)
    return q


def to_gguf(m: dict, kind: int = Q8_0) -> bytes:
    """to_gguf (ferrum_model/src/gguf/gpt2.rs:179-233) without tokenizer: `kind` for every row
    whose length is whole 32-blocks, F32 otherwise."""
    d, h, v, ctx = m["dim"], m["hidden"], m["vocab"], m["ctx"]
    b = og.GgufBuilder()
    b.meta("general.architecture", og.V(og.STR, "gpt2"))
    b.meta("general.name", og.V(og.STR, "ferrum-gpu Transformer"))
    b.meta("general.quantization_version", og.V(og.U32, 2))
    for key, val in (("context_length", ctx), ("embedding_length", d), ("block_count", m["layers"]),
                     ("feed_forward_length", h), ("attention.head_count", m["heads"])):
        b.meta(f"gpt2.{key}", og.V(og.U32, val))
    b.meta("gpt2.attention.layer_norm_epsilon", og.V(og.F32, float(LN_EPS)))

    def rows(name, data, n_rows, ne0):
        ty = kind if ne0 % 32 == 0 else F32
        raw = encode(ty, data) if ty != F32 else np.ascontiguousarray(data, np.float32).view(np.uint8)
        b.tensor_raw(name, [ne0, n_rows], ty, raw.tobytes())

    def matrix(name, w, inp, out):
        rows(name, transpose(w, inp, out), out, inp)

    rows("token_embd.weight", m["tok"], v, d)
    b.tensor_f32("position_embd.weight", [d, ctx], m["pos"])
    for i, blk in enumerate(m["blocks"]):
        n = f"blk.{i}."
        b.tensor_f32(n + "attn_norm.weight", [d], blk["ln1_g"])
        b.tensor_f32(n + "attn_norm.bias", [d], blk["ln1_b"])
        qkv = np.concatenate([transpose(blk[w], d, d) for w in ("wq", "wk", "wv")])
        rows(n + "attn_qkv.weight", qkv, 3 * d, d)
        b.tensor_f32(n + "attn_qkv.bias", [3 * d], np.concatenate([blk["bq"], blk["bk"], blk["bv"]]))
        matrix(n + "attn_output.weight", blk["wo"], d, d)
        b.tensor_f32(n + "attn_output.bias", [d], blk["bo"])
        b.tensor_f32(n + "ffn_norm.weight", [d], blk["ln2_g"])
        b.tensor_f32(n + "ffn_norm.bias", [d], blk["ln2_b"])
        matrix(n + "ffn_up.weight", blk["w1"], d, h)
        b.tensor_f32(n + "ffn_up.bias", [h], blk["b1"])
        matrix(n + "ffn_down.weight", blk["w2"], h, d)
        b.tensor_f32(n + "ffn_down.bias", [d], blk["b2"])
    b.tensor_f32("output_norm.weight", [d], m["lnf_g"])
    b.tensor_f32("output_norm.bias", [d], m["lnf_b"])
    head_rows = transpose(m["head"], d, v)
    if not np.array_equal(head_rows, m["tok"]):
        rows("output.weight", head_rows, v, d)
    return b.into_bytes()


def from_gguf(data: bytes) -> dict:
    """The f32 model a `gpt2` GGUF of Q8_0/Q4_0/F32 tensors stores (ferrum_model's from_gguf
    reading, for the CPU side): matrices back to [in, out], the head tied when absent."""
    kv, tensors, base = og.parse(data)
    meta = {k: v.v for k, v in kv}
    by = {t["name"]: t for t in tensors}

    def f32(name):
        t = by[name]
        n = int(np.prod(t["dims"]))
        if t["type"] == F32:
            return np.frombuffer(data, np.float32, n, base + t["offset"]).copy()
        nb = n // 32 * BLOCK_BYTES[t["type"]]
        raw = np.frombuffer(data, np.uint8, nb, base + t["offset"])
        return decode(t["type"], raw, n)

    def matrix(name):  # GGUF rows [out][in] -> [in, out]
        ne0, n_rows = by[name]["dims"]
        return transpose(f32(name), n_rows, ne0)

    d, h = meta["gpt2.embedding_length"], meta["gpt2.feed_forward_length"]
    m = {"ctx": meta["gpt2.context_length"], "dim": d, "layers": meta["gpt2.block_count"], "hidden": h,
         "heads": meta["gpt2.attention.head_count"], "vocab": by["token_embd.weight"]["dims"][1]}
    m["tok"] = f32("token_embd.weight")
    m["pos"] = f32("position_embd.weight")
    m["blocks"] = []
    for i in range(m["layers"]):
        n = f"blk.{i}."
        qkv = matrix(n + "attn_qkv.weight").reshape(d, 3 * d)
        bias = f32(n + "attn_qkv.bias")
        blk = {"ln1_g": f32(n + "attn_norm.weight"), "ln1_b": f32(n + "attn_norm.bias"),
               "wq": np.ascontiguousarray(qkv[:, :d]).reshape(-1), "bq": bias[:d].copy(),
               "wk": np.ascontiguousarray(qkv[:, d:2 * d]).reshape(-1), "bk": bias[d:2 * d].copy(),
               "wv": np.ascontiguousarray(qkv[:, 2 * d:]).reshape(-1), "bv": bias[2 * d:].copy(),
               "wo": matrix(n + "attn_output.weight"), "bo": f32(n + "attn_output.bias"),
               "ln2_g": f32(n + "ffn_norm.weight"), "ln2_b": f32(n + "ffn_norm.bias"),
               "w1": matrix(n + "ffn_up.weight"), "b1": f32(n + "ffn_up.bias"),
               "w2": matrix(n + "ffn_down.weight"), "b2": f32(n + "ffn_down.bias")}
        m["blocks"].append(blk)
    m["lnf_g"] = f32("output_norm.weight")
    m["lnf_b"] = f32("output_norm.bias")
    m["head"] = matrix("output.weight") if "output.weight" in by else transpose(m["tok"], m["vocab"], d)
    return m


__all__ = ["gpt2_random", "tie_head", "fake_quantize", "to_gguf", "from_gguf", "Q4_0", "Q8_0",
           "GPT2_BLOCK_NAMES"]
