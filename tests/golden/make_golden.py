"""Regenerate the golden fixtures under tests/golden/ (run in the build container, where the
reference checkout is mounted; the GPU box never runs this).

1. ``model.gguf``: the reference's fixture ``fixtures/bpe/model.gguf`` copied byte for byte (a
   2-layer GPT-2 with Q8_0 matrices and F32 vectors, written by a different encoder, ferrum-cpu;
   sha256 623af38b...6ec as in the reference's fixtures/README.md ledger). It is data: the tests
   parse it with the native reader and with oracle/gguf.py.
   ``model_gguf_q8_0.bin`` / ``.json``: the raw bytes of its Q8_0 tensors and their directory,
   cut out by oracle/gguf.py's reader; nothing from the reference is executed.
2. ``codec_nasty.npz``: the reference's "nasty" inputs (ferrum_wgpu/src/ops/quant/tests.rs:11-23,
   ferrum_wgpu/src/ops/qat.rs:68-80) encoded to Q8_0 and Q4_0, decoded, and snapped (rows and
   columns) by the C oracle. Every byte and every float is cross-checked against the
   independent numpy restatement (oracle/np_oracle.py) before it is written.

Usage: ``python tests/golden/make_golden.py [path/to/model.gguf]``
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

import oracle  # noqa: E402
from oracle import gguf, np_oracle  # noqa: E402

GGUF_PATH = "/root/reference/fixtures/bpe/model.gguf"


def parse_gguf(path: str):
    """(file bytes, metadata dict, tensor list, data-section offset) by oracle/gguf.py's reader."""
    data = open(path, "rb").read()
    kv, tensors, base = gguf.parse(data)
    return data, {k: v for k, v in kv}, tensors, base


def nasty(n: int) -> np.ndarray:
    """ferrum_wgpu/src/ops/quant/tests.rs:11-23 (the same generator as ops/qat.rs:68-80)."""
    v = oracle.rand_vec(n, 9) * np.float32(3.0)
    i = np.arange(n)
    sel = (i // 32) % 7
    v = np.where(sel == 0, v * np.float32(1e-6), v)
    v = np.where(sel == 1, np.float32(0), v)
    v = np.where(sel == 2, v * np.float32(1e4), v)
    v = np.where(sel == 3, (i % 9).astype(np.float32) - np.float32(4), v)
    return v.astype(np.float32)


MODEL_SHA256 = "623af38b770ace7617725682bf84c0bb212d62ab78be1784e6b9775928af36ec"


def make_model_fixture(path: str) -> None:
    data, meta, tensors, base = parse_gguf(path)
    if hashlib.sha256(data).hexdigest() != MODEL_SHA256:
        raise SystemExit(f"{path} is not the ledger's model.gguf")
    with open(os.path.join(HERE, "model.gguf"), "wb") as f:
        f.write(data)
    blobs, table, off = [], [], 0
    for t in tensors:
        if t["type"] != oracle.Q8_0:
            continue
        n = int(np.prod(t["dims"]))
        nb = oracle.nbytes(oracle.Q8_0, n)
        raw = data[base + t["offset"]: base + t["offset"] + nb]
        blobs.append(raw)
        table.append({"name": t["name"], "dims": t["dims"], "elements": n, "offset": off,
                      "bytes": nb})
        off += nb
    blob = b"".join(blobs)
    with open(os.path.join(HERE, "model_gguf_q8_0.bin"), "wb") as f:
        f.write(blob)
    info = {
        "source": "reference fixtures/bpe/model.gguf (GPT-2 written by ferrum-cpu)",
        "source_sha256": hashlib.sha256(data).hexdigest(),
        "blob_sha256": hashlib.sha256(blob).hexdigest(),
        "tensors": table,
    }
    with open(os.path.join(HERE, "model_gguf_q8_0.json"), "w") as f:
        json.dump(info, f, indent=1)
    print(f"model fixture: {len(table)} Q8_0 tensors, {len(blob)} bytes, {len(blob) // 34} blocks")


def make_codec_fixture() -> None:
    x = nasty(32 * 64)  # 64 blocks: every one of the 7 nasty classes several times
    q8 = oracle.encode(oracle.Q8_0, x)
    q4 = oracle.encode(oracle.Q4_0, x)
    assert np.array_equal(q8, np_oracle.encode_q8_0(x)), "Q8_0 encode: C vs numpy"
    assert np.array_equal(q4, np_oracle.encode_q4_0(x)), "Q4_0 encode: C vs numpy"
    d8 = oracle.decode(oracle.Q8_0, q8, x.size)
    d4 = oracle.decode(oracle.Q4_0, q4, x.size)
    assert np.array_equal(d8.view(np.uint32), np_oracle.decode_q8_0(q8).view(np.uint32))
    assert np.array_equal(d4.view(np.uint32), np_oracle.decode_q4_0(q4).view(np.uint32))
    snap_r = oracle.snap_rows(x, 32)
    assert np.array_equal(snap_r.view(np.uint32), d8.view(np.uint32)), "snap_rows = decode(encode)"
    snap_c = oracle.snap_cols(x, 64, 32)  # [64 in, 32 out]: blocks down the columns
    np.savez(os.path.join(HERE, "codec_nasty.npz"), x=x, q8_0=q8, q4_0=q4, dq8_0=d8, dq4_0=d4,
             snap_rows=snap_r, snap_cols_64x32=snap_c)
    print("codec fixture: 64 nasty blocks, Q8_0 and Q4_0, C and numpy agree")


if __name__ == "__main__":
    if not os.path.exists(oracle.LIB_PATH):
        raise SystemExit("build the oracle first: make -C oracle")
    make_model_fixture(sys.argv[1] if len(sys.argv) > 1 else GGUF_PATH)
    make_codec_fixture()
