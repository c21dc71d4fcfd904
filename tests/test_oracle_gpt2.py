"""Pins the CPU GPT-2 oracle (oracle/gpt2.c, oracle/gpt2_model.py) that the device decoder's
token IDs are compared with.

* The cached decode (Gpt2::feed, ferrum_ref/src/models/gpt2/decode.rs:57-117) must give, at every
  position, the logits of an independent float64 full causal forward pass written here from the
  reference's Gpt2::forward_logits (ferrum_ref/src/models/gpt2/mod.rs:206-235) and nn ops
  (ferrum_ref/src/kernels/nn.rs): a wrong cache index, head split, transposition or bias fails it.
* fake_quantize (the snap restatement) must equal the decoded GGUF export (the writer
  restatement), which pins the export's row layout and transposes.
* The reference's fixture model.gguf survives from_gguf -> to_gguf with its tensor bytes intact.
"""
import os

import numpy as np
import pytest

from oracle import gguf as og
from oracle import gpt2_model as gm

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SMALL = {"vocab": 96, "ctx": 12, "dim": 64, "heads": 4, "layers": 2, "hidden": 128}


def forward_f64(m: dict, ids) -> np.ndarray:
    """Gpt2::forward_logits in float64: every position's logits, [len(ids), vocab]."""
    d, h, heads, v = m["dim"], m["hidden"], m["heads"], m["vocab"]
    hd = d // heads
    t = len(ids)
    f = lambda a: np.asarray(a, np.float64)

    def ln(x, g, b):
        mu = x.mean(axis=1, keepdims=True)
        var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
        return (x - mu) / np.sqrt(var + 1e-5) * f(g) + f(b)

    def gelu(x):
        return 0.5 * x * (1.0 + np.tanh(0.7978846 * (x + 0.044715 * x ** 3)))

    x = f(m["tok"]).reshape(v, d)[ids] + f(m["pos"]).reshape(-1, d)[:t]
    mask = np.triu(np.full((t, t), -np.inf), 1)
    for b in m["blocks"]:
        hh = ln(x, b["ln1_g"], b["ln1_b"])
        q = hh @ f(b["wq"]).reshape(d, d) + f(b["bq"])
        k = hh @ f(b["wk"]).reshape(d, d) + f(b["bk"])
        vv = hh @ f(b["wv"]).reshape(d, d) + f(b["bv"])
        a = np.zeros((t, d))
        for i in range(heads):
            s = slice(i * hd, (i + 1) * hd)
            sc = q[:, s] @ k[:, s].T / np.sqrt(hd) + mask
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            a[:, s] = p @ vv[:, s]
        x = x + a @ f(b["wo"]).reshape(d, d) + f(b["bo"])
        hh = ln(x, b["ln2_g"], b["ln2_b"])
        x = x + gelu(hh @ f(b["w1"]).reshape(d, h) + f(b["b1"])) @ f(b["w2"]).reshape(h, d) + f(b["b2"])
    return ln(x, m["lnf_g"], m["lnf_b"]) @ f(m["head"]).reshape(d, v)


def test_cached_decode_matches_a_float64_full_forward(orc):
    m = gm.gpt2_random(SMALL, 3)
    ids = [5, 17, 0, 95, 42, 42, 7, 63, 1, 30, 88, 2]  # the whole context
    want = forward_f64(m, ids)
    cpu = orc.Gpt2Cpu(m)
    for i, t in enumerate(ids):
        got = cpu.feed(t)
        e = np.abs(got - want[i]).max() / max(np.abs(want[i]).max(), 1.0)
        assert e < 2e-5, (i, e)
    with pytest.raises(ValueError):
        cpu.feed(1)  # context full


def test_generate_is_feed_plus_argmax(orc):
    m = gm.gpt2_random(SMALL, 4)
    prompt = [3, 9, 27]
    got = orc.gpt2_generate(m, prompt, 6)
    cpu = orc.Gpt2Cpu(m)
    for t in prompt:
        logits = cpu.feed(t)
    want = []
    for i in range(6):
        want.append(int(np.argmax(logits)))  # first maximum, as sampling.rs:32-40
        if i < 5:
            logits = cpu.feed(want[-1])
    assert got == want


def test_random_model_draw_order(orc):
    """Gpt2::random: s counts from seed*1000; block tensors first (16 per block), then tok, pos,
    lnf_g, lnf_b, head."""
    m = gm.gpt2_random(SMALL, 2)
    d = SMALL["dim"]
    assert np.array_equal(m["blocks"][0]["ln1_g"], (1 + np.float32(0.1) * orc.rand_vec(d, 2001)).astype(np.float32))
    assert np.array_equal(m["blocks"][0]["wq"], orc.rand_vec(d * d, 2003) * np.float32(0.5))
    assert np.array_equal(m["blocks"][1]["b2"], orc.rand_vec(d, 2032) * np.float32(0.1))
    assert np.array_equal(m["tok"], orc.rand_vec(SMALL["vocab"] * d, 2033))
    assert np.array_equal(m["head"], orc.rand_vec(d * SMALL["vocab"], 2037) * np.float32(0.5))


def test_init_model_scales_gains_and_biases(orc):
    """Gpt2::init (params.rs:160-180) on Gpt2::random's draws: gains exactly 1, block biases and
    LayerNorm shifts exactly 0; the weights keep random's draws (each tensor a positive multiple
    of it, so the draw order above carries over) at GPT-style spreads: the token embedding's std
    is 0.02 (uniform draws times 0.02 sqrt 3) and the tensors random scales by 0.5 (position
    embedding, block matrices, head) 0.01, each within 3% on these sizes. A dropped rescale (std
    0.29 / 0.58), a lost 0.5 (0.02 for a matrix) or a gain left random fails one of them."""
    cfg = {"vocab": 512, "ctx": 64, "dim": 64, "heads": 4, "layers": 2, "hidden": 256}
    r, m = gm.gpt2_random(cfg, 3), gm.gpt2_init(cfg, 3)
    for b in m["blocks"]:
        for k in ("ln1_g", "ln2_g"):
            assert np.all(b[k] == 1.0)
        for k in ("ln1_b", "bq", "bk", "bv", "bo", "ln2_b", "b1", "b2"):
            assert np.all(b[k] == 0.0) and not np.signbit(b[k]).any()
    assert np.all(m["lnf_g"] == 1.0) and np.all(m["lnf_b"] == 0.0)
    pairs = [(m["tok"], r["tok"], 0.02), (m["pos"], r["pos"], 0.01), (m["head"], r["head"], 0.01)]
    for bm, br in zip(m["blocks"], r["blocks"]):
        pairs += [(bm[k], br[k], 0.01) for k in ("wq", "wk", "wv", "wo", "w1", "w2")]
    for got, drawn, std in pairs:
        ratio = got.astype(np.float64)[drawn != 0] / drawn[drawn != 0]
        assert np.all(np.abs(ratio / ratio[0] - 1) < 1e-6) and ratio[0] > 0
        assert abs(float(np.std(got)) / std - 1) < 0.03, (std, float(np.std(got)))


@pytest.mark.parametrize("kind", [gm.Q8_0, gm.Q4_0])
def test_export_decodes_to_the_snapped_model(orc, kind):
    m = gm.gpt2_random(SMALL, 5)
    back = gm.from_gguf(gm.to_gguf(m, kind))
    if kind == gm.Q8_0:
        want = gm.fake_quantize(m)
    else:  # Q4_0 has no snap op in the reference: decode(encode) of the same rows
        want = None
    for key in ("tok", "pos", "lnf_g", "lnf_b", "head"):
        if want is not None:
            assert np.array_equal(back[key], want[key]), key
    for i, blk in enumerate(back["blocks"]):
        for name in gm.GPT2_BLOCK_NAMES:
            if want is not None:
                assert np.array_equal(blk[name], want["blocks"][i][name]), (i, name)
    if kind == gm.Q4_0:
        wq = orc.dequantised_in_out(orc.Q4_0, orc.quantise_matrix(orc.Q4_0, m["blocks"][0]["wq"], 64, 64), 64, 64)
        assert np.array_equal(back["blocks"][0]["wq"], wq)


def test_tied_head_is_omitted_and_restored(orc):
    m = gm.tie_head(gm.gpt2_random(SMALL, 6))
    data = gm.to_gguf(m, gm.Q8_0)
    _, tensors, _ = og.parse(data)
    assert "output.weight" not in [t["name"] for t in tensors]
    back = gm.from_gguf(data)
    assert np.array_equal(back["head"], gm.fake_quantize(m)["head"])


def test_reference_fixture_round_trips_through_the_export(orc):
    data = open(os.path.join(GOLDEN, "model.gguf"), "rb").read()
    m = gm.from_gguf(data)
    assert (m["vocab"], m["ctx"], m["dim"], m["heads"], m["layers"], m["hidden"]) == (320, 64, 64, 4, 2, 256)
    again = gm.to_gguf(m, gm.Q8_0)
    _, t1, b1 = og.parse(data)
    _, t2, b2 = og.parse(again)
    by2 = {t["name"]: t for t in t2}
    for t in t1:
        u = by2[t["name"]]
        assert (t["dims"], t["type"]) == (u["dims"], u["type"]), t["name"]
        n = int(np.prod(t["dims"]))
        nb = n * 4 if t["type"] == og.GGML_F32 else n // 32 * 34
        assert data[b1 + t["offset"]: b1 + t["offset"] + nb] == again[b2 + u["offset"]: b2 + u["offset"] + nb], t["name"]
