"""Pins the CPU Llama / Qwen2 oracle (oracle/llama.c, oracle/llama_model.py) that the device's
scoring forward is compared with.

* forward_logits (ferrum_ref/src/models/llama/mod.rs:166-259) must give the logits of an
  independent float64 forward written here from the reference's mathematics: a wrong RoPE
  pairing, table index, GQA head map, bias, norm or causal bound fails it.
* The ops' known answers restate the reference's own unit tests (ferrum_ref/src/models/llama/
  ops.rs:169-300): RMSNorm's formula and unit RMS, SiLU values, RoPE identity at position 0, pair
  norms, partial rotary, scaling by hand, one-position attention, GQA sharing.
* score (ferrum_ref/src/kernels/nn.rs:117-129) against a float64 log-softmax, ties included.
* Llama::random's draw order, dequantised() and the GGUF writer/reader restatements.
"""
import numpy as np
import pytest

from oracle import gguf as og
from oracle import llama_model as lm

V = 17


def cfg(**kw):
    """The reference's GPU test config (ferrum_wgpu/src/models/llama/tests.rs:10-25)."""
    c = lm.config(vocab=V, ctx=10, dim=32, heads=4, kv_heads=2, head_dim=8, layers=2, hidden=64, rope_dim=8,
                  rope_base=10000.0, neox=False, eps=1e-5)
    c.update(kw)
    return c


def variants():
    """(name, config, biases, tied) as ferrum_wgpu/src/models/llama/tests.rs:29-45."""
    return [("llama", cfg(), False, False), ("qwen", cfg(neox=True), True, True),
            ("mqa+partial", cfg(kv_heads=1, rope_dim=4), False, False),
            ("dim24", cfg(dim=24, heads=3, kv_heads=3, head_dim=8, rope_dim=8), True, False)]


IDS = [3, 16, 0, 9, 9, 4, 11, 2, 7, 5]


def forward_f64(m: dict, ids) -> np.ndarray:
    """The causal forward in float64 from the model's definition: RMSNorm, q/k/v (+ bias), RoPE
    at angle pos * base^(-2i/rope_dim) / ff_i / linear, GQA softmax attention over positions
    <= the query's, output projection, SwiGLU FFN, final norm, head."""
    f = lambda a: np.asarray(a, np.float64)
    d, h, heads, kvh, hd = m["dim"], m["hidden"], m["heads"], m["kv_heads"], m["head_dim"]
    qd, kvd, rd, t = heads * hd, kvh * hd, m["rope_dim"], len(ids)
    half = rd // 2
    i = np.arange(half, dtype=np.float64)
    freq = float(m["rope_base"]) ** (-2.0 * i / rd)
    if m.get("freq_factors") is not None:
        freq = freq / f(m["freq_factors"])
    theta = np.arange(t, dtype=np.float64)[:, None] * freq[None, :] / m.get("linear_factor", 1.0)
    cos, sin = np.cos(theta), np.sin(theta)

    def norm(x, g):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + m["eps"]) * f(g)

    def rope(x, nh):
        x = x.reshape(t, nh, hd).copy()
        if m["neox"]:
            a, b = x[:, :, :half].copy(), x[:, :, half:rd].copy()
        else:
            a, b = x[:, :, 0:rd:2].copy(), x[:, :, 1:rd:2].copy()
        c, s = cos[:, None, :], sin[:, None, :]
        ra, rb = a * c - b * s, a * s + b * c
        if m["neox"]:
            x[:, :, :half], x[:, :, half:rd] = ra, rb
        else:
            x[:, :, 0:rd:2], x[:, :, 1:rd:2] = ra, rb
        return x

    x = f(m["tok"]).reshape(m["vocab"], d)[ids]
    mask = np.triu(np.full((t, t), -np.inf), 1)
    for b in m["blocks"]:
        hh = norm(x, b["attn_norm"])
        lin = lambda w, k, n, bias: hh @ f(w).reshape(k, n) + (0 if bias is None else f(bias))
        q = rope(lin(b["wq"], d, qd, b["bq"]), heads)
        k = rope(lin(b["wk"], d, kvd, b["bk"]), kvh)
        v = lin(b["wv"], d, kvd, b["bv"]).reshape(t, kvh, hd)
        a = np.zeros((t, heads, hd))
        for j in range(heads):
            g = j // (heads // kvh)
            sc = q[:, j] @ k[:, g].T / np.sqrt(hd) + mask
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            a[:, j] = (p / p.sum(axis=1, keepdims=True)) @ v[:, g]
        x = x + a.reshape(t, qd) @ f(b["wo"]).reshape(qd, d)
        hh = norm(x, b["ffn_norm"])
        gt, up = hh @ f(b["gate"]).reshape(d, h), hh @ f(b["up"]).reshape(d, h)
        x = x + (gt / (1.0 + np.exp(-gt)) * up) @ f(b["down"]).reshape(h, d)
    return norm(x, m["out_norm"]) @ f(m["head"]).reshape(d, m["vocab"])


def rel(got, want) -> float:
    return float((np.abs(got - want) / np.maximum(np.abs(want), 1.0)).max())


@pytest.mark.parametrize("name,c,biases,tied", variants(), ids=[v[0] for v in variants()])
def test_forward_matches_a_float64_forward(orc, name, c, biases, tied):
    m = lm.llama_random(c, 2, biases, tied)
    want = forward_f64(m, IDS)
    got = orc.llama_forward(m, IDS)
    assert got.shape == (10, V)
    assert rel(got, want) < 2e-5, name


def test_rope_scaling_reaches_the_forward(orc):
    m = lm.llama_random(cfg(), 3, False, False)
    base = orc.llama_forward(m, IDS[:6])
    m["freq_factors"] = np.array([1.0, 2.0, 4.0, 8.0], np.float32)
    m["linear_factor"] = 2.0
    got = orc.llama_forward(m, IDS[:6])
    assert rel(got, forward_f64(m, IDS[:6])) < 2e-5
    assert np.abs(got - base).max() > 1e-4  # "scaling must matter"
    m["freq_factors"], m["linear_factor"] = np.ones(4, np.float32), 1.0
    assert np.array_equal(orc.llama_forward(m, IDS[:6]), base)  # unit factors are no scaling


def test_qwen2_shape_layer_against_float64(orc):
    """One layer at the Qwen2-0.5B widths (d 896, 14 q / 2 kv heads of 64, FFN 4864, NEOX RoPE
    base 1e6, biases, tied head) over 40 tokens; vocab cut to 512. At these widths the f32
    sequential sums round at ~1e-4 of logits that reach ~80, so the bound is normwise (the error
    over the largest logit): 2e-6 observed, where a wrong index or pairing gives O(1)."""
    c = lm.config(vocab=512, ctx=64, dim=896, heads=14, kv_heads=2, head_dim=64, layers=1, hidden=4864,
                  rope_base=1e6, neox=True, eps=1e-6)
    m = lm.llama_random(c, 4, True, True)
    ids = [int(t) for t in np.random.default_rng(0).integers(0, 512, 40)]
    got = orc.llama_forward(m, ids, threads=8)
    want = forward_f64(m, ids)
    assert np.abs(got - want).max() / np.abs(want).max() < 1e-5


def test_threads_and_prefixes_change_nothing(orc):
    m = lm.llama_random(cfg(neox=True), 5, True, False)
    one = orc.llama_forward(m, IDS, threads=1)
    assert np.array_equal(orc.llama_forward(m, IDS, threads=7), one)
    # causality: a prefix gives the prefix's rows (ferrum_ref/src/models/llama/tests.rs:106-111)
    assert np.array_equal(orc.llama_forward(m, IDS[:3]), one[:3])


def test_bad_input_is_refused(orc):
    m = lm.llama_random(cfg(), 1, False, False)
    for bad in ([], [0] * 11, [V]):
        with pytest.raises(ValueError):
            orc.llama_forward(m, bad)


def test_op_known_answers(orc):
    """ferrum_ref/src/models/llama/ops.rs:169-300"""
    y = orc.rmsnorm([3.0, 4.0], [1.0, 2.0], 1, 2, 0.0)
    inv = np.float32(1.0) / np.sqrt(np.float32(12.5))
    assert abs(y[0] - 3 * inv) < 1e-6 and abs(y[1] - 8 * inv) < 1e-6
    y = orc.rmsnorm(orc.rand_vec(24, 1), np.ones(8), 3, 8, 0.0).reshape(3, 8)
    assert np.all(np.abs((y * y).mean(axis=1) - 1) < 1e-4)
    assert orc.silu(0.0) == 0.0 and abs(orc.silu(1.0) - 0.7310586) < 1e-6
    assert abs(orc.silu(-20.0)) < 1e-6 and abs(orc.silu(20.0) - 20.0) < 1e-5
    h = orc.swiglu([1.0, 0.0], [2.0, 5.0])
    assert abs(h[0] - 2 * orc.silu(1.0)) < 1e-6 and h[1] == 0.0
    c, s = orc.rope_tables(0, 1, 4, 10000.0)
    assert list(c) == [1.0, 1.0] and list(s) == [0.0, 0.0]
    x = orc.rand_vec(8, 2)
    assert np.array_equal(orc.apply_rope(x, 1, 2, 4, 4, c, s, False), x)
    x0 = orc.rand_vec(8, 3)
    c, s = orc.rope_tables(5, 1, 8, 10000.0)
    n, e = orc.apply_rope(x0, 1, 1, 8, 8, c, s, False), orc.apply_rope(x0, 1, 1, 8, 8, c, s, True)
    for i in range(4):
        assert abs(x0[2 * i] ** 2 + x0[2 * i + 1] ** 2 - n[2 * i] ** 2 - n[2 * i + 1] ** 2) < 1e-5
        assert abs(x0[i] ** 2 + x0[i + 4] ** 2 - e[i] ** 2 - e[i + 4] ** 2) < 1e-5
    assert not np.array_equal(n, e)
    x = orc.rand_vec(8, 4)
    c, s = orc.rope_tables(3, 1, 4, 10000.0)
    r = orc.apply_rope(x, 1, 1, 8, 4, c, s, True)
    assert np.array_equal(r[4:], x[4:]) and not np.array_equal(r[:4], x[:4])
    c, s = orc.rope_tables(8, 1, 4, 100.0, [2.0, 1.0], 4.0)
    f1 = np.float32(100.0) ** np.float32(-0.5)
    w0, w1 = np.float32(8.0 / 2.0 / 4.0), np.float32(8.0) * f1 / np.float32(4.0)
    assert abs(c[0] - np.cos(w0)) < 1e-6 and abs(s[0] - np.sin(w0)) < 1e-6
    assert abs(c[1] - np.cos(w1)) < 1e-6 and abs(s[1] - np.sin(w1)) < 1e-6
    a = orc.rope_tables(7, 3, 4, 1e4, [1.0, 1.0], 1.0)
    b = orc.rope_tables(7, 3, 4, 1e4)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # one position: each head returns its KV head's v
    q, k, v = orc.rand_vec(12, 5), orc.rand_vec(6, 6), orc.rand_vec(6, 7)
    o = orc.attend_row(q, k, v, 1, 4, 2, 3)
    for hh in range(4):
        g = (hh // 2) * 3
        assert np.array_equal(o[hh * 3:(hh + 1) * 3], v[g:g + 3])
    q1 = orc.rand_vec(4, 8)
    q = np.concatenate([q1, q1])
    o = orc.attend_row(q, orc.rand_vec(12, 9), orc.rand_vec(12, 10), 3, 2, 1, 4)
    assert np.array_equal(o[:4], o[4:])
    o2 = orc.attend_row(q, orc.rand_vec(24, 11), orc.rand_vec(24, 12), 3, 2, 2, 4)
    assert not np.array_equal(o2[:4], o2[4:])


def test_score_is_the_log_softmax_and_the_first_maximum(orc):
    rows, vocab = 5, 6
    logits = orc.rand_vec(rows * vocab, 11) * np.float32(4.0)
    logits[vocab:2 * vocab] = 1.5  # a fully tied row: index 0 is the first maximum
    targets = [0, 0, 3, 5, 1]
    lp, hit = orc.score(logits, targets, vocab)
    x = logits.astype(np.float64).reshape(rows, vocab)
    want = x[np.arange(rows), targets] - x.max(1) - np.log(np.exp(x - x.max(1, keepdims=True)).sum(1))
    assert np.abs(lp - want).max() < 1e-5
    assert list(hit) == [int(np.argmax(x[i])) == targets[i] for i in range(rows)]
    assert hit[1] and abs(lp[1] + np.log(6.0)) < 1e-6
    lp2, hit2 = orc.llama_score(lm.llama_random(cfg(), 8, True, True), [4, 8, 15, 16, 0, 1])
    assert lp2.shape == (5,) and np.all(lp2 <= 0)


def test_random_model_draw_order(orc):
    """Llama::random (params.rs:38-93): s from seed*1000; attn_norm, wq, bq, wk, bk, wv, bv, wo,
    ffn_norm, gate, up, down per block, then tok, head (untied), out_norm."""
    c = cfg()
    m = lm.llama_random(c, 2, True, False)
    qk = np.float32(0.5) * np.sqrt(np.float32(8.0) / np.float32(32))
    assert np.array_equal(m["blocks"][0]["attn_norm"], np.float32(1) + np.float32(0.1) * orc.rand_vec(32, 2001))
    assert np.array_equal(m["blocks"][0]["wq"], orc.rand_vec(32 * 32, 2002) * qk)
    assert np.array_equal(m["blocks"][0]["bq"], orc.rand_vec(32, 2003) * np.float32(0.1))
    assert np.array_equal(m["blocks"][1]["down"], orc.rand_vec(64 * 32, 2024) * np.float32(0.5))
    assert np.array_equal(m["tok"], orc.rand_vec(V * 32, 2025))
    assert np.array_equal(m["head"], orc.rand_vec(32 * V, 2026) * np.float32(0.5))
    assert np.array_equal(m["out_norm"], np.float32(1) + np.float32(0.1) * orc.rand_vec(32, 2027))
    t = lm.llama_random(c, 2, False, True)
    assert np.array_equal(t["head"], orc.transpose(t["tok"], V, 32))
    assert np.array_equal(t["out_norm"], np.float32(1) + np.float32(0.1) * orc.rand_vec(32, 2020))
    assert np.array_equal(t["tok"], orc.rand_vec(V * 32, 2019))
    assert t["blocks"][0]["bq"] is None


@pytest.mark.parametrize("kind", [lm.Q8_0, lm.Q4_0])
@pytest.mark.parametrize("name,c,biases,tied", variants(), ids=[v[0] for v in variants()])
def test_gguf_round_trip_is_the_dequantised_model(orc, kind, name, c, biases, tied):
    """from_gguf(to_gguf(m)) decodes to dequantised(m) except the embedding, which the file
    stores as rows (ferrum_wgpu/src/models/llama/tests.rs:92-112: requantising a loaded model is
    the identity)."""
    m = lm.llama_random(c, 4, biases, tied)
    data = lm.to_gguf(m, kind)
    back = lm.from_gguf(data)
    want = lm.dequantised(m, kind)
    for key in lm.CONFIG_KEYS:
        assert back[key] == pytest.approx(m[key]), key
    for i, blk in enumerate(back["blocks"]):
        for key in lm.LLAMA_BLOCK_NAMES:
            a, b = blk[key], want["blocks"][i][key]
            assert (a is None and b is None) or np.array_equal(a, b), (name, i, key)
    again = lm.dequantised(back, kind)
    for i, blk in enumerate(again["blocks"]):
        for key in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
            assert np.array_equal(blk[key], back["blocks"][i][key])
    assert np.array_equal(again["head"], back["head"])
    assert back["tied"] == tied
    names = [t["name"] for t in og.parse(data)[1]]
    assert ("output.weight" in names) == (not tied)
    assert ("blk.0.attn_q.bias" in names) == biases
    kv = {k: v.v for k, v in og.parse(data)[0]}
    assert kv["general.architecture"] == ("qwen2" if c["neox"] else "llama")


def test_tied_quantised_head_is_the_embeddings_rows(orc):
    m = lm.llama_random(cfg(neox=True), 6, True, True)
    back = lm.from_gguf(lm.to_gguf(m, lm.Q4_0))
    assert np.array_equal(back["head"], orc.transpose(back["tok"], V, 32))
    assert np.array_equal(back["tok"], orc.decode(lm.Q4_0, orc.encode(lm.Q4_0, m["tok"]), V * 32))
