"""Llama / Qwen2 full-sequence forward and scoring on the device against the CPU oracle
(ferrum_ref's Llama::forward_logits and nn::score on the weights the GGUF stores). Mirrors
ferrum_wgpu/src/models/llama/tests.rs (forward_all per variant, quantised GGUF models, score,
RoPE scaling, bad input) on packed Q8_0 / Q4_0 weights, plus the Qwen2-0.5B shape of the scoring
benchmark.

Tolerances. The precise path (FH_PATH_TILED) keeps the reference's FORWARD bound on logits,
max |g - w| / max(|w|, 1) < 1e-5 (ferrum_wgpu/src/tolerance.rs:11), and its score bound,
|g - w| < 1e-4 max(|w|, 1) per log-probability with identical first-argmax flags
(ferrum_wgpu/src/models/llama/tests.rs:177-194). The fast scoring path (FH_PATH_TILED_FAST) runs
every product with x rounded to f16 plus an e4m3 correction (relative error ~3e-5 per product);
its log-probabilities are held to FAST_LOGPROB = 5e-4 relative (observed 1.2e-4 at the
Qwen2-0.5B shape, 3e-5 on the small variants; the MFMA-GEMM tolerance is 2e-3). The dequant-f16
path (FH_PATH_TILED_F16) rounds x and every weight d q to f16 (2^-11 each) and is held to
F16_LOGPROB = 1e-2 relative (observed 3.8e-3 at the Qwen2-0.5B shape, whose 24 layers of
uniformly drawn weights amplify the roundings, and 5e-4 to 9e-4 on the small variants)."""
import os
import time

import numpy as np
import pytest

from oracle import llama_model as lm

pytestmark = pytest.mark.gpu
FORWARD = 1e-5
SCORE = 1e-4
FAST_LOGPROB = 5e-4
F16_LOGPROB = 1e-2
V = 17
IDS = [3, 16, 0, 9, 9, 4, 11, 2, 7, 5]


def say(*a):
    print(*a, flush=True)


def cfg(**kw):
    """ferrum_wgpu/src/models/llama/tests.rs:10-25"""
    c = lm.config(vocab=V, ctx=10, dim=32, heads=4, kv_heads=2, head_dim=8, layers=2, hidden=64, rope_dim=8,
                  rope_base=10000.0, neox=False, eps=1e-5)
    c.update(kw)
    return c


def variants():
    """tests.rs:29-45: llama-like, qwen-like with biases and a tied head, partial rotary with MQA,
    and dim24, whose 24-wide matrices (q/k/v, output, gate/up, the embedding and head) have no
    Q8_0/Q4_0 form: the GGUF stores them F32 and the device multiplies them as f32 (Lin::upload,
    ferrum_wgpu/src/models/llama/lin.rs:30-62), while ffn_down (64 wide) stays packed."""
    return [("llama", cfg(), False, False), ("qwen", cfg(neox=True), True, True),
            ("mqa+partial", cfg(kv_heads=1, rope_dim=4), False, False),
            ("dim24", cfg(dim=24, heads=3, kv_heads=3, head_dim=8, rope_dim=8), True, False)]


@pytest.fixture(scope="module")
def fh():
    import ferrum_hip

    return ferrum_hip


@pytest.fixture(scope="module")
def g(fh):
    gpu = fh.Gpu.open_for_test()
    if gpu is None:
        pytest.skip("no gfx950 device")
    yield gpu
    gpu.close()


def load(fh, g, data: bytes, path=None):
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.llama import GpuLlama

    return GpuLlama.from_gguf(g, Gguf.parse(data), fh.QPath.Tiled if path is None else path)


def rel(got, want) -> float:
    """ferrum_wgpu/src/tolerance.rs:14-26"""
    return float((np.abs(got - want) / np.maximum(np.abs(want), 1.0)).max())


def lp_err(got, want) -> float:
    return float((np.abs(got - want) / np.maximum(np.abs(want), 1.0)).max())


@pytest.mark.parametrize("kind", [lm.Q8_0, lm.Q4_0])
@pytest.mark.parametrize("name,c,biases,tied", variants(), ids=[v[0] for v in variants()])
def test_forward_all_matches_the_oracle_for_every_variant(fh, g, orc, kind, name, c, biases, tied):
    """tests.rs:92-131: a model loaded from a quantised GGUF, every prefix length, FORWARD."""
    data = lm.to_gguf(lm.llama_random(c, 5, biases, tied), kind)
    ref = lm.from_gguf(data)
    dev = load(fh, g, data)
    cf = dev.config()
    assert (cf.vocab, cf.dim, cf.heads, cf.kv_heads, cf.head_dim, cf.rope_dim, cf.neox, cf.tied) == \
        (V, c["dim"], c["heads"], c["kv_heads"], c["head_dim"], c["rope_dim"], c["neox"], tied)
    for t in (1, 2, 7, 10):
        e = rel(dev.forward_all(IDS[:t]), orc.llama_forward(ref, IDS[:t]))
        say(f"{name} kind {kind} t={t}: {e:.2e}")
        assert e < FORWARD, (name, t, e)


def test_bad_input_is_refused_with_the_reference_messages(fh, g, orc):
    dev = load(fh, g, lm.to_gguf(lm.llama_random(cfg(), 1, False, False), lm.Q8_0))
    for bad, msg in (([], "sequence length 0 must be in 1..=10"), ([0] * 11, "sequence length 11"),
                     ([V], "token 17 is out of range for vocab 17")):
        with pytest.raises(fh.GpuError) as err:
            dev.forward_all(bad)
        assert msg in str(err.value)
    with pytest.raises(fh.GpuError) as err:
        dev.score([1])
    assert "scoring needs at least 2 tokens" in str(err.value)
    with pytest.raises(fh.GpuError) as err:
        dev.score([1, 2, V])
    assert "out of range" in str(err.value)
    assert dev.forward_all([1, 2]).shape == (2, V)  # still usable


def test_score_matches_the_oracle(fh, g, orc):
    """tests.rs:177-194: Llama::random(cfg, 8, biases, tied), ids [4, 8, 15, 16, 0, 1]."""
    data = lm.to_gguf(lm.llama_random(cfg(), 8, True, True), lm.Q8_0)
    ref = lm.from_gguf(data)
    ids = [4, 8, 15, 16, 0, 1]
    want_lp, want_hit = orc.llama_score(ref, ids)
    dev = load(fh, g, data)
    got = dev.score(ids)
    assert len(got) == 5
    for i, ((glp, ghit), wlp, whit) in enumerate(zip(got, want_lp, want_hit)):
        assert abs(glp - wlp) < SCORE * max(abs(wlp), 1.0), (i, glp, wlp)
        assert ghit == bool(whit), i
    # a longer run over the whole context, flags included
    lp, hit = dev.score_arrays(IDS)
    wlp, whit = orc.llama_score(ref, IDS)
    assert lp_err(lp, wlp) < SCORE and np.array_equal(hit, whit)


def test_score_device_matches_score(fh, g, orc):
    data = lm.to_gguf(lm.llama_random(cfg(neox=True), 9, True, False), lm.Q4_0)
    dev = load(fh, g, data)
    lp, hit = dev.score_arrays(IDS)
    ids = g.upload_bytes(np.asarray(IDS, np.int32).view(np.uint8))
    out = g.zeros(2 * (len(IDS) - 1))
    dev.score_device(ids, len(IDS), out)
    pairs = g.read(out).reshape(-1, 2)
    assert np.array_equal(pairs[:, 0], lp)
    assert np.array_equal(pairs[:, 1] == 1.0, hit)


def test_rope_scaling_is_honoured_on_the_device(fh, g, orc):
    """tests.rs:152-175: rope_freqs.weight and linear scaling from the GGUF."""
    m = lm.llama_random(cfg(), 7, False, False)
    m["freq_factors"] = np.array([1.0, 2.0, 4.0, 8.0], np.float32)
    m["linear_factor"] = 2.0
    data = lm.to_gguf(m, lm.Q8_0)
    ref = lm.from_gguf(data)
    assert ref["linear_factor"] == 2.0 and np.array_equal(ref["freq_factors"], m["freq_factors"])
    plain = dict(ref, freq_factors=None, linear_factor=1.0)
    want = orc.llama_forward(ref, IDS[:6])
    assert np.abs(want - orc.llama_forward(plain, IDS[:6])).max() > 1e-3  # scaling must matter
    assert rel(load(fh, g, data).forward_all(IDS[:6]), want) < FORWARD


@pytest.mark.parametrize("kind", [lm.Q8_0, lm.Q4_0])
def test_unpackable_widths_run_as_f32(fh, g, orc, kind):
    """dim24 (tests.rs:36-41): the 24-wide matrices load as f32 rows (4 bytes a weight), the
    64-wide ffn_down packed; the fast scoring path, whose fused producers need packed
    consumers, runs its unfused form; every path scores like the oracle."""
    c = cfg(dim=24, heads=3, kv_heads=3, head_dim=8, rope_dim=8)
    data = lm.to_gguf(lm.llama_random(c, 1, True, False), kind)
    ref = lm.from_gguf(data)
    d, h, L = 24, 64, 2
    f32_bytes = 4 * (V * d + L * (d * (3 * d) + d * d + d * 2 * h))  # head, q/k/v, o, gate/up (untied: the
    # embedding is a lookup table, not a product's weight)
    packed = L * (h // 32) * d * (34 if kind == lm.Q8_0 else 18)  # ffn_down
    wlp, whit = orc.llama_score(ref, IDS)
    for path, bar in (("Tiled", SCORE), ("TiledFast", FAST_LOGPROB), ("TiledF16", F16_LOGPROB)):
        dev = load(fh, g, data, fh.QPath[path])
        assert dev.weight_bytes() == f32_bytes + packed
        assert dev.device_bytes() >= f32_bytes + packed
        lp, hit = dev.score_arrays(IDS)
        e = lp_err(lp, wlp)
        say(f"dim24 kind {kind} {path}: log-prob rel err {e:.2e}")
        assert e < bar, (path, e)


@pytest.mark.parametrize("path", ["TiledFast", "TiledF16"])
@pytest.mark.parametrize("name,c,biases,tied", variants(), ids=[v[0] for v in variants()])
def test_fast_paths_stay_within_their_bounds(fh, g, orc, name, c, biases, tied, path):
    data = lm.to_gguf(lm.llama_random(c, 11, biases, tied), lm.Q4_0)
    ref = lm.from_gguf(data)
    dev = load(fh, g, data, fh.QPath[path])
    assert dev.config().path == fh.QPath[path]
    lp, hit = dev.score_arrays(IDS)
    wlp, whit = orc.llama_score(ref, IDS)
    e = lp_err(lp, wlp)
    say(f"{path} {name}: log-prob rel err {e:.2e}, logits {rel(dev.forward_all(IDS), orc.llama_forward(ref, IDS)):.2e}")
    assert e < (FAST_LOGPROB if path == "TiledFast" else F16_LOGPROB)


@pytest.mark.parametrize("path", ["Tiled", "TiledFast"])
def test_score_epilogue_matches_the_logits_and_score_kernel(fh, g, orc, path):
    """The score folded into the head GEMM's epilogue (per row and 256-column tile the maximum, the
    sum of exponentials, the first maximum's column and the target's logit, merged per row) against
    the same model with FERRUM_HIP_SCORE_UNFUSED=1 (the logits written, then score_kernel): the same
    logits, summed in another order, so log-probabilities within 1e-6 and identical first-argmax
    flags; and both against the oracle. Vocab 1000 is four column tiles, the last 232 wide; 299
    scored rows are two row tiles, the second partly filled; targets include every tile's first and
    last column."""
    c = cfg(vocab=1000, ctx=300, dim=64, heads=4, kv_heads=2, head_dim=16, hidden=128, rope_dim=16)
    data = lm.to_gguf(lm.llama_random(c, 13, True, False), lm.Q8_0)
    ref = lm.from_gguf(data)
    fused = load(fh, g, data, fh.QPath[path])
    old = os.environ.get("FERRUM_HIP_SCORE_UNFUSED")
    os.environ["FERRUM_HIP_SCORE_UNFUSED"] = "1"
    try:
        plain = load(fh, g, data, fh.QPath[path])
    finally:
        if old is None:
            os.environ.pop("FERRUM_HIP_SCORE_UNFUSED")
        else:
            os.environ["FERRUM_HIP_SCORE_UNFUSED"] = old
    ids = [int(t) for t in np.random.default_rng(5).integers(0, 1000, 300)]
    ids[1:9] = [0, 255, 256, 511, 512, 767, 768, 999]
    lp, hit = fused.score_arrays(ids)
    lp0, hit0 = plain.score_arrays(ids)
    assert lp.shape == (299,) and np.all(np.isfinite(lp))
    assert np.array_equal(hit, hit0)
    e = lp_err(lp, lp0)
    wlp, whit = orc.llama_score(ref, ids)
    say(f"{path}: fused vs unfused log-prob rel err {e:.2e}; vs oracle {lp_err(lp, wlp):.2e}; hits {int(hit.sum())}")
    assert e < 1e-6
    assert lp_err(lp, wlp) < (SCORE if path == "Tiled" else FAST_LOGPROB)
    if path == "Tiled":
        assert np.array_equal(hit, whit)


def load_env(fh, g, data, path, var):
    """The model loaded with environment variable `var` set to 1 (a load-time switch)."""
    old = os.environ.get(var)
    os.environ[var] = "1"
    try:
        return load(fh, g, data, path)
    finally:
        if old is None:
            os.environ.pop(var)
        else:
            os.environ[var] = old


@pytest.mark.parametrize("shape", ["epilogue", "epilogue_odd_blocks", "fallback"])
def test_swiglu_epilogue_is_bit_identical_to_the_swiglu_pass(fh, g, orc, shape):
    """The fast path's SwiGLU in the gate/up GEMM's epilogue (gate and up rows interleaved in runs
    of 32 at load) against the same model loaded with FERRUM_HIP_SWIGLU_UNFUSED=1 (the stacked
    product, then swiglu_split_kernel): the same accumulators and the same activation function,
    so logits and log-probabilities bit-identical. "epilogue": d 64 (one pipeline stage, never
    split along K), so the epilogue runs; "epilogue_odd_blocks" the same with an FFN of 96 (three
    32-unit blocks, so the epilogue also writes the empty block that completes the down product's
    last x lo pair). "fallback": d 512 with 16 tiles, which the GEMM splits
    along K, so the interleaved weight goes through the plain product and the interleave-aware
    SwiGLU pass instead."""
    if shape.startswith("epilogue"):
        hid = 96 if shape == "epilogue_odd_blocks" else 256
        c = cfg(vocab=500, ctx=256, dim=64, heads=4, kv_heads=2, head_dim=16, hidden=hid, rope_dim=16)
        n_ids = 201
    else:
        c = cfg(vocab=500, ctx=256, dim=512, heads=8, kv_heads=4, head_dim=64, hidden=512, rope_dim=64)
        n_ids = 101
    data = lm.to_gguf(lm.llama_random(c, 17, True, False), lm.Q4_0)
    fused = load(fh, g, data, fh.QPath.TiledFast)
    plain = load_env(fh, g, data, fh.QPath.TiledFast, "FERRUM_HIP_SWIGLU_UNFUSED")
    ids = [int(t) for t in np.random.default_rng(8).integers(0, 500, n_ids)]
    lf, lp = fused.forward_all(ids), plain.forward_all(ids)
    assert np.all(np.isfinite(lf))
    same = np.array_equal(np.asarray(lf, np.float32).view(np.uint32), np.asarray(lp, np.float32).view(np.uint32))
    sf, hf = fused.score_arrays(ids)
    sp, hp = plain.score_arrays(ids)
    wlp, _ = orc.llama_score(lm.from_gguf(data), ids)
    say(f"{shape}: logits bit-identical {same}; log-probs vs oracle {lp_err(sf, wlp):.2e}")
    assert same
    assert np.array_equal(np.asarray(sf, np.float32).view(np.uint32), np.asarray(sp, np.float32).view(np.uint32))
    assert np.array_equal(hf, hp)
    assert lp_err(sf, wlp) < FAST_LOGPROB


@pytest.mark.parametrize("kind,head_dim,heads,kv_heads,dim", [(lm.Q4_0, 32, 3, 1, 128), (lm.Q8_0, 64, 4, 2, 256),
                                                              (lm.Q4_0, 128, 2, 1, 256)])
def test_attention_split_output_is_bit_identical_to_the_split_pass(fh, g, kind, head_dim, heads, kv_heads, dim):
    """On the fast path the split attention writes the output product's split x itself (per
    32-dim block: hi in the weight kind's operand order, lo in the pair order, the block's scale)
    instead of f32 rows that split_x_kernel then splits (FERRUM_HIP_ATTN_SPLIT_UNFUSED=1 at load):
    the same values, so logits and log-probabilities bit-identical. Both operand orders, head dims
    32, 64 and 128, and 3 heads of 32 (an odd block count: the last pair's empty block), at a
    ragged length."""
    c = lm.config(vocab=300, ctx=128, dim=dim, heads=heads, kv_heads=kv_heads, head_dim=head_dim, layers=2,
                  hidden=256, rope_base=10000.0, neox=True, eps=1e-5)
    data = lm.to_gguf(lm.llama_random(c, 29, True, False), kind)
    fused = load(fh, g, data, fh.QPath.TiledFast)
    plain = load_env(fh, g, data, fh.QPath.TiledFast, "FERRUM_HIP_ATTN_SPLIT_UNFUSED")
    ids = [int(t) for t in np.random.default_rng(head_dim).integers(0, 300, 97)]
    lf, lp = fused.forward_all(ids), plain.forward_all(ids)
    assert np.all(np.isfinite(lf))
    assert np.array_equal(np.asarray(lf, np.float32).view(np.uint32), np.asarray(lp, np.float32).view(np.uint32))
    sf, hf = fused.score_arrays(ids)
    sp, hp = plain.score_arrays(ids)
    assert np.array_equal(np.asarray(sf, np.float32).view(np.uint32), np.asarray(sp, np.float32).view(np.uint32))
    assert np.array_equal(hf, hp)


@pytest.fixture(scope="module")
def qwen(fh, g):
    """The scoring benchmark's model: Qwen2-0.5B shapes (24 layers, d 896, FFN 4864, 14 q / 2 kv
    heads of 64, NEOX RoPE base 1e6, q/k/v biases, vocab 151936, tied head), Q4_0, with
    Llama::random-distributed synthetic weights; and its decoded f32 form for the oracle."""
    from ferrum_hip.llama import QWEN2_0_5B, random_gguf

    t0 = time.time()
    data = random_gguf(g, dict(QWEN2_0_5B, ctx=4096), fh.QKind.Q4_0, seed=1)
    ref = lm.from_gguf(data)
    say(f"qwen2-0.5b model built in {time.time() - t0:.1f} s ({len(data) / 1e6:.1f} MB GGUF)")
    return data, ref


@pytest.mark.parametrize("path", ["Tiled", "TiledFast", "TiledF16"])
def test_qwen2_0_5b_scoring_matches_the_oracle(fh, g, orc, qwen, path):
    data, ref = qwen
    dev = load(fh, g, data, fh.QPath[path])
    assert dev.weight_bytes() == 277_853_184  # the packed Q4_0 bytes of every matrix and the head
    # the device footprint: padded planes, vectors, tables; the fast path adds a byte per weight
    db = dev.device_bytes()
    say(f"{path}: device bytes {db / 1e6:.1f} MB")
    assert db > 277_853_184
    if path == "TiledFast":
        assert db > 277_853_184 + 493_961_216
    ids = [int(t) for t in np.random.default_rng(2024).integers(0, 151936, 129)]
    t0 = time.time()
    wlp, whit = orc.llama_score(ref, ids, threads=min(16, os.cpu_count() or 1))
    say(f"oracle score of 128 rows in {time.time() - t0:.1f} s")
    lp, hit = dev.score_arrays(ids)
    e = lp_err(lp, wlp)
    say(f"{path}: log-prob rel err {e:.2e} (abs {np.abs(lp - wlp).max():.2e}); lp range {wlp.min():.1f}..{wlp.max():.1f}")
    bound = {"Tiled": SCORE, "TiledFast": FAST_LOGPROB, "TiledF16": F16_LOGPROB}[path]
    assert e < bound
    if path == "Tiled":
        assert np.array_equal(hit, whit)
    # causality at the benchmark lengths: the 512- and 2048-row passes agree on the first rows
    more = ids + [int(t) for t in np.random.default_rng(7).integers(0, 151936, 2048 - 128)]
    lp512, _ = dev.score_arrays(more[:513])
    lp2048, hit2048 = dev.score_arrays(more)
    assert lp512.shape == (512,) and lp2048.shape == (2048,)
    assert np.all(np.isfinite(lp2048)) and np.all(lp2048 <= 0)
    assert lp_err(lp512[:128], wlp) < bound and lp_err(lp2048[:512], lp512) < bound


@pytest.mark.parametrize("head_dim,neox,rope_dim", [(32, True, None), (64, True, None), (128, True, None),
                                                     (64, False, 32)])
def test_split_attention_head_dims_match_the_oracle(fh, g, orc, head_dim, neox, rope_dim):
    """Head dims 32, 64 and 128 take the f16-split attention (q, k, v on a power-of-two scale in
    two f16 parts, k and v stored in the kernel's fragment order); grouped kv heads, sequence
    lengths that leave some wavefronts without a key tile (1, 33) and span several query blocks
    and key tiles with a ragged last one (97); NEOX pairing over the whole head, and NORM pairing
    over half of it (rope_dim 32 of 64). Logits against the oracle within SCORE (1e-4
    relative to max(|w|, 1)), not FORWARD: at these widths (dim 128 to 512, logits up to 26) the
    f32 oracle is itself 1.2e-5 to 4.3e-5 from an f64 evaluation of the same model (measured), so
    1e-5 would test the oracle's rounding. A misplaced fragment element gives O(1) errors and an
    f16-only operand (the lo part lost) errors of the order of f16 rounding, 2^-11 = 4.9e-4."""
    c = lm.config(vocab=300, ctx=128, dim=4 * head_dim, heads=4, kv_heads=2, head_dim=head_dim, layers=2,
                  hidden=256, rope_dim=rope_dim, rope_base=10000.0, neox=neox, eps=1e-5)
    data = lm.to_gguf(lm.llama_random(c, 17, True, False), lm.Q8_0)
    ref = lm.from_gguf(data)
    dev = load(fh, g, data)
    # the RoPE and the split as two kernels (what q/k/v rows too wide for one workgroup's LDS take)
    os.environ["FERRUM_HIP_ROPE_UNFUSED"] = "1"
    try:
        two = load(fh, g, data)
    finally:
        del os.environ["FERRUM_HIP_ROPE_UNFUSED"]
    ids = [int(t) for t in np.random.default_rng(head_dim).integers(0, 300, 97)]
    for t in (1, 33, 97):
        got = dev.forward_all(ids[:t])
        e = rel(got, orc.llama_forward(ref, ids[:t]))
        say(f"head_dim {head_dim} t={t}: {e:.2e}")
        assert e < SCORE, (head_dim, t, e)
        assert np.array_equal(got, two.forward_all(ids[:t])), (head_dim, t)


@pytest.mark.parametrize("head_dim", [32, 64, 128])
def test_rope_split_tiles_are_bit_identical_to_the_two_pass_split(fh, g, head_dim):
    """qkv_rope_split_kernel takes 32-row tiles when they give at least two workgroups per CU
    (here 8 head slots x 64 tiles at t = 2048) and 16-row tiles below that (t = 1000, ragged):
    each writes whole k' and v' fragment lines from one workgroup. Both against the two-pass
    RoPE and split (FERRUM_HIP_ROPE_UNFUSED=1), logits bit for bit, for head dims 32, 64 and 128
    (a row's lane group of 8, 16 or 32 lanes). dim 1024 against 4 heads splits the QKV product
    along K at both lengths, so the tiles add partial sums."""
    c = lm.config(vocab=300, ctx=2048, dim=1024, heads=4, kv_heads=2, head_dim=head_dim, layers=2, hidden=256,
                  rope_base=10000.0, neox=False, eps=1e-5)
    data = lm.to_gguf(lm.llama_random(c, 23, True, False), lm.Q8_0)
    dev = load(fh, g, data, fh.QPath.TiledFast)
    os.environ["FERRUM_HIP_ROPE_UNFUSED"] = "1"
    try:
        two = load(fh, g, data, fh.QPath.TiledFast)
    finally:
        del os.environ["FERRUM_HIP_ROPE_UNFUSED"]
    ids = [int(t) for t in np.random.default_rng(5).integers(0, 300, 2048)]
    for t in (2048, 1000):
        got = dev.forward_all(ids[:t])
        assert np.all(np.isfinite(got)), t
        assert np.array_equal(got, two.forward_all(ids[:t])), t


@pytest.mark.parametrize("kind", [lm.Q8_0, lm.Q4_0])
def test_fast_path_with_narrow_attention_and_ffn(fh, g, orc, kind):
    """heads * key_length and the FFN width both below dim (ferrum_model/src/gguf/llama/mod.rs:133
    reads key_length from the file): the attention-output and down products are narrower than
    dim, and at t = 160 both split along K. Their partial sums are added by the next RMSNorm while
    it writes the next product's split x, which is dim wide; the two must not share memory."""
    c = lm.config(vocab=300, ctx=160, dim=1024, heads=8, kv_heads=2, head_dim=64, layers=2, hidden=512,
                  rope_base=10000.0, neox=True, eps=1e-5)
    data = lm.to_gguf(lm.llama_random(c, 13, True, False), kind)
    ref = lm.from_gguf(data)
    ids = [int(t) for t in np.random.default_rng(3).integers(0, 300, 160)]
    wlp, whit = orc.llama_score(ref, ids, threads=min(16, os.cpu_count() or 1))
    precise = load(fh, g, data, fh.QPath.Tiled)
    plp, phit = precise.score_arrays(ids)
    assert lp_err(plp, wlp) < SCORE and np.array_equal(phit, whit)
    fast = load(fh, g, data, fh.QPath.TiledFast)
    for rep in range(3):
        lp, hit = fast.score_arrays(ids)
        e = lp_err(lp, wlp)
        say(f"kind {kind} fast path rep {rep}: log-prob rel err {e:.2e}")
        assert e < FAST_LOGPROB, (rep, e)
