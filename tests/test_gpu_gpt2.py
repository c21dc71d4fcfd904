"""GPT-2 decode on the device against the CPU oracle (ferrum_ref's Gpt2::feed on the same stored
weights): logits within the reference's FORWARD tolerance (1e-5, ferrum_wgpu/src/tolerance.rs),
greedy token IDs identical. Mirrors ferrum_wgpu/src/models/gpt2.rs:433-520 (feed row by row,
reset, greedy generation, GGUF round trip) on packed Q8_0 / Q4_0 weights, plus the reference's
fixture model.gguf and the GPT-2-small shape of the decode benchmark."""
import os
import time

import numpy as np
import pytest

from oracle import gpt2_model as gm

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORWARD = 1e-5
SMALL = {"vocab": 96, "ctx": 12, "dim": 64, "heads": 4, "layers": 2, "hidden": 128}
MID = {"vocab": 1000, "ctx": 128, "dim": 256, "heads": 4, "layers": 3, "hidden": 1024}


def say(*a):
    print(*a, flush=True)


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


def load(g, data: bytes):
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.gpt2 import GpuGpt2

    return GpuGpt2.from_gguf(g, Gguf.parse(data))


def rel(got, want) -> float:
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1.0))


def margin(logits) -> float:
    s = np.sort(logits)
    return float(s[-1] - s[-2])


def test_fixture_feed_matches_the_oracle_row_by_row(g, orc):
    data = open(os.path.join(GOLDEN, "model.gguf"), "rb").read()
    m = gm.from_gguf(data)
    dev = load(g, data)
    cfg = dev.config()
    assert (cfg.vocab, cfg.ctx, cfg.dim, cfg.heads, cfg.layers, cfg.hidden) == (320, 64, 64, 4, 2, 256)
    cpu = orc.Gpt2Cpu(m)
    ids = [int(t) for t in np.random.default_rng(1).integers(0, 320, 64)]  # the whole context
    for i, t in enumerate(ids):
        e = rel(dev.feed(t), cpu.feed(t))
        assert e < FORWARD, (i, e)
    assert dev.pos() == 64
    with pytest.raises(Exception) as err:
        dev.feed(1)
    assert "full" in str(err.value)
    assert dev.pos() == 64


@pytest.mark.parametrize("kind", [gm.Q8_0, gm.Q4_0])
def test_random_model_feed_reset_and_errors(g, orc, kind):
    m = gm.gpt2_random(SMALL, 2)
    data = gm.to_gguf(m, kind)
    dev = load(g, data)
    cpu = orc.Gpt2Cpu(gm.from_gguf(data))
    ids = [3, 16, 0, 9, 9, 4, 11, 2, 7, 5, 95, 1]
    first = []
    for i, t in enumerate(ids):
        got = dev.feed(t)
        first.append(got)
        e = rel(got, cpu.feed(t))
        say(f"kind {kind} pos {i}: max rel err {e:.2e}")
        assert e < FORWARD, (i, e)
    with pytest.raises(Exception) as err:
        dev.feed(0)
    assert "full" in str(err.value)
    dev.reset()
    assert dev.pos() == 0
    with pytest.raises(Exception) as err:
        dev.feed(96)
    assert "out of range for vocab 96" in str(err.value)
    assert dev.pos() == 0
    again = [dev.feed(t) for t in ids[:4]]
    for a, b in zip(first, again):  # the same answers, bit for bit, after a reset
        assert np.array_equal(a, b)


@pytest.mark.parametrize("tied", [False, True])
def test_greedy_generation_matches_the_oracle_token_for_token(g, orc, tied):
    m = gm.gpt2_random(MID, 6)
    if tied:
        m = gm.tie_head(m)
    data = gm.to_gguf(m, gm.Q8_0)
    ref = gm.from_gguf(data)
    dev = load(g, data)
    prompt = [int(t) for t in np.random.default_rng(7).integers(0, MID["vocab"], 16)]
    want = orc.gpt2_generate(ref, prompt, 100)
    got = dev.generate(prompt, 100)
    assert got == want
    assert dev.pos() == 16 + 99
    # feed with the same history agrees with generate's picks
    dev.reset()
    for t in prompt:
        logits = dev.feed(t)
    for i in range(10):
        assert int(np.argmax(logits)) == want[i]
        logits = dev.feed(want[i])


def test_generate_continues_from_the_current_position(g, orc):
    m = gm.gpt2_random(SMALL, 8)
    data = gm.to_gguf(m, gm.Q8_0)
    dev = load(g, data)
    a = dev.generate([1, 2, 3], 3)       # positions 0..4
    b = dev.generate([a[-1], 7], 4)      # continues at position 5
    cpu = orc.Gpt2Cpu(gm.from_gguf(data))
    seq = [1, 2, 3] + a[:-1] + [a[-1], 7] + b[:-1]
    picks = [int(np.argmax(cpu.feed(t))) for t in seq]
    assert picks[2:5] == a and picks[-4:] == b
    with pytest.raises(Exception) as err:
        dev.generate([1], 4)  # needs 4 more positions, 2 left
    assert "full" in str(err.value)


@pytest.mark.parametrize("init", ["reference", "gpt2"])
def test_gpt2_small_shape_decodes_the_oracles_tokens(fh, g, orc, init):
    """The decode benchmark's model: GPT-2-small shapes (12 layers, d 768, 12 heads, vocab 50257,
    ctx 1024, tied head), stored Q8_0 by the device encoder; 32 uniform-random prompt tokens, 256
    greedy tokens, identical IDs, and the logits of the first 8 steps within FORWARD. The file the
    device writes is byte for byte the oracle's export of the same weights. Weights: "reference"
    is ferrum_ref's Gpt2::init (params.rs:160-180) with the head tied (Gpt2::tie_head, mod.rs:
    119-123); "gpt2" is GPT-2's published initialisation (ferrum_hip.gpt2.gpt2_init, the bench's
    model). (Gpt2::random's raw weights, uniform +-0.5, make this shape numerically chaotic: the
    CPU's own f32 logits leave the float64 ones by 1e-1 within 40 tokens, so no differently
    rounded implementation can follow them token for token; Gpt2::init rescales those draws.)"""
    from ferrum_hip.gpt2 import gpt2_init, to_gguf

    cfg = {"vocab": 50257, "ctx": 1024, "dim": 768, "heads": 12, "layers": 12, "hidden": 3072}
    t0 = time.time()
    if init == "reference":
        m = gm.gpt2_init(cfg, 1)
        m["head"] = None  # tied: the transposed token embedding
    else:
        m = gpt2_init(cfg, 1)
    data = to_gguf(g, m, fh.QKind.Q8_0)
    om = dict(m)
    om["head"] = orc.transpose(m["tok"], cfg["vocab"], cfg["dim"])
    assert data == gm.to_gguf(om, gm.Q8_0)
    ref = gm.from_gguf(data)
    say(f"gpt2-small ({init} init) built and checked in {time.time() - t0:.1f} s ({len(data) / 1e6:.1f} MB GGUF)")
    prompt = [int(t) for t in np.random.default_rng(2024).integers(0, cfg["vocab"], 32)]
    dev = load(g, data)
    assert dev.step_bytes() == 131_252_784
    got = dev.generate(prompt, 256)
    t0 = time.time()
    want = orc.gpt2_generate(ref, prompt, 256)
    say(f"oracle decode {time.time() - t0:.1f} s")
    assert got == want
    # the logits along the way: the first 8 steps against the oracle's
    dev.reset()
    cpu = orc.Gpt2Cpu(ref)
    worst = 0.0
    for t in prompt[:8]:
        worst = max(worst, rel(dev.feed(t), cpu.feed(t)))
    say(f"gpt2-small ({init} init) logits max rel err over 8 steps: {worst:.2e}")
    assert worst < FORWARD
