"""The four-launch GPT-2 decode step (per layer: LN1 + QKV with the residual row formed from the
previous layer's partial rows; one workgroup per head running its attention in one pass over the
caches and its columns of the output projection; LN2 + FFN-up + GELU; FFN-down split along K;
each launch adds the partial rows it consumes in a fixed order) against the CPU oracle
(ferrum_ref's Gpt2::feed, ferrum_ref/src/models/gpt2/decode.rs:57-117): logits within FORWARD
(1e-5, ferrum_wgpu/src/tolerance.rs) at every position of the context, greedy token IDs
identical, and agreement with the five-launch step of the same model. The shapes cover every
attention variant (head widths 64, 128 and 256), FFN widths split 1 to 6 ways, Q8_0 and Q4_0.
Form 1 is the one-launch step (the four-launch step's phases in one launch, with the head and the
pick): on every shape whose workgroups all fit on the chip at once (hd64: 64 workgroups, hd128:
40), the same tests; hd256 needs 440 and keeps the four-launch step."""
import os

import numpy as np
import pytest

from oracle import gpt2_model as gm

pytestmark = pytest.mark.gpu
FORWARD = 1e-5
CFGS = {
    # head width 64; FFN-down split 4 ways
    "hd64": {"vocab": 500, "ctx": 40, "dim": 256, "heads": 4, "layers": 2, "hidden": 1024},
    # head width 128; FFN width 320 (ten blocks, the last batch of eight half empty), split 2 ways
    "hd128": {"vocab": 300, "ctx": 24, "dim": 256, "heads": 2, "layers": 2, "hidden": 320},
    # head width 256; FFN-down split 11 ways (one chunk of 16 partial rows in the consumer)
    "hd256": {"vocab": 300, "ctx": 20, "dim": 512, "heads": 2, "layers": 1, "hidden": 8448},
}


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def g():
    import ferrum_hip

    gpu = ferrum_hip.Gpu.open_for_test()
    if gpu is None:
        pytest.skip("no gfx950 device")
    yield gpu
    gpu.close()


def load(g, data: bytes, form: int):
    """The model with the decode step of `form` launches per layer (5 or 4; 1: the one-launch step
    where it fits)."""
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.gpt2 import GpuGpt2

    os.environ["FERRUM_HIP_DECODE_STEP"] = str(form)
    try:
        return GpuGpt2.from_gguf(g, Gguf.parse(data))
    finally:
        del os.environ["FERRUM_HIP_DECODE_STEP"]


def launches(cfg: dict, form: int) -> int:
    if form == 1:  # the one-launch step where its workgroups fit: not hd256's 440 (FFN width 8448)
        return 1 if cfg["hidden"] < 8448 else 4 * cfg["layers"] + 3
    return {5: 5 * cfg["layers"] + 4, 4: 4 * cfg["layers"] + 3}[form]


def rel(got, want) -> float:
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1.0))


@pytest.mark.parametrize("form", [4, 1])
@pytest.mark.parametrize("kind", [gm.Q8_0, gm.Q4_0])
@pytest.mark.parametrize("name", list(CFGS))
def test_four_launch_step_feeds_the_whole_context_like_the_oracle(g, orc, name, kind, form):
    cfg = CFGS[name]
    m = gm.gpt2_init(cfg, 3)
    if name == "hd64":
        m = gm.tie_head(m)
    data = gm.to_gguf(m, kind)
    say(f"{name} kind {kind} form {form}: loading")
    dev = load(g, data, form)
    assert dev.step_launches() == launches(cfg, form)
    five = load(g, data, 5)
    assert five.step_launches() == launches(cfg, 5)
    cpu = orc.Gpt2Cpu(gm.from_gguf(data))
    ids = [int(t) for t in np.random.default_rng(11).integers(0, cfg["vocab"], cfg["ctx"])]
    first, worst, worst5 = [], 0.0, 0.0
    for i, t in enumerate(ids):
        got = dev.feed(t)
        want = cpu.feed(t)
        other = five.feed(t)
        first.append(got)
        e, e5, eo = rel(got, want), rel(got, other), rel(other, want)
        say(f"pos {i}: four-launch vs cpu {e:.2e}, four-launch vs five-launch {e5:.2e}, five-launch vs cpu {eo:.2e}")
        worst, worst5 = max(worst, e), max(worst5, e5)
    say(f"{name} kind {kind}: {cfg['ctx']} positions, max rel err {worst:.2e} (vs five-launch step {worst5:.2e})")
    assert worst < FORWARD and worst5 < FORWARD
    with pytest.raises(Exception) as err:
        dev.feed(0)
    assert "full" in str(err.value)
    dev.reset()
    again = [dev.feed(t) for t in ids[:4]]
    for a, b in zip(first, again):  # the same answers, bit for bit, after a reset
        assert np.array_equal(a, b)
    dev.free()
    five.free()


@pytest.mark.parametrize("form", [4, 1])
def test_four_launch_greedy_generation_matches_the_oracle(g, orc, form):
    cfg = dict(CFGS["hd64"], ctx=128)
    m = gm.gpt2_init(cfg, 6)
    data = gm.to_gguf(m, gm.Q8_0)
    dev = load(g, data, form)
    assert dev.step_launches() == launches(cfg, form)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, cfg["vocab"], 12)]
    want = orc.gpt2_generate(gm.from_gguf(data), prompt, 100)
    got = dev.generate(prompt, 100)
    assert got == want
    dev.free()


@pytest.mark.parametrize("form", [4, 1])
@pytest.mark.parametrize("kind", [gm.Q8_0, gm.Q4_0])
def test_four_launch_step_on_raw_random_weights_is_no_further_from_the_oracle(g, orc, kind, form):
    """Gpt2::random's raw weights (uniform +-0.5) amplify every rounding along the context, so the
    five-launch step itself leaves the CPU by about 1e-5 there: the four-launch step, which adds
    the same products in another order, must stay as close (within twice the five-launch step's
    distance, and 2e-5)."""
    cfg = CFGS["hd64"]
    m = gm.gpt2_random(cfg, 3)
    data = gm.to_gguf(m, kind)
    dev, five = load(g, data, form), load(g, data, 5)
    cpu = orc.Gpt2Cpu(gm.from_gguf(data))
    ids = [int(t) for t in np.random.default_rng(11).integers(0, cfg["vocab"], cfg["ctx"])]
    worst, worst_five = 0.0, 0.0
    for i, t in enumerate(ids):
        want = cpu.feed(t)
        e, eo = rel(dev.feed(t), want), rel(five.feed(t), want)
        say(f"pos {i}: four-launch vs cpu {e:.2e}, five-launch vs cpu {eo:.2e}")
        worst, worst_five = max(worst, e), max(worst_five, eo)
    say(f"kind {kind}: four-launch {worst:.2e}, five-launch {worst_five:.2e}")
    assert worst <= max(2 * worst_five, FORWARD) and worst < 2 * FORWARD
    dev.free()
    five.free()
