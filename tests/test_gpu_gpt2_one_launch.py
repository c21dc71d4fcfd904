"""The one-launch GPT-2 decode step (every layer, the head and the greedy pick in one launch; phase
counters between its workgroups) against the four-launch step (one launch per layer phase, then
the head and the pick) on the same model.

Both run the same lane-level arithmetic in the same order (the same workgroup tasks, wavefront
batches, LayerNorm sums and partial-row sums), so every logit must be bit-identical and greedy
generation must pick the same tokens. The four-launch step is itself held to the CPU oracle by
test_gpu_gpt2.py (logits within 1e-5, ferrum_wgpu/src/tolerance.rs:7, token IDs equal), which now
runs the one-launch step too, since it is the default wherever it fits.

Cases: GPT-2-small shapes (the decode benchmark's model: 240 workgroups, 12 layers) and a
three-layer model with d 256; feeds, reset, generate continuing from the current position, and two
models alive at once (each has its own counters)."""
import os

import numpy as np
import pytest

from oracle import gpt2_model as gm

pytestmark = pytest.mark.gpu
MID = {"vocab": 1000, "ctx": 160, "dim": 256, "heads": 4, "layers": 3, "hidden": 1024}
GPT2_SMALL = {"vocab": 50257, "ctx": 1024, "dim": 768, "heads": 12, "layers": 12, "hidden": 3072}


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


def load(g, data: bytes, form=None):
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.gpt2 import GpuGpt2

    old = os.environ.get("FERRUM_HIP_DECODE_STEP")
    try:
        if form is None:
            os.environ.pop("FERRUM_HIP_DECODE_STEP", None)
        else:
            os.environ["FERRUM_HIP_DECODE_STEP"] = str(form)
        return GpuGpt2.from_gguf(g, Gguf.parse(data))
    finally:
        if old is None:
            os.environ.pop("FERRUM_HIP_DECODE_STEP", None)
        else:
            os.environ["FERRUM_HIP_DECODE_STEP"] = old


def model_bytes(fh, g, cfg, seed):
    if cfg is GPT2_SMALL:
        from ferrum_hip.gpt2 import gpt2_init, to_gguf

        return to_gguf(g, gpt2_init(cfg, seed), fh.QKind.Q8_0)
    return gm.to_gguf(gm.gpt2_random(cfg, seed), gm.Q8_0)


def same_bits(a, b) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("name", ["mid", "gpt2_small"])
def test_one_launch_step_is_bit_identical_to_the_four_launch_step(fh, g, name):
    cfg = MID if name == "mid" else GPT2_SMALL
    data = model_bytes(fh, g, cfg, 3)
    one, four = load(g, data), load(g, data, form=4)
    assert one.step_launches() == 1, one.step_launches()
    assert four.step_launches() == 4 * cfg["layers"] + 3
    prompt = [int(t) for t in np.random.default_rng(11).integers(0, cfg["vocab"], 24)]
    say(f"{name}: feeding {len(prompt)} tokens to both steps")
    for i, t in enumerate(prompt):
        a, b = one.feed(t), four.feed(t)
        assert np.all(np.isfinite(a))
        assert same_bits(a, b), (i, float(np.abs(a - b).max()))
    # generate continues from the current position (24), then again after a reset
    ga, gb = one.generate([prompt[-1]], 40), four.generate([prompt[-1]], 40)
    assert ga == gb
    one.reset()
    four.reset()
    ga, gb = one.generate(prompt[:8], 64), four.generate(prompt[:8], 64)
    say(f"{name}: 64 generated tokens equal: {ga == gb}; first {ga[:6]}")
    assert ga == gb
    a, b = one.feed(ga[-1]), four.feed(gb[-1])
    assert same_bits(a, b)
    one.free()
    four.free()


def test_two_one_launch_models_alive_at_once(fh, g):
    """Interleaved steps of two models: each keeps its own phase counters and epoch."""
    d1, d2 = model_bytes(fh, g, MID, 5), model_bytes(fh, g, MID, 6)
    m1, m2 = load(g, d1), load(g, d2)
    r1, r2 = load(g, d1, form=4), load(g, d2, form=4)
    assert m1.step_launches() == 1 and m2.step_launches() == 1
    prompt = [int(t) for t in np.random.default_rng(12).integers(0, MID["vocab"], 10)]
    for t in prompt:
        a1, a2 = m1.feed(t), m2.feed(t)
        assert same_bits(a1, r1.feed(t)) and same_bits(a2, r2.feed(t))
    assert m1.generate([prompt[-1]], 20) == r1.generate([prompt[-1]], 20)
    assert m2.generate([prompt[-1]], 20) == r2.generate([prompt[-1]], 20)
    for m in (m1, m2, r1, r2):
        m.free()
