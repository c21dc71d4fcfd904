"""Benchmark of the quantized-weight hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): batch-1 Q4_0 GEMV at the Qwen2-0.5B layer shapes
K x N in {896 x 1152, 896 x 4864, 4864 x 896}, in HBM GB/s and as a fraction of the 8 TB/s peak.

A step is one pass of the batch-1 GEMV over a pool of distinct resident Q4_0 weights of those
three shapes (about 1 GiB, four times the 256 MB last-level cache, so every byte comes from
HBM), each with its own x and y, launched as one grouped launch per width class. Inputs are
resident in HBM before the timed region. Weights are seeded N(0, 0.02), x ~ N(0, 1) (synthetic).

Also reported (extra keys): the Q8_0 GPT-2 QKV GEMV (config 0), the MFMA dequant-GEMM at the
Qwen2 scoring shapes (M = 512, 2048) in TFLOP/s, the GPT-2-small Q8_0 greedy decode in tokens/s
(config 2) with its one-thread CPU counterpart, and the CPU baseline (the reference's CPU path
restated in C: f32 GEMV on the dequantised weights, one thread).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [REPO, os.path.join(REPO, "ferrum-gpu_amd")]

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
QWEN_SHAPES = [(896, 1152), (896, 4864), (4864, 896)]
# TinyLlama-1.1B layer products (K x N): fused QKV (2048 + 2 * 256), o, fused gate+up, down
LLAMA1B_SHAPES = [(2048, 2560), (2048, 2048), (2048, 11264), (5632, 2048)]
# one grouped launch per input width (the two 896-wide products share a kernel instantiation)
QWEN_GROUPS = [[(896, 1152), (896, 4864)], [(4864, 896)]]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(kind_bytes: int, k: int, n: int) -> int:
    """Algorithmic bytes of one batch-1 product: the packed weight, x and y."""
    return (k // 32) * n * kind_bytes + 4 * k + 4 * n


class HipEvents:
    """HIP events recorded on the library's own stream (the one its kernels run on), through the
    HIP runtime libferrum_hip already loaded (RTLD_NOLOAD: never a second runtime)."""

    DISABLE_SYSTEM_FENCE = 0x20000000  # hipEventDisableSystemFence

    def __init__(self, g):
        self.hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD | ctypes.RTLD_GLOBAL)
        self.stream = ctypes.c_void_p(g.stream())
        for name in ("hipEventCreateWithFlags", "hipEventRecord", "hipEventSynchronize", "hipEventElapsedTime",
                     "hipEventDestroy"):
            getattr(self.hip, name).restype = ctypes.c_int
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = ctypes.c_void_p()
            # timing events without a system-scope fence: a device-scope release is enough to
            # order them after the kernels on the stream, and the system fence costs microseconds
            if self.hip.hipEventCreateWithFlags(ctypes.byref(e), self.DISABLE_SYSTEM_FENCE) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            evs.append(e)
        return evs

    def record(self, e):
        if self.hip.hipEventRecord(e, self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def ms(self, e0, e1):
        if self.hip.hipEventSynchronize(e1) != 0:
            raise RuntimeError("hipEventSynchronize failed")
        out = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(out), e0, e1) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return out.value

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


def measured_traffic(bytes_per_launch):
    """HBM bytes per launch of this workload from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes (calibrated against the copy kernel), when they were taken on the same launch (same
    algorithmic bytes); None otherwise."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gemv_q4_0_qwen_pool.json")
    try:
        with open(path) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    L = d.get("launches", {}).get(str(bytes_per_launch))
    return L and {"traffic_bytes": L["traffic_bytes"], "source": d.get("source", path)}


PREWARM_S = 0.1


def prewarm(g, run, seconds=PREWARM_S):
    """Untimed load before a measurement: the GPU takes several milliseconds of sustained work
    to reach its steady clocks (a 20-step loop straight after 5 warm-up steps measured 4-6% below
    the same loop after 40 more steps). Runs `run` until `seconds` of wall time have passed."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            run()
        g.sync()
    return time.perf_counter() - t0


def bench_gemv_pool(fh, g, ev, kind, groups, pool_bytes, steps, warmup, seed=0):
    """Batch-1 GEMV over a pool of distinct resident weights, all in one plan run per step.
    `groups` lists the shapes of each of the plan's launches (the plan gives the products up to
    112 blocks wide one launch and the wider ones another, whose prepared x the first launch
    writes). The K timed steps run back to back between two HIP events (the step time); a second
    pass of K steps records an event pair around every launch (fh_gemv_plan_run_launch), so each
    launch's average duration is known too."""
    rng = np.random.default_rng(seed)
    kb = kind.file_bytes()
    shapes = [s for grp in groups for s in grp]
    set_bytes = sum((k // 32) * n * kb for k, n in shapes)
    copies = max(1, int(pool_bytes // set_bytes))
    packed = {}  # packed once on the device, then uploaded as distinct copies
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        packed[(k, n)] = fh.upload_quantised(g, kind, w, k, n).read_gguf()
    keep, probs = [], []
    for c in range(copies):
        for grp in groups:
            for k, n in grp:
                qw = fh.upload_qweight(g, kind, packed[(k, n)], k, n)
                gx = g.upload(rng.standard_normal(k).astype(np.float32))
                gy = g.zeros(n)
                keep += [qw, gx, gy]
                probs.append((qw, gx.device_ptr(), gy.device_ptr()))
    plan = fh.GemvPlan(g, probs)
    npl = plan.launches()
    assert npl == len(groups), "each group must be one of the plan's launches"
    warm_s = prewarm(g, plan.run)
    for _ in range(warmup):
        plan.run()
    g.sync()
    # the timed steps
    e0, e1 = ev.create(2)
    t0 = time.perf_counter()
    ev.record(e0)
    for s in range(steps):
        plan.run()
    ev.record(e1)
    g.sync()
    wall = time.perf_counter() - t0
    step_ms = ev.ms(e0, e1) / steps
    ev.destroy([e0, e1])
    # per-launch durations
    evs = ev.create(steps * npl * 2)
    for s in range(steps):
        for i in range(npl):
            ev.record(evs[2 * (s * npl + i)])
            plan.run_launch(i)
            ev.record(evs[2 * (s * npl + i) + 1])
    g.sync()
    launch_ms = [[ev.ms(evs[2 * (s * npl + i)], evs[2 * (s * npl + i) + 1]) for s in range(steps)]
                 for i in range(npl)]
    ev.destroy(evs)
    step_bytes = plan.bytes()
    launches = []
    for grp, ms in zip(groups, launch_ms):
        avg = float(np.mean(ms))
        lb = copies * sum((k // 32) * n * kb + 4 * k + 4 * n for k, n in grp)
        launches.append({"shapes": grp, "products": copies * len(grp), "bytes": lb,
                         "avg_ms": avg, "gbs": lb / (avg * 1e-3) / 1e9})
    assert sum(L["bytes"] for L in launches) == step_bytes
    plan.free()
    del keep
    return {"copies": copies, "products": copies * len(shapes), "launches_per_step": npl,
            "bytes_per_step": step_bytes, "ms_per_step": step_ms,
            "wall_ms_per_step": wall * 1e3 / steps,
            "gbs": step_bytes / (step_ms * 1e-3) / 1e9, "launches": launches, "prewarm_s": round(warm_s, 3)}


def bench_gemm(fh, g, ev, kind, m, shapes, steps, seed=0, path=None, copies=1, bound=False):
    """One step = every product of `shapes` (times `copies` distinct weight copies, to exceed the
    last-level cache for the HBM-bound small-M rates). Returns flops and algorithmic bytes per step.
    With `bound`, also the fraction of outputs outside the MFMA-GEMM bound |g - w| <= 1e-3 +
    2e-3 |w|, w taken from the precise path (QPath.Tiled, itself within 1e-5 of the CPU oracle)."""
    path = fh.QPath.Tiled if path is None else path
    rng = np.random.default_rng(seed)
    items = []
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        for _ in range(copies):
            qw = fh.upload_quantised(g, kind, w, k, n)
            gx = g.upload(rng.standard_normal(m * k).astype(np.float32))
            gy = g.zeros(m * n)
            items.append((qw, gx, gy, n))
    flops = copies * sum(2 * m * k * n for k, n in shapes)
    nbytes = copies * sum((k // 32) * n * kind.file_bytes() + 4 * m * k + 4 * m * n for k, n in shapes)
    for qw, gx, gy, _ in items:
        fh.linear_q_with(g, gx, qw, gy, m, path)
    g.sync()
    e0, e1 = ev.create(2)
    ev.record(e0)
    for _ in range(steps):
        for qw, gx, gy, _ in items:
            fh.linear_q_with(g, gx, qw, gy, m, path)
    ev.record(e1)
    g.sync()
    ms = ev.ms(e0, e1) / steps
    ev.destroy([e0, e1])
    out = {"m": m, "flops_per_step": flops, "ms_per_step": ms, "tflops": flops / (ms * 1e-3) / 1e12,
           "bytes_per_step": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9}
    if bound and path != fh.QPath.Tiled:
        outside = total = 0
        worst = 0.0
        for qw, gx, gy, n in items[::copies]:
            ref = g.zeros(m * n)
            fh.linear_q_with(g, gx, qw, ref, m, fh.QPath.Tiled)
            got, want = g.read(gy), g.read(ref)
            ref.free()
            lim = 1e-3 + 2e-3 * np.abs(want)
            r = np.abs(got - want) / lim
            outside += int(np.count_nonzero(r > 1.0))
            total += got.size
            worst = max(worst, float(r.max()))
        out["outside_bound_frac"] = outside / total
        out["worst_of_bound"] = round(worst, 4)
    return out


def bench_single_calls(fh, g, ev, kind, shapes, reps=3, seed=4):
    """One linear_q per product (batch 1, the library's own path choice): microseconds per call
    at each shape, over enough distinct weight copies (about 512 MB) that every call reads HBM;
    a decode step that calls the library once per matrix pays this per matrix."""
    rng = np.random.default_rng(seed)
    out = {}
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        data = fh.upload_quantised(g, kind, w, k, n).read_gguf()
        copies = max(2, int(512e6 // data.size))
        qs = [fh.upload_qweight(g, kind, data, k, n) for _ in range(copies)]
        xs = [g.upload(rng.standard_normal(k).astype(np.float32)) for _ in range(copies)]
        ys = [g.zeros(n) for _ in range(copies)]
        for i in range(copies):
            fh.linear_q(g, xs[i], qs[i], ys[i], 1)
        g.sync()
        e0, e1 = ev.create(2)
        ev.record(e0)
        for _ in range(reps):
            for i in range(copies):
                fh.linear_q(g, xs[i], qs[i], ys[i], 1)
        ev.record(e1)
        g.sync()
        ms = ev.ms(e0, e1) / (reps * copies)
        ev.destroy([e0, e1])
        out[f"{k}x{n}"] = {"us": round(ms * 1e3, 2), "gbs": round((data.size + 4 * k + 4 * n) / (ms * 1e-3) / 1e9, 1)}
        for q in qs:
            q.free()
    return out


CHOOSE_MS = (2, 4, 8, 16, 24, 32, 48, 64, 96, 128)


def bench_choose_sweep(fh, g, ev, shapes, kinds, ms=CHOOSE_MS, pool_bytes=256e6, reps=3, seed=9):
    """The measurement behind fh_choose's few-row / GEMM boundary (ferrum_wgpu/src/ops/quant.rs:
    303-323 says its thresholds must be re-measured per adapter): one linear_q per product, the
    few-row kernel (QPath.Rows, up to 64 rows) against the precise MFMA GEMM (QPath.Tiled) and the
    library's own choice (QPath.Auto), at each row count, over enough distinct weight copies
    (about `pool_bytes`) that every call reads its weight from HBM. Microseconds per call, the
    median of `reps` passes over the copies."""
    rng = np.random.default_rng(seed)
    out = {}
    for kind in kinds:
        for k, n in shapes:
            w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
            data = fh.upload_quantised(g, kind, w, k, n).read_gguf()
            copies = max(2, int(pool_bytes // data.size))
            qs = [fh.upload_qweight(g, kind, data, k, n) for _ in range(copies)]
            for m in ms:
                xs = [g.upload(rng.standard_normal(m * k).astype(np.float32)) for _ in range(copies)]
                ys = [g.zeros(m * n) for _ in range(copies)]
                row = {"auto": fh.choose(m, kind, k, n).name}
                for path in (fh.QPath.Rows, fh.QPath.Tiled, fh.QPath.Auto):
                    if path == fh.QPath.Rows and m > 64:
                        continue
                    for i in range(copies):
                        fh.linear_q_with(g, xs[i], qs[i], ys[i], m, path)
                    g.sync()
                    times = []
                    for _ in range(reps):
                        e0, e1 = ev.create(2)
                        ev.record(e0)
                        for i in range(copies):
                            fh.linear_q_with(g, xs[i], qs[i], ys[i], m, path)
                        ev.record(e1)
                        g.sync()
                        times.append(ev.ms(e0, e1) * 1e3 / copies)
                        ev.destroy([e0, e1])
                    row[path.name.lower() + "_us"] = round(float(np.median(times)), 2)
                best = min(v for key, v in row.items() if key in ("rows_us", "tiled_us"))
                row["auto_over_best"] = round(row["auto_us"] / best, 3)
                out[f"{kind.label()} {k}x{n} M={m}"] = row
                log(f"choose sweep {kind.label()} {k}x{n} M={m}: {row}")
                for b in xs + ys:
                    b.free()
            for q in qs:
                q.free()
    return out


def bench_ext_gemm(fh, g, ev, kinds, cases, reps=5, seed=6):
    """Multi-row products on the other weight formats through linear_q (QPath.Tiled: the MFMA GEMM
    on the GGUF rows, x split included): TFLOP/s per (format, M, K, N)."""
    rng = np.random.default_rng(seed)
    out = {}
    for kind in kinds:
        r = {}
        for m, k, n in cases:
            w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
            q = fh.upload_quantised(g, kind, w, k, n)
            x, y = g.upload(rng.standard_normal(m * k).astype(np.float32)), g.zeros(m * n)
            for _ in range(2):
                fh.linear_q_with(g, x, q, y, m, fh.QPath.Tiled)
            g.sync()
            e0, e1 = ev.create(2)
            ev.record(e0)
            for _ in range(reps):
                fh.linear_q_with(g, x, q, y, m, fh.QPath.Tiled)
            ev.record(e1)
            g.sync()
            ms = ev.ms(e0, e1) / reps
            ev.destroy([e0, e1])
            tf = 2 * m * k * n / (ms * 1e-3) / 1e12
            r[f"m{m}_{k}x{n}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1),
                                  "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4)}
            q.free()
        out[kind.label()] = r
    return out


def bench_rows_pool(fh, g, ev, kind, m, shapes, steps, copies=12, seed=0):
    """Config 5's few-row products as one grouped launch pair (RowsPlan: x split, then the
    few-row kernel over every product): `copies` distinct copies of `shapes` (12 copies of the
    TinyLlama-1.1B products hold about 300 MB of Q4_0 weights, more than the 256 MB last-level
    cache). One step = one run of the plan; algorithmic bytes = packed weights + x + y."""
    rng = np.random.default_rng(seed)
    keep, probs = [], []
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        packed = fh.upload_quantised(g, kind, w, k, n).read_gguf()
        for _ in range(copies):
            qw = fh.upload_qweight(g, kind, packed, k, n)
            gx = g.upload(rng.standard_normal(m * k).astype(np.float32))
            gy = g.zeros(m * n)
            keep += [qw, gx, gy]
            probs.append((qw, gx.device_ptr(), gy.device_ptr(), m))
    plan = fh.RowsPlan(g, probs)
    prewarm(g, plan.run)
    e0, e1 = ev.create(2)
    ev.record(e0)
    for _ in range(steps):
        plan.run()
    ev.record(e1)
    g.sync()
    ms = ev.ms(e0, e1) / steps
    ev.destroy([e0, e1])
    nbytes = plan.bytes()
    wbytes = copies * sum((k // 32) * n * kind.file_bytes() for k, n in shapes)
    flops = copies * sum(2 * m * k * n for k, n in shapes)
    launches = plan.launches()
    plan.free()
    return {"m": m, "ms_per_step": ms, "bytes_per_step": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9,
            "weight_gbs": wbytes / (ms * 1e-3) / 1e9, "tflops": flops / (ms * 1e-3) / 1e12,
            "products": len(probs), "launches": launches}


def bench_copy(g, ev, nbytes=512 * 2**20, reps=10):
    """A plain device copy (Gpu::copy_f32, one 16-byte-vector kernel) of a known size: the
    measured HBM ceiling for a read+write stream, and the known-size dispatch that calibrates the
    FETCH_SIZE / WRITE_SIZE counters (it is the first kernel this script launches)."""
    n = nbytes // 4
    src, dst = g.zeros(n), g.zeros(n)
    g.copy_f32(src, 0, dst, 0, n)  # calibration dispatch (also a warm-up)
    g.sync()
    e0, e1 = ev.create(2)
    ev.record(e0)
    for _ in range(reps):
        g.copy_f32(src, 0, dst, 0, n)
    ev.record(e1)
    ms = ev.ms(e0, e1) / reps
    ev.destroy([e0, e1])
    src.free()
    dst.free()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "avg_ms": ms, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9}


GPT2_SMALL = {"vocab": 50257, "ctx": 1024, "dim": 768, "heads": 12, "layers": 12, "hidden": 3072}


def bench_decode(fh, g, n_prompt=32, n_new=256, reps=3, cpu=True):
    """GPT-2-small (GPT-2 initialisation, tied head) with Q8_0 weights, KV-cached
    greedy decode of n_new tokens from an n_prompt-token seeded uniform-random prompt. One rep is one
    fh_gpt2_generate call from position 0 (the prompt is fed token by token, so a rep is
    n_prompt + n_new - 1 decode steps); the median rep is reported."""
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.gpt2 import GpuGpt2, gpt2_init, to_gguf

    cfg = GPT2_SMALL
    m = gpt2_init(cfg, 1)
    data = to_gguf(g, m, fh.QKind.Q8_0)
    model = GpuGpt2.from_gguf(g, Gguf.parse(data))
    prompt = [int(t) for t in np.random.default_rng(2024).integers(0, cfg["vocab"], n_prompt)]
    model.generate(prompt, 8)  # graph capture and warm-up
    times, toks = [], None
    for _ in range(reps):
        model.reset()
        t0 = time.perf_counter()
        toks = model.generate(prompt, n_new)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    steps = n_prompt + n_new - 1
    out = {"tok_s": n_new / t, "steps_per_s": steps / t, "ms_per_step": t / steps * 1e3,
           "weight_gbs": model.step_bytes() * steps / t / 1e9, "step_bytes": model.step_bytes(),
           "first_tokens": toks[:8], "reps": reps, "launches_per_step": model.step_launches()}
    if cpu:  # ferrum_ref's Gpt2::feed (restated in C) on the fake-quantised f32 weights, one thread
        import oracle as orc
        from oracle import gpt2_model as gm

        cpu_m = orc.Gpt2Cpu(gm.from_gguf(data))
        for tkn in prompt[:2]:
            cpu_m.feed(tkn)
        t0, n = time.perf_counter(), 0
        while time.perf_counter() - t0 < 5.0 or n < 5:
            cpu_m.feed(prompt[2 + n % 30])
            n += 1
        out["cpu_tok_s"] = n / (time.perf_counter() - t0)
        out["cpu_sample"] = f"{n} Gpt2::feed steps at positions 2..{n + 1}, f32 weights, 1 thread"
    model.free()
    return out


QWEN_LINEAR_WEIGHTS = 493_961_216  # packed weights one Qwen2-0.5B forward multiplies by (head included)


def bench_scoring(fh, g, ev, ms=(512, 2048), paths=None, reps=5, cpu=True, cpu_rows=64):
    """full-sequence scoring with the random-init Qwen2-0.5B-shape model (24
    layers, d 896, FFN 4864 SwiGLU, RMSNorm, NEOX RoPE base 1e6, q/k/v biases, vocab 151936, tied
    head), Q4_0 weights, M seeded uniform-random token IDs (M + 1 IDs, M scored rows). One rep is
    one fh_llama_score_device call with the IDs already on the device; the median of `reps` reps
    (HIP events on the device stream). TFLOP/s counts the linear layers only (2 M x 493.96M, the
    reference's formula); the causal attention adds 2 x 2 x 14 x 64 x M (M + 1) / 2 x 24 flops.
    The CPU leg runs the oracle's forward + score (all host threads, f32 decoded weights) on
    `cpu_rows` rows and reports its rate and the device's largest log-probability error on them."""
    from ferrum_hip.gguf import Gguf
    from ferrum_hip.llama import QWEN2_0_5B, GpuLlama, random_gguf

    paths = paths or (fh.QPath.TiledFast, fh.QPath.Tiled)
    data = random_gguf(g, QWEN2_0_5B, fh.QKind.Q4_0, seed=1)
    gg = Gguf.parse(data)
    rng = np.random.default_rng(2024)
    ids_all = rng.integers(0, QWEN2_0_5B["vocab"], max(ms) + 1).astype(np.int32)
    out = {"weights": QWEN_LINEAR_WEIGHTS, "gguf_bytes": len(data)}
    for path in paths:
        model = GpuLlama.from_gguf(g, gg, path)
        tag = "fast" if path == fh.QPath.TiledFast else "precise"
        for m in ms:
            ids = g.upload_bytes(ids_all[: m + 1].view(np.uint8))
            res = g.zeros(2 * m)
            for _ in range(2):
                model.score_device(ids, m + 1, res)
            g.sync()
            times = []
            for _ in range(reps):
                e0, e1 = ev.create(2)
                ev.record(e0)
                model.score_device(ids, m + 1, res)
                ev.record(e1)
                g.sync()
                times.append(ev.ms(e0, e1))
                ev.destroy([e0, e1])
            t = float(np.median(times))
            lp = g.read(res)[0::2]
            flops = 2 * m * QWEN_LINEAR_WEIGHTS
            attn = 2 * 2 * 14 * 64 * m * (m + 1) // 2 * 24
            out[f"{tag}_m{m}"] = {"ms": round(t, 4), "tok_s": round(m / (t * 1e-3), 1),
                                  "linear_tflops": round(flops / (t * 1e-3) / 1e12, 2),
                                  "frac": round(flops / (t * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                                  "attention_gflop": round(attn / 1e9, 1), "finite": bool(np.isfinite(lp).all()),
                                  "mean_logprob": round(float(lp.mean()), 3)}
            ids.free()
            res.free()
        if cpu:
            import oracle as orc
            from oracle import llama_model as lm

            ref = out.get("_ref") or lm.from_gguf(data)
            out["_ref"] = ref
            sample = [int(t) for t in ids_all[: cpu_rows + 1]]
            threads = min(16, os.cpu_count() or 1)
            t0 = time.perf_counter()
            wlp, whit = orc.llama_score(ref, sample, threads=threads)
            dt = time.perf_counter() - t0
            glp, ghit = model.score_arrays(sample)
            err = float((np.abs(glp - wlp) / np.maximum(np.abs(wlp), 1.0)).max())
            out[f"{tag}_logprob_rel_err_vs_cpu"] = err
            out[f"{tag}_logprob_abs_err_vs_cpu"] = float(np.abs(glp - wlp).max())
            out[f"{tag}_first_argmax_flags_equal"] = bool(np.array_equal(ghit, whit))
            out["cpu_tok_s"] = round(cpu_rows / dt, 2)
            out["cpu_sample"] = (f"oracle Llama::forward_logits + nn::score on {cpu_rows} rows, f32 decoded weights, "
                                 f"{threads} threads, {dt:.2f} s")
            out["cpu_threads"] = threads
        model.free()
    out.pop("_ref", None)
    return out


# TinyLlama-1.1B block matrices, [in, out]: q, k, v, o, gate, up, down; 22 blocks
LLAMA1B_MATRICES = [(2048, 2048), (2048, 256), (2048, 256), (2048, 2048), (2048, 5632), (2048, 5632), (5632, 2048)]
LLAMA1B_LAYERS = 22
EXT_GEMM_CASES = [(512, 2048, 2048), (4096, 2048, 5632)]


def ext_kinds(fh):
    return (fh.QKind.F16, fh.QKind.Fp8E4M3, fh.QKind.Fp8E5M2, fh.QKind.Fp4, fh.QKind.Q2K)


def bench_codec(fh, g, ev, reps=5, copies=8):
    """The block codec on the device at the TinyLlama-1.1B gate matrix (2048 x 5632 = 11.5M values),
    inputs resident: encode (f32 -> GGUF blocks), decode (blocks -> f32), snap rows and columns
    (f32 -> f32), and the weight's dequantise (tiles -> the [k, n] f32 weight); GB/s of the bytes
    each reads and writes. Each line rotates over `copies` distinct source and destination
    buffers (8 x 92 MB, more than the 256 MB last-level cache), so every call streams from HBM.
    Then config 5's QAT fake-quant pass: the column snap of every block matrix of the 1.1B model
    (the seven matrices of each of its 22 blocks, each its own buffer: 3.9 GB in, 3.9 GB out), as
    one grouped launch and as one call per matrix."""
    rng = np.random.default_rng(3)
    k, n = 2048, 5632
    vals = k * n
    host = (rng.standard_normal(vals) * 0.02).astype(np.float32)
    srcs = [g.upload(host) for _ in range(copies)]
    dsts = [g.zeros(vals) for _ in range(copies)]
    out = {}

    def timed(fn, nbytes, calls):
        for c in range(calls):
            fn(c)
        g.sync()
        e0, e1 = ev.create(2)
        ev.record(e0)
        for _ in range(reps):
            for c in range(calls):
                fn(c)
        ev.record(e1)
        g.sync()
        ms = ev.ms(e0, e1) / (reps * calls)
        ev.destroy([e0, e1])
        return {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}

    for kind, tag in ((fh.QKind.Q8_0, "q8_0"), (fh.QKind.Q4_0, "q4_0")):
        pb = fh.nbytes(kind, vals)
        blocks = [g.bytes_zeros(pb) for _ in range(copies)]
        out[f"encode_{tag}"] = timed(lambda c: fh.encode(g, kind, srcs[c], vals, blocks[c]), 4 * vals + pb, copies)
        out[f"decode_{tag}"] = timed(lambda c: fh.decode(g, kind, blocks[c], vals, dsts[c]), 4 * vals + pb, copies)
        gguf = g.read_bytes(blocks[0])
        qws = [fh.upload_qweight(g, kind, gguf, k, n) for _ in range(copies)]
        out[f"dequantise_{tag}"] = timed(
            lambda c: fh._check(fh.lib().fh_qweight_dequantise(g.handle, qws[c].handle, dsts[c].handle)),
            4 * vals + pb, copies)
        for q in qws:
            q.free()
        # GGUF bytes from the host into the tiled planes (allocation, PCIe copy, repack kernel): wall
        # time, PCIe-inclusive; the repack kernel's own time is in the kernel trace
        t0 = time.perf_counter()
        for _ in range(3):
            fh.upload_qweight(g, kind, gguf, k, n).free()
        g.sync()
        out[f"upload_gguf_{tag}_pcie_inclusive_ms"] = round((time.perf_counter() - t0) / 3 * 1e3, 3)
        for b in blocks:
            b.free()
    out["snap_rows"] = timed(lambda c: fh.q8_snap_rows(g, srcs[c], dsts[c], k), 8 * vals, copies)
    out["snap_cols"] = timed(lambda c: fh.q8_snap_cols(g, srcs[c], dsts[c], (k, n)), 8 * vals, copies)
    for b in srcs + dsts:
        b.free()
    # the QAT pass: every matrix of every block its own source and destination
    mats = []
    for a, b in LLAMA1B_MATRICES:
        h = (rng.standard_normal(a * b) * 0.02).astype(np.float32)
        mats += [(g.upload(h), g.zeros(a * b), a, b) for _ in range(LLAMA1B_LAYERS)]
    pass_vals = sum(a * b for _, _, a, b in mats)

    def qat_pass(_):
        for s_, d_, a, b in mats:
            fh.q8_snap_cols(g, s_, d_, (a, b))

    plan = fh.SnapPlan(g, [(fh.SNAP_COLS, s_, d_, (a, b)) for s_, d_, a, b in mats])
    r = timed(lambda _: plan.run(), 8 * pass_vals, 1)
    r["values"] = pass_vals
    r["launches"] = 1
    r["form"] = "one grouped launch (fh_snap_plan_run)"
    out["qat_fake_quant_pass_llama1b"] = r
    plan.free()
    r1 = timed(qat_pass, 8 * pass_vals, 1)
    r1["launches"] = len(mats)
    r1["form"] = "one q8_snap_cols call per matrix"
    out["qat_fake_quant_pass_llama1b_single_calls"] = r1
    for s_, d_, _, _ in mats:
        s_.free()
        d_.free()
    out["shape"] = (f"{k} x {n} ({vals} values), {copies} rotating copies; QAT pass: {LLAMA1B_LAYERS} x "
                    f"{LLAMA1B_MATRICES} [in, out], distinct buffers")
    return out


def compact(extra):
    """One number per configuration for the final JSON line (the driver keeps only the tail of
    stdout, so the line stays under 4 kB); the full detail goes to stderr as `bench detail:`."""
    def pick(key, *fields):
        d = extra.get(key)
        if not isinstance(d, dict):
            return None
        return {f: d[f] for f in fields if f in d} or None

    out = {"q8_0_gemv_768x2304_pool": pick("q8_0_gemv_768x2304", "gbs", "frac")}
    gemm = {}  # TFLOP/s per path (fast = QPath.TiledFast, precise = QPath.Tiled, f16 = QPath.TiledF16)
    for name in ("q4_0_gemm_llama1b", "q8_0_gemm_llama1b", "q4_0_gemm_qwen"):
        for m in (512, 2048, 4096):
            row = {}
            for tag, label in (("", "fast"), ("_precise", "precise"), ("_f16", "f16")):
                d = extra.get(f"{name}{tag}_m{m}")
                if isinstance(d, dict):
                    row[label] = round(d["tflops"], 1)
                    if d.get("outside_bound_frac"):
                        row[label + "_outside_bound"] = d["outside_bound_frac"]
            if row:
                gemm[f"{name[:4]}_{name.split('_')[-1]}_m{m}"] = row
    out["gemm_tflops"] = gemm or None
    for tag in ("q4_0", "q8_0"):
        for m in (8, 64):
            v = pick(f"{tag}_gemm_llama1b_m{m}", "gbs", "frac_hbm", "single_calls_gbs")
            if v:
                out[f"{tag}_rows_llama1b_m{m}"] = v
    sc = extra.get("qwen2_0_5b_q4_0_scoring")
    if isinstance(sc, dict):
        out["qwen2_0_5b_scoring_ms"] = {k: v["ms"] for k, v in sc.items() if isinstance(v, dict) and "ms" in v}
        out["qwen2_0_5b_scoring_logprob_rel_err_vs_cpu"] = {
            k.split("_")[0]: v for k, v in sc.items() if k.endswith("logprob_rel_err_vs_cpu")}
    dec = extra.get("gpt2_small_q8_0_decode")
    if isinstance(dec, dict):
        out["gpt2_small_q8_0_decode"] = {k: dec[k] for k in ("tok_s", "ms_per_step", "weight_gbs", "cpu_tok_s")
                                         if k in dec}
    codec = extra.get("codec_llama1b")
    if isinstance(codec, dict) and isinstance(codec.get("qat_fake_quant_pass_llama1b"), dict):
        out["qat_fake_quant_pass_llama1b_gbs"] = codec["qat_fake_quant_pass_llama1b"].get("gbs")
    return {k: v for k, v in out.items() if v is not None}


def host_info():
    """The host's core count and CPU model (for the CPU baseline's report)."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model}


def cpu_matmul_tuned(threads, m=64, k=2048, n=2048, budget_s=3.0):
    """ferrum_ref's matmul_tuned (kernels/tuned.rs:99-134, the oracle's restatement) on `threads`
    threads at a config-5 shape: GFLOP/s, median of repeats (bench_util::time_ms)."""
    import oracle as orc

    rng = np.random.default_rng(2)
    x = rng.standard_normal(m * k).astype(np.float32)
    w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
    orc.matmul_tuned(x, w, m, k, n, threads)
    times, t0 = [], time.perf_counter()
    while time.perf_counter() - t0 < budget_s or len(times) < 7:
        t1 = time.perf_counter()
        orc.matmul_tuned(x, w, m, k, n, threads)
        times.append(time.perf_counter() - t1)
    med = float(np.median(times))
    return {"gflops": round(2 * m * k * n / med / 1e9, 2), "threads": threads, "shape": f"{m} x {k} x {n}",
            "ms": round(med * 1e3, 3)}


def cpu_baseline(shapes, kind_bytes, budget_s=12.0):
    """The reference's CPU decode path restated in C (oracle/gemv: f32 weights [k, n], ascending
    k, one thread), on the same shapes; the rate is the same algorithmic bytes (the packed
    weights' size) over CPU time, plus the f32 bytes it actually streams."""
    import oracle as orc

    rng = np.random.default_rng(1)
    mats = [((rng.standard_normal(k * n) * 0.02).astype(np.float32), rng.standard_normal(k).astype(np.float32), k, n)
            for k, n in shapes]
    for w, x, k, n in mats:  # warm-up (bench_util::time_ms: one warm-up, then the median)
        orc.gemv(x, w, None, k, n)
    times, t_start = [], time.perf_counter()
    while time.perf_counter() - t_start < budget_s or len(times) < 7:
        t0 = time.perf_counter()
        for w, x, k, n in mats:
            orc.gemv(x, w, None, k, n)
        times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    alg = sum(gemv_bytes(kind_bytes, k, n) for k, n in shapes)
    f32b = sum(4 * k * n for k, n in shapes)
    hi = host_info()
    return {"value": alg / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} reps (median) of one pass over {shapes} Q4_0-sized work on f32 "
                      f"dequantised weights, {sum(x[2]*x[3] for x in mats)} weights; f32 stream "
                      f"{f32b / med / 1e9:.2f} GB/s; {med * 1e3:.3f} ms per pass; host {hi['nproc']} "
                      f"cores, {hi['cpu_model']}",
            "f32_gbs": f32b / med / 1e9, "ms_per_pass": med * 1e3, "host_nproc": hi["nproc"],
            "host_cpu_model": hi["cpu_model"]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--pool-gib", type=float, default=1.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the GPT-2-small decode (config 2), one JSON line (for profiling)")
    ap.add_argument("--gemm-path", default="TiledFast", choices=["Tiled", "TiledFast", "TiledF16"],
                    help="the GEMM --gemm-only measures")
    ap.add_argument("--score-only", action="store_true",
                    help="only the Qwen2-0.5B Q4_0 scoring forward (config 4), one JSON line (for profiling)")
    ap.add_argument("--codec-only", action="store_true",
                    help="only the codec and QAT-pass lines at the TinyLlama-1.1B sizes, one JSON line (for profiling)")
    ap.add_argument("--rows-only", action="store_true",
                    help="only config 5's grouped few-row products (M = 8, 64), one JSON line (for profiling)")
    ap.add_argument("--ext-only", action="store_true",
                    help="only the one-row GEMV on the other weight formats (F16, FP8, MXFP4, Q2_K), one JSON line")
    ap.add_argument("--choose-sweep", action="store_true",
                    help="only the few-row kernel against the precise GEMM, one linear_q per product, M = 2..128 "
                         "at the config 2 and config 5 shapes (the measurement behind fh_choose)")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the scoring GEMM at the TinyLlama-1.1B shapes, M = 4096, one JSON line (for profiling)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported (the path shards by "
              "output rows with no exchange; see the sharding design)", file=sys.stderr)
        sys.exit(2)

    import ferrum_hip as fh

    g = fh.Gpu(0)
    if a.decode_only:
        dec = bench_decode(fh, g, cpu=not a.no_cpu)
        print(json.dumps({"metric": "GPT-2-small Q8_0 greedy decode tokens/s", "value": round(dec["tok_s"], 2),
                          "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "detail": dec}))
        g.close()
        return
    ev = HipEvents(g)
    if a.score_only:
        r = bench_scoring(fh, g, ev, paths=(fh.QPath.TiledFast,), cpu=not a.no_cpu)
        best = r["fast_m2048"]
        print(json.dumps({"metric": "Qwen2-0.5B Q4_0 scoring tokens/s, M = 2048", "value": best["tok_s"],
                          "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "detail": r}))
        g.close()
        return
    if a.codec_only:
        r = bench_codec(fh, g, ev)
        print(json.dumps({"metric": "Q8_0 QAT fake-quant pass over TinyLlama-1.1B's block matrices, GB/s",
                          "value": r["qat_fake_quant_pass_llama1b"]["gbs"], "unit": "GB/s", "n_gpus": 1,
                          "higher_is_better": True, "detail": r}))
        g.close()
        return
    if a.rows_only:
        det = {}
        for kind, tag in ((fh.QKind.Q4_0, "q4_0"), (fh.QKind.Q8_0, "q8_0")):
            for m in (8, 64):
                det[f"{tag}_m{m}"] = bench_rows_pool(fh, g, ev, kind, m, LLAMA1B_SHAPES, a.steps)
        print(json.dumps({"metric": "config 5 few-row products, weight GB/s", "value": det["q4_0_m8"]["weight_gbs"],
                          "unit": "GB/s", "n_gpus": 1, "higher_is_better": True, "detail": det}))
        g.close()
        return
    if a.ext_only:
        ext = {}
        for kind in ext_kinds(fh):
            shapes = [(8192, 8192), (1024 if kind == fh.QKind.Q2K else 896, 151936)]
            ext[kind.label()] = bench_single_calls(fh, g, ev, kind, shapes, reps=2, seed=5)
        gemm = bench_ext_gemm(fh, g, ev, ext_kinds(fh), EXT_GEMM_CASES)
        print(json.dumps({"metric": "one-row GEMV GB/s on the other weight formats, 8192 x 8192",
                          "value": ext["MXFP4"]["8192x8192"]["gbs"], "unit": "GB/s", "n_gpus": 1,
                          "higher_is_better": True, "detail": ext, "gemm": gemm}))
        g.close()
        return
    if a.choose_sweep:
        r = bench_choose_sweep(fh, g, ev, QWEN_SHAPES + LLAMA1B_SHAPES, (fh.QKind.Q4_0, fh.QKind.Q8_0))
        worst = max(v["auto_over_best"] for v in r.values())
        print(json.dumps({"metric": "fh_choose: worst ratio of AUTO's time to the faster path's", "value": worst,
                          "unit": "ratio", "n_gpus": 1, "higher_is_better": False, "detail": r}))
        g.close()
        return
    if a.gemm_only:
        r = bench_gemm(fh, g, ev, fh.QKind.Q4_0, 4096, LLAMA1B_SHAPES, a.steps, path=fh.QPath[a.gemm_path])
        print(json.dumps({"metric": "Q4_0 scoring GEMM TFLOP/s, TinyLlama-1.1B layer shapes, M = 4096",
                          "value": round(r["tflops"], 2), "unit": "TFLOP/s", "n_gpus": 1, "higher_is_better": True,
                          "frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4), "detail": r}))
        g.close()
        return
    name, cus = g.info()
    log(f"device {name}, {cus} CUs")
    copy = bench_copy(g, ev)
    log("copy:", copy)

    head = bench_gemv_pool(fh, g, ev, fh.QKind.Q4_0, QWEN_GROUPS, a.pool_gib * 2**30, a.steps, a.warmup)
    log("Q4_0 GEMV pool:", head)
    extra = {}
    if not a.no_extra:
        q8 = bench_gemv_pool(fh, g, ev, fh.QKind.Q8_0, [[(768, 2304)]], a.pool_gib * 2**30, a.steps, a.warmup,
                             seed=1)
        log("Q8_0 GEMV pool:", q8)
        extra["q8_0_gemv_768x2304"] = {"gbs": round(q8["gbs"], 2), "frac": round(q8["gbs"] / HBM_PEAK_GBS, 4),
                                       "ms_per_step": q8["ms_per_step"], "bytes_per_step": q8["bytes_per_step"],
                                       "products_per_step": q8["products"]}
        for name, kind, shapes, ms in (("q4_0_gemm_qwen", fh.QKind.Q4_0, QWEN_SHAPES, (512, 2048)),
                                       ("q4_0_gemm_llama1b", fh.QKind.Q4_0, LLAMA1B_SHAPES, (512, 4096)),
                                       ("q8_0_gemm_llama1b", fh.QKind.Q8_0, LLAMA1B_SHAPES, (512, 4096))):
            for m in ms:
                for tag, path in (("", fh.QPath.TiledFast), ("_f16", fh.QPath.TiledF16), ("_precise", fh.QPath.Tiled)):
                    r = bench_gemm(fh, g, ev, kind, m, shapes, 10, path=path, bound=True)
                    log(f"{name}{tag} M={m}:", r)
                    extra[f"{name}{tag}_m{m}"] = {"tflops": round(r["tflops"], 2),
                                                  "frac": round(r["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                                                  "ms_per_step": r["ms_per_step"],
                                                  "flops_per_step": r["flops_per_step"]}
                    if "outside_bound_frac" in r:
                        extra[f"{name}{tag}_m{m}"].update(outside_bound_frac=r["outside_bound_frac"],
                                                          worst_of_bound=r["worst_of_bound"])
        # config 5's small M (HBM-bound): 12 distinct copies of the four products (about 300 MB of
        # Q4_0 weights, more than the 256 MB last-level cache), as one grouped launch of the few-row
        # kernel, and as one linear_q per product with the library's own path choice
        for kind, tag in ((fh.QKind.Q4_0, "q4_0"), (fh.QKind.Q8_0, "q8_0")):
            for m in (8, 64):
                r = bench_rows_pool(fh, g, ev, kind, m, LLAMA1B_SHAPES, 20)
                log(f"{tag} few-row products M={m}, grouped:", r)
                r1 = bench_gemm(fh, g, ev, kind, m, LLAMA1B_SHAPES, 10, path=fh.QPath.Auto, copies=12)
                log(f"{tag} few-row products M={m}, one linear_q each:", r1)
                extra[f"{tag}_gemm_llama1b_m{m}"] = {
                    "gbs": round(r["gbs"], 2), "frac_hbm": round(r["gbs"] / HBM_PEAK_GBS, 4),
                    "weight_gbs": round(r["weight_gbs"], 2), "tflops": round(r["tflops"], 2),
                    "ms_per_step": r["ms_per_step"], "bytes_per_step": r["bytes_per_step"],
                    "path": "rows plan (QPath.Rows), one launch pair for 48 products",
                    "single_calls_gbs": round(r1["gbs"], 2), "single_calls_ms_per_step": r1["ms_per_step"]}
        for kind, tag in ((fh.QKind.Q4_0, "q4_0"), (fh.QKind.Q8_0, "q8_0")):
            sc1 = bench_single_calls(fh, g, ev, kind, QWEN_SHAPES + LLAMA1B_SHAPES)
            log(f"{tag} single-call GEMV:", sc1)
            extra[f"{tag}_gemv_single_call_us"] = sc1
        ext = {}
        for kind in ext_kinds(fh):
            shapes = [(8192, 8192), (1024 if kind == fh.QKind.Q2K else 896, 151936)]
            ext[kind.label()] = bench_single_calls(fh, g, ev, kind, shapes, reps=2, seed=5)
        log("other formats, single-call GEMV:", ext)
        extra["ext_formats_gemv_single_call"] = {
            "kernel": "ext_gemv_rows_kernel: GGUF rows decoded in registers, x shared by up to 8 rows per lane, "
                      "f32 accumulation; one launch per call, launch gaps included",
            "by_format": ext}
        eg = bench_ext_gemm(fh, g, ev, ext_kinds(fh), EXT_GEMM_CASES)
        log("other formats, MFMA GEMM:", eg)
        extra["ext_formats_gemm"] = {
            "kernel": "gemm_ext_kernel: x as two f16 parts, f16-exact decoded values times per-block f32 scales "
                      "(Q2_K: per 16-element sub-block, minus dmin times the x sums) on f16 MFMA; x split included",
            "by_format": eg}
        codec = bench_codec(fh, g, ev)
        log("codec:", codec)
        extra["codec_llama1b"] = codec
        sc = bench_scoring(fh, g, ev, cpu=not a.no_cpu)
        log("Qwen2-0.5B Q4_0 scoring:", sc)
        extra["qwen2_0_5b_q4_0_scoring"] = sc
        dec = bench_decode(fh, g, cpu=not a.no_cpu)
        log("GPT-2-small Q8_0 decode:", dec)
        extra["gpt2_small_q8_0_decode"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in dec.items()}
        extra["gemm_operands"] = ("scoring GEMM (QPath.TiledFast): x as f16 times exact f16 integer quants on f16 "
                                  "MFMA with the f32 block scale per block, plus an e4m3 correction (x's f16 "
                                  "residual times e4m3 d*q) on the scaled fp8 MFMA; _precise: x as two f16 parts "
                                  "(QPath.Tiled); f32 accumulate")

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(QWEN_SHAPES, 18)
        log("cpu baseline:", cpu)
        if not a.no_extra:  # the CPU matmul on all host cores, beside the GEMM lines
            cores = min(16, os.cpu_count() or 1)
            extra["cpu_matmul_tuned"] = cpu_matmul_tuned(cores)
            log("cpu matmul_tuned:", extra["cpu_matmul_tuned"])

    gbs = head["gbs"]
    dom = max(head["launches"], key=lambda L: L["avg_ms"])  # the launch that takes the most time
    traffic = measured_traffic(dom["bytes"])
    out = {
        "metric": "Q4_0 batch-1 GEMV HBM GB/s at Qwen2-0.5B layer shapes",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights (exact int8 quants); x on a per-32-block fixed-point grid of 30 bits "
                 "(2^-30 of the block's largest |x|, four int8 limbs) on int8 MFMA with exact int32 block "
                 "sums; f32 block scales and accumulation",
        "data": "synthetic: seeded N(0,0.02) weights packed Q4_0, x ~ N(0,1)",
        "config": {"workload": "Q4_0 GEMV sweep, K x N in {896x1152, 896x4864, 4864x896}, "
                               f"{head['copies']} distinct copies each ({head['bytes_per_step'] / 2**30:.2f} GiB per step)",
                   "products_per_step": head["products"], "launches_per_step": head["launches_per_step"],
                   "prewarm_s": head["prewarm_s"]},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic and traffic["traffic_bytes"],
                     "kernel": f"grouped Q4_0 GEMV launch over {dom['shapes']} x {head['copies']} (one product "
                               "kernel; the 896-wide launch prepares its x in LDS and also writes the 4864-wide "
                               "launch's prepared x, which then runs no preparation kernel)",
                     "bytes_per_launch": dom["bytes"], "avg_launch_ms": round(dom["avg_ms"], 5),
                     "traffic_source": traffic and traffic["source"]},
        "launches": [{k: (round(v, 5) if isinstance(v, float) else v) for k, v in L.items()}
                     for L in head["launches"]],
        "cpu_baseline": cpu and {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample", "host_nproc",
                                                     "host_cpu_model")},
        "extra": compact(extra),
        "hbm_copy_gbs": round(copy["gbs"], 1),
    }
    log("bench detail: " + json.dumps(extra))
    print(json.dumps(out))
    g.close()


if __name__ == "__main__":
    main()
