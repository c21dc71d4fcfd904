"""Benchmark of the quantized-weight hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): batch-1 Q4_0 GEMV at the Qwen2-0.5B layer shapes
K x N in {896 x 1152, 896 x 4864, 4864 x 896}, in HBM GB/s and as a fraction of the 8 TB/s peak.

A step is one pass of the batch-1 GEMV over a pool of distinct resident Q4_0 weights of those
three shapes (about 1 GiB, four times the 256 MB last-level cache, so every byte comes from
HBM), each with its own x and y, launched as one grouped launch per width class. Inputs are
resident in HBM before the timed region. Weights are seeded N(0, 0.02), x ~ N(0, 1) (synthetic).

Also reported (extra keys): the Q8_0 GPT-2 QKV GEMV (config 0), the MFMA dequant-GEMM at the
Qwen2 scoring shapes (M = 512, 2048) in TFLOP/s, and the CPU baseline (the reference's CPU
path restated in C: f32 GEMV on the dequantised weights, one thread).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(kind_bytes: int, k: int, n: int) -> int:
    """Algorithmic bytes of one batch-1 product: the packed weight, x and y."""
    return (k // 32) * n * kind_bytes + 4 * k + 4 * n


class Timer:
    """HIP events on the library's own stream (the stream the kernels run on)."""

    def __init__(self, g):
        import torch

        self.torch = torch
        self.stream = torch.cuda.ExternalStream(g.stream())

    def event(self):
        e = self.torch.cuda.Event(enable_timing=True)
        e.record(self.stream)
        return e


def bench_gemv_pool(fh, g, timer, kind, shapes, pool_bytes, steps, warmup, seed=0):
    rng = np.random.default_rng(seed)
    kb = kind.file_bytes()
    set_bytes = sum((k // 32) * n * kb for k, n in shapes)
    copies = max(1, int(pool_bytes // set_bytes))
    packed = []  # packed once on the device, then uploaded as distinct copies
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        packed.append(fh.upload_quantised(g, kind, w, k, n).read_gguf())
    keep, probs = [], []
    for c in range(copies):
        for (k, n), b in zip(shapes, packed):
            qw = fh.upload_qweight(g, kind, b, k, n)
            gx = g.upload(rng.standard_normal(k).astype(np.float32))
            gy = g.zeros(n)
            keep += [qw, gx, gy]
            probs.append((qw, gx.device_ptr(), gy.device_ptr()))
    plan = fh.GemvPlan(g, probs)
    step_bytes = plan.bytes()
    for _ in range(warmup):
        plan.run()
    g.sync()
    t0 = time.perf_counter()
    e0 = timer.event()
    for _ in range(steps):
        plan.run()
    e1 = timer.event()
    g.sync()
    wall = time.perf_counter() - t0
    ev_ms = e0.elapsed_time(e1)
    res = {
        "copies": copies, "products": len(probs), "launches_per_step": plan.launches(),
        "bytes_per_step": step_bytes, "ms_per_step": ev_ms / steps,
        "wall_ms_per_step": wall * 1e3 / steps,
        "gbs": step_bytes * steps / (ev_ms * 1e-3) / 1e9,
    }
    plan.free()
    del keep
    return res


def bench_gemm(fh, g, timer, kind, m, shapes, steps, seed=0):
    rng = np.random.default_rng(seed)
    items = []
    for k, n in shapes:
        w = (rng.standard_normal(k * n) * 0.02).astype(np.float32)
        qw = fh.upload_quantised(g, kind, w, k, n)
        gx = g.upload(rng.standard_normal(m * k).astype(np.float32))
        gy = g.zeros(m * n)
        items.append((qw, gx, gy))
    flops = sum(2 * m * k * n for k, n in shapes)
    for qw, gx, gy in items:
        fh.linear_q_with(g, gx, qw, gy, m, fh.QPath.Tiled)
    g.sync()
    e0 = timer.event()
    for _ in range(steps):
        for qw, gx, gy in items:
            fh.linear_q_with(g, gx, qw, gy, m, fh.QPath.Tiled)
    e1 = timer.event()
    g.sync()
    ms = e0.elapsed_time(e1) / steps
    return {"m": m, "flops_per_step": flops, "ms_per_step": ms, "tflops": flops / (ms * 1e-3) / 1e12}


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
    return {"value": alg / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} reps (median) of one pass over {shapes} Q4_0-sized work on f32 "
                      f"dequantised weights, {sum(x[2]*x[3] for x in mats)} weights; f32 stream "
                      f"{f32b / med / 1e9:.2f} GB/s; {med * 1e3:.3f} ms per pass",
            "f32_gbs": f32b / med / 1e9, "ms_per_pass": med * 1e3}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--pool-gib", type=float, default=1.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported (the path shards by "
              "output rows with no exchange; see the sharding design)", file=sys.stderr)
        sys.exit(2)

    import ferrum_hip as fh

    g = fh.Gpu(0)
    timer = Timer(g)
    name, cus = g.info()
    log(f"device {name}, {cus} CUs")

    head = bench_gemv_pool(fh, g, timer, fh.QKind.Q4_0, QWEN_SHAPES, a.pool_gib * 2**30, a.steps, a.warmup)
    log("Q4_0 GEMV pool:", head)
    extra = {}
    if not a.no_extra:
        q8 = bench_gemv_pool(fh, g, timer, fh.QKind.Q8_0, [(768, 2304)], a.pool_gib * 2**30, a.steps, a.warmup, seed=1)
        log("Q8_0 GEMV pool:", q8)
        extra["q8_0_gemv_768x2304"] = {"gbs": q8["gbs"], "frac": q8["gbs"] / HBM_PEAK_GBS, "ms_per_step": q8["ms_per_step"],
                                       "bytes_per_step": q8["bytes_per_step"]}
        for m in (512, 2048):
            r = bench_gemm(fh, g, timer, fh.QKind.Q4_0, m, QWEN_SHAPES, 10)
            log(f"Q4_0 GEMM M={m}:", r)
            extra[f"q4_0_gemm_m{m}"] = {"tflops": r["tflops"], "frac": r["tflops"] / MFMA_F16_PEAK_TFLOPS,
                                        "ms_per_step": r["ms_per_step"], "flops_per_step": r["flops_per_step"],
                                        "operands": "split-f16 x (hi+lo) x exact integer q, f32 accumulate, f32 block scale"}

    cpu = None
    if not a.no_cpu:
        cpu = cpu_baseline(QWEN_SHAPES, 18)
        log("cpu baseline:", cpu)

    gbs = head["gbs"]
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
        "dtype": "q4_0 weights, f32 activations and accumulation",
        "data": "synthetic: seeded N(0,0.02) weights packed Q4_0, x ~ N(0,1)",
        "config": {"workload": "Q4_0 GEMV sweep, K x N in {896x1152, 896x4864, 4864x896}, "
                               f"{head['copies']} distinct copies each ({head['bytes_per_step'] / 2**30:.2f} GiB per step)",
                   "products_per_step": head["products"], "launches_per_step": head["launches_per_step"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu and {k: cpu[k] for k in ("value", "unit", "cores", "kind", "sample")},
        "extra": extra,
    }
    print(json.dumps(out))
    g.close()


if __name__ == "__main__":
    main()
