#!/usr/bin/env python3
"""Benchmark of the Q4_0 x Q8_0 decode GEMV hot path on one MI355X.

Workload (one "step"): the four OpenLLaMA-7B-shape decode GEMVs, M = 1,
[4096->4096], [4096->11008], [11008->4096], [4096->32000], each a full
tensor_matvec (Q8 activation quantization + Q4_0 x Q8 GEMV) through the C ABI.
Weights are N(0, 0.02) quantized to Q4_0, activations N(0, 1) with 0.1%
+-20 outliers; weights rotate over enough copies (> 600 MB) that every step
reads them from HBM, not from the 256 MB Infinity Cache.

`value` = algorithmic bytes of the step (weights + Q8 activation + scales +
fp32 output, per GEMV) / measured time, in GB/s.  `roofline` times the
dominant kernel alone (the Q4_0 GEMV launches, pre-quantized input) with HIP
events on the backend's stream.  `cpu_baseline` runs the compiled reference's
tensor_matvec (oracle/_ref, else the C restatement) on the host cores over a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "tg128 tok/s + achieved HBM GB/s (7B-shape Q4_0); pp512 prefill tok/s"
SHAPES = [("blk.0.attn_q.weight", 4096, 4096), ("blk.0.ffn_up.weight", 4096, 11008),
          ("blk.0.ffn_down.weight", 11008, 4096), ("output.weight", 4096, 32000)]  # (name, K, N)
HBM_PEAK_GBS = 8000.0


def gemv_bytes(k: int, n: int) -> int:
    """Algorithmic bytes of one Q4_0 x Q8 GEMV: weights + int8 act + f32 scales + f32 out."""
    return n * (k // 32) * 18 + k + 4 * (k // 32) + 4 * n


def make_weights(seed: int):
    import numpy as np

    from memvanta_amd import synth

    rng = np.random.default_rng(seed)
    out = []
    for name, k, n in SHAPES:
        w = synth.quantize_q4_0(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        out.append((name, k, n, w))
    return out


def cpu_baseline(weights, xs, budget_s: float = 12.0):
    """Time the reference CPU tensor_matvec on the same bytes (bounded sample)."""
    import numpy as np

    from memvanta_amd import synth
    from oracle import pyoracle

    threads = len(os.sched_getaffinity(0))
    step_bytes = sum(gemv_bytes(k, n) for _, k, n, _ in weights)
    if pyoracle.ref_available():
        kind = "reference"
        path = os.path.join(tempfile.gettempdir(), f"mv_bench_gemv_{os.getpid()}.gguf")
        w = synth.GgufWriter()
        w.add_str("general.architecture", "matrices")
        for name, k, n, data in weights:
            w.add_tensor(name, (k, n), synth.Q4_0, data.nbytes, lambda d=data: iter([d.tobytes()]))
        w.write(path)
        g = pyoracle.Ref().gguf(path)
        run = lambda name, k, n, data, x: g.matvec(name, x, n, threads)  # noqa: E731
    else:
        kind, path = "port", None
        o = pyoracle.Oracle()
        run = lambda name, k, n, data, x: o.matvec(data, synth.Q4_0, n, k, x, threads)  # noqa: E731
    for (name, k, n, data), x in zip(weights, xs):  # warm-up
        run(name, k, n, data, x)
    steps, t0 = 0, time.perf_counter()
    while True:
        for (name, k, n, data), x in zip(weights, xs):
            run(name, k, n, data, x)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 200:
            break
    if path:
        del g
        os.unlink(path)
    return {"value": round(steps * step_bytes / el / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"{steps} steps of the 4 GEMVs (tensor_matvec incl. Q8 quantization), {el:.1f} s, "
                      f"{threads} threads, warm host memory"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=6, help="weight copies rotated per step (cold HBM)")
    ap.add_argument("--kernel-launches", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from memvanta_amd import capi, synth

    ctx = capi.Context(0)
    stream = torch.cuda.ExternalStream(ctx.stream)
    weights = make_weights(1234)
    rng = np.random.default_rng(99)
    xs = [synth.activations(rng, 1, k)[0] for _, k, _, _ in weights]

    # R copies of every weight, each its own HBM allocation
    copies = [[ctx.upload(name, synth.Q4_0, k, n, w) for name, k, n, w in weights] for _ in range(args.copies)]
    xd = [torch.from_numpy(x).cuda() for x in xs]
    yd = [torch.empty(n, dtype=torch.float32, device="cuda") for _, _, n, _ in weights]
    qd = [torch.empty(k, dtype=torch.int8, device="cuda") for _, k, _, _ in weights]
    dd = [torch.empty(k // 32, dtype=torch.float32, device="cuda") for _, k, _, _ in weights]
    torch.cuda.synchronize()
    step_bytes = sum(gemv_bytes(k, n) for _, k, n, _ in weights)

    def step(i):
        ts = copies[i % args.copies]
        for j in range(len(ts)):
            ctx.matvec(ts[j], xd[j], yd[j])

    def capture(fn):
        # HIP graph of the C-ABI launches on the backend's stream (µs kernels
        # would otherwise be timed at the host's launch rate)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        ctx.synchronize()
        return g

    for i in range(args.warmup):
        step(i)
    ctx.synchronize()
    g_steps = capture(lambda: [step(i) for i in range(args.copies)])
    replays = max(1, (args.steps + args.copies - 1) // args.copies)
    n_steps = replays * args.copies
    with torch.cuda.stream(stream):
        g_steps.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(replays):
            g_steps.replay()
        e1.record(stream)
    e1.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_step = e0.elapsed_time(e1) / n_steps
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # dominant kernel alone: Q4_0 x Q8 GEMV on a pre-quantized input
    for j in range(len(weights)):
        ctx.quantize_q8(xd[j], qd[j], dd[j])
    ctx.synchronize()
    per_shape = []
    tot_bytes, tot_ms = 0, 0.0
    launches = max(args.copies, args.kernel_launches // args.copies * args.copies)
    for j, (name, k, n, _) in enumerate(weights):
        g = capture(lambda j=j: [ctx.matvec_q8(copies[i % args.copies][j], qd[j], dd[j], yd[j])
                                 for i in range(launches)])
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            g.replay()
            a.record(stream)
            for _ in range(3):
                g.replay()
            b.record(stream)
        b.synchronize()
        ms = a.elapsed_time(b) / (3 * launches)
        gb = gemv_bytes(k, n)
        per_shape.append({"shape": f"{k}->{n}", "us": round(ms * 1e3, 2), "GB/s": round(gb / ms / 1e6, 1)})
        tot_bytes += gb
        tot_ms += ms
    achieved = tot_bytes / tot_ms / 1e6

    traffic = None
    pmc = os.path.join(ROOT, "profiles", "gemv_q4_0_7b_shapes_traffic.json")
    if os.path.exists(pmc):
        with open(pmc) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    cpu = None if args.no_cpu else cpu_baseline(weights, xs)
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": n_steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8 (int8 dot, f32 accumulate)",
        "data": "synthetic",
        "config": {"workload": "7B-shape Q4_0 x Q8_0 decode GEMV, M=1: 4096->4096, 4096->11008, 11008->4096, "
                               "4096->32000 (tensor_matvec incl. Q8 quantization)",
                   "weight_copies_rotated": args.copies, "bytes_per_step": step_bytes,
                   "wall_s": round(wall, 3), "timing": "HIP graph replays, events on the backend stream",
                   "per_shape_kernel": per_shape},
        "roofline": {"bound": "hbm", "kernel": "gemv_q4_0_kernel<8>", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "avg_launch_us": round(tot_ms / len(weights) * 1e3, 2),
                     "algorithmic_bytes_per_launch": tot_bytes // len(weights)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))
    ctx.close()


if __name__ == "__main__":
    main()
