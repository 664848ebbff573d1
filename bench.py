#!/usr/bin/env python3
"""bench.py -- fp8 (e4m3) W8A16 linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 15]

Headline (``value``): BASELINE config 1, the decode-step GEMV set of one attention block and
one MLP block at M = 1 (q 3136->5120, k/v 3136->1024, o 5120->3136, up 3136->12544,
down 12544->3136), six launches per step in the engine's order, replayed from a HIP graph.
A step's algorithmic bytes are sum(N*K + 4N + 2K + 2N) = 117,427,456 B.  Weights rotate over
ten copies (1.17 GB > the 256 MB Infinity Cache + L2), so every step streams from HBM.
``value`` = bytes per step / measured time per step (GB/s, whole job, launch gaps included).

``roofline`` -- the GEMV kernel (the dominant kernel of the step): its algorithmic bytes per
launch over its average launch duration, from HIP events around each launch in a separate
pass over the same rotated weights (HBM-bound; peak 8 TB/s).

Also reported (same line): ``prefill_gemm`` (config 3, M = 2048, TFLOP/s vs 2.5 PFLOP/s dense
bf16 MFMA), ``decode_stream`` (config 4, 92 GEMVs over a 42-layer weight set),
``skinny`` (config 2, M in {2,4,8,16}) and ``cpu_baseline``: the torch CPU reference path
(fp32 dequant then F.linear, oracle/linear.py) on a bounded sample of config 1.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fp8 W8A16 GEMV achieved HBM GB/s (% of peak) at M=1; prefill GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
ROTATION_BYTES = 1 << 30


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-extras", action="store_true", help="headline and roofline only")
    return p.parse_args()


class Events:
    """Elapsed GPU time between events on torch's current stream (our launch stream)."""

    def __init__(self, n):
        import torch

        self.ev = [torch.cuda.Event(enable_timing=True) for _ in range(n)]

    def ms(self, i, j):
        return self.ev[i].elapsed_time(self.ev[j])


def prime_queue(ms=20):
    """Spin the GPU briefly so the host can enqueue ahead of it (event deltas then measure GPU
    time, not host launch latency)."""
    import torch

    try:
        torch.cuda._sleep(int(ms * 2.0e6))
    except Exception:
        pass


def decode_set_weights(dev, rotation_bytes):
    """Config-1 weights: seeded on the CPU (the same bytes feed the CPU baseline), copied to
    the GPU, then cloned into enough copies to defeat the caches."""
    import torch

    from nemotron_infer_amd import synth

    host, dset = [], []
    for i, lin in enumerate(synth.DECODE_SET):
        w, s = synth.make_weight(lin.N, lin.K, 1000 + i, "cpu")
        x = synth.make_act(1, lin.K, 1100 + i, "cpu", kind=lin.act)
        host.append((lin, x, w, s))
    set_bytes = sum(l.weight_bytes for l in synth.DECODE_SET)
    copies = max(2, math.ceil(rotation_bytes / set_bytes))
    base = [(lin, x.to(dev), w.to(dev), s.to(dev)) for lin, x, w, s in host]
    for _ in range(copies):
        dset.append([(lin, x, w.clone(), s.clone(),
                      torch.empty((1, lin.N), dtype=torch.bfloat16, device=dev)) for lin, x, w, s in base])
    return host, dset


def capture(fn, stream):
    import torch

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    return g


def bench_decode_set(args, dev):
    import torch

    from nemotron_infer_amd import ops, synth

    host, dset = decode_set_weights(dev, ROTATION_BYTES)
    R = len(dset)
    step_bytes = sum(synth.linear_bytes(1, l.N, l.K) for l in synth.DECODE_SET)

    def step(r):
        for lin, x, w, s, y in dset[r]:
            ops.linear_fp8_w8a16(x, w, s, out=y)

    # eager warm-up (also initialises per-device state before capture)
    for i in range(max(args.warmup, R)):
        step(i % R)
    torch.cuda.synchronize()

    stream = torch.cuda.Stream()
    graph_all = capture(lambda: [step(r) for r in range(R)], stream)
    tail = args.steps % R
    graph_tail = capture(lambda: [step(r) for r in range(tail)], stream) if tail else None
    for _ in range(max(1, args.warmup // R)):
        graph_all.replay()
    torch.cuda.synchronize()

    ev = Events(2)
    torch.cuda.synchronize()
    ev.ev[0].record()
    for _ in range(args.steps // R):
        graph_all.replay()
    if graph_tail is not None:
        graph_tail.replay()
    ev.ev[1].record()
    torch.cuda.synchronize()
    ms_total = ev.ms(0, 1)
    ms_per_step = ms_total / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    # Kernel durations: one event between consecutive launches, eager, queue primed.
    reps = max(4, min(args.steps, 40))
    n = reps * len(synth.DECODE_SET)
    kev = Events(n + 1)
    prime_queue()
    i = 0
    kev.ev[0].record()
    for rep in range(reps):
        for lin, x, w, s, y in dset[rep % R]:
            ops.linear_fp8_w8a16(x, w, s, out=y)
            i += 1
            kev.ev[i].record()
    torch.cuda.synchronize()
    per = {l.name: [] for l in synth.DECODE_SET}
    for k in range(n):
        lin = synth.DECODE_SET[k % len(synth.DECODE_SET)]
        per[lin.name].append(kev.ms(k, k + 1))
    kernels = {}
    tot_b, tot_ms = 0, 0.0
    for lin in synth.DECODE_SET:
        d = sorted(per[lin.name])[len(per[lin.name]) // 2]
        b = synth.linear_bytes(1, lin.N, lin.K)
        kernels[lin.name] = {"N": lin.N, "K": lin.K, "us": round(d * 1e3, 2),
                             "GB/s": round(b / (d * 1e-3) / 1e9, 1)}
        tot_b += b
        tot_ms += d
    achieved = tot_b / (tot_ms * 1e-3) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "gemv_fp8_m1_kernel",
                "per_launch_bytes_avg": tot_b // len(synth.DECODE_SET),
                "per_launch_us_avg": round(tot_ms * 1e3 / len(synth.DECODE_SET), 2)}
    return dict(value=value, ms_per_step=ms_per_step, step_bytes=step_bytes, copies=R,
                roofline=roofline, kernels=kernels, host=host)


def bench_prefill(dev, reps=20):
    import torch

    from nemotron_infer_amd import ops, synth

    out = {}
    tot_f, tot_ms = 0, 0.0
    for i, lin in enumerate(synth.PREFILL_SET):
        M = synth.PREFILL_M
        w, s = synth.make_weight(lin.N, lin.K, 3000 + i, dev)
        x = synth.make_act(M, lin.K, 3100 + i, dev, kind=lin.act, outlier_frac=0.001)
        y = torch.empty((M, lin.N), dtype=torch.bfloat16, device=dev)
        for _ in range(3):
            ops.gemm_fp8_w8a16(x, w, s, out=y)
        torch.cuda.synchronize()
        ev = Events(reps + 1)
        prime_queue(5)
        ev.ev[0].record()
        for r in range(reps):
            ops.gemm_fp8_w8a16(x, w, s, out=y)
            ev.ev[r + 1].record()
        torch.cuda.synchronize()
        d = sorted(ev.ms(r, r + 1) for r in range(reps))[reps // 2]
        fl = synth.linear_flops(M, lin.N, lin.K)
        out[lin.name] = {"M": M, "N": lin.N, "K": lin.K, "us": round(d * 1e3, 1),
                         "TFLOP/s": round(fl / (d * 1e-3) / 1e12, 1)}
        tot_f += fl
        tot_ms += d
        del w, s, x, y
    tf = tot_f / (tot_ms * 1e-3) / 1e12
    return {"workload": "config3_prefill_m2048", "tflops": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4), "kernel": "gemm_fp8_w8a16_kernel",
            "shapes": out}


def bench_decode_stream(dev, reps=5):
    import torch

    from nemotron_infer_amd import ops, synth

    layers = synth.decode_stream_layers()
    acts = {}
    mats = []
    for li, kind, lins in layers:
        for j, lin in enumerate(lins):
            w, s = synth.make_weight(lin.N, lin.K, 40000 + 10 * li + j, dev)
            if (lin.K, lin.act) not in acts:
                acts[(lin.K, lin.act)] = synth.make_act(1, lin.K, 41000 + lin.K, dev, kind=lin.act)
            y = torch.empty((1, lin.N), dtype=torch.bfloat16, device=dev)
            mats.append((lin, acts[(lin.K, lin.act)], w, s, y))
    total_bytes = sum(synth.linear_bytes(1, l.N, l.K) for l, *_ in mats)
    weight_bytes = sum(l.N * l.K for l, *_ in mats)

    def run():
        for lin, x, w, s, y in mats:
            ops.linear_fp8_w8a16(x, w, s, out=y)

    run()
    torch.cuda.synchronize()
    g = capture(run, torch.cuda.Stream())
    g.replay()
    torch.cuda.synchronize()
    ev = Events(2)
    ev.ev[0].record()
    for _ in range(reps):
        g.replay()
    ev.ev[1].record()
    torch.cuda.synchronize()
    ms = ev.ms(0, 1) / reps
    gbs = total_bytes / (ms * 1e-3) / 1e9
    n_gemv = len(mats)
    del mats
    return {"workload": "config4_42layer_decode_stream", "gemvs": n_gemv,
            "bytes": total_bytes, "weight_bytes": weight_bytes, "ms": round(ms, 4),
            "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "tok_per_s_ceiling": round(1e3 / ms, 1)}


def bench_skinny(dev, host_sets, reps=20):
    import torch

    from nemotron_infer_amd import ops, synth

    res = {}
    copies = []
    set_bytes = sum(l.weight_bytes for l in synth.DECODE_SET)
    R = max(2, math.ceil(ROTATION_BYTES / set_bytes))
    base = [(lin, w.to(dev), s.to(dev)) for lin, x, w, s in host_sets]
    for _ in range(R):
        copies.append([(lin, w.clone(), s.clone()) for lin, w, s in base])
    for M in (2, 4, 8, 16):
        xs = [synth.make_act(M, lin.K, 2200 + M, dev, kind=lin.act) for lin in synth.DECODE_SET]
        ys = [torch.empty((M, lin.N), dtype=torch.bfloat16, device=dev) for lin in synth.DECODE_SET]

        def step(r):
            for (lin, w, s), x, y in zip(copies[r], xs, ys):
                ops.linear_fp8_w8a16(x, w, s, out=y)

        for r in range(R):
            step(r)
        torch.cuda.synchronize()
        g = capture(lambda: [step(r) for r in range(R)], torch.cuda.Stream())
        g.replay()
        torch.cuda.synchronize()
        ev = Events(2)
        ev.ev[0].record()
        for _ in range(max(1, reps // R)):
            g.replay()
        ev.ev[1].record()
        torch.cuda.synchronize()
        nsteps = max(1, reps // R) * R
        ms = ev.ms(0, 1) / nsteps
        b = sum(synth.linear_bytes(M, l.N, l.K) for l in synth.DECODE_SET)
        f = sum(synth.linear_flops(M, l.N, l.K) for l in synth.DECODE_SET)
        res[f"M={M}"] = {"us_per_step": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                         "TFLOP/s": round(f / (ms * 1e-3) / 1e12, 2)}
    del copies
    return {"workload": "config2_skinny_decode_set", "results": res}


def cpu_baseline(host_sets, seconds):
    """The reference's CPU path (tools/ref_full_model.py:44-49,137, restated in
    oracle/linear.py): fp32 dequant of W, F.linear in fp32, bf16 rounding -- on config 1's
    bytes, for about ``seconds`` of work."""
    import numpy as np
    import torch

    from nemotron_infer_amd import synth
    from oracle import linear as olin

    data = [(x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy()) for _, x, w, s in host_sets]
    step_bytes = sum(synth.linear_bytes(1, l.N, l.K) for l, *_ in host_sets)
    threads = torch.get_num_threads()
    olin.linear_fp8_w8a16(*data[0])          # warm-up
    t0 = time.perf_counter()
    steps = 0
    while True:
        for x, w, s in data:
            olin.linear_fp8_w8a16(x, w, s)
        steps += 1
        if time.perf_counter() - t0 >= seconds and steps >= 2:
            break
    dt = time.perf_counter() - t0
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(step_bytes * steps / dt / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "ms_per_step": round(dt / steps * 1e3, 1),
            "sample": f"config 1 decode set (6 GEMVs, M=1), {steps} steps in {dt:.1f} s: "
                      f"torch CPU fp32 dequant + F.linear + bf16 round (oracle/linear.py), "
                      f"{threads} threads of os.cpu_count()={os.cpu_count()} ({model})"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the fp8 linear "
              f"path is single-GPU, multi-GPU sharding is a design note in DESIGN.md", file=sys.stderr)
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs the GPU"
    dev = "cuda:0"
    torch.cuda.set_device(0)
    t0 = time.time()
    log("decode set (config 1) ...")
    d = bench_decode_set(args, dev)
    log(f"decode set: {d['value']:.1f} GB/s, {d['ms_per_step'] * 1e3:.2f} us/step; kernel {d['roofline']['achieved']} GB/s")
    extras = {}
    if not args.no_extras:
        log("prefill GEMM (config 3) ...")
        extras["prefill_gemm"] = bench_prefill(dev)
        log(f"prefill: {extras['prefill_gemm']['tflops']} TFLOP/s")
        log("skinny M (config 2) ...")
        extras["skinny"] = bench_skinny(dev, d["host"])
        log("decode stream (config 4) ...")
        extras["decode_stream"] = bench_decode_stream(dev)
        log(f"stream: {extras['decode_stream']['GB/s']} GB/s")
    torch.cuda.empty_cache()
    log("cpu baseline ...")
    cpu = cpu_baseline(d["host"], args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(d["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights -> e4m3 per-tensor scale; bf16 N(0,1) / relu^2 activations)",
        "config": {"workload": "config1_decode_gemv_set_m1",
                   "shapes": {k: [v["N"], v["K"]] for k, v in d["kernels"].items()},
                   "M": 1, "bytes_per_step": d["step_bytes"],
                   "weight_copies_rotated": d["copies"],
                   "operands": "W e4m3 [N,K] + f32 per-row scale, x bf16, y bf16, f32 accumulate",
                   "launch": "HIP graph of the six GEMV launches per step"},
        "roofline": d["roofline"],
        "cpu_baseline": cpu,
        "kernels": d["kernels"],
        **extras,
        "wall_s": round(time.time() - t0, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
