#!/usr/bin/env python3
"""bench.py -- fp8 (e4m3) W8A16 linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20] [--cpu-seconds 15] [--no-extras]
                    [--only stream|decode|prefill|prefill_small|block|skinny|attn|mamba|engine|prefill_attn|prefill_mamba]

Headline (``value``): config 4 of the reference's benchmark, the full decode-step weight stream at M = 1 -- 4
attention layers (q|k|v grouped: they share one normed input, model/attention_block.cuh:400-402;
then o), 17 MLP layers (up, down) and 21 Mamba layers (in_proj with ragged N = 14690, out_proj
with K = 6272): 92 GEMVs over 2.87 GB of e4m3 weights, each GEMV on its own seeded activation.
A step is one GEMV chain launch (nmi_gemv_chain, 84 phases) replayed from a HIP graph; the
stream is larger than the 256 MB Infinity Cache, so every step reads W from HBM.  A step's
algorithmic bytes are sum(N*K + 4N + 2K + 2N) over the 92 matrices = 2,877,242,812 B; ``value``
= bytes per step / time per step (GB/s); the north star's target is >= 80% of 8 TB/s on it.

``roofline`` -- the chain kernel (one launch per step): algorithmic bytes per launch over the
launch duration, both from the timed region (graph replay, HIP events on the replay stream);
HBM-bound, peak 8 TB/s; ``traffic`` -- HBM bytes per launch from rocprofv3 FETCH_SIZE /
WRITE_SIZE (profiles/gemv_chain_config4_decode_stream.md).  Beside it: the same GEMVs as 84
separate launches, and as a dependent chain (every phase waits for its predecessor).

Also reported (same line): ``decode_set`` (config 1, one attention and one MLP block at M = 1,
ten rotated weight copies: one chain launch per step, the engine's four launches, each launch
alone, six separate launches, the dependent chain), ``prefill_gemm`` (config 3, M = 2048,
TFLOP/s against 2.5 PFLOP/s dense bf16 MFMA; steady state: timed after 0.3 s of untimed
replays), ``skinny`` (config 2, M in {2,4,8,16}, four launches per step), ``mlp_block`` (the fp8
MLP block, decode and prefill, fused against the reference's five-launch structure) and
``cpu_baseline``: the torch CPU reference path (per call: fp32 dequant of W, then F.linear in
fp32, bf16 rounding -- tools/ref_full_model.py:44-49,137, restated in oracle/linear.py) on a
bounded sample of config 4's layers on this host's cores, with the matmul-only time (W
dequantized once, outside the timed region) and config 1 and config 3 samples beside it.
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
# HBM bytes per launch of the headline (config 4 as one chain launch), from rocprofv3
# FETCH_SIZE / WRITE_SIZE runs of `bench.py --only stream` scaled by a 256 MiB copy
# (profiles/gemv_chain_config4_decode_stream.md).  Re-measured when the GEMV kernels change;
# reported as roofline.traffic next to the algorithmic bytes.  None until measured.
MEASURED_TRAFFIC = {"chain_config4": 2902926840}


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--no-extras", action="store_true", help="headline, roofline and CPU baseline only")
    p.add_argument("--only", choices=["stream", "decode", "prefill", "block", "skinny", "attn", "mamba", "engine", "prefill_attn", "prefill_mamba",
                                       "prefill_small"],
                   help="run one extra leg alone and print its JSON record (for profiling that leg); "
                        "not the bench contract line")
    p.add_argument("--pmc-calibration", action="store_true",
                   help="first copy 256 MiB device-to-device three times (a kernel of known traffic "
                        "that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    return p.parse_args()


class Timer:
    """HIP events on a dedicated stream; everything timed is launched on that stream."""

    def __init__(self):
        import torch

        self.stream = torch.cuda.Stream()
        self.t0 = torch.cuda.Event(enable_timing=True)
        self.t1 = torch.cuda.Event(enable_timing=True)

    def capture(self, fn):
        import torch

        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            fn()
        return g

    def time_replays(self, graphs):
        """Run ``graphs`` (a list, replayed in order) between two events; return ms."""
        import torch

        torch.cuda.synchronize()
        with torch.cuda.stream(self.stream):
            self.t0.record(self.stream)
            for g in graphs:
                g.replay()
            self.t1.record(self.stream)
        torch.cuda.synchronize()
        return self.t0.elapsed_time(self.t1)


def rotated(dev, host, copies):
    import torch

    base = [(w.to(dev), s.to(dev)) for w, s in host]
    return [[(w.clone(), s.clone()) for w, s in base] for _ in range(copies)]


def decode_inputs():
    """Config-1 weights and activations, seeded on the CPU (the same bytes feed the CPU
    baseline)."""
    from nemotron_infer_amd import synth

    host = []
    for i, lin in enumerate(synth.DECODE_SET):
        w, s = synth.make_weight(lin.N, lin.K, 1000 + i, "cpu")
        x = synth.make_act(1, lin.K, 1100 + i, "cpu", kind=lin.act)
        host.append((lin, x, w, s))
    return host


def make_step(ops, xs, mats, ys, ws_use=True):
    """One decode step over one weight copy: q|k|v grouped, then o, up, down."""
    (wq, sq), (wk, sk), (wv, sv), (wo, so), (wu, su), (wd, sd) = mats
    x_attn, x_o, x_up, x_down = xs
    y_qkv, y_o, y_up, y_down = ys

    def step():
        ops.linear_fp8_w8a16_grouped(x_attn, [(wq, sq), (wk, sk), (wv, sv)], outs=y_qkv,
                                     use_workspace=ws_use)
        ops.linear_fp8_w8a16(x_o, wo, so, out=y_o, use_workspace=ws_use)
        ops.linear_fp8_w8a16(x_up, wu, su, out=y_up, use_workspace=ws_use)
        ops.linear_fp8_w8a16(x_down, wd, sd, out=y_down, use_workspace=ws_use)

    return step


def make_batch_step(ops, xs, mats, ys):
    """The same step as one nmi_linear_fp8_w8a16_batch call: six jobs (q, k and v on the one
    attention activation, o, up and down on their own), one launch of the skinny kernel."""
    (wq, sq), (wk, sk), (wv, sv), (wo, so), (wu, su), (wd, sd) = mats
    x_attn, x_o, x_up, x_down = xs
    y_qkv, y_o, y_up, y_down = ys
    jobs = [(x_attn, wq, sq), (x_attn, wk, sk), (x_attn, wv, sv), (x_o, wo, so), (x_up, wu, su), (x_down, wd, sd)]
    outs = list(y_qkv) + [y_o, y_up, y_down]

    def step():
        ops.linear_fp8_w8a16_batch(jobs, outs=outs)

    return step


def step_buffers(dev, M, K_attn=3136):
    import torch

    from nemotron_infer_amd import synth

    L = synth.DECODE_SET
    y_qkv = [torch.empty((M, l.N), dtype=torch.bfloat16, device=dev) for l in L[:3]]
    return (y_qkv, torch.empty((M, L[3].N), dtype=torch.bfloat16, device=dev),
            torch.empty((M, L[4].N), dtype=torch.bfloat16, device=dev),
            torch.empty((M, L[5].N), dtype=torch.bfloat16, device=dev))


def make_chain(ops, xs, mats, ys, dependent=False):
    """The step as one GEMV chain launch: phases q|k|v, o, up, down.  dependent: each phase reads
    the previous phase's output (q -> o -> up -> down chain by shape: 5120, 3136, 12544) and
    waits for it; otherwise every phase reads its own config-1 activation."""
    (wq, sq), (wk, sk), (wv, sv), (wo, so), (wu, su), (wd, sd) = mats
    x_attn, x_o, x_up, x_down = xs
    y_qkv, y_o, y_up, y_down = ys
    if dependent:
        x_o, x_up, x_down = y_qkv[0], y_o, y_up
    return ops.GemvChain([(x_attn, [(wq, sq, y_qkv[0]), (wk, sk, y_qkv[1]), (wv, sv, y_qkv[2])], False),
                          (x_o, [(wo, so, y_o)], dependent), (x_up, [(wu, su, y_up)], dependent),
                          (x_down, [(wd, sd, y_down)], dependent)])


def bench_decode_set(args, dev, host):
    import torch

    from nemotron_infer_amd import ops, synth

    set_bytes = sum(l.weight_bytes for l in synth.DECODE_SET)
    R = max(2, math.ceil(ROTATION_BYTES / set_bytes))
    copies = rotated(dev, [(w, s) for _, _, w, s in host], R)
    xs = (host[0][1].to(dev), host[3][1].to(dev), host[4][1].to(dev), host[5][1].to(dev))
    ys = step_buffers(dev, 1)
    chains = [make_chain(ops, xs, copies[r], ys) for r in range(R)]
    step_bytes = sum(synth.linear_bytes(1, l.N, l.K) for l in synth.DECODE_SET)

    for i in range(2 * R):                        # eager warm-up, also before any capture
        chains[i % R].launch()
    torch.cuda.synchronize()
    T = Timer()
    g_all = T.capture(lambda: [c.launch() for c in chains])
    T.time_replays([g_all] * 2)
    reps = 20
    ms_per_step = T.time_replays([g_all] * reps) / (reps * R)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    def timed(fn, reps=5):
        g = T.capture(lambda: [fn(r) for r in range(R)])
        T.time_replays([g])
        t = T.time_replays([g] * reps) / (reps * R)
        del g
        return {"us_per_step": round(t * 1e3, 2), "GB/s": round(step_bytes / (t * 1e-3) / 1e9, 1)}

    # The engine's launch structure: q|k|v grouped, o, up, down (four launches).
    steps = [make_step(ops, xs, copies[r], ys) for r in range(R)]
    engine = {"launches": 4, **timed(lambda r: steps[r]())}
    # Each of those launches alone: a graph of that launch over the R copies.
    L = synth.DECODE_SET
    launches = {}
    groups = [("qkv_grouped", [0, 1, 2]), ("o_proj", [3]), ("up_proj", [4]), ("down_proj", [5])]
    for name, idx in groups:
        def one(r, idx=idx):
            if len(idx) > 1:
                ops.linear_fp8_w8a16_grouped(xs[0], [copies[r][i] for i in idx], outs=ys[0])
            else:
                i = idx[0]
                ops.linear_fp8_w8a16(xs[{3: 1, 4: 2, 5: 3}[i]], *copies[r][i], out=ys[{3: 1, 4: 2, 5: 3}[i]])
        g = T.capture(lambda: [one(r) for r in range(R)])
        T.time_replays([g])
        t = T.time_replays([g] * 5) / (5 * R)
        b = sum(synth.linear_bytes(1, L[i].N, L[i].K) for i in idx)
        launches[name] = {"N": sum(L[i].N for i in idx), "K": L[idx[0]].K, "bytes": b,
                          "us": round(t * 1e3, 2), "GB/s": round(b / (t * 1e-3) / 1e9, 1)}
        del g

    # The six matrices as six separate launches (the reference's launch structure).
    def six(r):
        for i, l in enumerate(L):
            xi = xs[0] if i < 3 else xs[{3: 1, 4: 2, 5: 3}[i]]
            yi = ys[0][i] if i < 3 else ys[{3: 1, 4: 2, 5: 3}[i]]
            ops.linear_fp8_w8a16(xi, *copies[r][i], out=yi)
    separate = {"launches": 6, **timed(six)}
    # The dependent chain: each phase waits for and reads the previous phase's output (a launch
    # per phase, ordered by the stream).
    dep = [make_chain(ops, xs, copies[r], ys, dependent=True) for r in range(R)]
    for c in dep:
        c.launch()
    torch.cuda.synchronize()
    dependent = {"launches": dep[0].launches, **timed(lambda r: dep[r].launch())}
    del copies, chains, steps, dep, g_all
    return {"workload": "config1_decode_gemv_set_m1", "bytes_per_step": step_bytes, "weight_copies_rotated": R,
            "chain_one_launch": {"launches": 1, "us_per_step": round(ms_per_step * 1e3, 2),
                                 "GB/s": round(value, 1), "frac": round(value / HBM_PEAK_GBS, 4)},
            "engine_four_launches": engine, "launches": launches, "six_separate_launches": separate,
            "chain_dependent": dependent}


def steady(T, graph, seconds=0.3):
    """Untimed replays for about `seconds`: under sustained MFMA load the GPU takes ~0.1 s to
    raise its clock (measured: the first replays of a prefill GEMM run ~20% slower), and a real
    prefill runs its layers' GEMMs back to back."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        T.time_replays([graph])


def bench_prefill(dev, reps=20):
    import torch

    from nemotron_infer_amd import ops, synth

    out = {}
    tot_f, tot_ms = 0, 0.0
    T = Timer()
    for i, lin in enumerate(synth.PREFILL_SET):
        M = synth.PREFILL_M
        w, s = synth.make_weight(lin.N, lin.K, 3000 + i, dev)
        x = synth.make_act(M, lin.K, 3100 + i, dev, kind=lin.act, outlier_frac=0.001)
        y = torch.empty((M, lin.N), dtype=torch.bfloat16, device=dev)
        for _ in range(3):
            ops.gemm_fp8_w8a16(x, w, s, out=y)
        g = T.capture(lambda: [ops.gemm_fp8_w8a16(x, w, s, out=y) for _ in range(reps)])
        steady(T, g)
        d = T.time_replays([g]) / reps
        fl = synth.linear_flops(M, lin.N, lin.K)
        out[lin.name] = {"M": M, "N": lin.N, "K": lin.K, "us": round(d * 1e3, 1),
                         "TFLOP/s": round(fl / (d * 1e-3) / 1e12, 1)}
        tot_f += fl
        tot_ms += d
        del w, s, x, y, g
    tf = tot_f / (tot_ms * 1e-3) / 1e12
    return {"workload": "config3_prefill_m2048", "tflops": round(tf, 1), "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4), "kernel": "gemm_fp8_w8a16_dma_kernel (4 waves, 256x256 or 128x256 tiles by round count, DMA-fed LDS)",
            "shapes": out}


def bench_prefill_small_m(dev, reps=20):
    """Short prompts: the three config-3 shapes at M = 64, 128, 256 (the GEMM path below the
    256x256 DMA kernel's M >= 512).  Weights rotated over copies of >= 1 GiB, since at these M
    the launch also streams W (the arithmetic intensity is about 2M flop/B, below MI355X's
    ~315 flop/B ridge up to M ~ 150)."""
    import torch

    from nemotron_infer_amd import ops, synth

    T = Timer()
    set_bytes = sum(l.N * l.K for l in synth.PREFILL_SET)
    R = max(2, math.ceil(ROTATION_BYTES / set_bytes))
    ws = [synth.make_weight(l.N, l.K, 3000 + i, dev) for i, l in enumerate(synth.PREFILL_SET)]
    copies = [[(w.clone(), s.clone()) for (w, s) in ws] for _ in range(R)]
    del ws
    res = {}
    for M in (64, 128, 256):
        shapes = {}
        tot_f = tot_b = tot_ms = 0.0
        for i, lin in enumerate(synth.PREFILL_SET):
            x = synth.make_act(M, lin.K, 3200 + M + i, dev, kind=lin.act)
            y = torch.empty((M, lin.N), dtype=torch.bfloat16, device=dev)
            calls = [lambda r=r: ops.gemm_fp8_w8a16(x, copies[r][i][0], copies[r][i][1], out=y) for r in range(R)]
            for c in calls:
                c()
            g = T.capture(lambda: [c() for c in calls])
            steady(T, g, 0.1)
            n = max(1, reps // R)
            d = T.time_replays([g] * n) / (n * R)
            fl = synth.linear_flops(M, lin.N, lin.K)
            by = synth.linear_bytes(M, lin.N, lin.K)
            shapes[lin.name] = {"us": round(d * 1e3, 2), "TFLOP/s": round(fl / (d * 1e-3) / 1e12, 1),
                                "GB/s": round(by / (d * 1e-3) / 1e9, 1)}
            tot_f += fl
            tot_b += by
            tot_ms += d
            del g, calls, x, y
        res[f"M={M}"] = {"TFLOP/s": round(tot_f / (tot_ms * 1e-3) / 1e12, 1),
                         "GB/s": round(tot_b / (tot_ms * 1e-3) / 1e9, 1), "shapes": shapes}
    del copies
    return {"workload": "config3 shapes at short-prompt M", "weight_copies_rotated": R, "results": res}


def bench_skinny(dev, reps=20):
    """Config 2: the config-1 shapes at M in {2, 4, 8, 16}, weights with per-row log-uniform
    scales, every activation row its own N(0, 1) draw (down_proj included)."""
    import torch

    from nemotron_infer_amd import ops, synth

    L = synth.SKINNY_SET
    set_bytes = sum(l.weight_bytes for l in L)
    R = max(2, math.ceil(ROTATION_BYTES / set_bytes))
    base = [synth.make_weight(l.N, l.K, 2100 + i, dev, scales="log_uniform") for i, l in enumerate(L)]
    copies = [[(w.clone(), s.clone()) for w, s in base] for _ in range(R)]
    del base
    res = {}
    T = Timer()
    for M in synth.SKINNY_M:
        xs = tuple(synth.make_act(M, L[i].K, 2200 + M + i, dev, kind=L[i].act) for i in (0, 3, 4, 5))
        ys = step_buffers(dev, M)
        b = sum(synth.linear_bytes(M, l.N, l.K) for l in L)
        f = sum(synth.linear_flops(M, l.N, l.K) for l in L)
        rec = {}
        for form, make in (("four_launches", make_step), ("batch_one_launch", make_batch_step)):
            steps = [make(ops, xs, copies[r], ys) for r in range(R)]
            for s in steps:
                s()
            torch.cuda.synchronize()
            g = T.capture(lambda: [s() for s in steps])
            T.time_replays([g])
            n = max(1, reps // R)
            ms = T.time_replays([g] * n) / (n * R)
            rec[form] = {"us_per_step": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                         "TFLOP/s": round(f / (ms * 1e-3) / 1e12, 2)}
            del g, steps
        res[f"M={M}"] = dict(rec["four_launches"], batch_one_launch=rec["batch_one_launch"])
    del copies
    return {"workload": "config2_skinny_decode_set", "launches_per_step": 4,
            "note": "per-M figures: q|k|v grouped, o, up, down as four launches (the engine's form); "
                    "batch_one_launch: the six linears as one nmi_linear_fp8_w8a16_batch launch",
            "results": res}


def bench_decode_stream(args, dev):
    """Config 4 (the headline): the 84-phase chain launch per step, timed over args.steps
    replays after args.warmup; beside it the same GEMVs as separate launches and as a dependent
    chain."""
    import torch

    from nemotron_infer_amd import ops, synth

    layers = synth.decode_stream_layers()
    phases, calls, total_bytes, weight_bytes, _ = synth.decode_stream_chain(dev)

    def run():
        for c in calls:
            if c[0] == "grouped":
                ops.linear_fp8_w8a16_grouped(c[1], c[2], outs=c[3])
            else:
                ops.linear_fp8_w8a16(c[1], c[2], c[3], out=c[4])

    chain = ops.GemvChain(phases)
    run()
    for _ in range(max(1, args.warmup)):          # eager warm-up, also before any capture
        chain.launch()
    torch.cuda.synchronize()
    T = Timer()
    # graphs of up to 20 launches, replayed to make exactly args.steps launches
    per_g = min(20, args.steps)
    g = T.capture(lambda: [chain.launch() for _ in range(per_g)])
    tail = args.steps % per_g
    g_tail = T.capture(lambda: [chain.launch() for _ in range(tail)]) if tail else None
    T.time_replays([g] * max(1, args.warmup // per_g))
    ms = T.time_replays([g] * (args.steps // per_g) + ([g_tail] if g_tail is not None else []))
    ms_per_step = ms / args.steps
    value = total_bytes / (ms_per_step * 1e-3) / 1e9

    def timed(fn, reps=5):
        gg = T.capture(fn)
        T.time_replays([gg])
        t = T.time_replays([gg] * reps) / reps
        del gg
        gbs = total_bytes / (t * 1e-3) / 1e9
        return {"ms": round(t, 4), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                "tok_per_s_ceiling": round(1e3 / t, 1)}

    sep = timed(run)
    dep_chain = ops.GemvChain([(x, grp, i > 0) for i, (x, grp, _) in enumerate(phases)])
    dep_chain.launch()
    torch.cuda.synchronize()
    dep = timed(dep_chain.launch)
    roofline = {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBS, 4), "traffic": MEASURED_TRAFFIC["chain_config4"],
                "traffic_source": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE per launch of `bench.py --only stream` "
                                  "(x2.0 / x1.0 copy calibration), profiles/gemv_chain_config4_decode_stream.md",
                "kernel": "gemv_stream_kernel (chain form, one launch per step)",
                "launches_per_step": 1, "per_launch_bytes_avg": total_bytes,
                "per_launch_us_avg": round(ms_per_step * 1e3, 2)}
    n_gemv = sum(len(l[2]) for l in layers)
    out = dict(value=value, ms_per_step=ms_per_step, step_bytes=total_bytes, weight_bytes=weight_bytes,
               gemvs=n_gemv, phases=len(phases), roofline=roofline,
               tok_per_s_ceiling=round(1e3 / ms_per_step, 1),
               separate_launches={"launches": len(calls), **sep},
               dependent_chain={"launches": dep_chain.launches, **dep})
    del calls, chain, dep_chain, phases, g, g_tail
    torch.cuda.empty_cache()
    return out


def bench_mlp_block(dev, reps=5):
    """The fp8 MLP block (mlp_forward_fp8): RMSNorm -> up -> relu^2 -> down -> residual.
    Decode (M = 1, weights rotated over copies totalling > 1 GB): the fused block (two
    launches) against separate launches in the reference's order (rmsnorm, up, relu^2, down,
    add; relu^2 as two torch bf16 ops, so six launches where the reference has five).  Prefill
    (M = 2048): three launches."""
    import torch

    from nemotron_infer_amd import ops, synth

    H, I = synth.HIDDEN, synth.INTER
    up = synth.make_weight(I, H, 5000, dev)
    dn = synth.make_weight(H, I, 5001, dev)
    nw = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator(device=dev).manual_seed(5002), device=dev)).float()
    blk_bytes = synth.linear_bytes(1, I, H) + synth.linear_bytes(1, H, I) + 4 * H + 2 * H
    R = max(2, math.ceil(ROTATION_BYTES / (2 * H * I)))
    copies = [(up[0].clone(), up[1].clone(), dn[0].clone(), dn[1].clone()) for _ in range(R)]
    x = synth.make_act(1, H, 5003, dev)
    out = torch.empty_like(x)
    h = torch.empty_like(x)
    yu = torch.empty((1, I), dtype=torch.bfloat16, device=dev)
    act = torch.empty_like(yu)
    yd = torch.empty_like(x)

    def fused(r):
        uw, us, dw, ds = copies[r]
        ops.mlp_forward_fp8(x, nw, uw, us, dw, ds, out=out)

    def unfused(r):
        uw, us, dw, ds = copies[r]
        ops.rmsnorm_bf16(x, nw, out=h)
        ops.linear_fp8_w8a16(h, uw, us, out=yu)
        torch.relu_(yu)
        torch.mul(yu, yu, out=act)
        ops.linear_fp8_w8a16(act, dw, ds, out=yd)
        torch.add(x, yd, out=out)

    T = Timer()
    res = {}
    for name, fn in (("fused_2_launches", fused), ("separate_6_launches", unfused)):
        for r in range(R):
            fn(r)
        torch.cuda.synchronize()
        g = T.capture(lambda: [fn(r) for r in range(R)])
        T.time_replays([g])
        t = T.time_replays([g] * reps) / (reps * R)
        res[name] = {"us": round(t * 1e3, 2), "GB/s": round(blk_bytes / (t * 1e-3) / 1e9, 1)}
        del g
    del copies
    # prefill chunk
    M = synth.PREFILL_M
    xp = synth.make_act(M, H, 5004, dev)
    op = torch.empty_like(xp)
    for _ in range(2):
        ops.mlp_forward_fp8(xp, nw, *up, *dn, out=op)
    torch.cuda.synchronize()
    g = T.capture(lambda: [ops.mlp_forward_fp8(xp, nw, *up, *dn, out=op) for _ in range(reps)])
    steady(T, g)
    t = T.time_replays([g]) / reps
    fl = synth.linear_flops(M, I, H) + synth.linear_flops(M, H, I)
    del g
    return {"workload": "mlp_forward_fp8 block (hidden 3136, inter 12544)",
            "decode_m1": {"bytes": blk_bytes, "weight_copies_rotated": R, **res},
            "prefill_m2048": {"us": round(t * 1e3, 1), "TFLOP/s": round(fl / (t * 1e-3) / 1e12, 1),
                              "launches": 3,
                              "steps": "rmsnorm; up GEMM + relu^2; down GEMM (128 x 256 tiles) + residual"}}


def bench_attn_decode(dev, reps=5):
    """The fp8 attention block at decode (attn_decode_fp8; 40 query heads, 8 KV heads of 128)
    at cache lengths S, weights and caches rotated over copies totalling > 1 GB: the block
    (q|k|v GEMV with the RMSNorm, SDPA split [+ combine], o GEMV + residual) against the
    reference's launch structure on this library's kernels (rmsnorm, q, k, v, SDPA, o, add);
    and the SDPA kernel(s) alone, priced on the K/V bytes they read."""
    import torch

    from nemotron_infer_amd import ops, synth

    H, HQ, HKV, D = synth.HIDDEN, 40, 8, 128
    mats = [synth.make_weight(r, c, 9000 + i, dev)
            for i, (r, c) in enumerate([(HQ * D, H), (HKV * D, H), (HKV * D, H), (H, HQ * D)])]
    nw = (1.0 + 0.1 * torch.randn(H, generator=torch.Generator(device=dev).manual_seed(9010), device=dev)).float()
    wbytes = sum(synth.linear_bytes(1, w.shape[0], w.shape[1]) for w, _ in mats)
    x = synth.make_act(1, H, 9011, dev)
    out = torch.empty_like(x)
    T = Timer()
    res = {}
    for S in (1024, 4096, 32768):
        cap = S + 1
        kv_bytes = 2 * HKV * S * D * 2
        R = max(2, math.ceil(ROTATION_BYTES / (wbytes + 2 * kv_bytes)))
        g = torch.Generator(device=dev).manual_seed(9100 + S)
        caches = [(torch.randn((HKV, cap, D), generator=g, device=dev).to(torch.bfloat16),
                   torch.randn((HKV, cap, D), generator=g, device=dev).to(torch.bfloat16)) for _ in range(R)]
        copies = [[(w.clone(), sc.clone()) for w, sc in mats] for _ in range(R)]
        q = torch.empty((HQ, D), dtype=torch.bfloat16, device=dev)
        kn = torch.empty((HKV, D), dtype=torch.bfloat16, device=dev)
        vn = torch.empty_like(kn)
        o = torch.empty_like(q)
        h = torch.empty_like(x)
        att = torch.empty_like(x)

        def block(r):
            (qw, qs), (kw, ks), (vw, vs), (ow, os_) = copies[r]
            ops.attn_decode_fp8(x, nw, qw, qs, kw, ks, vw, vs, ow, os_, *caches[r], S, out=out)

        def separate(r):
            (qw, qs), (kw, ks), (vw, vs), (ow, os_) = copies[r]
            ops.rmsnorm_bf16(x, nw, out=h)
            ops.linear_fp8_w8a16(h, qw, qs, out=q.view(1, -1))
            ops.linear_fp8_w8a16(h, kw, ks, out=kn.view(1, -1))
            ops.linear_fp8_w8a16(h, vw, vs, out=vn.view(1, -1))
            ops.sdpa_decode_bf16(q, *caches[r], kn, vn, S, out=o)
            ops.linear_fp8_w8a16(o.view(1, -1), ow, os_, out=att)
            torch.add(x, att, out=out)

        def sdpa(r):
            ops.sdpa_decode_bf16(q, *caches[r], kn, vn, S, out=o)

        row = {"kv_bytes": kv_bytes, "weight_copies_rotated": R}
        for name, fn, nbytes in (("block", block, wbytes + kv_bytes), ("separate_7_launches", separate,
                                                                        wbytes + kv_bytes),
                                 ("sdpa_only", sdpa, kv_bytes)):
            for r in range(R):
                fn(r)
            torch.cuda.synchronize()
            gr = T.capture(lambda: [fn(r) for r in range(R)])
            T.time_replays([gr])
            t = T.time_replays([gr] * reps) / (reps * R)
            row[name] = {"us": round(t * 1e3, 2), "GB/s": round(nbytes / (t * 1e-3) / 1e9, 1)}
            del gr
        res[f"S={S}"] = row
        del caches, copies
        torch.cuda.empty_cache()
    return {"workload": "attn_decode_fp8 block (hidden 3136, 40 q heads, 8 KV heads, head 128)",
            "weight_bytes": wbytes, **res}


def bench_attn_prefill(dev, reps=10):
    """Causal attention over a prompt (sdpa_prefill, 40 query heads, 8 KV heads of 128) at
    S = 512 / 2048 / 8192, priced on its causal flops (2 S (S + 1) / 2 x 128 x 2 per head for
    Q.K^T and P.V), and the fp8 attention block attn_forward_fp8 at S = 2048."""
    import torch

    from nemotron_infer_amd import ops, synth

    HQ, HKV, D = 40, 8, 128
    T = Timer()
    res = {}
    for S in (512, 2048, 8192):
        g = torch.Generator(device=dev).manual_seed(9300 + S)
        qkv = torch.randn((S, (HQ + 2 * HKV) * D), generator=g, device=dev).to(torch.bfloat16)
        q, k, v = qkv[:, :HQ * D], qkv[:, HQ * D:(HQ + HKV) * D], qkv[:, (HQ + HKV) * D:]
        o = torch.empty((S, HQ * D), dtype=torch.bfloat16, device=dev)
        ops.sdpa_prefill_bf16(q, k, v, HQ, HKV, out=o)
        torch.cuda.synchronize()
        gr = T.capture(lambda: [ops.sdpa_prefill_bf16(q, k, v, HQ, HKV, out=o) for _ in range(reps)])
        steady(T, gr, 0.2)
        t = T.time_replays([gr]) / reps
        fl = 2 * 2 * (S * (S + 1) // 2) * D * HQ
        res[f"sdpa_S={S}"] = {"us": round(t * 1e3, 1), "TFLOP/s": round(fl / (t * 1e-3) / 1e12, 1)}
        del gr, qkv, o
    S, hid = 2048, synth.HIDDEN
    mats = [synth.make_weight(r, c, 9400 + i, dev)
            for i, (r, c) in enumerate([(HQ * D, hid), (HKV * D, hid), (HKV * D, hid), (hid, HQ * D)])]
    nw = 1.0 + 0.1 * torch.randn(hid, device=dev)
    x = synth.make_act(S, hid, 9410, dev)
    out = torch.empty_like(x)
    kc = torch.empty((HKV, S, D), dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    args = [t for m in mats for t in m]
    ops.attn_forward_fp8(x, nw, *args, k_cache=kc, v_cache=vc, out=out)
    torch.cuda.synchronize()
    gr = T.capture(lambda: [ops.attn_forward_fp8(x, nw, *args, k_cache=kc, v_cache=vc, out=out) for _ in range(reps)])
    steady(T, gr, 0.2)
    t = T.time_replays([gr]) / reps
    fl = sum(synth.linear_flops(S, w.shape[0], w.shape[1]) for w, _ in mats) + 2 * 2 * (S * (S + 1) // 2) * D * HQ
    res["attn_forward_block_S=2048"] = {"us": round(t * 1e3, 1), "TFLOP/s": round(fl / (t * 1e-3) / 1e12, 1),
                                        "launches": 5}
    del gr
    return {"workload": "causal attention prefill (40 q heads, 8 KV heads, head 128) and attn_forward_fp8", **res}


def _mamba_layer(dev, seed):
    """Real-model Mamba-2 layer (hidden 3136, 96 heads of 80, 8 groups, state 128): fp8 in_proj
    [17504, 3136] and out_proj [3136, 7680], float32 parameters and states."""
    import torch

    from nemotron_infer_amd import synth

    H, P, G, N, hid = 96, 80, 8, 128, synth.HIDDEN
    inter, conv_dim = H * P, H * P + 2 * G * N
    g = torch.Generator(device=dev).manual_seed(seed)
    f = dict(device=dev, dtype=torch.float32)
    return dict(norm=1.0 + 0.1 * torch.randn(hid, generator=g, **f),
                inp=synth.make_weight(inter + conv_dim + H, hid, seed + 1, dev),
                out=synth.make_weight(hid, inter, seed + 2, dev),
                conv_w=0.3 * torch.randn((conv_dim, 4), generator=g, **f),
                conv_b=0.1 * torch.randn(conv_dim, generator=g, **f),
                A_log=torch.rand(H, generator=g, **f) * 2.5 - 1.0,
                D=torch.randn(H, generator=g, **f),
                dt_bias=0.5 * torch.randn(H, generator=g, **f),
                gnorm_w=1.0 + 0.1 * torch.randn(inter, generator=g, **f),
                conv_state=torch.zeros((1, conv_dim, 3), **f),
                ssm_state=torch.zeros((1, H, P, N), **f))


def _mamba_args(L):
    return (L["norm"], *L["inp"], L["conv_w"], L["conv_b"], L["A_log"], L["D"], L["dt_bias"], L["gnorm_w"],
            *L["out"], L["conv_state"], L["ssm_state"])


def bench_mamba_prefill(dev, reps=5):
    """The fp8 Mamba-2 block over a prompt (mamba_forward_fp8) at S = 2048 with its final states:
    block time and TFLOP/s of its two linears, and the conv + scan kernels' share (kernel trace)."""
    import torch

    from nemotron_infer_amd import ops, synth

    H, P, G = 96, 80, 8
    L = _mamba_layer(dev, 9600)
    res = {}
    for S in (512, 2048):
        x = synth.make_act(S, synth.HIDDEN, 9601, dev)
        out = torch.empty_like(x)
        args = (L["norm"], *L["inp"], L["conv_w"], L["conv_b"], L["A_log"], L["D"], L["dt_bias"], L["gnorm_w"],
                *L["out"])

        def run():
            ops.mamba_forward_fp8(x, *args, H, P, G, conv_state_out=L["conv_state"], ssm_state_out=L["ssm_state"],
                                  out=out)

        run()
        torch.cuda.synchronize()
        T = Timer()
        g = T.capture(lambda: [run() for _ in range(reps)])
        steady(T, g, 0.2)
        t = T.time_replays([g]) / reps
        fl = sum(synth.linear_flops(S, w.shape[0], w.shape[1]) for w, _ in (L["inp"], L["out"]))
        res[f"S={S}"] = {"us": round(t * 1e3, 1), "linear_TFLOP/s_equiv": round(fl / (t * 1e-3) / 1e12, 1),
                         "launches": 6}
        del g
    return {"workload": "mamba_forward_fp8 block (hidden 3136, 96 heads x 80, 8 groups, state 128)", **res}


def bench_mamba_decode(dev, reps=5):
    """The fp8 Mamba-2 block at decode (mamba_decode_fp8), layers rotated over copies totalling
    > 1 GB: the block (4 launches) against the reference's launch structure on this library's
    kernels (rmsnorm, in_proj, mixer, out_proj, add: 6 launches; the reference has 12, counting
    its three in_proj slices and three split copies)."""
    import torch

    from nemotron_infer_amd import ops, synth

    H, P, G = 96, 80, 8
    L0 = _mamba_layer(dev, 9500)
    wbytes = sum(synth.linear_bytes(1, w.shape[0], w.shape[1]) for w, _ in (L0["inp"], L0["out"]))
    state_bytes = 2 * (L0["ssm_state"].numel() * 4 + L0["conv_state"].numel() * 4)
    R = max(2, math.ceil(ROTATION_BYTES / wbytes))
    layers = [L0] + [{k: (tuple(t.clone() for t in v) if isinstance(v, tuple) else v.clone()) for k, v in L0.items()}
                     for _ in range(R - 1)]
    x = synth.make_act(1, synth.HIDDEN, 9501, dev)
    out = torch.empty_like(x)
    h = torch.empty_like(x)
    proj = torch.empty((1, L0["inp"][0].shape[0]), dtype=torch.bfloat16, device=dev)
    mix = torch.empty_like(x)

    def blk(r):
        ops.mamba_decode_fp8(x, *_mamba_args(layers[r]), H, P, G, out=out)

    def separate(r):
        Lr = layers[r]
        ops.rmsnorm_bf16(x, Lr["norm"], out=h)
        ops.linear_fp8_w8a16(h, *Lr["inp"], out=proj)
        _, g = ops.mamba_mixer_decode(proj, Lr["conv_w"], Lr["conv_b"], Lr["A_log"], Lr["D"], Lr["dt_bias"],
                                      Lr["gnorm_w"], Lr["conv_state"], Lr["ssm_state"], H, P, G)
        ops.linear_fp8_w8a16(g, *Lr["out"], out=mix)
        torch.add(x, mix, out=out)

    T = Timer()
    res = {"weight_bytes": wbytes, "state_bytes_read_written": state_bytes, "weight_copies_rotated": R}
    for name, fn in (("block_4_launches", blk), ("separate_6_launches", separate)):
        for r in range(R):
            fn(r)
        torch.cuda.synchronize()
        g = T.capture(lambda: [fn(r) for r in range(R)])
        T.time_replays([g])
        t = T.time_replays([g] * reps) / (reps * R)
        res[name] = {"us": round(t * 1e3, 2), "GB/s": round((wbytes + state_bytes) / (t * 1e-3) / 1e9, 1)}
        del g
    return {"workload": "mamba_decode_fp8 block (hidden 3136, 96 heads x 80, 8 groups, state 128)", **res}


def bench_engine_decode(dev, s_cache=1024, reps=5):
    """A whole decode step of the 42-layer stack through the three block entries, in the
    engine's order (engine.py:252-265; config 4's layer pattern at the real model's Mamba
    dimensions): 21 mamba_decode_fp8, 17 mlp_forward_fp8, 4 attn_decode_fp8 at S_cache
    positions, each reading the previous layer's output.  One HIP graph per step."""
    import torch

    from nemotron_infer_amd import ops, synth

    H, P, G, hid = 96, 80, 8, synth.HIDDEN
    HQ, HKV, D = 40, 8, 128
    kinds = [k for _, k, _ in synth.decode_stream_layers()]
    layers = []
    wbytes = 0
    for i, kind in enumerate(kinds):
        if kind == "mamba":
            L = _mamba_layer(dev, 20000 + 10 * i)
            wbytes += sum(synth.linear_bytes(1, w.shape[0], w.shape[1]) for w, _ in (L["inp"], L["out"]))
        elif kind == "mlp":
            L = dict(norm=1.0 + 0.1 * torch.randn(hid, device=dev),
                     up=synth.make_weight(synth.INTER, hid, 20000 + 10 * i, dev),
                     down=synth.make_weight(hid, synth.INTER, 20001 + 10 * i, dev))
            wbytes += synth.linear_bytes(1, synth.INTER, hid) + synth.linear_bytes(1, hid, synth.INTER)
        else:
            mats = [synth.make_weight(r, c, 20000 + 10 * i + j, dev)
                    for j, (r, c) in enumerate([(HQ * D, hid), (HKV * D, hid), (HKV * D, hid), (hid, HQ * D)])]
            g = torch.Generator(device=dev).manual_seed(20005 + 10 * i)
            L = dict(norm=1.0 + 0.1 * torch.randn(hid, device=dev), mats=mats,
                     kc=torch.randn((HKV, s_cache + 1, D), generator=g, device=dev).to(torch.bfloat16),
                     vc=torch.randn((HKV, s_cache + 1, D), generator=g, device=dev).to(torch.bfloat16))
            wbytes += sum(synth.linear_bytes(1, w.shape[0], w.shape[1]) for w, _ in mats)
        layers.append((kind, L))
    bufs = [synth.make_act(1, hid, 20999, dev), torch.empty((1, hid), dtype=torch.bfloat16, device=dev)]

    def step():
        cur, nxt = bufs
        for kind, L in layers:
            if kind == "mamba":
                ops.mamba_decode_fp8(cur, *_mamba_args(L), H, P, G, out=nxt)
            elif kind == "mlp":
                ops.mlp_forward_fp8(cur, L["norm"], *L["up"], *L["down"], out=nxt)
            else:
                (qw, qs), (kw, ks), (vw, vs), (ow, os_) = L["mats"]
                ops.attn_decode_fp8(cur, L["norm"], qw, qs, kw, ks, vw, vs, ow, os_, L["kc"], L["vc"], s_cache, out=nxt)
            cur, nxt = nxt, cur

    step()
    torch.cuda.synchronize()
    T = Timer()
    g = T.capture(step)
    T.time_replays([g])
    t = T.time_replays([g] * reps) / reps
    del g, layers
    torch.cuda.empty_cache()
    return {"workload": "42-layer decode step through the block entries (21 Mamba, 17 MLP, 4 attention; "
                        f"S_cache {s_cache})", "launches": 21 * 4 + 17 * 2 + 4 * 4, "weight_bytes": wbytes,
            "us_per_token": round(t * 1e3, 1), "tok_per_s": round(1e3 / t, 1),
            "weight_GB/s": round(wbytes / (t * 1e-3) / 1e9, 1)}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(host, seconds):
    """The reference's CPU path (tools/ref_full_model.py:44-49,137, restated in
    oracle/linear.py): per call, fp32 dequant of W, F.linear in fp32, bf16 rounding -- with
    torch's intra-op threads on this host.  Timed on a bounded sample of config 4 (one Mamba, one
    MLP and one attention layer: 14 % of its bytes; ``value``, GB/s), plus the matmul-only time
    of the same sample (W dequantized once, outside the timed region), config 1's six matrices,
    and one config-3 prefill GEMM (up_proj at M = 2048)."""
    import numpy as np
    import torch

    from nemotron_infer_amd import synth
    from oracle import linear as olin

    threads = torch.get_num_threads()
    budget = seconds / 4.0

    def loop(fn, budget_s, min_iters=2):
        fn()                                       # warm-up
        t0 = time.perf_counter()
        n = 0
        while True:
            fn()
            n += 1
            if time.perf_counter() - t0 >= budget_s and n >= min_iters:
                break
        return (time.perf_counter() - t0) / n

    # config 4 sample: one layer of each kind, on the CPU, same generator as the GPU stream
    sample = []
    for li, kind, lins in synth.decode_stream_layers():
        if (kind, li) in (("mamba", 0), ("mlp", 1), ("attn", 41)):
            for j, lin in enumerate(lins):
                w, s = synth.make_weight(lin.N, lin.K, 40000 + 10 * li + j, "cpu")
                x = synth.make_act(1, lin.K, 41000 + lin.K, "cpu", kind=lin.act)
                sample.append((x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy(), lin))
    sbytes = sum(synth.linear_bytes(1, l.N, l.K) for *_, l in sample)
    t_ref = loop(lambda: [olin.linear_fp8_w8a16(x, w, s) for x, w, s, _ in sample], budget)
    deq = [(torch.from_numpy(olin.bf16_to_f32(x)).view(1, -1),
            torch.from_numpy(olin.dequant_f32(w, s))) for x, w, s, _ in sample]
    t_mm = loop(lambda: [torch.nn.functional.linear(x, w) for x, w in deq], budget)
    del deq
    # config 1: the six matrices, per call dequant
    c1 = [(x.view(torch.int16).numpy().view(np.uint16), w.numpy(), s.numpy()) for _, x, w, s in host]
    c1_bytes = sum(synth.linear_bytes(1, l.N, l.K) for l, *_ in host)
    t_c1 = loop(lambda: [olin.linear_fp8_w8a16(x, w, s) for x, w, s in c1], budget)
    # config 3: one prefill GEMM (up_proj, M = 2048), per call dequant and matmul only
    lin = synth.PREFILL_SET[0]
    M = synth.PREFILL_M
    w3, s3 = synth.make_weight(lin.N, lin.K, 3000, "cpu")
    x3 = synth.make_act(M, lin.K, 3100, "cpu", outlier_frac=0.001).float()
    w3t = w3.view(torch.float8_e4m3fn)
    w3d = w3t.float() * s3[:, None]
    t_c3_mm = loop(lambda: torch.nn.functional.linear(x3, w3d), budget / 2, min_iters=1)
    t_c3 = loop(lambda: torch.nn.functional.linear(x3, w3t.float() * s3[:, None]), budget / 2, min_iters=1)
    fl3 = synth.linear_flops(M, lin.N, lin.K)
    where = f"{threads} threads of os.cpu_count()={os.cpu_count()} ({_cpu_model()})"
    return {"value": round(sbytes / t_ref / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 4 layers 0 (Mamba), 1 (MLP), 41 (attention): 8 GEMVs, {sbytes} B per pass, "
                      f"{t_ref * 1e3:.1f} ms per pass: torch CPU per-call fp32 dequant + F.linear + bf16 round "
                      f"(oracle/linear.py), {where}",
            "matmul_only": {"value": round(sbytes / t_mm / 1e9, 3), "unit": "GB/s",
                            "ms_per_pass": round(t_mm * 1e3, 2),
                            "note": "same sample, W dequantized once outside the timed region, F.linear fp32"},
            "config1": {"value": round(c1_bytes / t_c1 / 1e9, 3), "unit": "GB/s", "ms_per_step": round(t_c1 * 1e3, 1)},
            "config3_prefill_up_proj": {"M": M, "N": lin.N, "K": lin.K,
                                        "per_call_dequant": {"ms": round(t_c3 * 1e3, 1),
                                                             "TFLOP/s": round(fl3 / t_c3 / 1e12, 3)},
                                        "matmul_only": {"ms": round(t_c3_mm * 1e3, 1),
                                                        "TFLOP/s": round(fl3 / t_c3_mm / 1e12, 3)}}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the fp8 linear "
              f"path is single-GPU here; how it would shard is a design note, not code", file=sys.stderr)
        sys.exit(2)
    import torch

    from nemotron_infer_amd import synth

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    t0 = time.time()
    if args.pmc_calibration:
        a = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
    if args.only:
        if args.only == "skinny":
            leg = bench_skinny(dev)
        elif args.only == "stream":
            leg = bench_decode_stream(args, dev)
            leg = {k: v for k, v in leg.items()}
        elif args.only == "decode":
            leg = bench_decode_set(args, dev, decode_inputs())
        elif args.only == "attn":
            leg = bench_attn_decode(dev)
        elif args.only == "mamba":
            leg = bench_mamba_decode(dev)
        elif args.only == "prefill_attn":
            leg = bench_attn_prefill(dev)
        elif args.only == "prefill_mamba":
            leg = bench_mamba_prefill(dev)
        elif args.only == "prefill_small":
            leg = bench_prefill_small_m(dev)
        elif args.only == "engine":
            leg = bench_engine_decode(dev)
        else:
            leg = bench_prefill(dev) if args.only == "prefill" else bench_mlp_block(dev)
        print(json.dumps(leg), flush=True)
        return
    log("decode stream (config 4, headline) ...")
    d = bench_decode_stream(args, dev)
    log(f"decode stream: {d['value']:.1f} GB/s, {d['ms_per_step'] * 1e3:.1f} us/step")
    host = decode_inputs()
    extras = {}
    if not args.no_extras:
        log("decode set (config 1) ...")
        extras["decode_set"] = bench_decode_set(args, dev, host)
        log(f"decode set: {extras['decode_set']['chain_one_launch']}")
        log("prefill GEMM (config 3) ...")
        extras["prefill_gemm"] = bench_prefill(dev)
        log(f"prefill: {extras['prefill_gemm']['tflops']} TFLOP/s")
        extras["prefill_small_m"] = bench_prefill_small_m(dev)
        log(f"prefill small M: { {k: v['TFLOP/s'] for k, v in extras['prefill_small_m']['results'].items()} }")
        log("skinny M (config 2) ...")
        extras["skinny"] = bench_skinny(dev)
        log("mlp block ...")
        extras["mlp_block"] = bench_mlp_block(dev)
        log(f"mlp block: {extras['mlp_block']['decode_m1']}")
        log("attention decode block ...")
        extras["attn_decode"] = bench_attn_decode(dev)
        log(f"attention decode: {extras['attn_decode']['S=4096']}")
        log("attention prefill ...")
        extras["attn_prefill"] = bench_attn_prefill(dev)
        log(f"attention prefill: {extras['attn_prefill']['sdpa_S=2048']}")
        log("mamba prefill block ...")
        extras["mamba_prefill"] = bench_mamba_prefill(dev)
        log(f"mamba prefill: {extras['mamba_prefill']['S=2048']}")
        log("mamba decode block ...")
        extras["mamba_decode"] = bench_mamba_decode(dev)
        log(f"mamba decode: {extras['mamba_decode']['block_4_launches']}")
        log("42-layer decode step through the blocks ...")
        extras["engine_decode_step"] = bench_engine_decode(dev)
        log(f"engine decode step: {extras['engine_decode_step']['us_per_token']} us")
    torch.cuda.empty_cache()
    log("cpu baseline ...")
    cpu = cpu_baseline(host, args.cpu_seconds)
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
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights -> e4m3 per-tensor scale; bf16 N(0,1) / relu^2 activations)",
        "config": {"workload": "config4_42layer_decode_stream",
                   "layers": {"attention": 4, "mlp": 17, "mamba": 21}, "gemvs": d["gemvs"],
                   "phases_per_launch": d["phases"], "M": 1, "bytes_per_step": d["step_bytes"],
                   "weight_bytes": d["weight_bytes"],
                   "operands": "W e4m3 [N,K] (converted exactly to bf16) + f32 per-row scale, x bf16, "
                               "f32 accumulation, y bf16",
                   "launch": "HIP graph; per step one GEMV chain launch of 84 phases (q|k|v grouped, o; up, "
                             "down; in_proj, out_proj per layer), each on its own activation"},
        "roofline": d["roofline"],
        "cpu_baseline": cpu,
        "tok_per_s_ceiling": d["tok_per_s_ceiling"],
        "separate_launches": d["separate_launches"],
        "dependent_chain": d["dependent_chain"],
        **extras,
        "wall_s": round(time.time() - t0, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
