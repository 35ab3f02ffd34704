#!/usr/bin/env python3
"""Benchmark of the gfx950 GEMM hot path (one MI355X).

Headline (BASELINE.json metric): bf16 GEMM TFLOPS at 4096^3 (config 2: NN layout,
N(0,1) inputs, fp32 accumulate, bf16 output) as a fraction of the dense bf16
MFMA peak, plus the W4A16 decode GEMM (config 4: M=16, K=4096, N=11008, int4
weights, group 128, zero point 8, bf16 out) in HBM GB/s against the HBM peak.

A "step" is one launch of the GEMM over the 4096^3 problem with inputs already
resident in HBM.  Kernel time is measured with HIP events on the stream the
kernels are launched on (the t0mi runtime launches on torch's current stream).
The W4A16 timing rotates over >= 512 MB of distinct weight copies so the
256 MB Infinity Cache cannot serve repeats.

The default run also times, as extra keys of the same JSON line, config 3
("skinny"), config 5 ("prefill": the default route, and "prefill_fused": the
dequant inside the MFMA K loop) and the 16 x 4096 x 1376 W4A16 decode shard
("shard"), each with its own roofline object and CPU baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only LEG] [--no-cpu]
       [--config PRESET] [--split-k S] [--stages S] [--tune] [--clocks] [--rows R]
LEG: all (default) | gemm | w4a16 | skinny | prefill | shard (one leg alone) |
     copy (FETCH/WRITE_SIZE calibration) | dispatch | persistent | split
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "rust-gpu_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E (published)
METRIC = "bf16 GEMM TFLOPS @4096³ (% MFMA peak); W4A16 decode HBM GB/s (% peak)"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", choices=["all", "gemm", "w4a16", "skinny", "prefill", "shard", "copy", "dispatch",
                                      "persistent", "split"],
                   default="all",
                   help="'copy' runs only a plain 1 GiB fp32 copy kernel (torch): the calibration for "
                        "rocprofv3 FETCH_SIZE/WRITE_SIZE readings; 'dispatch' times batched submission (a "
                        "batch of small GEMM dispatches: synchronous, DispatchQueue, HIP graph); 'gemm', "
                        "'w4a16', 'skinny', 'prefill' and 'shard' time one leg of the default run alone "
                        "(BASELINE configs 2, 4, 3, 5 and the 1376-column W4A16 decode shard); 'persistent' "
                        "times the persistent decode preset beside the one-shot auto_select configuration; "
                        "'split' times the dequant-once W4A16 route with its planned column split against "
                        "one launch of the head config")
    p.add_argument("--clocks", action="store_true",
                   help="with --only gemm / w4a16: sample the GPU clock and power (amd-smi) during ~3 s of "
                        "sustained launches and report their medians")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--config", default=None, help="GEMM preset name to force (default: auto_select)")
    p.add_argument("--split-k", type=int, default=0, help="with --config: the split-K factor to force")
    p.add_argument("--stages", type=int, default=0, help="with --config: the LDS stage count to force")
    p.add_argument("--rows", type=int, default=16,
                   help="with --only w4a16: activation rows of the decode GEMM (default 16, BASELINE config 4)")
    p.add_argument("--tune", action="store_true",
                   help="with --only gemm/skinny: also run GemmTuner on the shape (fresh cache) and report "
                        "its measured pick beside auto_select's")
    return p.parse_args()


def load_traffic(kernel_key):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary (FETCH_SIZE /
    WRITE_SIZE, scaled by a copy-kernel calibration), or None if not measured."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(kernel_key)
    except (OSError, ValueError):
        return None


def warm_up(torch, launch, n: int, min_s: float = 0.3):
    """n untimed launches, then more until min_s seconds of back-to-back work have run:
    the clock and power state settle within a few hundred milliseconds of sustained load,
    and the timed region should see that steady state, not the first milliseconds."""
    for _ in range(n):
        launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < min_s:
        for _ in range(20):
            launch()
        torch.cuda.synchronize()


def bench_gemm(args, torch, t0mi, rt):
    M = N = K = 4096
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7402)
    a = torch.randn(M, K, device="cuda:0", generator=g).to(torch.bfloat16)
    b = torch.randn(K, N, device="cuda:0", generator=g).to(torch.bfloat16)
    y = torch.empty(M, N, device="cuda:0", dtype=torch.bfloat16)
    if args.config:
        cfg = t0mi.preset(args.config)
    else:
        cfg = t0mi.auto_select_layout(M, K, N, t0mi.NN, t0mi.OUT_BF16)
    cfg = cfg.copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16)
    args.tuned = run_tuner(t0mi, rt, M, N, K, t0mi.NN, t0mi.OUT_BF16) if args.tune else None
    pa, pb, py = a.data_ptr(), b.data_ptr(), y.data_ptr()
    warm_up(torch, lambda: rt.gemm(cfg, pa, pb, py, M, N, K), args.warmup)
    t_host0 = time.perf_counter()
    us, batches = timed_batches(torch, lambda i: rt.gemm(cfg, pa, pb, py, M, N, K), args.steps)
    t_host = time.perf_counter() - t_host0
    ms = us * 1e-3
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    print(f"[bench] gemm {cfg.name()} 4096^3 NN bf16-out: {us:.1f} us/launch (median of {len(batches)} batches "
          f"of {args.steps}: {', '.join(f'{b:.1f}' for b in batches)}), {tflops:.1f} TFLOPS "
          f"({100*tflops/PEAK_BF16_TFLOPS:.1f}% of peak); host wall {t_host:.3f}s", file=sys.stderr, flush=True)
    args.gemm_clocks = smi_sample(3.0, lambda: rt.gemm(cfg, pa, pb, py, M, N, K), torch) if args.clocks else None
    return cfg, ms, tflops, batches


def run_tuner(t0mi, rt, m, n, k, transpose, out_dtype):
    """GemmTuner::tune on a fresh cache: the measured pick among the cost model's top
    candidates, and the tuner's own report of every candidate it timed."""
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        tuner = t0mi.GemmTuner(cache_dir=d, max_candidates=8, n_iters=10)
        cfg, tflops, _ = tuner.tune(rt, m, n, k, transpose, out_dtype)
        report = tuner.report()
        del tuner
    print(f"[bench] tuner {m}x{n}x{k}: {cfg.name()} {tflops:.1f} TFLOPS\n{report}", file=sys.stderr, flush=True)
    return {"config": cfg.name(), "tflops": round(tflops, 2)}


BATCHES = 5


def time_calls(torch, launch, calls, start=0):
    """Microseconds per launch over `calls` back-to-back launches, from HIP events recorded
    on torch's current stream (the stream the t0mi runtime launches on)."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(calls):
        launch(start + i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / calls


def timed_batches(torch, launch, calls, batches=BATCHES):
    """The median over `batches` event-timed batches of `calls` launches each (launch(i) gets a
    running index, so rotations continue across batches), and every batch's value."""
    vals = [time_calls(torch, launch, calls, start=b * calls) for b in range(batches)]
    return sorted(vals)[len(vals) // 2], vals


def bench_skinny(args, torch, t0mi, rt):
    """Config 3: 128 x 4096 x 4096 NN, N(0, 0.02) bf16, bf16 out.  HBM-bound; B (32 MB) is
    rotated over >= 512 MB of copies so the Infinity Cache cannot serve repeats.  One call
    is the GEMM plus, when the chosen config splits K, its reduce."""
    M, N, K = 128, 4096, 4096
    copies = 16
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7503)
    a = (torch.randn(M, K, device="cuda:0", generator=g) * 0.02).to(torch.bfloat16)
    bs = [(torch.randn(K, N, device="cuda:0", generator=g) * 0.02).to(torch.bfloat16) for _ in range(copies)]
    y = torch.empty(M, N, device="cuda:0", dtype=torch.bfloat16)
    cfg = t0mi.preset(args.config) if args.config else t0mi.auto_select_layout(M, K, N, t0mi.NN, t0mi.OUT_BF16)
    cfg = cfg.copy(transpose=t0mi.NN, out_dtype=t0mi.OUT_BF16)
    if args.config and args.split_k:
        cfg = cfg.copy(split_k=args.split_k)
    if args.config and args.stages:
        cfg = cfg.copy(stages=args.stages)
    tuned = run_tuner(t0mi, rt, M, N, K, t0mi.NN, t0mi.OUT_BF16) if args.tune else None
    pa, py = a.data_ptr(), y.data_ptr()

    def launch(i):
        rt.gemm(cfg, pa, bs[i % copies].data_ptr(), py, M, N, K)
    rot = [0]

    def launch_rot():
        launch(rot[0])
        rot[0] += 1
    warm_up(torch, launch_rot, max(args.warmup, copies))
    us, batches = timed_batches(torch, launch, max(args.steps * 4, 2 * copies))
    alg_bytes = 2 * M * K + 2 * K * N + 2 * M * N
    gbs = alg_bytes / (us * 1e-6) / 1e9
    print(f"[bench] skinny {cfg.name()} 128x4096x4096 NN bf16-out: {us:.2f} us/call (median of "
          f"{', '.join(f'{b:.2f}' for b in batches)}), {gbs:.0f} GB/s "
          f"({100*gbs/PEAK_HBM_GBS:.1f}% of HBM peak)", file=sys.stderr, flush=True)
    return cfg, us, gbs, alg_bytes, tuned


def bench_prefill(args, torch, t0mi, rt):
    """Config 5: A[4096,4096] bf16 x int4 W[4096,14336], group 128, per-group int4 zero
    points, bf16 scales, bf16 out, through t0mi_w4a16_gemm (whichever route it takes for
    4096 rows).  MFMA-bound."""
    M, K, N, G = 4096, 4096, 14336, 128
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7505)
    a = torch.randn(M, K, device="cuda:0", generator=g).to(torch.bfloat16)
    w = torch.randint(-2**31, 2**31 - 1, (K // 8, N), device="cuda:0", dtype=torch.int32, generator=g)
    s = (torch.rand(K // G, N, device="cuda:0", generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    z = torch.randint(-2**31, 2**31 - 1, (K // G, N // 8), device="cuda:0", dtype=torch.int32, generator=g)
    y = torch.empty(M, N, device="cuda:0", dtype=torch.bfloat16)
    args_ = (a.data_ptr(), w.data_ptr(), s.data_ptr(), z.data_ptr(), 0, y.data_ptr(), M, K, N, G, t0mi.OUT_BF16)

    def launch(i=0):
        rt.w4a16_gemm(*args_)
    res = {}
    # The default route, then the fused route a caller gets with a zero workspace limit
    # (dequant inside the K loop, no bf16 weight buffer).
    for route, limit in (("default", 2**64 - 1), ("fused", 0)):
        rt.set_w4a16_workspace_limit(limit)
        warm_up(torch, launch, args.warmup)
        us, batches = timed_batches(torch, launch, args.steps)
        tflops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        res[route] = (us, tflops)
        print(f"[bench] prefill w4a16 4096x4096x14336 g128 zeros, {route} route: {us:.1f} us/call (median of "
              f"{', '.join(f'{b:.1f}' for b in batches)}), {tflops:.1f} TFLOPS "
              f"({100*tflops/PEAK_BF16_TFLOPS:.1f}% of peak)", file=sys.stderr, flush=True)
    rt.set_w4a16_workspace_limit(2**64 - 1)
    return res["default"][0], res["default"][1], res["fused"]


SHARD_N = 1376  # config 4's N = 11008 over 8 GPUs, column-parallel


def bench_shard(args, torch, t0mi, rt):
    """The one-GPU stand-in for config 4's column-parallel shard over 8 GPUs: the W4A16 decode
    GEMM 16 x 4096 x 1376 (22 strips of 64 columns; the K range split over 8 workgroups per
    strip inside the launch), weights rotated over >= 512 MB of copies, direct launches and a
    HIP-graph replay of the same calls."""
    Mw, Kw, Nw, G = 16, 4096, SHARD_N, 128
    wbytes, sbytes = Kw // 8 * Nw * 4, Kw // G * Nw * 2
    copies = max(2, -(-512 * 1024 * 1024 // (wbytes + sbytes)))
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7506)
    a = torch.randn(Mw, Kw, device="cuda:0", generator=g).to(torch.bfloat16)
    ws = torch.randint(-2**31, 2**31 - 1, (copies, Kw // 8, Nw), device="cuda:0", dtype=torch.int32, generator=g)
    ss = (torch.rand(copies, Kw // G, Nw, device="cuda:0", generator=g) * 0.015 + 0.005).to(torch.bfloat16)
    y = torch.empty(Mw, Nw, device="cuda:0", dtype=torch.bfloat16)
    pa, py = a.data_ptr(), y.data_ptr()
    wp = [(ws[i].data_ptr(), ss[i].data_ptr()) for i in range(copies)]

    def launch_i(i):
        pw, ps = wp[i % copies]
        rt.w4a16_gemm(pa, pw, ps, 0, 8, py, Mw, Kw, Nw, G, t0mi.OUT_BF16)
    warm_up(torch, lambda: launch_i(0), max(args.warmup, copies))
    us, batches = timed_batches(torch, launch_i, max(args.steps * 4, 2 * copies))
    gus = graph_replay_us(torch, t0mi, lambda r, i: r.w4a16_gemm(pa, wp[i % copies][0], wp[i % copies][1], 0, 8, py,
                                                                 Mw, Kw, Nw, G, t0mi.OUT_BF16), 4 * copies)
    alg_bytes = 2 * Mw * Kw + Kw * Nw // 2 + 2 * (Kw // G) * Nw + 2 * Mw * Nw
    gbs = alg_bytes / (us * 1e-6) / 1e9
    print(f"[bench] shard w4a16 decode 16x4096x{Nw} g128: {us:.2f} us/call (median of "
          f"{', '.join(f'{b:.2f}' for b in batches)}), {gbs:.0f} GB/s; graph replay {gus} us", file=sys.stderr,
          flush=True)
    return {"us_per_call": round(us, 3), "value": round(gbs, 1), "unit": "GB/s", "batch_us": [round(b, 3) for b in batches],
            "graph_replay_us_per_call": gus, "algorithmic_bytes": alg_bytes, "weight_copies_rotated": copies,
            "workload": f"W4A16 decode A[16,4096] bf16 x int4 W[4096,{Nw}] g128 zp=8, bf16 out: config 4's "
                        f"column-parallel shard over 8 GPUs, run on one",
            "roofline": roofline("hbm", gbs, load_traffic("w4a16_shard"))}


def bench_w4a16(args, torch, t0mi, rt):
    Mw, Kw, Nw, G = args.rows, 4096, 11008, 128
    wbytes = Kw // 8 * Nw * 4
    sbytes = Kw // G * Nw * 2
    copies = max(2, -(-512 * 1024 * 1024 // (wbytes + sbytes)))
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7502)
    a = torch.randn(Mw, Kw, device="cuda:0", generator=g).to(torch.bfloat16)
    ws = [torch.randint(-2**31, 2**31 - 1, (Kw // 8, Nw), device="cuda:0", dtype=torch.int32, generator=g)
          for _ in range(copies)]
    ss = [(torch.rand(Kw // G, Nw, device="cuda:0", generator=g) * 0.015 + 0.005).to(torch.bfloat16)
          for _ in range(copies)]
    y = torch.empty(Mw, Nw, device="cuda:0", dtype=torch.bfloat16)
    calls = max(args.steps * 4, 2 * copies)
    rot = [0]

    def launch():
        j = rot[0] % copies
        rot[0] += 1
        rt.w4a16_gemm(a.data_ptr(), ws[j].data_ptr(), ss[j].data_ptr(), 0, 8, y.data_ptr(), Mw, Kw, Nw, G,
                      t0mi.OUT_BF16)
    warm_up(torch, launch, max(args.warmup, copies))
    pa, py = a.data_ptr(), y.data_ptr()
    wp = [(w.data_ptr(), s.data_ptr()) for w, s in zip(ws, ss)]

    def launch_i(i):
        pw, ps = wp[i % copies]
        rt.w4a16_gemm(pa, pw, ps, 0, 8, py, Mw, Kw, Nw, G, t0mi.OUT_BF16)
    us, batches = timed_batches(torch, launch_i, calls)
    args.w4_graph_us = w4a16_graph_us(torch, t0mi, pa, wp, py, Mw, Kw, Nw, G, copies)
    args.w4_clocks = smi_sample(3.0, launch, torch) if args.clocks else None
    alg_bytes = 2 * Mw * Kw + Kw * Nw // 2 + 2 * (Kw // G) * Nw + 2 * Mw * Nw
    gbs = alg_bytes / (us * 1e-6) / 1e9
    print(f"[bench] w4a16 decode {Mw}x4096x11008 g128: {us:.2f} us/call (median of {len(batches)} batches of "
          f"{calls}: {', '.join(f'{b:.2f}' for b in batches)}), {gbs:.0f} GB/s "
          f"({100*gbs/PEAK_HBM_GBS:.1f}% of HBM peak), {copies} weight copies rotated", file=sys.stderr, flush=True)
    return us, gbs, alg_bytes, copies, batches


def w4a16_graph_us(torch, t0mi, pa, wp, py, Mw, Kw, Nw, G, copies):
    """Per-call time of the same decode calls replayed from a HIP graph (captured with the
    runtime's capture API on its own stream): the kernels back to back without the host's
    enqueue cost (~4 us per call from Python), which bounds what direct launches can show
    once a call's kernel time falls below it.  Median of the replays' per-call times."""
    rt2 = t0mi.Runtime(device=0)
    try:
        ext = torch.cuda.ExternalStream(rt2.stream)
        torch.cuda.synchronize()
        for pw, ps in wp:  # grow the runtime's buffers before capturing
            rt2.w4a16_gemm(pa, pw, ps, 0, 8, py, Mw, Kw, Nw, G, t0mi.OUT_BF16)
        t0mi.check(rt2.wait_idle())
        n = 4 * copies
        rt2.capture_begin()
        for i in range(n):
            pw, ps = wp[i % copies]
            rt2.w4a16_gemm(pa, pw, ps, 0, 8, py, Mw, Kw, Nw, G, t0mi.OUT_BF16)
        graph = rt2.capture_end()
        vals = []
        for rep in range(3 + BATCHES):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(ext)
            graph.launch()
            e1.record(ext)
            t0mi.check(rt2.wait_idle())
            e1.synchronize()
            if rep >= 3:
                vals.append(e0.elapsed_time(e1) * 1e3 / n)
        graph.destroy()
        vals.sort()
        return round(vals[len(vals) // 2], 3)
    finally:
        rt2.close()


def graph_replay_us(torch, t0mi, call, n):
    """Per-call time of n calls call(rt, i) captured into a HIP graph on a fresh runtime's
    stream and replayed (no host enqueue cost); call(rt, 0) runs once first so the runtime's
    buffers exist before the capture.  Median over BATCHES replays."""
    rt2 = t0mi.Runtime(device=0)
    try:
        ext = torch.cuda.ExternalStream(rt2.stream)
        torch.cuda.synchronize()
        call(rt2, 0)
        t0mi.check(rt2.wait_idle())
        rt2.capture_begin()
        for i in range(n):
            call(rt2, i)
        graph = rt2.capture_end()
        vals = []
        for rep in range(3 + BATCHES):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(ext)
            graph.launch()
            e1.record(ext)
            t0mi.check(rt2.wait_idle())
            e1.synchronize()
            if rep >= 3:
                vals.append(e0.elapsed_time(e1) * 1e3 / n)
        graph.destroy()
        vals.sort()
        return round(vals[len(vals) // 2], 3)
    finally:
        rt2.close()


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo) and its logical CPU count."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs visible)"


def cpu_baseline(which, budget_s: float = 10.0):
    """The oracle (C restatement of cpu_gemm_nt_bf16 -- one fp32 accumulator per output, k
    ascending -- with OpenMP over output rows; for W4A16 the exact fp32 dequant first) timed
    on this host's cores for about budget_s seconds of CPU work (at least one full call),
    on the same shape as the GPU leg; the 4096^3 leg adds a one-core rate from 64 rows."""
    import numpy as np  # noqa: F401
    import oracle  # the CPU baseline leg is the only bench code that uses the oracle
    threads = oracle.num_threads()
    model = cpu_model()

    def timed(fn):
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 > budget_s:
                return (time.perf_counter() - t0) / reps, reps

    def gemm_leg(M, N, K, sd, seed, what):
        a = oracle.normal_bf16((M, K), seed, 0.0, sd)
        b = oracle.normal_bf16((K, N), seed + 1, 0.0, sd)
        dt, reps = timed(lambda: oracle.gemm_bf16(a, b, "nn"))
        return dt, reps, {"sample": f"full {what} NN GEMM x{reps} ({dt:.3f} s each) with OpenMP over rows; "
                                    f"sequential fp32 per output as cpu_gemm_nt_bf16 (src/t0/tile_ir.rs:5021-5038)"}

    def w4_leg(M, K, N, G, zeros, what):
        a = oracle.normal_bf16((M, K), 1, 0.0, 1.0)
        w = oracle.pack_qweight(oracle.nibbles((K, N), 2))
        s = oracle.uniform_bf16((K // G, N), 3, 0.005, 0.02)
        z = oracle.pack_qzeros(oracle.nibbles((K // G, N), 4)) if zeros else None
        dt, reps = timed(lambda: oracle.w4a16_gemm(a, w, s, z, G, 8))
        return dt, reps, {"sample": f"full {what} GEMM x{reps} ({dt * 1e3:.0f} ms each): exact fp32 dequant "
                                    f"((q - z) * s, quant_kernels.rs:24) then the sequential-fp32 loop, OpenMP over rows"}

    base = {"cores": threads, "kind": "port", "cpu_model": model}
    if which == "gemm":
        M = N = K = 4096
        dt, reps, info = gemm_leg(M, N, K, 1.0, 0x7501, "4096^3")
        a = oracle.normal_bf16((64, K), 0x7501, 0.0, 1.0)
        b = oracle.normal_bf16((K, N), 0x7502, 0.0, 1.0)
        t1 = time.perf_counter()
        oracle.gemm_bf16(a, b, "nn", nthreads=1)
        one = 2.0 * 64 * N * K / (time.perf_counter() - t1) / 1e12
        return {"value": round(2.0 * M * N * K / dt / 1e12, 4), "unit": "TFLOPS", **base,
                "one_core_TFLOPS": round(one, 5), **info}
    if which == "skinny":
        M, N, K = 128, 4096, 4096
        dt, reps, info = gemm_leg(M, N, K, 0.02, 0x7503, "128x4096x4096")
        return {"value": round((2 * M * K + 2 * K * N + 2 * M * N) / dt / 1e9, 3), "unit": "GB/s", **base, **info}
    if which == "prefill":
        M, K, N, G = 4096, 4096, 14336, 128
        dt, reps, info = w4_leg(M, K, N, G, True, "4096x4096x14336 g128 W4A16 prefill")
        return {"value": round(2.0 * M * N * K / dt / 1e12, 4), "unit": "TFLOPS", **base, **info}
    Mw, Kw, Nw, G = 16, 4096, (1376 if which == "shard" else 11008), 128
    dt, reps, info = w4_leg(Mw, Kw, Nw, G, False, f"16x4096x{Nw} decode")
    alg_bytes = 2 * Mw * Kw + Kw * Nw // 2 + 2 * (Kw // G) * Nw + 2 * Mw * Nw
    return {"value": round(alg_bytes / dt / 1e9, 3), "unit": "GB/s", **base, **info}


def roofline(bound, achieved, traffic):
    peak = PEAK_HBM_GBS if bound == "hbm" else PEAK_BF16_TFLOPS
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": "GB/s" if bound == "hbm" else "TFLOP/s",
            "frac": round(achieved / peak, 4), "traffic": traffic}


def copy_calibration(args, torch):
    """A plain elementwise copy of known size (1 GiB read + 1 GiB written per launch).  Under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE its readings give the counters' scale factor."""
    n = 1 << 28
    x = torch.ones(n, device="cuda:0", dtype=torch.float32)
    y = torch.empty_like(x)
    for _ in range(max(1, args.warmup)):
        torch.add(x, 1.0, out=y)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        torch.add(x, 1.0, out=y)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    nbytes = 2 * 4 * n
    print(json.dumps({"calibration": "fp32 copy y = x + 1", "read_bytes": 4 * n, "write_bytes": 4 * n,
                      "ms_per_launch": round(ms, 4), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1)}), flush=True)


def smi_sample(duration_s, launch, torch):
    """GFX clocks (MHz, averaged over the XCDs) and socket power (W) read with amd-smi
    every ~0.3 s while `launch` runs back to back for duration_s; medians and samples."""
    import re
    import subprocess
    import threading
    samples, stop = [], threading.Event()

    def poll():
        while not stop.is_set():
            try:
                out = subprocess.run(["amd-smi", "metric", "-g", "0", "-c", "-p"], capture_output=True, text=True,
                                     timeout=10).stdout
            except (OSError, subprocess.SubprocessError):
                return
            clks = [int(v) for v in re.findall(r"GFX_\d+:\s*\n\s*CLK:\s*(\d+)\s*MHz", out)]
            pw = re.findall(r"(?:SOCKET_POWER|POWER)\s*:\s*([\d.]+)\s*W", out)
            if clks:
                samples.append((sum(clks) / len(clks), float(pw[0]) if pw else None))
            stop.wait(0.3)
    th = threading.Thread(target=poll, daemon=True)
    t0 = time.perf_counter()
    th.start()
    while time.perf_counter() - t0 < duration_s:
        for _ in range(10):
            launch()
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    # the first sample may predate the load's steady state
    use = samples[1:] if len(samples) > 2 else samples
    med = lambda v: sorted(v)[len(v) // 2] if v else None
    return {"gfx_clock_MHz_median": med([c for c, _ in use]),
            "power_W_median": med([p for _, p in use if p is not None]),
            "samples": len(use), "clock_MHz_samples": [round(c) for c, _ in use]}


def bench_persistent(args, torch, t0mi):
    """The persistent preset tile_persistent_decode (tile_ir.rs:540-561) through t0mi_tile_gemm: one
    launch of the persistent decode kernel, beside the one-shot configuration the cost model picks
    for the same call (auto_select: split-K GEMM + reduce).  N(0,1) bf16 operands, f32 out; B is
    rotated over copies totalling >= 512 MB so the Infinity Cache cannot serve repeats.  Bytes
    per call: A, B and Y once."""
    rt = t0mi.Runtime.on_torch_stream(0)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7901)
    res = {}
    cases = ((1, 4096, 4096, t0mi.NT), (16, 4096, 4096, t0mi.NT), (1, 4096, 4096, t0mi.NN),
             (16, 4096, 4096, t0mi.NN), (32, 4096, 4096, t0mi.NT), (64, 4096, 4096, t0mi.NT),
             (16, 11008, 4096, t0mi.NT))
    preset = t0mi.tile_preset("tile_persistent_decode")
    for m, n, k, tr in cases:
        copies = max(2, -(-(512 << 20) // (2 * n * k)))
        a = torch.randn(m, k, device="cuda:0", generator=g).to(torch.bfloat16)
        shape_b = (k, n) if tr == t0mi.NN else (n, k)
        bs = [torch.randn(*shape_b, device="cuda:0", generator=g).to(torch.bfloat16) for _ in range(copies)]
        y = torch.empty(m, n, device="cuda:0", dtype=torch.float32)
        spec = preset.copy(transpose=tr)
        cfg = t0mi.auto_select_layout(m, k, n, tr, t0mi.OUT_F32).copy(transpose=tr, out_dtype=t0mi.OUT_F32)
        pa, py = a.data_ptr(), y.data_ptr()
        bp = [b.data_ptr() for b in bs]
        alg = 2 * n * k + 2 * m * k + 4 * m * n
        name = f"{m}x{n}x{k}_{'NN' if tr == t0mi.NN else 'NT'}"
        row = {"bytes": alg}
        for who, fn, gcall in (
                ("persistent", lambda i: rt.tile_gemm(spec, pa, bp[i % copies], py, m, n, k),
                 lambda r, i: r.tile_gemm(spec, pa, bp[i % copies], py, m, n, k)),
                ("one_shot:" + cfg.name(), lambda i: rt.gemm(cfg, pa, bp[i % copies], py, m, n, k),
                 lambda r, i: r.gemm(cfg, pa, bp[i % copies], py, m, n, k))):
            warm_up(torch, lambda fn=fn: fn(0), max(args.warmup, copies))
            us, batches = timed_batches(torch, fn, max(args.steps, 2 * copies))
            gbs = alg / (us * 1e-6) / 1e9
            gus = graph_replay_us(torch, t0mi, gcall, 4 * copies)
            row[who] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                        "batch_us": [round(b, 2) for b in batches], "graph_replay_us": gus,
                        "graph_GB/s": round(alg / (gus * 1e-6) / 1e9, 1)}
        res[name] = row
        print(f"[bench] persistent {name}: " + ", ".join(f"{k_} {v['us']} us ({v['GB/s']} GB/s; graph "
                                                       f"{v['graph_replay_us']} us)"
                                                       for k_, v in row.items() if k_ != "bytes"),
              file=sys.stderr, flush=True)
    rt.close()
    print(json.dumps({"metric": "tile_persistent_decode vs the one-shot auto_select config, us per call",
                      "unit": "us", "higher_is_better": False, "results": res}), flush=True)


SPLIT_SHAPES = ((4096, 14336, 4096), (1536, 11008, 4096), (2048, 11008, 4096), (1536, 14336, 4096),
                (2048, 14336, 4096))


def bench_split(args, torch, t0mi):
    """The column split of the auto-scheduled GEMMs (t0mi_auto_gemm_plan) on the dequant-once
    W4A16 route: per shape, t0mi_w4a16_gemm (dequant to bf16, then the planned pair of launches)
    against the same dequant followed by one launch of the head configuration over all columns
    (the schedule without the split).  Operands as the prefill leg (N(0,1) activations, random
    nibbles and zero points, group 128, bf16 out); median of 5 event-timed batches, the two
    schedules alternated three times and the middle of those medians kept."""
    rt = t0mi.Runtime.on_torch_stream(0)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7509)
    G = 128
    res = []
    for (m, n, k) in SPLIT_SHAPES:
        a = torch.randn(m, k, device="cuda:0", generator=g).to(torch.bfloat16)
        w = torch.randint(-2**31, 2**31 - 1, (k // 8, n), device="cuda:0", dtype=torch.int32, generator=g)
        s = (torch.rand(k // G, n, device="cuda:0", generator=g) * 0.015 + 0.005).to(torch.bfloat16)
        z = torch.randint(-2**31, 2**31 - 1, (k // G, n // 8), device="cuda:0", dtype=torch.int32, generator=g)
        y = torch.empty(m, n, device="cuda:0", dtype=torch.bfloat16)
        wb = torch.empty(k, n, device="cuda:0", dtype=torch.bfloat16)
        head, n1, tail = t0mi.auto_gemm_plan(m, n, k, t0mi.NN, t0mi.OUT_BF16)
        q = (w.data_ptr(), s.data_ptr(), z.data_ptr(), 0)

        def planned(i=0):
            rt.w4a16_gemm(a.data_ptr(), *q, y.data_ptr(), m, k, n, G, t0mi.OUT_BF16)

        def one_launch(i=0):
            rt.dequant_int4(*q, wb.data_ptr(), k, n, G, 2)
            rt.gemm(head, a.data_ptr(), wb.data_ptr(), y.data_ptr(), m, n, k)
        t = {"planned": [], "one_launch": []}
        for _ in range(3):
            for name, f in (("planned", planned), ("one_launch", one_launch)):
                warm_up(torch, f, 3, min_s=0.1)
                t[name].append(timed_batches(torch, f, 20)[0])
        us = {name: sorted(v)[1] for name, v in t.items()}
        r = {"shape": [m, n, k], "head": head.name(), "n_main": n1, "tail": tail.name() if n1 < n else None,
             "planned_us": round(us["planned"], 1), "one_launch_us": round(us["one_launch"], 1),
             "ratio": round(us["planned"] / us["one_launch"], 3)}
        res.append(r)
        print(f"[bench] split {m}x{n}x{k}: planned {r['planned_us']} us ({head.name()} to column {n1}"
              f"{', then ' + r['tail'] if r['tail'] else ''}), one launch {r['one_launch_us']} us",
              file=sys.stderr, flush=True)
        del a, w, s, z, y, wb
    rt.close()
    print(json.dumps({"metric": "W4A16 dequant-once route: planned column split / one launch", "unit": "ratio",
                      "higher_is_better": False, "results": res}), flush=True)


def bench_dispatch(args, torch, t0mi):
    """Host-visible cost per dispatch of a batch of small GEMMs (the prefill_dispatch.rs
    scenario: dozens of layers x a few kernels), three ways: a synchronous dispatch per
    kernel (GpuRuntime::dispatch), one DispatchQueue flush per batch, and one replay of
    the batch captured as a HIP graph.  Wall time from the first submit to the end of
    the final wait, median over repeats; the kernels are the same in all three."""
    batch, reps = 128, max(5, min(args.steps, 50))
    cfg = t0mi.preset("tile_64x64_k32")
    m = n = 128
    k = 256
    rt = t0mi.Runtime(device=0)  # own stream: a graph cannot be captured on the null stream
    kern = rt.kernel(cfg)
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0x7601)
    a = torch.randn(m, k, device="cuda:0", generator=g).to(torch.bfloat16)
    bs = [torch.randn(n, k, device="cuda:0", generator=g).to(torch.bfloat16) for _ in range(8)]
    ys = [torch.empty(m, n, device="cuda:0", dtype=torch.float32) for _ in range(batch)]
    torch.cuda.synchronize()
    grid = t0mi.compute_grid_auto(cfg, m, n)
    kas = [t0mi.build_kernargs(a.data_ptr(), bs[i % 8].data_ptr(), ys[i].data_ptr(), k, n, m, cfg)
           for i in range(batch)]

    def sync_each():
        for ka in kas:
            t0mi.check(rt.dispatch(kern, grid, ka, sync=True))

    def queued():
        dq = t0mi.DispatchQueue(rt)
        for ka in kas:
            dq.submit(kern, grid, ka)
        assert dq.flush() == batch

    rt.capture_begin()
    for ka in kas:
        t0mi.check(rt.dispatch(kern, grid, ka, sync=False))
    graph = rt.capture_end()

    def replay():
        graph.launch()
        t0mi.check(rt.wait_idle())

    # GPU time of one replay (kernels plus the gaps between them), from events
    # recorded on the runtime's own stream.
    ext = torch.cuda.ExternalStream(rt.stream)
    replay()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(ext)
    graph.launch()
    e1.record(ext)
    t0mi.check(rt.wait_idle())
    e1.synchronize()
    gpu_us = e0.elapsed_time(e1) * 1e3 / batch

    res = {}
    for name, fn in (("sync", sync_each), ("queue", queued), ("graph", replay)):
        for _ in range(3):
            fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        ts.sort()
        res[name] = round(ts[len(ts) // 2] / batch * 1e6, 3)
    graph.destroy()
    rt.close()
    print(json.dumps({"metric": "host-visible time per dispatch in a batch (us)", "unit": "us/dispatch",
                      "higher_is_better": False, "batch": batch, "repeats": reps, "per_dispatch_us": res,
                      "gpu_us_per_dispatch_in_graph": round(gpu_us, 3),
                      "config": {"workload": f"{batch} dispatches of a {m}x{n}x{k} NT bf16 GEMM, f32 out",
                                 "kernel": cfg.name()}}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the GEMM path "
              f"is not sharded across GPUs here.", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.init()
    if args.only == "copy":
        copy_calibration(args, torch)
        return
    import t0mi
    if args.only == "dispatch":
        bench_dispatch(args, torch, t0mi)
        return
    if args.only == "persistent":
        bench_persistent(args, torch, t0mi)
        return
    if args.only == "split":
        bench_split(args, torch, t0mi)
        return
    rt = t0mi.Runtime.on_torch_stream(0)
    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic"}
    legs = ("gemm", "w4a16", "skinny", "prefill", "shard") if args.only == "all" else (args.only,)
    cpu = {}

    def baseline(which):
        if args.no_cpu:
            return None
        try:
            return cpu_baseline(which, budget_s=10.0 if which in ("gemm", "w4a16") else 5.0)
        except Exception as e:  # the baseline is reported, never required
            return {"value": None, "error": str(e)}

    if "gemm" in legs:
        cfg, ms, tflops, batches = bench_gemm(args, torch, t0mi, rt)
        out.update({"value": round(tflops, 2), "unit": "TFLOPS", "ms_per_step": round(ms, 5),
                    "timing": f"median of {len(batches)} batches of {args.steps} launches (HIP events)",
                    "batch_us": [round(b, 2) for b in batches],
                    "config": {"workload": "bf16 GEMM M=N=K=4096, A[M,K] x B[K,N] row-major (NN), N(0,1), "
                                           "fp32 accumulate, bf16 out (BASELINE config 2)",
                               "M": 4096, "N": 4096, "K": 4096, "kernel": cfg.name()},
                    "roofline": roofline("mfma", tflops, load_traffic("gemm_4096"))})
        if args.tuned:
            out["tuned"] = args.tuned
        if args.gemm_clocks:
            out["clocks_during_sustained_launches"] = args.gemm_clocks
        cpu["gemm"] = baseline("gemm")
    if "w4a16" in legs:
        us, gbs, alg_bytes, copies, wb = bench_w4a16(args, torch, t0mi, rt)
        w = {"value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(us, 3),
             "batch_us": [round(b, 3) for b in wb],
             "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "algorithmic_bytes": alg_bytes,
             "graph_replay_us_per_call": args.w4_graph_us,
             **({"clocks_during_sustained_launches": args.w4_clocks} if args.w4_clocks else {}),
             "weight_copies_rotated": copies,
             "workload": f"W4A16 decode A[{args.rows},4096] bf16 x int4 W[4096,11008] g128 zp=8, bf16 out"
                         + (" (BASELINE config 4)" if args.rows == 16 else "")}
        out["w4a16_decode"] = w
        out["roofline_w4a16"] = roofline("hbm", gbs, load_traffic("w4a16_decode") if args.rows == 16 else None)
        cpu["w4a16"] = baseline("w4a16")
    if "skinny" in legs:
        cfg, us, gbs, alg_bytes, tuned = bench_skinny(args, torch, t0mi, rt)
        out["skinny"] = {"value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(us, 3),
                         "algorithmic_bytes": alg_bytes, "kernel": cfg.name(),
                         "workload": "bf16 GEMM M=128, N=4096, K=4096 NN, N(0,0.02), bf16 out (BASELINE config 3), "
                                     "B rotated over 16 copies",
                         "roofline": roofline("hbm", gbs, load_traffic("gemm_skinny"))}
        if tuned:
            out["skinny"]["tuned"] = tuned
        cpu["skinny"] = baseline("skinny")
    if "prefill" in legs:
        us, tflops, (fus_us, fus_tf) = bench_prefill(args, torch, t0mi, rt)
        work = ("W4A16 A[4096,4096] bf16 x int4 W[4096,14336] g128, per-group zero points, bf16 out "
                "(BASELINE config 5); one call = t0mi_w4a16_gemm")
        out["prefill"] = {"value": round(tflops, 2), "unit": "TFLOPS", "us_per_call": round(us, 2), "workload": work,
                          "route": "default (t0mi_w4a16_gemm as called)",
                          "roofline": roofline("mfma", tflops, load_traffic("w4a16_prefill"))}
        out["prefill_fused"] = {"value": round(fus_tf, 2), "unit": "TFLOPS", "us_per_call": round(fus_us, 2),
                                "workload": work,
                                "route": "t0mi_set_w4a16_workspace_limit(ctx, 0): dequant inside the MFMA K loop",
                                "roofline": roofline("mfma", fus_tf, (load_traffic("w4a16_prefill_fused_detail")
                                                                      or {}).get("call_bytes"))}
        cpu["prefill"] = baseline("prefill")
    if "shard" in legs:
        out["shard"] = bench_shard(args, torch, t0mi, rt)
        cpu["shard"] = baseline("shard")
    rt.close()
    if args.only != "all":
        # One leg alone: its figures are the line's own.
        leg = {"gemm": None, "w4a16": "w4a16_decode", "skinny": "skinny", "prefill": "prefill", "shard": "shard"}
        key = leg.get(args.only)
        if key:
            o = out.pop(key)
            out["metric"] = {"w4a16_decode": "W4A16 decode HBM GB/s (% peak)", "skinny": "skinny bf16 GEMM HBM GB/s (% peak)",
                             "prefill": "W4A16 prefill TFLOPS (% MFMA peak)",
                             "shard": "W4A16 decode shard HBM GB/s (% peak)"}[key]
            us = o.get("us_per_call")
            out.update({"value": o["value"], "unit": o["unit"], "ms_per_step": round(us * 1e-3, 6),
                        "config": {"workload": o["workload"], **({"kernel": o["kernel"]} if "kernel" in o else {})},
                        "roofline": out.pop("roofline_w4a16") if key == "w4a16_decode" else o.pop("roofline")})
            if key == "prefill":
                out["fused_route"] = out.pop("prefill_fused")
            out[key + "_detail"] = o
        c = cpu.get(args.only)
        if c:
            out["cpu_baseline"] = c
    else:
        if cpu.get("gemm"):
            out["cpu_baseline"] = cpu["gemm"]
        for key, leg in (("w4a16", "cpu_baseline_w4a16"), ("skinny", "skinny"), ("prefill", "prefill"),
                         ("shard", "shard")):
            c = cpu.get(key)
            if not c:
                continue
            if key == "w4a16":
                out[leg] = c
            else:
                out[leg]["cpu_baseline"] = c
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
