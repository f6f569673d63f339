#!/usr/bin/env python3
"""Benchmark of the gfx950 attention forward at the headline shape.

Workload (one "step" = one fav4_bshd_forward launch over one batch):
B=32, H=8, Sq=Sk=4096, D=128, BF16 BSHD, Q/K/V iid N(0,1) (synthetic,
seeded), scale 1/sqrt(128), LSE off -- timed dense (the JSON ``value``) and
top-left causal (reported beside it).  Timing follows the reference harness,
benchmarks/bshd.py:34-51,163: a HIP graph of W launches is replayed as warmup,
then a graph of exactly K launches is replayed between two GPU events on the
launch stream; six such observations are taken and the mean is reported.  The
FLOP convention is the reference's (bshd.py:169-170, README.md:59): useful
QK+PV only, dense 4*B*H*D*S^2, causal 4*B*H*D*S(S+1)/2.

Before timing, each timed output is checked against the FP64 oracle on the
reference's sampled rows (bshd.py:147-148) for a subset of (b, h) pairs.

The ``cpu_baseline`` leg times the FP64 oracle on this host's cores on a
bounded sample of (b, h) slices of the same dense workload (a baseline only).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_TFLOPS = 2516.6      # MI355X dense BF16 MFMA: 256 CU x 4 SIMD x 1024 FLOP/clk x 2.4 GHz
HBM_TBPS = 8.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_fmha_fwd_dense_b32h8s4096.md"


def parse_args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", type=int, default=0)
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--seq", type=int, default=4096)
    p.add_argument("--observations", type=int, default=6)
    p.add_argument("--no-causal", action="store_true", help="time dense only")
    p.add_argument("--no-check", action="store_true", help="skip the sampled-row FP64 check")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    p.add_argument("--sweep", default="", help="comma list of extra sequence lengths to time (report only)")
    p.add_argument("--pmc-pass", action="store_true",
                   help="profiling mode for counter runs: two eager launches per mask type, then a "
                        "plain 1 GiB device copy (HBM counter calibration); prints no JSON")
    return p.parse_args()


def pmc_pass(torch, runner, args):
    """Eager launches for rocprofv3 --pmc runs (no graphs, one dispatch per launch)."""
    b, h, s = args.batch, args.heads, args.seq
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    for causal in (False, True):
        for _ in range(2):
            runner.call(q, k, v, o, None, causal, args.config)
        torch.cuda.synchronize()
        print(f"# pmc-pass launched B{b} H{h} S{s} causal={causal} x2", flush=True)
    del q, k, v, o
    src = torch.ones(1 << 28, device="cuda", dtype=torch.float32)    # 1 GiB
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("# pmc-pass copy: 1073741824 bytes read + 1073741824 bytes written per dispatch", flush=True)


def make_inputs(torch, b, h, s, seed=11939):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    shape = (b, s, h, 128)
    q = torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    k = torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    v = torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    return q, k, v


def bits(torch, t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def check_rows(torch, orc, q, k, v, o, causal, pairs):
    """FP64 oracle on the reference's sampled rows for the given (b, h) pairs."""
    s = q.shape[1]
    rows = orc.sample_rows(s)
    qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
    ref, _ = orc.attention_fp64(qb, kb, vb, orc.DEFAULT_SCALE, causal, rows=rows, heads=pairs)
    got = bits(torch, o[:, rows])
    sel_ref = np.stack([ref[b, :, h] for b, h in pairs])
    sel_got = np.stack([got[b, :, h] for b, h in pairs])
    return orc.errors(sel_got, None, sel_ref, None), rows


def time_graph(torch, fn, steps, warmup, observations, stream):
    """Per-launch microseconds from HIP-graph replays bracketed by events on `stream`."""
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g_timed = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_timed, stream=stream):
            for _ in range(steps):
                fn()
        g_warm = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_warm, stream=stream):
            for _ in range(warmup):
                fn()
    samples = []
    for _ in range(observations):
        with torch.cuda.stream(stream):
            g_warm.replay()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(stream)
            g_timed.replay()
            end.record(stream)
        end.synchronize()
        samples.append(start.elapsed_time(end) * 1000.0 / steps)
    torch.cuda.synchronize()
    return samples


def cpu_baseline(torch, orc, q, k, v, budget_s):
    """FP64 oracle on host cores over (b, h) slices of the dense workload until
    the time budget is spent.  Threads: one slice per worker, BLAS single-threaded."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    b, s, h, d = q.shape
    cores = min(len(os.sched_getaffinity(0)), 16)
    qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
    pairs = [(i, j) for i in range(b) for j in range(h)]
    done = 0
    t0 = time.perf_counter()
    with threadpool_limits(1), ThreadPoolExecutor(cores) as ex:
        while done < len(pairs) and time.perf_counter() - t0 < budget_s:
            chunk = pairs[done:done + cores]
            list(ex.map(lambda p: orc.attention_fp64(qb, kb, vb, orc.DEFAULT_SCALE, False, heads=[p]),
                        chunk))
            done += len(chunk)
    elapsed = time.perf_counter() - t0
    flop = orc.flops(1, 1, s, s, False) * done
    return dict(value=flop / elapsed / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                sample=f"FP64 numpy oracle, {done} of {len(pairs)} (b,h) slices of B{b} H{h} "
                       f"S{s} D{d} dense, {elapsed:.1f} s on {cores} threads (one slice per thread, "
                       f"single-threaded BLAS); extrapolated whole-job time "
                       f"{elapsed * len(pairs) / done:.1f} s")


def read_traffic():
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    from oracle import attention as orc
    import __graft_entry__
    pkg = __graft_entry__.import_package()
    runner = pkg.Runner()
    if args.pmc_pass:
        pmc_pass(torch, runner, args)
        return

    b, h, s = args.batch, args.heads, args.seq
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    stream = torch.cuda.Stream()
    pairs = [(0, 0), (b // 2, h // 2), (b - 1, h - 1)]
    results = {}
    for causal in ([False] if args.no_causal else [False, True]):
        fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        check = None
        if not args.no_check:
            o.fill_(float("nan"))
            with torch.cuda.stream(stream):
                fn()
            torch.cuda.synchronize()
            check, _ = check_rows(torch, orc, q, k, v, o, causal, pairs)
            if not orc.check_north_star_tolerance(check):
                raise SystemExit(f"sampled-row check failed (causal={causal}): {check}")
        samples = time_graph(torch, fn, args.steps, args.warmup, args.observations, stream)
        flop = orc.flops(b, h, s, s, causal)
        us = statistics.mean(samples)
        results[causal] = dict(us=us, median_us=statistics.median(samples), samples_us=samples,
                               tflops=flop / us / 1e6, flop=flop, check=check)
        print(f"# B{b} H{h} S{s} causal={causal}: {us:.1f} us/launch, {flop / us / 1e6:.1f} TFLOP/s "
              f"({flop / us / 1e6 / PEAK_BF16_TFLOPS * 100:.1f}% of peak) check={check}",
              file=sys.stderr, flush=True)

    sweep = {}
    for n in [int(x) for x in args.sweep.split(",") if x]:
        del q, k, v, o
        torch.cuda.empty_cache()
        q, k, v = make_inputs(torch, b, h, n)
        o = torch.empty_like(q)
        for causal in (False, True):
            fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
            sm = time_graph(torch, fn, args.steps, args.warmup, 2, stream)
            us = statistics.mean(sm)
            tf = orc.flops(b, h, n, n, causal) / us / 1e6
            sweep[f"S{n}_{'causal' if causal else 'dense'}"] = dict(us=round(us, 2), tflops=round(tf, 1))
            print(f"# sweep S{n} causal={causal}: {us:.1f} us, {tf:.1f} TFLOP/s", file=sys.stderr, flush=True)

    dense = results[False]
    traffic = read_traffic()
    compulsory = 2 * b * h * 128 * (2 * s + 2 * s)
    roofline = dict(bound="mfma", achieved=round(dense["tflops"], 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                    frac=round(dense["tflops"] / PEAK_BF16_TFLOPS, 4), traffic=traffic,
                    kernel="fav4::fwd_kernel (dense)", flop_per_launch=dense["flop"],
                    avg_launch_us=round(dense["us"], 3), compulsory_hbm_bytes=compulsory)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(torch, orc, q, k, v, args.cpu_seconds) if not sweep else None
    line = {
        "metric": "fwd TFLOP/s + % BF16 MFMA peak, B32 H8 D128 S4096 dense & causal",
        "value": round(dense["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dense["us"] / 1000.0, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) BF16 Q/K/V generated on the GPU)",
        "config": {"workload": f"FMHA fwd BSHD B{b} H{h} Sq=Sk={s} D128 BF16, scale 1/sqrt(128), LSE off",
                   "global_batch": b, "seq_len": s, "heads": h, "head_dim": 128,
                   "config_id": args.config, "parallelism": "single GPU"},
        "frac_of_peak_dense": round(dense["tflops"] / PEAK_BF16_TFLOPS, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if True in results:
        c = results[True]
        line["causal"] = dict(value=round(c["tflops"], 2), unit="TFLOP/s", us_per_launch=round(c["us"], 3),
                              frac_of_peak=round(c["tflops"] / PEAK_BF16_TFLOPS, 4),
                              samples_us=[round(x, 2) for x in c["samples_us"]])
    line["dense_samples_us"] = [round(x, 2) for x in dense["samples_us"]]
    if sweep:
        line["sweep"] = sweep
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
