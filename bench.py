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

The ``comparator`` leg times torch's scaled_dot_product_attention on the same
device and inputs (contiguous BHSD copies, its fused flash backend, else its
memory-efficient one; never the unfused math path), interleaved with this
library's kernel in A-B-B-A order, and reports the speedup and the largest
difference between the two outputs.  ``provenance`` records what was measured:
library and source hashes, toolchain and torch versions, device and clocks.
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
SWEEP_SPIN_MS = 50.0           # untimed spin-up before each sweep shape (report-only rows)


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
    p.add_argument("--sweep", default="512,1024,8192,16384,32768",
                   help="comma list of the long-sequence sweep's lengths (B and H as the headline; dense and causal)")
    p.add_argument("--no-sweep", action="store_true", help="skip the long-sequence sweep")
    p.add_argument("--no-comparator", action="store_true", help="skip the torch SDPA comparator")
    p.add_argument("--no-splitkv", action="store_true", help="skip the split-KV report (B1 H8 Sq1024 Sk32768; B1 H1 S16384 causal)")
    p.add_argument("--no-api", action="store_true", help="skip the GQA / varlen report")
    p.add_argument("--no-telemetry", action="store_true",
                   help="start no child processes (amd-smi clocks, hipcc version), e.g. under a profiler")
    p.add_argument("--mfma-ceiling", action="store_true",
                   help="MFMA-only ceiling: a probe kernel streaming BF16 MFMAs (32x32x16 and 16x16x32) at the "
                        "forward's occupancy, graph-timed with clock and power under load, beside the dense and "
                        "causal headline in the same process; prints one JSON line")
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


def mfma_ceiling(torch, runner, pkg, args):
    """The MFMA rate with nothing else on the chip (libfav4_mfma_ceiling.so,
    built by build()), at the clock the board's power limit allows, beside
    the headline kernels measured the same way. One workgroup of 8 waves per
    CU streams BF16 MFMAs on pseudo-random register operands; shape 0 is
    32x32x16 (the forward's), shape 1 16x16x32 at equal FLOPs."""
    import ctypes as C
    lib = C.CDLL(str(pkg.CEILING_LIB_PATH))
    lib.fav4_probe_mfma_ceiling.argtypes = [C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
    lib.fav4_probe_mfma_ceiling.restype = C.c_int
    stream = torch.cuda.Stream()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 2048                                   # about 2 ms per launch
    out = torch.empty(cus * 512, device="cuda", dtype=torch.float32)
    res = {}
    for shape, name in ((0, "mfma_32x32x16"), (1, "mfma_16x16x32")):
        fn = lambda: lib.fav4_probe_mfma_ceiling(shape, cus, iters, out.data_ptr(), stream.cuda_stream)
        with torch.cuda.stream(stream):
            st = fn()
        torch.cuda.synchronize()
        if st:
            raise SystemExit(f"mfma ceiling probe: HIP status {st}")
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
        flop = cus * 8 * iters * 1048576
        res[name] = dict(us=round(us, 2), tflops=round(flop / us / 1e6, 1),
                         frac_of_peak=round(flop / us / 1e6 / PEAK_BF16_TFLOPS, 4),
                         telemetry_under_load=loaded_telemetry(torch, fn, stream) if _TELEMETRY else None)
        print(f"# {name}: {us:.1f} us, {flop / us / 1e6:.1f} TFLOP/s", file=sys.stderr, flush=True)
    b, h, s = args.batch, args.heads, args.seq
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    for causal in (False, True):
        fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
        tflops = flops(b, h, s, s, causal) / us / 1e6
        res["fwd_causal" if causal else "fwd_dense"] = dict(
            us=round(us, 2), tflops=round(tflops, 1), frac_of_peak=round(tflops / PEAK_BF16_TFLOPS, 4),
            telemetry_under_load=loaded_telemetry(torch, fn, stream) if _TELEMETRY else None)
        print(f"# B{b} H{h} S{s} causal={causal}: {us:.1f} us, {tflops:.1f} TFLOP/s", file=sys.stderr, flush=True)
    res["fwd_dense_of_ceiling"] = round(res["fwd_dense"]["tflops"] / res["mfma_32x32x16"]["tflops"], 4)
    print(json.dumps({"mode": "mfma_ceiling", "workload": f"B{b} H{h} Sq=Sk={s} D128 BF16, LSE off, config "
                      f"{args.config}", "cus": cus, "iters_per_wave": iters, **res}), flush=True)


def flops(b, h, sq, sk, causal):
    """Useful QK+PV FLOPs, the reference's convention (benchmarks/bshd.py:169-170):
    4*B*H*128*Sq*Sk dense; top-left causal counts the keys each row sees,
    4*B*H*128*sum_{i<Sq} min(i+1, Sk)."""
    if not causal:
        return 4 * b * h * 128 * sq * sk
    full = min(sq, sk)
    return 4 * b * h * 128 * (full * (full + 1) // 2 + max(0, sq - sk) * sk)


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


def check_rows(torch, orc, q, k, v, o, causal, pairs, lse=None):
    """FP64 oracle on the reference's sampled rows for the given (b, h) pairs
    (and the LSE of those rows when `lse` is given).  Only those slices are
    copied to the host (a full S32768 tensor is 2 GiB)."""
    s = q.shape[1]
    rows = orc.sample_rows(s)
    rows_t = torch.from_numpy(rows).to(q.device)
    refs, gots, ref_l, got_l = [], [], [], []
    for b, h in pairs:
        sl = lambda t: bits(torch, t[b:b + 1, :, h:h + 1])
        ref, rl = orc.attention_fp64(sl(q), sl(k), sl(v), orc.DEFAULT_SCALE, causal, rows=rows)
        refs.append(ref[0, :, 0])
        gots.append(bits(torch, o[b:b + 1].index_select(1, rows_t)[:, :, h:h + 1])[0, :, 0])
        if lse is not None:
            ref_l.append(rl[0, 0])
            got_l.append(lse[b, h].index_select(0, rows_t).cpu().numpy())
    if lse is None:
        return orc.errors(np.stack(gots), None, np.stack(refs), None), rows
    return orc.errors(np.stack(gots), np.stack(got_l), np.stack(refs), np.stack(ref_l)), rows


def time_graph(torch, fn, steps, warmup, observations, stream, spin_ms=0.0):
    """Per-launch microseconds from HIP-graph replays bracketed by events on `stream`.

    spin_ms > 0: before the observations, replay the warmup graph (untimed)
    until that much wall time has passed, so that short launches are timed at
    the loaded clock rather than while the GPU ramps up from idle."""
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
    if spin_ms > 0:
        t_end = time.perf_counter() + spin_ms / 1000.0
        while time.perf_counter() < t_end:
            with torch.cuda.stream(stream):
                g_warm.replay()
            torch.cuda.synchronize()
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


def cpu_info():
    """Host CPU description: lscpu's model name (else /proc/cpuinfo's), sockets,
    and the cores this process may run on."""
    info = {"model": None, "sockets": None, "affinity_cores": len(os.sched_getaffinity(0))}
    txt = _run(["lscpu"], force=True)
    for ln in (txt or "").splitlines():
        key, _, val = ln.partition(":")
        key, val = key.strip(), val.strip()
        if key == "Model name" and not info["model"]:
            info["model"] = val
        elif key == "BIOS Model name":
            info["bios_model"] = val
        elif key == "Socket(s)":
            info["sockets"] = int(val) if val.isdigit() else val
    # /proc/cpuinfo's identification of the first core: a virtual machine's
    # model name can be as short as "AMD EPYC", and family / model / stepping
    # still name the part.
    try:
        with open("/proc/cpuinfo") as f:
            first = {}
            for ln in f:
                if not ln.strip():
                    break
                key, _, val = ln.partition(":")
                first[key.strip()] = val.strip()
        if not info["model"]:
            info["model"] = first.get("model name")
        info["cpuinfo"] = {k: first.get(k) for k in ("model name", "cpu family", "model", "stepping", "cpu MHz",
                                                       "cache size")}
    except OSError:
        pass
    return info


def cpu_threads():
    """Worker threads for the CPU baseline: every core of this process's
    affinity set, capped by OMP_NUM_THREADS when the launcher sets it (the
    CPU share granted beside one GPU, 16 on the MI355X boxes used here)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return (min(n, int(cap)) if cap.isdigit() and int(cap) > 0 else n), n


def _attention_fp32_slice(qb, kb, vb, bh, scale):
    """Dense FP32 attention of one (b, h) slice (numpy, textbook form)."""
    from oracle import attention as orc
    b, h = bh
    q = orc.bf16_to_f32(qb[b, :, h]).reshape(qb.shape[1], -1)
    k = orc.bf16_to_f32(kb[b, :, h]).reshape(kb.shape[1], -1)
    v = orc.bf16_to_f32(vb[b, :, h]).reshape(vb.shape[1], -1)
    s = (q @ k.T) * np.float32(scale)
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ v) / p.sum(axis=1, keepdims=True)


def cpu_baseline(torch, orc, q, k, v, budget_s):
    """FP64 oracle (and an FP32 textbook attention) on host cores over (b, h)
    slices of the dense workload until each time budget is spent.  Threads: one
    slice per worker, BLAS single-threaded."""
    from concurrent.futures import ThreadPoolExecutor
    from threadpoolctl import threadpool_limits
    b, s, h, d = q.shape
    cores, affinity = cpu_threads()
    qb, kb, vb = bits(torch, q), bits(torch, k), bits(torch, v)
    pairs = [(i, j) for i in range(b) for j in range(h)]

    def run(fn, budget):
        done = 0
        t0 = time.perf_counter()
        with threadpool_limits(1), ThreadPoolExecutor(cores) as ex:
            while done < len(pairs) and time.perf_counter() - t0 < budget:
                chunk = pairs[done:done + cores]
                list(ex.map(fn, chunk))
                done += len(chunk)
        return done, time.perf_counter() - t0

    done, elapsed = run(lambda p: orc.attention_fp64(qb, kb, vb, orc.DEFAULT_SCALE, False, heads=[p]), budget_s)
    done32, elapsed32 = run(lambda p: _attention_fp32_slice(qb, kb, vb, p, orc.DEFAULT_SCALE), budget_s / 2)
    flop1 = flops(1, 1, s, s, False)
    host = cpu_info()
    return dict(value=flop1 * done / elapsed / 1e12, unit="TFLOP/s", cores=cores, kind="port",
                sample=f"FP64 numpy oracle, {done} of {len(pairs)} (b,h) slices of B{b} H{h} "
                       f"S{s} D{d} dense, {elapsed:.1f} s on {cores} threads (one slice per thread, "
                       f"single-threaded BLAS; {affinity} cores in the affinity set, threads capped by "
                       f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}); extrapolated "
                       f"whole-job time {elapsed * len(pairs) / done:.1f} s",
                fp32=dict(value=round(flop1 * done32 / elapsed32 / 1e12, 4), unit="TFLOP/s",
                          sample=f"FP32 numpy textbook attention, {done32} slices in {elapsed32:.1f} s"),
                cpu_model=host.get("model"), bios_model=host.get("bios_model"), sockets=host.get("sockets"),
                affinity_cores=affinity, cpuinfo=host.get("cpuinfo"))


def time_eager(torch, fn, steps, warmup, stream):
    """Per-launch microseconds of `steps` eager launches between events on `stream`."""
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(steps):
            fn()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


def comparator(torch, orc, runner, q, k, v, o, stream, args, causal_list):
    """torch SDPA (fused backends only) vs this library on the same inputs, A-B-B-A."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    b, s, h, d = q.shape
    qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    scale = 1.0 / math.sqrt(d)
    backend = None
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([be]):
                F.scaled_dot_product_attention(qh[:1, :1, :256], kh[:1, :1, :256], vh[:1, :1, :256], scale=scale)
            torch.cuda.synchronize()
            backend = (name, be)
            break
        except RuntimeError:
            continue
    if backend is None:
        return None
    out = {"name": f"torch.nn.functional.scaled_dot_product_attention, {backend[0]} backend "
                   f"(torch {torch.__version__})",
           "layout": "contiguous BHSD copies of the same Q/K/V (its preferred layout; copies not timed)"}
    for causal in causal_list:
        ref = [None]

        def theirs():
            with sdpa_kernel([backend[1]]):
                ref[0] = F.scaled_dot_product_attention(qh, kh, vh, is_causal=causal, scale=scale)

        ours = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        t = {"ours": [], "theirs": []}
        for who in ("ours", "theirs", "theirs", "ours"):
            t[who].append(time_eager(torch, ours if who == "ours" else theirs, args.steps, args.warmup, stream))
        torch.cuda.synchronize()
        diff = (ref[0].transpose(1, 2).float() - o.float()).abs().max().item()
        flop = flops(b, h, s, s, causal)
        us_o, us_t = statistics.mean(t["ours"]), statistics.mean(t["theirs"])
        out["causal" if causal else "dense"] = dict(
            tflops=round(flop / us_t / 1e6, 2), us_per_launch=round(us_t, 3),
            ours_tflops_eager=round(flop / us_o / 1e6, 2), speedup=round(us_t / us_o, 4),
            max_abs_diff_vs_ours=round(diff, 5))
        print(f"# comparator causal={causal}: SDPA {flop / us_t / 1e6:.1f} TFLOP/s, ours {flop / us_o / 1e6:.1f} "
              f"(eager, ABBA), speedup {us_t / us_o:.3f}, max|diff| {diff:.4f}", file=sys.stderr, flush=True)
    del qh, kh, vh
    return out


def splitkv_report(torch, orc, runner, args, stream):
    """Few (b, h, q tile) items and long keys: the single-pass forward against the
    split-KV forward (Auto chunk count), both graph-timed, each output checked on
    sampled rows first.  B1 H8 Sq1024 Sk32768 dense and causal (causal rows see
    only the first 1024 keys: Auto keeps the unsplit forward there), and a
    single-head causal prefill of 16384 tokens."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11939)
    out = {}
    for label, b, h, sq, sk, causal in (("dense", 1, 8, 1024, 32768, False), ("causal", 1, 8, 1024, 32768, True),
                                        ("causal_long", 1, 1, 16384, 16384, True)):
        mk = lambda s: torch.randn((b, s, h, 128), device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
        q, k, v = mk(sq), mk(sk), mk(sk)
        o = torch.empty_like(q)
        splits = runner.splitkv_select(b, h, sq, sk, causal)
        ws = torch.empty(max(runner.splitkv_workspace_size(b, h, sq, sk, causal, 0), 1), device="cuda",
                         dtype=torch.uint8)
        plain = lambda: runner.call(q, k, v, o, None, causal, 0, stream=stream.cuda_stream)
        split = lambda: runner.call_splitkv(q, k, v, o, None, causal, 0, workspace=ws, stream=stream.cuda_stream)
        flop = flops(b, h, sq, sk, causal)
        res = {"workload": f"B{b} H{h} Sq={sq} Sk={sk} D128 BF16 {'causal' if causal else 'dense'}, LSE off",
               "splits": splits, "workspace_bytes": ws.numel()}
        for name, fn in (("plain", plain), ("splitkv", split)):
            o.fill_(float("nan"))
            torch.cuda.synchronize()   # the fill runs on the default stream
            with torch.cuda.stream(stream):
                fn()
            torch.cuda.synchronize()
            err, _ = check_rows(torch, orc, q, k, v, o, causal, [(0, 0), (0, h - 1)])
            if not orc.check_acceptance_tolerance(err):
                raise SystemExit(f"split-KV report: {name} check failed ({label}): {err}")
            us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
            res[name] = dict(us=round(us, 2), tflops=round(flop / us / 1e6, 1))
        res["speedup"] = round(res["plain"]["us"] / res["splitkv"]["us"], 2)
        out[label] = res
        print(f"# splitkv B{b} H{h} {sq}x{sk} causal={causal}: plain {res['plain']['tflops']} TFLOP/s, "
              f"split-KV ({splits} chunks) {res['splitkv']['tflops']} TFLOP/s, x{res['speedup']}",
              file=sys.stderr, flush=True)
        del q, k, v, o, ws
    torch.cuda.empty_cache()
    return out


def api_report(torch, orc, runner, args, stream, b=32, h=8, s=4096, kvh=2):
    """The GQA and varlen entry points at the headline token count (B*S rows, H8):
    GQA with `kvh` K/V heads; varlen with B ragged sequences of seeded lengths in
    [S/4, 7S/4]; and a GQA decode through split-KV.  Graph-timed, each output
    first checked against the FP64 oracle on sampled rows of two (sequence,
    head) pairs of two sequences."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11939)
    mk = lambda *shape: torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    out = {}

    def measure(name, fn, o, checks, flop):
        o.fill_(float("nan"))
        torch.cuda.synchronize()   # the fill runs on the default stream
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        for qc, kc, vc, oc, causal in checks():
            err, _ = check_rows(torch, orc, qc, kc, vc, oc, causal, [(0, 0), (0, h - 1)])
            if not orc.check_acceptance_tolerance(err):
                raise SystemExit(f"api report: {name} check failed: {err}")
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream))
        print(f"# {name}: {us:.1f} us, {flop / us / 1e6:.1f} TFLOP/s", file=sys.stderr, flush=True)
        return dict(us=round(us, 2), tflops=round(flop / us / 1e6, 1))

    q, k, v = mk(b, s, h, 128), mk(b, s, kvh, 128), mk(b, s, kvh, 128)
    o = torch.empty_like(q)
    grp = h // kvh
    res = {"workload": f"B{b} H{h} KV heads {kvh} Sq=Sk={s} D128 BF16, LSE off"}
    for causal in (False, True):
        fn = lambda: runner.call_gqa(q, k, v, o, None, causal, 0, stream=stream.cuda_stream)
        checks = lambda: [(q[i:i + 1], k[i:i + 1].repeat_interleave(grp, dim=2),
                           v[i:i + 1].repeat_interleave(grp, dim=2), o[i:i + 1], causal) for i in (0, b - 1)]
        res["causal" if causal else "dense"] = measure(f"gqa causal={causal}", fn, o, checks,
                                                       flops(b, h, s, s, causal))
    out["gqa"] = res
    del q, k, v, o

    lens = np.random.default_rng(11939).integers(s // 4, 7 * s // 4 + 1, size=b)
    cu_h = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    total, maxlen = int(cu_h[-1]), int(lens.max())
    cu = torch.from_numpy(cu_h).cuda()
    q, k, v = mk(total, h, 128), mk(total, h, 128), mk(total, h, 128)
    o = torch.empty_like(q)
    res = {"workload": f"{b} sequences, lengths {int(lens.min())}..{maxlen} (seeded), {total} tokens, "
                       f"H{h} D128 BF16, LSE off"}
    for causal in (False, True):
        fn = lambda: runner.call_varlen(q, k, v, o, None, cu, cu, maxlen, maxlen, causal, stream=stream.cuda_stream)
        sel = (0, int(np.argmax(lens)))
        checks = lambda: [tuple(x[cu_h[i]:cu_h[i + 1]][None] for x in (q, k, v, o)) + (causal,) for i in sel]
        flop = sum(flops(1, h, int(n), int(n), causal) for n in lens)
        res["causal" if causal else "dense"] = measure(f"varlen causal={causal}", fn, o, checks, flop)
    out["varlen"] = res
    del q, k, v, o
    torch.cuda.empty_cache()

    # GQA decode through split-KV: one query per sequence against a long
    # cache; the query heads of a K/V head share its stream.  Reported as K+V
    # bandwidth (the bound).
    db, dh, dkvh, dsk = 4, 32, 8, 32768
    q, k, v = mk(db, 1, dh, 128), mk(db, dsk, dkvh, 128), mk(db, dsk, dkvh, 128)
    o = torch.empty_like(q)
    need = runner.splitkv_workspace_size(db, dh, 1, dsk, False, 0, kv_heads=dkvh)
    ws = torch.empty(max(need, 256), device="cuda", dtype=torch.uint8)
    fn = lambda: runner.call_splitkv(q, k, v, o, None, False, 0, workspace=ws, stream=stream.cuda_stream)
    o.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    grp = dh // dkvh
    for i in (0, db - 1):
        err, _ = check_rows(torch, orc, q[i:i + 1], k[i:i + 1].repeat_interleave(grp, dim=2),
                            v[i:i + 1].repeat_interleave(grp, dim=2), o[i:i + 1], False, [(0, 0), (0, dh - 1)])
        if not orc.check_acceptance_tolerance(err):
            raise SystemExit(f"api report: gqa decode check failed: {err}")
    us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
    kv_bytes = 2 * db * dsk * dkvh * 256
    splits = runner.splitkv_select(db, dh, 1, dsk, False, kv_heads=dkvh)
    print(f"# gqa decode (split-KV, {splits} chunks): {us:.1f} us, K+V {kv_bytes / us / 1e6:.2f} TB/s",
          file=sys.stderr, flush=True)
    out["gqa_decode"] = {"workload": f"B{db} H{dh} KV heads {dkvh} Sq=1 Sk={dsk} D128 BF16 dense, split-KV Auto",
                         "splits": splits, "us": round(us, 2), "kv_tbps": round(kv_bytes / us / 1e6, 2)}
    del q, k, v, o, ws
    torch.cuda.empty_cache()

    # Continuous-batching decode: packed sequences, one new query each, ragged
    # cache lengths; split-KV over the packed batch against the unsplit packed
    # forward.  Reported as K+V bandwidth.
    vb, vh, vkvh = 32, 32, 8
    klens = np.random.default_rng(4242).integers(1024, 32768 + 1, size=vb)
    cuk_h = np.concatenate([[0], np.cumsum(klens)]).astype(np.int32)
    cuq_h = np.arange(vb + 1, dtype=np.int32)
    tk, mk_len = int(cuk_h[-1]), int(klens.max())
    cuq, cuk = torch.from_numpy(cuq_h).cuda(), torch.from_numpy(cuk_h).cuda()
    q, k, v = mk(vb, vh, 128), mk(tk, vkvh, 128), mk(tk, vkvh, 128)
    o = torch.empty_like(q)
    need = runner.splitkv_varlen_workspace_size(vb, vh, vkvh, 1, mk_len, vb, tk, False)
    ws = torch.empty(max(need, 256), device="cuda", dtype=torch.uint8)
    splits = runner.splitkv_varlen_select(vb, vh, vkvh, 1, mk_len, vb, tk, False)
    kv_bytes = 2 * tk * vkvh * 256
    grp = vh // vkvh
    res = {"workload": f"{vb} sequences x 1 query, cache lengths {int(klens.min())}..{mk_len} (seeded), {tk} keys, "
                       f"H{vh} KV heads {vkvh} D128 BF16 dense", "splits": splits}
    fns = (("plain", lambda: runner.call_varlen(q, k, v, o, None, cuq, cuk, 1, mk_len, False,
                                                stream=stream.cuda_stream)),
           ("splitkv", lambda: runner.call_splitkv_varlen(q, k, v, o, None, cuq, cuk, 1, mk_len, False, 0,
                                                          workspace=ws, stream=stream.cuda_stream)))
    for name, fn in fns:
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        for i in (0, int(np.argmax(klens))):
            ks, ke = int(cuk_h[i]), int(cuk_h[i + 1])
            err, _ = check_rows(torch, orc, q[i:i + 1][None], k[ks:ke][None].repeat_interleave(grp, dim=2),
                                v[ks:ke][None].repeat_interleave(grp, dim=2), o[i:i + 1][None], False,
                                [(0, 0), (0, vh - 1)])
            if not orc.check_acceptance_tolerance(err):
                raise SystemExit(f"api report: varlen decode {name} check failed: {err}")
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
        res[name] = {"us": round(us, 2), "kv_tbps": round(kv_bytes / us / 1e6, 2)}
        print(f"# varlen decode {name}: {us:.1f} us, K+V {kv_bytes / us / 1e6:.2f} TB/s", file=sys.stderr, flush=True)
    res["speedup"] = round(res["plain"]["us"] / res["splitkv"]["us"], 2)

    # The same decode batch over paged K/V caches: 64-key pages in a random
    # order, Auto chunk count; checked like the packed run.
    ps = 64
    npg = [-(-int(n) // ps) for n in klens]
    perm = torch.randperm(sum(npg), generator=torch.Generator().manual_seed(5)).cuda()
    kc = torch.zeros((sum(npg), ps, vkvh, 128), device="cuda", dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    table = torch.zeros((vb, max(npg)), device="cuda", dtype=torch.int32)
    at = 0
    for i, n in enumerate(npg):
        ids = perm[at:at + n]
        at += n
        table[i, :n] = ids.to(torch.int32)
        ks, ke = int(cuk_h[i]), int(cuk_h[i + 1])
        for src, dst in ((k, kc), (v, vc)):
            pad = torch.zeros((n * ps, vkvh, 128), device="cuda", dtype=torch.bfloat16)
            pad[:ke - ks] = src[ks:ke]
            dst[ids] = pad.view(n, ps, vkvh, 128)
    seqlens = torch.from_numpy(klens.astype(np.int32)).cuda()
    pws = torch.empty(max(runner.splitkv_paged_workspace_size(vb, vh, vkvh, 1, mk_len, vb, tk, ps, max(npg), sum(npg)),
                          256), device="cuda", dtype=torch.uint8)
    fn = lambda: runner.call_splitkv_paged(q, kc, vc, o, None, cuq, seqlens, table, 1, mk_len, 0, workspace=pws,
                                           total_k=tk, stream=stream.cuda_stream)
    o.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    for i in (0, int(np.argmax(klens))):
        ks, ke = int(cuk_h[i]), int(cuk_h[i + 1])
        err, _ = check_rows(torch, orc, q[i:i + 1][None], k[ks:ke][None].repeat_interleave(grp, dim=2),
                            v[ks:ke][None].repeat_interleave(grp, dim=2), o[i:i + 1][None], False,
                            [(0, 0), (0, vh - 1)])
        if not orc.check_acceptance_tolerance(err):
            raise SystemExit(f"api report: paged decode check failed: {err}")
    us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SWEEP_SPIN_MS))
    res["paged"] = {"page_size": ps, "splits": runner.splitkv_paged_select(vb, vh, vkvh, 1, mk_len, vb, tk, ps,
                                                                            max(npg), sum(npg)),
                    "us": round(us, 2), "kv_tbps": round(kv_bytes / us / 1e6, 2)}
    print(f"# varlen decode paged ({ps}-key pages): {us:.1f} us, K+V {kv_bytes / us / 1e6:.2f} TB/s", file=sys.stderr,
          flush=True)
    out["varlen_decode"] = res
    del q, k, v, o, ws, kc, vc, pws
    torch.cuda.empty_cache()
    return out


_TELEMETRY = True


def _run(cmd, timeout=20, force=False):
    import subprocess
    if not (_TELEMETRY or force):
        return None
    try:
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        return r.stdout if r.returncode == 0 else None
    except (OSError, subprocess.SubprocessError):
        return None


def gpu_clocks():
    """Current clocks in MHz per domain ({"GFX_0": 2398, ..., "MEM_0": 2000}) from amd-smi, or None."""
    txt = _run(["amd-smi", "metric", "-c"])
    if not txt:
        return None
    clocks, domain = {}, None
    for ln in txt.splitlines():
        t = ln.strip()
        if t.endswith(":") and " " not in t:
            domain = t[:-1]
        elif t.startswith("CLK:") and domain and t.endswith("MHz"):
            try:
                clocks[domain] = int(float(t.split()[1]))
            except ValueError:
                pass
    return {d: c for d, c in clocks.items() if d.startswith(("GFX", "MEM"))} or None


def gpu_telemetry():
    """One amd-smi snapshot: GFX clock (mean / min / max over the XCDs, MHz),
    memory clock, power, temperatures and activity, or None."""
    txt = _run(["amd-smi", "metric", "-c", "-p", "-t", "-u", "--json"])
    if not txt:
        return None
    try:
        start = min(i for i in (txt.find("{"), txt.find("[")) if i >= 0)
        doc = json.loads(txt[start:])
    except ValueError:
        return None
    gpus = doc.get("gpu_data", doc) if isinstance(doc, dict) else doc
    if not isinstance(gpus, list) or not gpus or not isinstance(gpus[0], dict):
        return None
    g = gpus[0]
    out = {}
    clk = g.get("clock") or {}
    gfx = [d["clk"]["value"] for n, d in clk.items()
           if n.lower().startswith("gfx") and isinstance(d, dict) and isinstance(d.get("clk"), dict)
           and isinstance(d["clk"].get("value"), (int, float))]
    if gfx:
        out["gfx_mhz"] = dict(mean=round(statistics.mean(gfx)), min=min(gfx), max=max(gfx))
    mem = (clk.get("mem_0") or {}).get("clk") if isinstance(clk.get("mem_0"), dict) else None
    if isinstance(mem, dict) and isinstance(mem.get("value"), (int, float)):
        out["mem_mhz"] = mem["value"]

    def flat(x, path, sink):
        if isinstance(x, dict):
            if isinstance(x.get("value"), (int, float)):
                sink[path] = x["value"]
                return
            for key, val in x.items():
                flat(val, f"{path}.{key}" if path else key, sink)
        elif isinstance(x, (int, float)) and not isinstance(x, bool):
            sink[path] = x

    for sec in ("power", "temperature", "usage"):
        sink = {}
        flat(g.get(sec), "", sink)
        if sink:
            out[sec] = sink
    return out or None


def timed_with_telemetry(fn):
    """(fn(), amd-smi snapshots before and after it)."""
    before = gpu_telemetry()
    res = fn()
    return res, {"before": before, "after": gpu_telemetry()}


def loaded_telemetry(torch, fn, stream, launches=50, max_s=20.0):
    """One amd-smi snapshot (clocks, power, temperatures, activity) read from a
    child process while graphs of `launches` x fn replay back to back; the
    replays continue until the snapshot is taken (amd-smi's start-up time
    varies), at most `max_s` seconds."""
    import threading
    with torch.cuda.stream(stream):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(launches):
                fn()
    got = {}
    # amd-smi's activity figure averages over about a second: start it a
    # second into the replays so the window holds load only.
    reader = threading.Thread(target=lambda: (time.sleep(1.0), got.update(t=gpu_telemetry())))
    t_end = time.perf_counter() + max_s
    with torch.cuda.stream(stream):
        g.replay()
        reader.start()
        while reader.is_alive() and time.perf_counter() < t_end:
            g.replay()
            stream.synchronize()
    torch.cuda.synchronize()
    reader.join()
    del g
    return got.get("t")


def provenance(torch, lib_path):
    import hashlib
    h = lambda p: hashlib.sha256(Path(p).read_bytes()).hexdigest()
    src = ROOT / "flash-attention-v4-rocm_amd" / "csrc"
    srcs = sorted(src.glob("*")) + [ROOT / "include" / "fav4_bshd.h"]
    digest = hashlib.sha256()
    for p in srcs:
        digest.update(p.name.encode())
        digest.update(p.read_bytes())
    hipcc = _run(["hipcc", "--version"])
    prop = torch.cuda.get_device_properties(0)
    lib_sha = h(lib_path)
    manifest = None
    mpath = Path(lib_path).parent / "build-manifest.json"
    if mpath.exists():
        try:
            manifest = json.loads(mpath.read_text())
        except ValueError:
            manifest = {"error": "unreadable build-manifest.json"}
    lib_entry = ((manifest or {}).get("libraries") or {}).get(Path(lib_path).name) or {}
    return {"library": str(Path(lib_path).relative_to(ROOT)), "library_sha256": lib_sha,
            "sources_sha256": digest.hexdigest(),
            "build_manifest": manifest,
            "library_matches_manifest": (lib_entry.get("sha256") == lib_sha) if lib_entry else None,
            "hipcc": next((ln for ln in (hipcc or "").splitlines() if "HIP version" in ln), None),
            "torch": torch.__version__, "device": f"{prop.name} {prop.gcnArchName} {prop.multi_processor_count} CUs",
            "clocks_before": gpu_clocks()}


def read_traffic(lib_sha):
    """HBM bytes per dense headline launch from the committed counter summary,
    and whether those counters were taken on the library being timed."""
    if not TRAFFIC_FILE.exists():
        return None, None, None
    traffic = counters_sha = None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            traffic = int(float(line.split(":", 1)[1]))
        elif line.startswith("library_sha256:"):
            counters_sha = line.split(":", 1)[1].strip()
    return traffic, counters_sha, (counters_sha != lib_sha)


def headline(torch, orc, runner, args, b, h, s, stream, pairs, spin_ms=0.0, observations=None):
    """Sampled-row check, then graph timing of the dense and causal forward at
    B{b} H{h} S{s}, each with amd-smi snapshots around its timed region."""
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    out = {}
    for causal in ([False] if args.no_causal else [False, True]):
        fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        check = check_lse = None
        if not args.no_check:
            o.fill_(float("nan"))
            torch.cuda.synchronize()   # the fill runs on the default stream
            with torch.cuda.stream(stream):
                fn()
            torch.cuda.synchronize()
            check, _ = check_rows(torch, orc, q, k, v, o, causal, pairs)
            if not orc.check_acceptance_tolerance(check):
                raise SystemExit(f"sampled-row check failed (B{b} H{h} S{s} causal={causal}): {check}")
            # The same rows with the LSE written (benchmarks/bshd.py:147-156
            # checks every timed shape with and without it).
            lse = torch.full((b, h, s), float("nan"), device=q.device, dtype=torch.float32)
            o.fill_(float("nan"))
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                runner.call(q, k, v, o, lse, causal, args.config, stream=stream.cuda_stream)
            torch.cuda.synchronize()
            check_lse, _ = check_rows(torch, orc, q, k, v, o, causal, pairs, lse=lse)
            del lse
            if not orc.check_acceptance_tolerance(check_lse):
                raise SystemExit(f"sampled-row LSE check failed (B{b} H{h} S{s} causal={causal}): {check_lse}")
        samples, tel = timed_with_telemetry(
            lambda: time_graph(torch, fn, args.steps, args.warmup, observations or args.observations, stream,
                               spin_ms=spin_ms))
        flop = flops(b, h, s, s, causal)
        us = statistics.mean(samples)
        out[causal] = dict(us=us, median_us=statistics.median(samples), samples_us=samples,
                           tflops=flop / us / 1e6, flop=flop, check=check, check_lse=check_lse, telemetry=tel)
        print(f"# B{b} H{h} S{s} causal={causal}: {us:.1f} us/launch, {flop / us / 1e6:.1f} TFLOP/s "
              f"({flop / us / 1e6 / PEAK_BF16_TFLOPS * 100:.1f}% of peak) check={check} "
              f"lse_max_abs={None if check_lse is None else check_lse['lse_max_abs']}",
              file=sys.stderr, flush=True)
    return out, (q, k, v, o)


def main():
    args = parse_args()
    global _TELEMETRY
    _TELEMETRY = not args.no_telemetry
    if args.gpus != 1:
        print(json.dumps({"error": "this library runs on one GPU only; --gpus must be 1",
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
    if args.mfma_ceiling:
        mfma_ceiling(torch, runner, pkg, args)
        return

    b, h, s = args.batch, args.heads, args.seq
    prov = provenance(torch, pkg.LIB_PATH)
    stream = torch.cuda.Stream()
    pairs = [(0, 0), (b // 2, h // 2), (b - 1, h - 1)]
    results, (q, k, v, o) = headline(torch, orc, runner, args, b, h, s, stream, pairs)
    dense = results[False]
    # Clocks, power and temperatures while each headline kernel runs (the
    # snapshots around the timed regions land when the GPU is already idle).
    under_load = {}
    if _TELEMETRY:
        for causal in results:
            under_load["causal" if causal else "dense"] = loaded_telemetry(
                torch, lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream), stream)
    clk = ((under_load.get("dense") or {}).get("gfx_mhz") or {}).get("mean")
    # The CPU baseline times the oracle on slices of the same dense inputs.
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch, orc, q, k, v, args.cpu_seconds)

    cmp = None
    if not args.no_comparator:
        cmp = comparator(torch, orc, runner, q, k, v, o, stream, args, list(results))
    del q, k, v, o
    torch.cuda.empty_cache()
    skv = None if args.no_splitkv else splitkv_report(torch, orc, runner, args, stream)
    api = None if args.no_api else api_report(torch, orc, runner, args, stream)

    # Long-sequence sweep (B and H of the headline): each shape checked on
    # sampled rows, then graph-timed (2 observations) after an untimed spin-up.
    sweep = {}
    for n in ([] if args.no_sweep else [int(x) for x in args.sweep.split(",") if x]):
        res, bufs = headline(torch, orc, runner, args, b, h, n, stream, pairs, spin_ms=SWEEP_SPIN_MS,
                             observations=2)
        del bufs
        torch.cuda.empty_cache()
        for causal, r in res.items():
            sweep[f"S{n}_{'causal' if causal else 'dense'}"] = dict(
                us=round(r["us"], 2), tflops=round(r["tflops"], 1),
                frac_of_peak=round(r["tflops"] / PEAK_BF16_TFLOPS, 4), check=r["check"],
                check_lse=r["check_lse"], telemetry=r["telemetry"])

    traffic, counters_sha, stale = read_traffic(prov["library_sha256"])
    compulsory = 2 * b * h * 128 * (2 * s + 2 * s)
    roofline = dict(bound="mfma", achieved=round(dense["tflops"], 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                    frac=round(dense["tflops"] / PEAK_BF16_TFLOPS, 4), traffic=traffic,
                    traffic_library_sha256=counters_sha, traffic_stale=stale,
                    kernel="fav4::fwd_kernel (dense)", flop_per_launch=dense["flop"],
                    avg_launch_us=round(dense["us"], 3), compulsory_hbm_bytes=compulsory,
                    hbm_roofline_tflops=round(dense["flop"] / compulsory * HBM_TBPS, 1),
                    gfx_clock_mhz_under_load=clk, telemetry_under_load=under_load or None,
                    peak_at_loaded_clock=round(PEAK_BF16_TFLOPS * clk / 2400, 1) if clk else None,
                    frac_at_loaded_clock=round(dense["tflops"] / (PEAK_BF16_TFLOPS * clk / 2400), 4) if clk else None)
    line = {
        "metric": "fwd TFLOP/s + % BF16 MFMA peak, B32 H8 D128 S4096 dense & causal",
        "value": round(dense["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dense["us"] / 1000.0, 5),
        "median_us_per_step": round(dense["median_us"], 3),
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
                              median_us_per_launch=round(c["median_us"], 3),
                              frac_of_peak=round(c["tflops"] / PEAK_BF16_TFLOPS, 4),
                              samples_us=[round(x, 2) for x in c["samples_us"]], check=c["check"],
                              check_lse=c["check_lse"], telemetry=c["telemetry"])
    line["dense_samples_us"] = [round(x, 2) for x in dense["samples_us"]]
    line["dense_check"] = dense["check"]
    line["dense_check_lse"] = dense["check_lse"]
    line["dense_telemetry"] = dense["telemetry"]
    line["comparator"] = cmp
    line["splitkv"] = skv
    line["api"] = api
    prov["clocks_after"] = gpu_clocks()
    prov["host_cpu"] = cpu_info()
    line["provenance"] = prov
    if sweep:
        line["sweep"] = sweep
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
