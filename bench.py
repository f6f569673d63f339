#!/usr/bin/env python3
"""Benchmark of the gfx950 attention forward at the headline shape.

Workload (one "step" = one fav4_bshd_forward launch over one batch):
B=32, H=8, Sq=Sk=4096, D=128, BF16 BSHD, Q/K/V iid N(0,1) (synthetic,
seeded), scale 1/sqrt(128), LSE off -- timed dense (the JSON ``value``) and
top-left causal (reported beside it).  Timing follows the reference harness,
benchmarks/bshd.py:34-51,163: a HIP graph of W launches is replayed as warmup,
then a graph of exactly K launches is replayed between two GPU events on the
launch stream; six such observations are taken and the mean is reported.
Before the first observation of every timed shape the warmup graph replays,
untimed, for 50 ms: the FP64 checks run on the CPU while the GPU idles, and
without the spin-up the first observation caught the clock's ramp back to its
loaded value (3% slow dense, 8% causal, where the other five agree).  The
FLOP convention is the reference's (bshd.py:169-170, README.md:59): useful
QK+PV only, dense 4*B*H*D*S^2, causal 4*B*H*D*S(S+1)/2.

Every timed shape is first checked against the FP64 oracle on the
reference's sampled rows (bshd.py:147-148) for three (b, h) pairs, with and
without the LSE output.

The long-sequence sweep (B and H of the headline, S in 512..32768, dense and
causal) times this library against torch's scaled_dot_product_attention (its
fused flash backend, else its memory-efficient one; never the unfused math
path) on the same device and inputs the way the reference times itself
against CK (bshd.py:151-166): both are graph-captured, and their observations
interleave in the order ABBA BAAB ABBA, six each.  The headline shape gets
the same comparison after its own dedicated timing.

The ``cpu_baseline`` leg times the FP64 oracle on this host's cores on a
bounded sample of (b, h) slices of the same dense workload (a baseline only).

Output: stdout ends with ONE short JSON line (the driver's record; kept well
under 4 KB), the same way the reference prints one summary line per shape
and keeps bulky records for its --output file (bshd.py:183-185).  The full
record (checks, telemetry, provenance and build manifest, every sample) goes
to the --detail file.  Progress lines go to stderr, prefixed with '#'.
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

METRIC = "fwd TFLOP/s + % BF16 MFMA peak, B32 H8 D128 S4096 dense & causal"
PEAK_BF16_TFLOPS = 2516.6      # MI355X dense BF16 MFMA: 256 CU x 4 SIMD x 1024 FLOP/clk x 2.4 GHz
HBM_TBPS = 8.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_fmha_fwd_dense_b32h8s4096.md"
SPIN_MS = 50.0                 # untimed spin-up before each timed shape (headline and sweep)
DEFAULT_SWEEP = "512,1024,2048,8192,16384,32768"   # bshd.py:195 plus the long-sequence configs
ABBA = "ABBABAABABBA"          # bshd.py:151-166: six observations of each side
LINE_LIMIT = 4096              # bytes of the final stdout line


def parse_args(argv=None):
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
    p.add_argument("--sweep", default=DEFAULT_SWEEP,
                   help="comma list of the long-sequence sweep's lengths (B and H as the headline; dense and causal)")
    p.add_argument("--no-sweep", action="store_true", help="skip the long-sequence sweep")
    p.add_argument("--no-comparator", action="store_true", help="skip the torch SDPA comparator")
    p.add_argument("--splitkv", action="store_true",
                   help="also time the split-KV entry point (B1 H8 Sq1024 Sk32768; B1 H1 S16384 causal)")
    p.add_argument("--api", action="store_true", help="also time the GQA / varlen / decode entry points")
    p.add_argument("--detail", default=str(ROOT / "gpurun_out" / "bench_detail.json"),
                   help="file for the full record (checks, telemetry, provenance, samples)")
    p.add_argument("--no-telemetry", action="store_true",
                   help="start no child processes (amd-smi clocks, hipcc version), e.g. under a profiler")
    p.add_argument("--mfma-ceiling", action="store_true",
                   help="MFMA-only ceiling: a probe kernel streaming BF16 MFMAs (32x32x16 and 16x16x32) at the "
                        "forward's occupancy, graph-timed with clock and power under load, beside the dense and "
                        "causal headline in the same process; prints one JSON line")
    p.add_argument("--pmc-pass", action="store_true",
                   help="profiling mode for counter runs: two eager launches per mask type, then a "
                        "plain 1 GiB device copy (HBM counter calibration); prints no JSON")
    return p.parse_args(argv)


def log(msg):
    print(f"# {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# FLOPs, bytes, inputs, checks
# ---------------------------------------------------------------------------
def flops(b, h, sq, sk, causal):
    """Useful QK+PV FLOPs, the reference's convention (benchmarks/bshd.py:169-170):
    4*B*H*128*Sq*Sk dense; top-left causal counts the keys each row sees,
    4*B*H*128*sum_{i<Sq} min(i+1, Sk)."""
    if not causal:
        return 4 * b * h * 128 * sq * sk
    full = min(sq, sk)
    return 4 * b * h * 128 * (full * (full + 1) // 2 + max(0, sq - sk) * sk)


def compulsory_bytes(b, h, sq, sk, lse=False):
    """HBM bytes every implementation must move: Q and O ([B,Sq,H,128] BF16),
    K and V ([B,Sk,H,128] BF16), and the FP32 LSE when written."""
    return 2 * b * h * 128 * (2 * sq + 2 * sk) + (4 * b * h * sq if lse else 0)


def roofline_floor_us(b, h, sq, sk, causal):
    """The shape's roofline time: max(MFMA time at the nominal peak, compulsory
    bytes at 8 TB/s), in microseconds."""
    return max(flops(b, h, sq, sk, causal) / (PEAK_BF16_TFLOPS * 1e6),
               compulsory_bytes(b, h, sq, sk) / (HBM_TBPS * 1e6))


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


def run_once(torch, fn, stream):
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()


def checked(torch, orc, runner, q, k, v, o, causal, config, stream, pairs, what):
    """Sampled-row FP64 checks of one shape, without and with the LSE output
    (benchmarks/bshd.py:147-156 checks every timed shape both ways).  Raises
    when either misses the acceptance bar; returns both error dicts."""
    b, s, h, _ = q.shape
    o.fill_(float("nan"))
    torch.cuda.synchronize()   # the fill runs on the default stream
    run_once(torch, lambda: runner.call(q, k, v, o, None, causal, config, stream=stream.cuda_stream), stream)
    e, _ = check_rows(torch, orc, q, k, v, o, causal, pairs)
    if not orc.check_acceptance_tolerance(e):
        raise SystemExit(f"sampled-row check failed ({what} causal={causal}): {e}")
    lse = torch.full((b, h, s), float("nan"), device=q.device, dtype=torch.float32)
    o.fill_(float("nan"))
    torch.cuda.synchronize()
    run_once(torch, lambda: runner.call(q, k, v, o, lse, causal, config, stream=stream.cuda_stream), stream)
    e_lse, _ = check_rows(torch, orc, q, k, v, o, causal, pairs, lse=lse)
    del lse
    if not orc.check_acceptance_tolerance(e_lse):
        raise SystemExit(f"sampled-row LSE check failed ({what} causal={causal}): {e_lse}")
    return e, e_lse


# ---------------------------------------------------------------------------
# Timing (benchmarks/bshd.py:34-51, 151-166)
# ---------------------------------------------------------------------------
def capture(torch, fn, steps, warmup, stream):
    """(warmup graph, timed graph) of `warmup` and `steps` launches of fn on `stream`."""
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
    torch.cuda.synchronize()
    return g_warm, g_timed


def spin(torch, g_warm, stream, spin_ms):
    """Replay the warmup graph (untimed) until spin_ms of wall time has passed,
    so short launches are timed at the loaded clock, not while the GPU ramps
    up from idle."""
    t_end = time.perf_counter() + spin_ms / 1000.0
    while time.perf_counter() < t_end:
        with torch.cuda.stream(stream):
            g_warm.replay()
        torch.cuda.synchronize()


def observe(torch, graphs, steps, stream):
    """One observation: replay the warmup graph, then the timed graph between
    two events on `stream`; microseconds per launch."""
    g_warm, g_timed = graphs
    with torch.cuda.stream(stream):
        g_warm.replay()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g_timed.replay()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / steps


def time_graph(torch, fn, steps, warmup, observations, stream, spin_ms=0.0):
    """Per-launch microseconds of `observations` graph observations of fn."""
    graphs = capture(torch, fn, steps, warmup, stream)
    if spin_ms > 0:
        spin(torch, graphs[0], stream, spin_ms)
    samples = [observe(torch, graphs, steps, stream) for _ in range(observations)]
    del graphs
    torch.cuda.synchronize()
    return samples


def time_interleaved(torch, fa, fb, steps, warmup, stream, spin_ms=0.0, order=ABBA):
    """Graph-timed A and B with their observations interleaved in `order`
    (the reference's ABBA BAAB ABBA against CK, bshd.py:151-166)."""
    ga = capture(torch, fa, steps, warmup, stream)
    gb = capture(torch, fb, steps, warmup, stream)
    if spin_ms > 0:
        spin(torch, ga[0], stream, spin_ms / 2)
        spin(torch, gb[0], stream, spin_ms / 2)
    out = {"A": [], "B": []}
    for who in order:
        out[who].append(observe(torch, ga if who == "A" else gb, steps, stream))
    del ga, gb
    torch.cuda.synchronize()
    return out["A"], out["B"]


def sweep_launches(s, steps, warmup):
    """Launches per timed / warmup graph at sequence length s: the reference's
    20 / 5 up to S8192; fewer for the longest shapes (one S32768 dense launch
    takes about 0.12 s), so the interleaved comparison stays within a minute."""
    if s >= 32768:
        return min(steps, 3), min(warmup, 1)
    if s >= 16384:
        return min(steps, 6), min(warmup, 2)
    return steps, warmup


# ---------------------------------------------------------------------------
# Comparator: torch SDPA on the same device
# ---------------------------------------------------------------------------
def sdpa_backend(torch):
    """The first fused SDPA backend that runs here (flash, else
    memory-efficient), as (name, backend enum), or None."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    x = torch.zeros((1, 1, 256, 128), device="cuda", dtype=torch.bfloat16)
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([be]):
                F.scaled_dot_product_attention(x, x, x, scale=1.0 / math.sqrt(128))
            torch.cuda.synchronize()
            return name, be
        except RuntimeError:
            continue
    return None


class Sdpa:
    """torch SDPA over contiguous BHSD copies of Q/K/V (its preferred layout;
    the copies are not timed)."""

    def __init__(self, torch, backend, q, k, v):
        import torch.nn.functional as F
        from torch.nn.attention import sdpa_kernel
        self.F, self.sdpa_kernel, self.backend = F, sdpa_kernel, backend
        self.qh, self.kh, self.vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
        self.out = None

    def __call__(self, causal):
        with self.sdpa_kernel([self.backend[1]]):
            self.out = self.F.scaled_dot_product_attention(self.qh, self.kh, self.vh, is_causal=causal,
                                                           scale=1.0 / math.sqrt(128))

    def max_diff(self, torch, o, rows):
        """Largest |SDPA - ours| over the sampled rows (BSHD)."""
        rt = torch.from_numpy(rows).to(o.device)
        theirs = self.out.index_select(2, rt).transpose(1, 2).float()
        return (theirs - o.index_select(1, rt).float()).abs().max().item()


def compare(torch, orc, runner, sdpa, q, k, v, o, causal, config, stream, steps, warmup, spin_ms):
    """Ours (A) against SDPA (B), graph-timed and interleaved; plus the largest
    output difference on the sampled rows."""
    ours = lambda: runner.call(q, k, v, o, None, causal, config, stream=stream.cuda_stream)
    theirs = lambda: sdpa(causal)
    run_once(torch, theirs, stream)   # lazy init outside the capture
    a, bs = time_interleaved(torch, ours, theirs, steps, warmup, stream, spin_ms=spin_ms)
    run_once(torch, ours, stream)
    run_once(torch, theirs, stream)
    diff = sdpa.max_diff(torch, o, orc.sample_rows(q.shape[1]))
    return a, bs, diff


# ---------------------------------------------------------------------------
# CPU baseline
# ---------------------------------------------------------------------------
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
                sample=f"FP64 numpy oracle on {done} of {len(pairs)} (b,h) slices of the dense B{b} H{h} S{s} "
                       f"D{d} workload, {elapsed:.1f} s, one slice per thread",
                slices=done, seconds=round(elapsed, 2),
                extrapolated_whole_job_s=round(elapsed * len(pairs) / done, 1),
                fp32=dict(value=round(flop1 * done32 / elapsed32 / 1e12, 4), unit="TFLOP/s",
                          sample=f"FP32 numpy textbook attention, {done32} slices in {elapsed32:.1f} s"),
                threads_note=f"single-threaded BLAS; {affinity} cores in the affinity set, threads capped by "
                             f"OMP_NUM_THREADS={os.environ.get('OMP_NUM_THREADS', 'unset')}",
                cpu_model=host.get("model"), bios_model=host.get("bios_model"), sockets=host.get("sockets"),
                affinity_cores=affinity, cpuinfo=host.get("cpuinfo"))


# ---------------------------------------------------------------------------
# Opt-in reports of the other entry points (split-KV, GQA, varlen, decode)
# ---------------------------------------------------------------------------
def splitkv_report(torch, orc, runner, args, stream):
    """Few (b, h, q tile) items and long keys: the single-pass forward against the
    split-KV forward (Auto chunk count), both graph-timed, each output checked on
    sampled rows first."""
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
            torch.cuda.synchronize()
            run_once(torch, fn, stream)
            err, _ = check_rows(torch, orc, q, k, v, o, causal, [(0, 0), (0, h - 1)])
            if not orc.check_acceptance_tolerance(err):
                raise SystemExit(f"split-KV report: {name} check failed ({label}): {err}")
            us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SPIN_MS))
            res[name] = dict(us=round(us, 2), tflops=round(flop / us / 1e6, 1))
        res["speedup"] = round(res["plain"]["us"] / res["splitkv"]["us"], 2)
        out[label] = res
        log(f"splitkv B{b} H{h} {sq}x{sk} causal={causal}: plain {res['plain']['tflops']} TFLOP/s, "
            f"split-KV ({splits} chunks) {res['splitkv']['tflops']} TFLOP/s, x{res['speedup']}")
        del q, k, v, o, ws
    torch.cuda.empty_cache()
    return out


def api_report(torch, orc, runner, args, stream, b=32, h=8, s=4096, kvh=2):
    """The GQA and varlen entry points at the headline token count (B*S rows,
    H8), and a GQA decode through split-KV; graph-timed, each output first
    checked against the FP64 oracle on sampled rows."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11939)
    mk = lambda *shape: torch.randn(shape, device="cuda", dtype=torch.float32, generator=g).to(torch.bfloat16)
    out = {}

    def measure(name, fn, o, checks, flop):
        o.fill_(float("nan"))
        torch.cuda.synchronize()
        run_once(torch, fn, stream)
        for qc, kc, vc, oc, causal in checks():
            err, _ = check_rows(torch, orc, qc, kc, vc, oc, causal, [(0, 0), (0, h - 1)])
            if not orc.check_acceptance_tolerance(err):
                raise SystemExit(f"api report: {name} check failed: {err}")
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream))
        log(f"{name}: {us:.1f} us, {flop / us / 1e6:.1f} TFLOP/s")
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
    run_once(torch, fn, stream)
    grp = dh // dkvh
    for i in (0, db - 1):
        err, _ = check_rows(torch, orc, q[i:i + 1], k[i:i + 1].repeat_interleave(grp, dim=2),
                            v[i:i + 1].repeat_interleave(grp, dim=2), o[i:i + 1], False, [(0, 0), (0, dh - 1)])
        if not orc.check_acceptance_tolerance(err):
            raise SystemExit(f"api report: gqa decode check failed: {err}")
    us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SPIN_MS))
    kv_bytes = 2 * db * dsk * dkvh * 256
    splits = runner.splitkv_select(db, dh, 1, dsk, False, kv_heads=dkvh)
    log(f"gqa decode (split-KV, {splits} chunks): {us:.1f} us, K+V {kv_bytes / us / 1e6:.2f} TB/s")
    out["gqa_decode"] = {"workload": f"B{db} H{dh} KV heads {dkvh} Sq=1 Sk={dsk} D128 BF16 dense, split-KV Auto",
                         "splits": splits, "us": round(us, 2), "kv_tbps": round(kv_bytes / us / 1e6, 2)}
    del q, k, v, o, ws
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# Telemetry and provenance
# ---------------------------------------------------------------------------
_TELEMETRY = True


def _run(cmd, timeout=20, force=False):
    """stdout of cmd, or None.  The child runs in its own session; on a
    time-out its whole process group (helpers it started included) is
    killed and reaped, so nothing it started outlives the benchmark."""
    import signal
    import subprocess
    if not (_TELEMETRY or force):
        return None
    try:
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                                start_new_session=True)
    except OSError:
        return None
    try:
        out, _ = proc.communicate(timeout=timeout)
    except subprocess.TimeoutExpired:
        try:
            os.killpg(proc.pid, signal.SIGKILL)
        except OSError:
            pass
        proc.communicate()
        return None
    return out if proc.returncode == 0 else None


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
            "host_cpu": cpu_info()}


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


# ---------------------------------------------------------------------------
# The driver's line
# ---------------------------------------------------------------------------
def _r(x, n):
    return None if x is None else round(x, n)


def make_line(res: dict) -> dict:
    """The final stdout line from the collected results (pure: no GPU, no I/O).

    `res` keys: b, h, s, config, steps, warmup, dense / causal (us,
    median_us, tflops, flop, check, check_lse), clk_mhz, traffic,
    traffic_stale, cpu (cpu_baseline dict or None), comparator (per mask:
    speedup, sdpa_tflops, max_diff), sweep (name -> us, tflops, frac,
    roofline_frac, speedup), detail (path), lib_sha256."""
    b, h, s = res["b"], res["h"], res["s"]
    dense = res["dense"]
    clk = res.get("clk_mhz")
    watts = res.get("socket_w")
    compulsory = compulsory_bytes(b, h, s, s)
    frac = dense["tflops"] / PEAK_BF16_TFLOPS
    roofline = dict(bound="mfma", achieved=_r(dense["tflops"], 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                    frac=round(frac, 4), traffic=res.get("traffic"), traffic_stale=res.get("traffic_stale"),
                    kernel="fav4::fwd_kernel (dense)", avg_launch_us=_r(dense["us"], 3),
                    flop_per_launch=dense["flop"], compulsory_hbm_bytes=compulsory,
                    gfx_mhz_loaded=clk,
                    frac_at_loaded_clock=_r(dense["tflops"] / (PEAK_BF16_TFLOPS * clk / 2400), 4) if clk else None,
                    socket_w_loaded=watts,
                    energy_j_per_launch=_r(watts * dense["us"] * 1e-6, 4) if watts else None)
    cpu = res.get("cpu")
    cpu_line = None
    if cpu:
        cpu_line = dict(value=_r(cpu["value"], 5), unit=cpu["unit"], cores=cpu["cores"], kind=cpu["kind"],
                        sample=cpu["sample"][:240], fp32_value=(cpu.get("fp32") or {}).get("value"),
                        cpu_model=(cpu.get("cpu_model") or "")[:80] or None, sockets=cpu.get("sockets"))
    chk = lambda r: None if r.get("check") is None else [
        _r(r["check"]["max_abs"], 5), _r((r.get("check_lse") or {}).get("lse_max_abs"), 7)]
    line = {
        "metric": METRIC,
        "value": _r(dense["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": res["warmup"],
        "ms_per_step": _r(dense["us"] / 1000.0, 5),
        "median_us_per_step": _r(dense["median_us"], 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) BF16 Q/K/V generated on the GPU)",
        "config": {"workload": f"FMHA fwd BSHD B{b} H{h} Sq=Sk={s} D128 BF16, scale 1/sqrt(128), LSE off",
                   "global_batch": b, "seq_len": s, "heads": h, "head_dim": 128, "config_id": res["config"],
                   "parallelism": "single GPU"},
        "frac_of_peak_dense": round(frac, 4),
        "roofline": roofline,
        "cpu_baseline": cpu_line,
    }
    c = res.get("causal")
    if c:
        line["causal"] = dict(value=_r(c["tflops"], 2), us=_r(c["us"], 3),
                              frac=round(c["tflops"] / PEAK_BF16_TFLOPS, 4))
    line["checks_max_abs_lse"] = {"dense": chk(dense), **({"causal": chk(c)} if c else {})}
    cmp = res.get("comparator")
    if cmp:
        line["comparator"] = {"name": cmp.get("name", "")[:60], **{
            m: [v["speedup"], v["sdpa_tflops"], v["max_diff"]] for m, v in cmp.items() if isinstance(v, dict)}}
    sw = res.get("sweep")
    if sw:
        line["sweep_cols"] = ["us", "tflops", "frac_of_peak", "frac_of_roofline", "speedup_vs_sdpa"]
        line["sweep"] = {name: [_r(r["us"], 2), _r(r["tflops"], 1), _r(r["frac"], 4), _r(r["roofline_frac"], 4),
                                _r(r.get("speedup"), 3)] for name, r in sw.items()}
    line["library_sha256"] = (res.get("lib_sha256") or "")[:16]
    line["detail"] = res.get("detail")
    return line


def dump_line(line: dict) -> str:
    txt = json.dumps(line, separators=(",", ":"))
    if len(txt.encode()) >= LINE_LIMIT:
        raise SystemExit(f"bench line is {len(txt.encode())} bytes (limit {LINE_LIMIT})")
    return txt


# ---------------------------------------------------------------------------
# Special modes
# ---------------------------------------------------------------------------
def pmc_pass(torch, runner, args):
    """Eager launches for rocprofv3 --pmc runs (no graphs, one dispatch per launch)."""
    b, h, s = args.batch, args.heads, args.seq
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    for causal in ([False] if args.no_causal else [False, True]):
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
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SPIN_MS))
        flop = cus * 8 * iters * 1048576
        res[name] = dict(us=round(us, 2), tflops=round(flop / us / 1e6, 1),
                         frac_of_peak=round(flop / us / 1e6 / PEAK_BF16_TFLOPS, 4),
                         telemetry_under_load=loaded_telemetry(torch, fn, stream) if _TELEMETRY else None)
        log(f"{name}: {us:.1f} us, {flop / us / 1e6:.1f} TFLOP/s")
    b, h, s = args.batch, args.heads, args.seq
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    for causal in (False, True):
        fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        us = statistics.mean(time_graph(torch, fn, args.steps, args.warmup, 3, stream, spin_ms=SPIN_MS))
        tflops = flops(b, h, s, s, causal) / us / 1e6
        res["fwd_causal" if causal else "fwd_dense"] = dict(
            us=round(us, 2), tflops=round(tflops, 1), frac_of_peak=round(tflops / PEAK_BF16_TFLOPS, 4),
            telemetry_under_load=loaded_telemetry(torch, fn, stream) if _TELEMETRY else None)
        log(f"B{b} H{h} S{s} causal={causal}: {us:.1f} us, {tflops:.1f} TFLOP/s")
    res["fwd_dense_of_ceiling"] = round(res["fwd_dense"]["tflops"] / res["mfma_32x32x16"]["tflops"], 4)
    print(json.dumps({"mode": "mfma_ceiling", "workload": f"B{b} H{h} Sq=Sk={s} D128 BF16, LSE off, config "
                      f"{args.config}", "cus": cus, "iters_per_wave": iters, **res}), flush=True)


# ---------------------------------------------------------------------------
# Main
# ---------------------------------------------------------------------------
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
    masks = [False] if args.no_causal else [False, True]
    name = lambda n, causal: f"S{n}_{'causal' if causal else 'dense'}"
    detail = {"args": vars(args), "provenance": prov, "headline": {}, "sweep": {}}
    res = dict(b=b, h=h, s=s, config=args.config, steps=args.steps, warmup=args.warmup, lib_sha256=
               prov["library_sha256"], detail=os.path.relpath(args.detail, ROOT))

    # Headline: checks, then dedicated graph timing (6 observations).
    q, k, v = make_inputs(torch, b, h, s)
    o = torch.empty_like(q)
    for causal in masks:
        e = e_lse = None
        if not args.no_check:
            e, e_lse = checked(torch, orc, runner, q, k, v, o, causal, args.config, stream, pairs, f"B{b} H{h} S{s}")
        fn = lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream)
        samples = time_graph(torch, fn, args.steps, args.warmup, args.observations, stream, spin_ms=SPIN_MS)
        flop = flops(b, h, s, s, causal)
        us = statistics.mean(samples)
        r = dict(us=us, median_us=statistics.median(samples), tflops=flop / us / 1e6, flop=flop, check=e,
                 check_lse=e_lse, samples_us=samples)
        res["causal" if causal else "dense"] = r
        detail["headline"][name(s, causal)] = r
        log(f"B{b} H{h} S{s} causal={causal}: {us:.1f} us/launch, {r['tflops']:.1f} TFLOP/s "
            f"({r['tflops'] / PEAK_BF16_TFLOPS * 100:.1f}% of peak) check={e}")

    # Clocks, power and temperatures while each headline kernel runs.
    if _TELEMETRY:
        under = {}
        for causal in masks:
            under[name(s, causal)] = loaded_telemetry(
                torch, lambda: runner.call(q, k, v, o, None, causal, args.config, stream=stream.cuda_stream), stream)
        detail["telemetry_under_load"] = under
        loaded = under.get(name(s, False)) or {}
        res["clk_mhz"] = (loaded.get("gfx_mhz") or {}).get("mean")
        res["socket_w"] = next((v for k, v in (loaded.get("power") or {}).items() if "socket" in k), None)

    res["cpu"] = None if args.no_cpu_baseline else cpu_baseline(torch, orc, q, k, v, args.cpu_seconds)
    detail["cpu_baseline"] = res["cpu"]
    if res["cpu"]:
        log(f"cpu baseline: {res['cpu']['value']:.5f} TFLOP/s FP64 on {res['cpu']['cores']} threads")

    backend = None if args.no_comparator else sdpa_backend(torch)
    sweep = {}
    if backend:
        res["comparator"] = {"name": f"torch SDPA {backend[0]} (torch {torch.__version__})"}
        sdpa = Sdpa(torch, backend, q, k, v)
        for causal in masks:
            a, bs, diff = compare(torch, orc, runner, sdpa, q, k, v, o, causal, args.config, stream, args.steps,
                                  args.warmup, 0.0)
            flop = flops(b, h, s, s, causal)
            cm = dict(speedup=round(statistics.mean(bs) / statistics.mean(a), 3),
                      sdpa_tflops=round(flop / statistics.mean(bs) / 1e6, 1), max_diff=round(diff, 5))
            res["comparator"]["causal" if causal else "dense"] = cm
            detail["headline"][name(s, causal)]["comparator"] = dict(cm, ours_us=a, sdpa_us=bs, order=ABBA)
            log(f"comparator S{s} causal={causal}: SDPA {cm['sdpa_tflops']} TFLOP/s, ours (interleaved) "
                f"{flop / statistics.mean(a) / 1e6:.1f}, speedup {cm['speedup']}, max|diff| {diff:.4f}")
        del sdpa
    for causal in masks:
        r = res["causal" if causal else "dense"]
        sweep[name(s, causal)] = dict(us=r["us"], tflops=r["tflops"], frac=r["tflops"] / PEAK_BF16_TFLOPS,
                                      roofline_frac=roofline_floor_us(b, h, s, s, causal) / r["us"],
                                      speedup=(res.get("comparator") or {}).get(
                                          "causal" if causal else "dense", {}).get("speedup"))
    del q, k, v, o
    torch.cuda.empty_cache()

    # Long-sequence sweep: each shape checked on sampled rows, then timed
    # against SDPA (interleaved graphs) or alone when no comparator runs.
    for n in ([] if args.no_sweep else [int(x) for x in args.sweep.split(",") if x]):
        if n == s:
            continue
        steps, warmup = sweep_launches(n, args.steps, args.warmup)
        q, k, v = make_inputs(torch, b, h, n)
        o = torch.empty_like(q)
        sdpa = Sdpa(torch, backend, q, k, v) if backend else None
        for causal in masks:
            e = e_lse = None
            if not args.no_check:
                e, e_lse = checked(torch, orc, runner, q, k, v, o, causal, args.config, stream, pairs,
                                   f"B{b} H{h} S{n}")
            flop = flops(b, h, n, n, causal)
            rec = dict(steps=steps, warmup=warmup, check=e, check_lse=e_lse)
            if sdpa:
                a, bs, diff = compare(torch, orc, runner, sdpa, q, k, v, o, causal, args.config, stream, steps,
                                      warmup, SPIN_MS)
                rec.update(ours_us=a, sdpa_us=bs, order=ABBA, max_diff=diff,
                           speedup=statistics.mean(bs) / statistics.mean(a),
                           sdpa_tflops=flop / statistics.mean(bs) / 1e6)
            else:
                a = time_graph(torch, lambda: runner.call(q, k, v, o, None, causal, args.config,
                                                          stream=stream.cuda_stream),
                               steps, warmup, args.observations, stream, spin_ms=SPIN_MS)
                rec.update(ours_us=a)
            us = statistics.mean(a)
            rec.update(us=us, tflops=flop / us / 1e6, frac=flop / us / 1e6 / PEAK_BF16_TFLOPS,
                       roofline_frac=roofline_floor_us(b, h, n, n, causal) / us)
            sweep[name(n, causal)] = rec
            detail["sweep"][name(n, causal)] = rec
            log(f"B{b} H{h} S{n} causal={causal}: {us:.1f} us, {rec['tflops']:.1f} TFLOP/s "
                f"({rec['frac'] * 100:.1f}% of peak, {rec['roofline_frac'] * 100:.1f}% of roofline)"
                + (f", SDPA x{rec['speedup']:.3f}, max|diff| {rec['max_diff']:.4f}" if sdpa else "")
                + f", check max-abs {None if e is None else round(e['max_abs'], 5)}")
        del q, k, v, o, sdpa
        torch.cuda.empty_cache()
    res["sweep"] = dict(sorted(sweep.items(), key=lambda kv: (int(kv[0][1:].split("_")[0]), kv[0])))

    if args.splitkv:
        detail["splitkv"] = splitkv_report(torch, orc, runner, args, stream)
    if args.api:
        detail["api"] = api_report(torch, orc, runner, args, stream)

    traffic, counters_sha, stale = read_traffic(prov["library_sha256"])
    res.update(traffic=traffic, traffic_stale=stale)
    detail["traffic"] = dict(bytes_per_launch=traffic, counters_library_sha256=counters_sha, stale=stale)
    line = make_line(res)
    detail["line"] = line
    Path(args.detail).parent.mkdir(parents=True, exist_ok=True)
    Path(args.detail).write_text(json.dumps(detail, indent=1, default=str))
    log(f"full record written to {args.detail}")
    print(dump_line(line), flush=True)


if __name__ == "__main__":
    main()
