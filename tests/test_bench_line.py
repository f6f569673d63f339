"""The benchmark's final stdout line (no GPU): it must stay short enough for a
reader that keeps only the tail of stdout, parse back as JSON, and carry the
keys the headline record needs (metric, value, roofline, cpu_baseline, the
causal figure and the sweep).  Built from a synthetic result set as large as
a full default run produces: every sweep shape, both masks, the comparator
and a CPU baseline with long host strings."""
import json

import bench

REQUIRED = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
            "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "causal", "sweep")


def _shape(us, flop, causal):
    err = dict(max_abs=0.00390625, rms_rel=0.0021, max_tolerance_ratio=0.31, lse_max_abs=None, finite=True)
    return dict(us=us, median_us=us * 0.999, tflops=flop / us / 1e6, flop=flop, check=err,
                check_lse=dict(err, lse_max_abs=4.76837158203125e-07), samples_us=[us] * 6)


def _results():
    b, h, s = 32, 8, 4096
    sweep = {}
    for n in [int(x) for x in bench.DEFAULT_SWEEP.split(",")] + [s]:
        for causal in (False, True):
            flop = bench.flops(b, h, n, n, causal)
            us = flop / 1.1e9 + 11.123456
            sweep[f"S{n}_{'causal' if causal else 'dense'}"] = dict(
                us=us, tflops=flop / us / 1e6, frac=flop / us / 1e6 / bench.PEAK_BF16_TFLOPS,
                roofline_frac=bench.roofline_floor_us(b, h, n, n, causal) / us, speedup=1.7234567)
    cpu = dict(value=0.01234567891, unit="TFLOP/s", cores=16, kind="port",
               sample="FP64 numpy oracle on 48 of 256 (b,h) slices of the dense B32 H8 S4096 D128 workload, "
                      "12.3 s, one slice per thread " + "x" * 300,
               fp32=dict(value=0.0456, unit="TFLOP/s", sample="FP32 ..."),
               cpu_model="AMD EPYC 9575F 64-Core Processor " + "y" * 200, sockets=2, cpuinfo={"a": "b" * 500})
    return dict(b=b, h=h, s=s, config=0, steps=20, warmup=5, lib_sha256="ab" * 32,
                detail="gpurun_out/bench_detail.json",
                dense=_shape(1885.7, bench.flops(b, h, s, s, False), False),
                causal=_shape(1068.1, bench.flops(b, h, s, s, True), True),
                clk_mhz=1843, socket_w=1387, traffic=1502123456, traffic_stale=False, cpu=cpu,
                comparator={"name": "torch SDPA flash (torch 2.10.0+rocm7.0) " + "z" * 100,
                            "dense": dict(speedup=1.72, sdpa_tflops=678.1, max_diff=0.00098),
                            "causal": dict(speedup=2.61, sdpa_tflops=395.2, max_diff=0.0156)},
                sweep=sweep)


def test_line_fits_and_round_trips():
    line = bench.make_line(_results())
    txt = bench.dump_line(line)
    assert len(txt.encode()) < bench.LINE_LIMIT, len(txt)
    assert "\n" not in txt
    back = json.loads(txt)
    for key in REQUIRED:
        assert key in back, key
    assert back["metric"] == bench.METRIC
    assert back["value"] == round(bench.flops(32, 8, 4096, 4096, False) / 1885.7 / 1e6, 2)
    assert abs(back["ms_per_step"] - 1.8857) < 1e-9
    r = back["roofline"]
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic", "traffic_stale", "avg_launch_us",
                "flop_per_launch", "compulsory_hbm_bytes", "gfx_mhz_loaded", "frac_at_loaded_clock",
                "socket_w_loaded", "energy_j_per_launch"):
        assert key in r, key
    assert abs(r["energy_j_per_launch"] - 1387 * 1885.7e-6) < 1e-4
    assert r["frac"] == round(r["achieved"] / r["peak"], 4)
    assert r["compulsory_hbm_bytes"] == 2 * 32 * 8 * 128 * 4 * 4096
    c = back["cpu_baseline"]
    for key in ("value", "unit", "cores", "kind", "sample", "fp32_value", "cpu_model", "sockets"):
        assert key in c, key
    assert back["causal"]["frac"] == round(back["causal"]["value"] / bench.PEAK_BF16_TFLOPS, 4)
    assert len(back["sweep"]) == 14
    assert len(back["sweep"]["S512_dense"]) == len(back["sweep_cols"])
    assert back["comparator"]["dense"][0] == 1.72


def test_line_without_optional_legs():
    res = _results()
    for key in ("causal", "cpu", "comparator", "sweep", "clk_mhz", "socket_w"):
        res.pop(key)
    back = json.loads(bench.dump_line(bench.make_line(res)))
    assert back["cpu_baseline"] is None
    assert back["roofline"]["frac_at_loaded_clock"] is None
    assert back["roofline"]["energy_j_per_launch"] is None
    assert "causal" not in back and "sweep" not in back


def test_roofline_floor():
    # S4096 dense is MFMA-bound, S512 causal HBM-bound (arithmetic intensity
    # below the ridge of ~315 FLOP/B).
    assert abs(bench.roofline_floor_us(32, 8, 4096, 4096, False) - 2.199023255552e12 / 2516.6e6) < 1e-6
    assert abs(bench.roofline_floor_us(32, 8, 512, 512, True) - 2 * 32 * 8 * 128 * 4 * 512 / 8e6) < 1e-6


def test_sweep_launch_counts():
    assert bench.sweep_launches(4096, 20, 5) == (20, 5)
    assert bench.sweep_launches(8192, 20, 5) == (20, 5)
    assert bench.sweep_launches(16384, 20, 5) == (6, 2)
    assert bench.sweep_launches(32768, 20, 5) == (3, 1)
    assert bench.ABBA.count("A") == bench.ABBA.count("B") == 6


def _alive(pid):
    """True if pid is a live (not zombie) process."""
    try:
        with open(f"/proc/{pid}/status") as f:
            state = [ln for ln in f if ln.startswith("State:")][0]
    except (OSError, IndexError):
        return False
    return "Z" not in state.split()[1]


def test_run_helper_output_and_timeout(tmp_path):
    import time
    assert bench._run(["echo", "ok"], force=True) == "ok\n"
    assert bench._run(["false"], force=True) is None
    assert bench._run(["/nonexistent/tool"], force=True) is None
    # A command that outlives its time-out, with a helper of its own: both are
    # killed, and _run returns None.
    marker = tmp_path / "helper.pid"
    t0 = time.monotonic()
    out = bench._run(["bash", "-c", f"sleep 37 & echo $! > {marker}; wait"], timeout=1.0, force=True)
    assert out is None
    assert time.monotonic() - t0 < 10
    pid = int(marker.read_text())
    deadline = time.monotonic() + 5
    while _alive(pid) and time.monotonic() < deadline:
        time.sleep(0.05)
    assert not _alive(pid)
