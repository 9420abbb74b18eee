"""Benchmark of the decode hot path on one MI355X.

Headline (BASELINE.json metric, configs[1]): single-token Q4_K matvec at the
Llama FFN-up shape 14336 x 4096 in GB/s and as a fraction of the 8 TB/s HBM
peak.  A "step" is one matvec over one resident weight; 16 weight copies
(528 MB, above the 256 MB Infinity Cache) are rotated so HBM, not MALL,
serves them.  Inputs are synthetic (seeded counter-based generator) and
already resident in HBM when the timed region starts.

Prints ONE JSON line.  `roofline` comes from per-launch HIP events on the
library's stream; `cpu_baseline` times the AVX2 restatement of soso's CPU
kernels (oracle/) on the host cores for a bounded sample.  Other configs of
BASELINE.json are reported under "configs" (they are parity cases, not the
headline).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0
Q4K, Q8, Q6K, F32 = 3, 2, 13, 1
ROW_BYTES = {Q4K: lambda c: c // 256 * 144, Q8: lambda c: c // 32 * 36, Q6K: lambda c: c // 256 * 210}


def algo_bytes(dtype, rows, cols):
    """Algorithmic bytes of one matvec: weights + x + y, each moved once."""
    return rows * ROW_BYTES[dtype](cols) + 4 * cols + 4 * rows


def _capture(g, body):
    """Captures body() into a graph; the capture is always closed."""
    g.graph_begin()
    err = None
    try:
        body()
    except Exception as e:  # noqa: BLE001
        err = e
    gid = g.graph_end()
    if err is not None:
        g.graph_destroy(gid)
        raise err
    return gid


def time_matvec(g, dtype, rows, cols, copies, steps, warmup, seed=1):
    """Rotating resident copies; returns (ms_per_step_wall, ms_per_step_events, ms_kernel_mean)."""
    keys = [f"bench.{dtype}.{rows}x{cols}.{i}" for i in range(copies)]
    for i, k in enumerate(keys):
        g.weight_synth(k, dtype, rows, cols, seed, 1000 + i)
    x = g.dev_alloc(cols * 4)
    y = g.dev_alloc(rows * 4)
    g.synth_normal(x, cols, 1.0, seed, 7)
    try:
        for i in range(warmup):
            g.matvec_dev(keys[i % copies], x, y)
        g.sync()
        # graph of the timed steps: back-to-back launches with no host in between
        gid = _capture(g, lambda: [g.matvec_dev(keys[i % copies], x, y) for i in range(steps)])
        g.graph_launch(gid)  # first replay warms the graph itself
        g.sync()
        t0 = time.perf_counter()
        g.event_record(0)
        g.graph_launch(gid)
        g.event_record(1)
        g.sync()
        t1 = time.perf_counter()
        ms_wall = (t1 - t0) * 1e3 / steps
        ms_ev = g.event_elapsed(0, 1) / steps
        g.graph_destroy(gid)
        # per-launch kernel duration: HIP events around every launch, issued
        # while the GPU works through a queued backlog so it never waits for
        # the host; gaps between consecutive launches are reported too.
        n = min(steps, 2000)
        for i in range(min(400, 4 * n)):
            g.matvec_dev(keys[i % copies], x, y)
        for i in range(n):
            g.event_record(2 + 2 * i)
            g.matvec_dev(keys[i % copies], x, y)
            g.event_record(3 + 2 * i)
        g.sync()
        durs = [g.event_elapsed(2 + 2 * i, 3 + 2 * i) for i in range(n)]
        gaps = [g.event_elapsed(3 + 2 * i, 4 + 2 * i) for i in range(n - 1)]
        ms_kernel = sum(durs) / n
        time_matvec.last_gap_us = 1e3 * sum(gaps) / max(1, len(gaps))
        return ms_wall, ms_ev, ms_kernel
    finally:
        g.sync()
        g.dev_free(x)
        g.dev_free(y)
        for k in keys:
            g.weight_drop(k)


def copy_calibration(g, nbytes=512 << 20, reps=20):
    """A plain device-to-device copy of known size, for scaling rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters (run under --pmc)."""
    a, b = g.dev_alloc(nbytes), g.dev_alloc(nbytes)
    try:
        for _ in range(reps):
            g.d2d(b, a, nbytes)
        g.sync()
    finally:
        g.dev_free(a)
        g.dev_free(b)
    print(json.dumps({"copy_calibration_bytes": nbytes, "reps": reps}), flush=True)


def cpu_baseline(dtype, rows, cols, seconds, threads):
    """The AVX2+FMA restatement of soso's CPU matvec, contiguous row strips
    over `threads` host threads (HostPool), on a bounded sample."""
    from oracle import oracle as orc
    copies = 4  # 132 MB of Q4_K: above the host's last-level cache
    ws = [orc.synth(dtype, rows, cols, 1, 1000 + i) for i in range(copies)]
    x = orc.normal(cols, 1.0, 1, 7)
    orc.matvec(dtype, ws[0], rows, cols, x, threads=threads, avx2=True)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        orc.matvec(dtype, ws[n % copies], rows, cols, x, threads=threads, avx2=True)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return algo_bytes(dtype, rows, cols) / dt / 1e9, n, dt * 1e3


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/), if recorded."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        return json.load(open(p)).get(name)
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-threads", type=int, default=16)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="only the headline config")
    ap.add_argument("--copy-calibration", action="store_true", help="only run a 512 MiB D2D copy (PMC scaling)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the multi-GPU sharding is described in DESIGN.md, not run.", file=sys.stderr)
        sys.exit(2)

    from soso_amd.dispatch import HipGpu
    g = HipGpu(0)
    if args.copy_calibration:
        copy_calibration(g)
        g.close()
        return
    rows, cols = 14336, 4096
    nbytes = algo_bytes(Q4K, rows, cols)
    ms_wall, ms_ev, ms_k = time_matvec(g, Q4K, rows, cols, 16, args.steps, args.warmup)
    value = nbytes / (ms_wall * 1e-3) / 1e9
    achieved = nbytes / (ms_k * 1e-3) / 1e9
    line = {
        "metric": "Q4_K matvec GB/s (% HBM peak) at 14336x4096; decode tok/s on 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_wall, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights, f32 accumulate",
        "data": "synthetic (seeded counter-based generator, BASELINE configs[1] distributions)",
        "config": {"workload": "Q4_K matvec 14336x4096, batch 1, 16 rotating resident copies (528 MB)",
                   "rows": rows, "cols": cols, "bytes_per_step": nbytes, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": load_traffic("q4k_14336x4096"),
                     "kernel_us": round(ms_k * 1e3, 3), "step_us_events": round(ms_ev * 1e3, 3),
                     "inter_launch_gap_us": round(getattr(time_matvec, "last_gap_us", 0.0), 3)},
    }
    if not args.no_extra:
        extra = {}
        for name, dt, r, c, copies in (("q8_0_4096x4096", Q8, 4096, 4096, 28),
                                       ("q6_k_head_128256x4096", Q6K, 128256, 4096, 2),
                                       ("q4_k_down_4096x14336", Q4K, 4096, 14336, 16)):
            steps = max(20, args.steps // (10 if dt == Q6K else 1))
            w_, e_, k_ = time_matvec(g, dt, r, c, copies, steps, min(args.warmup, 10))
            b = algo_bytes(dt, r, c)
            extra[name] = {"us_kernel": round(k_ * 1e3, 3), "GB_s": round(b / (k_ * 1e-3) / 1e9, 1),
                           "frac_hbm": round(b / (k_ * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes": b}
        line["configs"] = extra
    if not args.no_cpu:
        gbs, n, ms = cpu_baseline(Q4K, rows, cols, args.cpu_seconds, args.cpu_threads)
        line["cpu_baseline"] = {"value": round(gbs, 2), "unit": "GB/s", "cores": args.cpu_threads, "kind": "port",
                                "sample": f"{n} AVX2 Q4_K matvecs 14336x4096 over 4 rotating copies "
                                          f"({ms:.2f} ms each) in ~{args.cpu_seconds:.0f} s",
                                "host_nproc": os.cpu_count()}
    g.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
