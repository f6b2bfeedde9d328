#!/usr/bin/env python3
"""Throughput of the reduction / scan hot path on one MI355X.

Metric: achieved HBM GB/s (and fraction of the 8 TB/s peak) for the u32
exclusive scan and the f32 sum-reduce at 2^28 elements.  A step is one
exclusive scan of the 2^28-element u32 operand (the
headline); inputs are generated in HBM before timing and every step is one
launch of the single-pass look-back scan kernel.

The default run also times, the same way, every other BASELINE.json
configuration and the f32 sum-reduce at 2^28 (the metric's second half),
under "secondary":
  cfg1  f32 full sum, n = 2^20 (the CPU reference device's plumbing case;
        cache-resident on the GPU)
  cfg3  f32 row-wise sum, max, argmax of fmaf(0.5, x, 0.25), 65536 x 4096
  cfg4  i32 segmented sum, n = 2^27, geometric(300) segment lengths
  cfg5  f32 inclusive scan, n = 2^30
Each line carries its roofline, the mean, median and minimum time per launch,
a CPU baseline (the oracle on this host over a bounded sample) and the check
of the GPU output.  "ceiling" times the best read+write streams on the same
device in the same run: the library's copy kernel and the runtime's
hipMemcpyAsync device-to-device blit, 1 GiB each way.

Timing: HIP events on the device stream, which every launch here uses.  Each
configuration first runs untimed for --settle-ms of device time (100 ms by
default; its first launches after set-up run slow), then `warmup` untimed
launches.  The mean comes from one pair of events around `steps` back-to-back launches;
median and minimum from five further batches of steps/5 back-to-back
launches, each between its own pair of events.  GB/s = algorithmic bytes per
launch / mean time per launch.

Usage: python bench.py [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_GBS = 8000.0  # MI355X HBM3E
WORKLOADS = ("scan_u32", "sum_f32", "sum_f32_2_20", "rows_f32", "segmented_i32", "scan_f32_2_30",
             "segmented_short_i32", "copy_u32", "dot_f32", "axpy_f32", "colsum_f32", "colscan_u32",
             "colscan_narrow_u32", "segmented_long_i32", "colscan_rowtile_u32", "colscan_rowtile_wide_u32",
             "colsum_period_f32", "rows_short_f32")
# Dominant kernel of each workload (substring of its name in rocprofv3 output).
KERNEL_OF = {"scan_u32": "scan_tiles_kernel", "sum_f32": "full_reduce_kernel<", "sum_f32_2_20": "full_reduce_kernel<",
             "rows_f32": "rows_kernel", "segmented_i32": "segmented_sum_kernel",
             "segmented_short_i32": "seg_short_kernel", "scan_f32_2_30": "scan_tiles_kernel",
             "copy_u32": "copy_tiles_kernel", "dot_f32": "map_reduce_kernel<", "axpy_f32": "vector_tiles_kernel<1",
             "colsum_f32": "cols_tiles_kernel", "colscan_u32": "col_lookback_kernel",
             "colscan_narrow_u32": "col_narrow_scan_kernel", "segmented_long_i32": "segmented_sum_kernel",
             "colscan_rowtile_u32": "col_rowtile_lookback_kernel", "colscan_rowtile_wide_u32": "col_rowtile_scan_kernel",
             "colsum_period_f32": "cols_period_kernel", "rows_short_f32": "rows_tile_kernel"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Untimed device time spent on each configuration before its warm-up steps.
# A configuration's first launches after its set-up run slow, and the timed
# region must see the steady state: measured on MI355X in batches of 10
# launches, the first batch of each ran 2-5x its steady time (segmented sum
# 185.8 us per launch against 85.0, the scan 1684 against 355), and the f32
# sum at 2^28 took 158 us per launch for its first ~60 ms before settling at
# 151.  With 10 warm-up launches alone, the segmented sum's mean over 100
# timed launches came out at 91.8 us against a median of 85.5.
SETTLE_MS = 100.0


def settle(dev, run, ms: float, chunk: int = 10, max_launches: int = 100000) -> int:
    """Launches `run` untimed until `ms` of device time has passed; returns
    the number of launches.  The first `chunk` launches time one launch; the
    rest go back to back in as few batches as that estimate allows, so the
    device never idles between host synchronisations (a launch-bound kernel
    synchronised every 10 launches ran with the device half idle, and its
    timed mean afterwards rose from 5.1 to 7.6 us)."""
    if ms <= 0:
        return 0
    start, stop = dev.event(), dev.event()
    start.record()
    n = 0
    while n < max_launches:
        for _ in range(chunk):
            run()
        n += chunk
        stop.record()
        stop.synchronize()
        elapsed = start.elapsed_ms(stop)
        if elapsed >= ms:
            break
        chunk = int(min(max_launches - n, max(10, (ms - elapsed) / (elapsed / n) + 1)))
    return n


def time_launches(dev, run, steps: int, warmup: int, batches: int = 5) -> dict:
    """Milliseconds per launch of `run`: the mean over one pair of events
    around `steps` back-to-back launches, then the median and minimum over
    `batches` further batches of steps/batches back-to-back launches, each
    between a pair of events.  (An event between every two launches would
    add its own fence to each launch.)  The settle launches and the
    `warmup` launches before them are untimed."""
    settled = settle(dev, run, SETTLE_MS)
    for _ in range(warmup):
        run()
    dev.synchronize()
    start, stop = dev.event(), dev.event()
    start.record()
    for _ in range(steps):
        run()
    stop.record()
    stop.synchronize()
    mean = start.elapsed_ms(stop) / steps
    per_batch = max(1, steps // batches)
    evs = [dev.event() for _ in range(batches + 1)]
    evs[0].record()
    for b in range(batches):
        for _ in range(per_batch):
            run()
        evs[b + 1].record()
    evs[-1].synchronize()
    per = [evs[b].elapsed_ms(evs[b + 1]) / per_batch for b in range(batches)]
    dev.synchronize()
    return {"mean_ms": mean, "median_ms": statistics.median(per), "min_ms": min(per), "settle_launches": settled}


def time_plan(dev, run, steps: int, warmup: int) -> float:
    """Mean milliseconds per launch (time_launches' first pass only)."""
    settle(dev, run, SETTLE_MS)
    for _ in range(warmup):
        run()
    dev.synchronize()
    start, stop = dev.event(), dev.event()
    start.record()
    for _ in range(steps):
        run()
    stop.record()
    stop.synchronize()
    dev.synchronize()
    return start.elapsed_ms(stop) / steps


def traffic_for(name: str):
    """(HBM bytes per launch, where that figure comes from) from the
    committed rocprofv3 PMC summary; (None, None) when it has no entry.
    The counters cannot be read in this run (rocprofv3 --pmc needs a run of
    its own), so the figure is the one committed under profiles/, with the
    command and run that measured it."""
    f = REPO / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None, None
    data = json.loads(f.read_text())
    entry = data.get(name)
    if entry is None:
        return None, None
    prov = data.get("_provenance", {})
    src = (f"profiles/pmc_traffic.json, not measured in this run: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, each "
           f"in its own run of `{prov.get('command', 'bench.py --workload ' + name)}`, scaled by the copy-kernel "
           f"calibration; measured {prov.get('measured', 'on an earlier lease')}")
    return entry.get("hbm_bytes_per_launch"), src


def roofline(bytes_per_launch: float, ms: float, name: str) -> dict:
    achieved = bytes_per_launch / (ms * 1e-3) / 1e9
    traffic, source = traffic_for(name)
    out = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
           "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic}
    if source:
        out["traffic_source"] = source
    return out


def gbs(nbytes: float, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


def _cpu_rate(run, bytes_per_pass: float, seconds: float = 2.0, max_reps: int = 50):
    """(GB/s, passes, ms per pass) of `run()` repeated for about `seconds`."""
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= max_reps:
            break
    per = el / reps
    return bytes_per_pass / per / 1e9, reps, per * 1e3


def _cpu_line(gbs_, reps, ms, sample):
    out = {"value": round(gbs_, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{sample}; {reps} passes, {ms:.1f} ms per pass"}
    return out


def host_cores() -> int:
    """Threads for the all-core CPU baselines: the cores this process may
    run on, at most 16 (one GPU's share of a GPU box's host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _multithread(run, bytes_per_pass: float, seconds: float, sample: str, max_reps: int = 50) -> dict:
    """The all-core figure: `run(cores)` repeated for about `seconds`."""
    cores = host_cores()
    gb, reps, ms = _cpu_rate(lambda: run(cores), bytes_per_pass, seconds, max_reps)
    return {"value": round(gb, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{sample}; {reps} passes, {ms:.1f} ms per pass"}


# ------------------------------------------------------------- workloads
# Each returns {"n", "bytes", "run", "verify"}: `run` is one step on the
# device stream, `verify()` checks the output of the last step against the
# oracle and returns a short record, `cpu(seconds)` times the oracle.

def wl_scan_u32(hx, dev):
    """cfg 2 (headline): u32 exclusive scan, n = 2^28, uniform ints in [0, 256)."""
    from hephaestus_amd import Layout, StridedView

    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=2, lo=0, hi=255)
    out = dev.alloc_uninitialized(np.uint32, n)
    lay = Layout.c_contiguous([n])
    plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                              StridedView(out, lay), hx.ScanKind.Exclusive)

    def cpu(seconds):
        from oracle import oracle

        host = dev.download_owned(x)
        got = dev.download_owned(out)
        ref = np.empty_like(host)
        gb, reps, ms = _cpu_rate(lambda: oracle.lib().hxo_scan_sum_u32(host.ctypes.data, n, 1, 0, ref.ctypes.data),
                                 8.0 * n, seconds)
        mt = np.empty_like(host)
        line = _cpu_line(gb, reps, ms, "the full 2^28-element u32 exclusive scan, sequential C oracle "
                                       "(oracle/hx_oracle.c hxo_scan_sum_u32)")
        line["multithread"] = _multithread(lambda c: oracle.scan_excl_u32_threads(host, mt, c), 8.0 * n, seconds / 2,
                                           "the full 2^28-element input, two-pass pthread scan "
                                           "hxo_scan_excl_u32_threads")
        line["multithread"]["equals_sequential"] = bool(np.array_equal(mt, ref))
        line["gpu_output_verified"] = bool(np.array_equal(got, ref))
        return line

    return {"n": n, "bytes": 8 * n, "run": plan.dispatch, "cpu": cpu, "verify": None,
            "keep": (x, out, plan), "dtype": "u32",
            "workload": "u32 exclusive prefix scan, n=2^28 (BASELINE configs[1], the headline)"}


def _sum_f32(hx, dev, n, seed):
    from hephaestus_amd import Layout, StridedView

    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=seed, lo=-1.0, hi=1.0)
    out = dev.alloc_zeroed(np.float32, 1)
    plan = hx.RocmFullReductionOps().prepare_reduce_full(dev, hx.SumOp, StridedView(x, Layout.c_contiguous([n])),
                                                         StridedView(out, Layout.c_contiguous([1])))

    def verify():
        from oracle import oracle

        ref, ab = oracle.full_sum(dev.download_owned(x))
        got = float(dev.download_owned(out)[0])
        tol = 2 * oracle.ceil_log2(n) * 2.0**-23 * ab
        return {"ok": abs(got - ref) <= tol, "check": "|gpu - f64 sum| <= 2*ceil(log2 n)*eps*sum|x|",
                "err_over_eps_abs": abs(got - ref) / (2.0**-23 * ab)}

    return plan, x, out, verify


def wl_sum_f32(hx, dev):
    """The metric's second half: f32 full sum, n = 2^28, uniform[-1, 1)."""
    n = 1 << 28
    plan, x, out, verify = _sum_f32(hx, dev, n, 1)

    def cpu(seconds):
        from oracle import oracle

        m = 1 << 26
        h = oracle.uniform_real(m, 1, -1.0, 1.0)
        line = _cpu_line(*_cpu_rate(lambda: oracle.full_sum(h), 4.0 * m, seconds),
                         "2^26 f32 (a quarter of the GPU input), oracle full_sum (compensated f64 accumulation)")
        full = dev.download_owned(x)
        line["multithread"] = _multithread(lambda c: oracle.sum_f32_threads(full, c), 4.0 * n, seconds,
                                           "the full 2^28-element GPU input, pthread f64 partial sums "
                                           "hxo_sum_f32_threads")
        return line

    return {"n": n, "bytes": 4 * n + 4, "run": plan.dispatch, "cpu": cpu, "verify": verify, "keep": (plan, x, out),
            "dtype": "f32", "workload": "f32 full sum-reduce, n=2^28, uniform[-1,1)"}


def wl_sum_f32_2_20(hx, dev):
    """cfg 1: f32 full sum, n = 2^20 (cache-resident on the GPU)."""
    n = 1 << 20
    plan, x, out, verify = _sum_f32(hx, dev, n, 1)

    def cpu(seconds):
        from oracle import oracle

        h = oracle.uniform_real(n, 1, -1.0, 1.0)
        line = _cpu_line(*_cpu_rate(lambda: oracle.full_sum(h), 4.0 * n, seconds, max_reps=2000),
                         "the full 2^20 f32 input, oracle full_sum (the CPU reference device's role)")
        line["multithread"] = _multithread(lambda c: oracle.sum_f32_threads(h, c), 4.0 * n, seconds,
                                           "the full 2^20 f32 input, pthread f64 partial sums hxo_sum_f32_threads",
                                           max_reps=2000)
        return line

    return {"n": n, "bytes": 4 * n + 4, "run": plan.dispatch, "cpu": cpu, "verify": verify, "keep": (plan, x, out),
            "dtype": "f32", "workload": "f32 full sum-reduce, n=2^20 (BASELINE configs[0]; 4 MiB, cache-resident)"}


def wl_rows_f32(hx, dev):
    """cfg 3: per-row sum, max, argmax of fmaf(0.5, x, 0.25), 65536 x 4096
    N(0,1) f32, one prepared launch."""
    rows, cols = 65536, 4096
    x = dev.alloc_uninitialized(np.float32, rows * cols)
    dev.fill_normal(x, seed=3)
    s = dev.alloc_uninitialized(np.float32, rows)
    m = dev.alloc_uninitialized(np.float32, rows)
    i = dev.alloc_uninitialized(np.uint32, rows)
    plan = hx.RocmAxisReductionOps().prepare_reduce_rows_fused(dev, x, rows, cols, prologue=(0.5, 0.25),
                                                               out_sum=s, out_max=m, out_argmax=i)

    def verify():
        from oracle import oracle

        s_ref, a_ref, m_ref, i_ref = oracle.rows(dev.download_owned(x), rows, cols, prologue=(0.5, 0.25))
        got = dev.download_owned(s).astype(np.float64)
        tol = 2 * oracle.ceil_log2(cols) * 2.0**-23 * a_ref
        ok = (np.array_equal(dev.download_owned(m), m_ref) and np.array_equal(dev.download_owned(i), i_ref)
              and bool(np.all(np.abs(got - s_ref) <= tol)))
        return {"ok": ok, "check": "max and argmax bit-exact, sums within 2*ceil(log2 cols)*eps*sum|y|"}

    def cpu(seconds):
        from oracle import oracle

        r = 4096
        h = oracle.normal(r * cols, 3)
        line = _cpu_line(*_cpu_rate(lambda: oracle.rows(h, r, cols, prologue=(0.5, 0.25)), 4.0 * r * cols + 12.0 * r,
                                    seconds),
                         "4096 x 4096 f32 (1/16 of the GPU rows), oracle rows (sum, max, argmax of fmaf(.5,x,.25))")
        full = dev.download_owned(x)
        line["multithread"] = _multithread(
            lambda c: oracle.rows_threads(full, rows, cols, c, prologue=(0.5, 0.25)), 4.0 * rows * cols + 12.0 * rows,
            seconds, "the full 65536 x 4096 GPU input, oracle rows on pthread row ranges (hxo_rows_f32_threads)")
        return line

    return {"n": rows * cols, "bytes": 4 * rows * cols + 12 * rows, "run": plan.dispatch, "cpu": cpu,
            "verify": verify, "keep": (x, s, m, i, plan), "dtype": "f32",
            "workload": "f32 row-wise sum+max+argmax of fmaf(0.5,x,0.25), 65536 x 4096 (BASELINE configs[2])"}


def wl_segmented_i32(hx, dev):
    """cfg 4: i32 segmented sum, n = 2^27, geometric(300) lengths."""
    from oracle import oracle  # geometric offsets are generated on the host

    n = 1 << 27
    x = dev.alloc_uninitialized(np.int32, n)
    dev.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    off = oracle.geometric_offsets(n, 300.0, seed=5)
    ob = dev.upload(off)
    out = dev.alloc_uninitialized(np.int32, off.size - 1)
    plan = hx.RocmSegmentedReductionOps().prepare_segmented_sum(dev, x, ob, out)
    segs = off.size - 1

    def verify():
        ok = np.array_equal(dev.download_owned(out), oracle.segmented_sum(dev.download_owned(x), off))
        return {"ok": bool(ok), "check": "bit-exact", "segments": int(segs)}

    def cpu(seconds):
        m = 1 << 25
        h = oracle.uniform_int(m, 4, -1000, 1000, dtype=np.int32)
        o = oracle.geometric_offsets(m, 300.0, seed=5)
        line = _cpu_line(*_cpu_rate(lambda: oracle.segmented_sum(h, o), 4.0 * m + 8.0 * (o.size - 1) + 4, seconds),
                         f"2^25 i32 values, {o.size - 1} geometric(300) segments, oracle segmented_sum")
        full = dev.download_owned(x)
        line["multithread"] = _multithread(
            lambda c: oracle.segmented_sum_threads(full, off, c), 4.0 * n + 4.0 * (segs + 1) + 4.0 * segs, seconds,
            f"the full 2^27-value GPU input and its {segs} segments, oracle segmented_sum on pthread segment ranges "
            "(hxo_segmented_sum_u32_threads)")
        return line

    return {"n": n, "bytes": 4 * n + 4 * (segs + 1) + 4 * segs, "run": plan.dispatch, "cpu": cpu, "verify": verify,
            "keep": (x, ob, out, plan), "dtype": "i32",
            "workload": f"i32 segmented sum, n=2^27, {segs} geometric(300) segments (BASELINE configs[3])"}


def wl_scan_f32_2_30(hx, dev):
    """cfg 5: f32 inclusive scan, n = 2^30, uniform[0, 1)."""
    from hephaestus_amd import Layout, StridedView

    n = 1 << 30
    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=6, lo=0.0, hi=1.0)
    out = dev.alloc_uninitialized(np.float32, n)
    lay = Layout.c_contiguous([n])
    plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                              StridedView(out, lay))
    head = 1 << 24

    def verify():
        # A prefix of a scan depends on nothing after it: the first 2^24
        # outputs are checked in full (the tests check all 2^30).
        from oracle import oracle

        hx_ = hx.RocmBuffer(dev, x.ptr, head, np.float32)
        ho = hx.RocmBuffer(dev, out.ptr, head, np.float32)
        try:
            xi, go = dev.download_owned(hx_), dev.download_owned(ho)
        finally:
            hx_.ptr = ho.ptr = None  # views of x and out
        bad, worst = oracle.check_scan_f32(xi, go, n_for_log=n)
        return {"ok": bad == 0, "check": f"first 2^24 outputs within 2*ceil(log2 2^30)*eps*sum|x|",
                "worst_err_over_eps_abs": worst}

    def cpu(seconds):
        from oracle import oracle

        m = 1 << 23
        h = oracle.uniform_real(m, 6, 0.0, 1.0)
        line = _cpu_line(*_cpu_rate(lambda: oracle.scan_sum(h), 8.0 * m, seconds),
                         "2^23 f32 (1/128 of the GPU input), oracle scan_sum (compensated f64 prefix and |prefix|)")
        full = dev.download_owned(x)
        res = np.empty_like(full)
        line["multithread"] = _multithread(
            lambda c: oracle.scan_incl_f32_threads(full, res, c), 8.0 * n, seconds,
            "the full 2^30-element GPU input to an f32 output, pthread reduce-then-scan with f64 carries "
            "(hxo_scan_incl_f32_threads)")
        del full, res
        return line

    return {"n": n, "bytes": 8 * n, "run": plan.dispatch, "cpu": cpu, "verify": verify, "keep": (x, out, plan),
            "dtype": "f32", "workload": "f32 inclusive prefix scan, n=2^30 (BASELINE configs[4])"}


def ceiling(hx, dev, steps: int, warmup: int) -> dict:
    """The best read+write streams on this device: the library's copy
    kernel (nt loads, nt|sc1 stores, 256 KiB tiles) and the runtime's
    hipMemcpyAsync device-to-device, each 1 GiB in and 1 GiB out."""
    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=7, lo=0, hi=255)
    y = dev.alloc_uninitialized(np.uint32, n)
    out = {}
    t = time_launches(dev, lambda: dev.copy_buffer_async(x, y), steps, warmup)
    out["copy_kernel"] = {"GB/s": round(gbs(8.0 * n, t["mean_ms"]), 1), **{k: round(v, 5) for k, v in t.items()}}
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]

    def blit():
        err = hip.hipMemcpyAsync(y.ptr, x.ptr, 4 * n, 3, dev.stream)  # hipMemcpyDeviceToDevice
        if err != 0:
            raise RuntimeError(f"hipMemcpyAsync failed: {err}")

    t = time_launches(dev, blit, steps, warmup)
    out["runtime_blit_hipMemcpyAsync"] = {"GB/s": round(gbs(8.0 * n, t["mean_ms"]), 1),
                                          **{k: round(v, 5) for k, v in t.items()}}
    # The two yardsticks a single-pass look-back scan is actually held to.
    # (1) The copy in the integer scan's own tile shape and order: block b
    # moves 128 KiB tile b, each wave a contiguous 16 KiB run; a look-back
    # needs every tile's predecessors dispatched first, so it cannot take
    # the XCD-contiguous order of the copy above.
    t = time_launches(dev, _raw("hx_debug_copy_scan_shape", dev.handle, x.ptr, y.ptr, 4 * n, None), steps, warmup)
    out["copy_scan_shape_block_order"] = {"GB/s": round(gbs(8.0 * n, t["mean_ms"]), 1),
                                          **{k: round(v, 5) for k, v in t.items()}}
    # (2) The headline's own kernel with no look-back: the same 2^28 u32
    # exclusive scan cut into 8192 lines of 32768 elements scanned along
    # axis 1, so every line is one 8 x 16 tile of the same kernel
    # instantiation and no tile has a predecessor to wait for.  A real,
    # checked workload (row-wise scans), not a switch in the kernel.
    from hephaestus_amd import Layout, StridedView

    lines, width = 8192, 32768
    lay = Layout.c_contiguous([lines, width])
    rows_plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 1,
                                                   hx.ScanDirection.Forward, StridedView(y, lay),
                                                   hx.ScanKind.Exclusive)
    t = time_launches(dev, rows_plan.dispatch, steps, warmup)
    from oracle import oracle

    host_x, host_y = dev.download_owned(x).reshape(lines, width), dev.download_owned(y).reshape(lines, width)
    sample = range(0, lines, 257)
    ok = all(np.array_equal(host_y[r], oracle.scan_sum(host_x[r], exclusive=True)) for r in sample)
    out["scan_rows_one_tile_no_lookback"] = {
        "GB/s": round(gbs(8.0 * n, t["mean_ms"]), 1), **{k: round(v, 5) for k, v in t.items()},
        "workload": "u32 exclusive scan of [8192, 32768] along axis 1: scan_tiles_kernel 8 x 16, one tile per line",
        "gpu_output_check": {"ok": bool(ok), "check": f"{len(sample)} sampled lines bit-exact against the oracle"}}
    out["bytes_per_launch"] = 8 * n
    rows_plan.destroy()
    x.free()
    y.free()
    return out


# ----------------------------------------------- extra workloads (--workload)
def bench_segmented_short_i32(hx, dev, args):
    """Short segments (geometric, mean 4): the segment-parallel path."""
    from oracle import oracle

    n = 1 << 27
    x = dev.alloc_uninitialized(np.int32, n)
    dev.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    off = oracle.geometric_offsets(n, 4.0, seed=5)
    ob = dev.upload(off)
    out = dev.alloc_uninitialized(np.int32, off.size - 1)
    plan = hx.RocmSegmentedReductionOps().prepare_segmented_sum(dev, x, ob, out)
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    s = off.size - 1
    return {"n": n, "ms": ms, "bytes": 4 * n + 4 * (s + 1) + 4 * s}


def bench_dot_f32(hx, dev, args):
    """Prepared f32 dot of two 2^28 vectors (DenseVectorOps::prepare_dot):
    reads 8n bytes; f64 accumulation of exact products."""
    n = 1 << 28
    a = dev.alloc_uninitialized(np.float32, n)
    b = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(a, seed=11, lo=-1.0, hi=1.0)
    dev.fill_uniform_real(b, seed=12, lo=-1.0, hi=1.0)
    lay = hx.Layout.c_contiguous([n])
    plan = hx.prepare_dot(dev, hx.StridedView(a, lay), hx.StridedView(b, lay))
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    return {"n": n, "ms": ms, "bytes": 8 * n + 4}


def bench_axpy_f32(hx, dev, args):
    """axpy over 2^28 f32 (target = fmaf(f, source, target)): reads 8n,
    writes 4n bytes."""
    n = 1 << 28
    t = dev.alloc_uninitialized(np.float32, n)
    s = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(t, seed=13, lo=-1.0, hi=1.0)
    dev.fill_uniform_real(s, seed=14, lo=-1.0, hi=1.0)
    ops = hx.RocmDenseVectorOps()
    ms = time_plan(dev, lambda: ops.axpy(dev, t, s, 0.5), args.steps, args.warmup)
    return {"n": n, "ms": ms, "bytes": 12 * n}


def bench_colsum_f32(hx, dev, args):
    """Axis-0 sum of a 65536 x 4096 row-major f32 matrix (4096 outputs)."""
    from hephaestus_amd import Layout, StridedView

    rows, cols = 65536, 4096
    x = dev.alloc_uninitialized(np.float32, rows * cols)
    dev.fill_normal(x, seed=7)
    out = dev.alloc_uninitialized(np.float32, cols)
    plan = hx.RocmAxisReductionOps().prepare_reduce_axis_into(
        dev, hx.SumOp, StridedView(x, Layout.c_contiguous([rows, cols])), 0,
        StridedView(out, Layout.c_contiguous([1, cols])))
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    return {"n": rows * cols, "ms": ms, "bytes": 4 * rows * cols + 4 * cols}


def bench_colscan_u32(hx, dev, args):
    """Axis-0 inclusive scan of a 65536 x 4096 row-major u32 matrix."""
    from hephaestus_amd import Layout, StridedView

    rows, cols = 65536, 4096
    x = dev.alloc_uninitialized(np.uint32, rows * cols)
    dev.fill_uniform_int(x, seed=8, lo=0, hi=255)
    out = dev.alloc_uninitialized(np.uint32, rows * cols)
    lay = Layout.c_contiguous([rows, cols])
    plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                              StridedView(out, lay))
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    return {"n": rows * cols, "ms": ms, "bytes": 8 * rows * cols}


def _colscans_u32(hx, dev, args, name, widths):
    """Axis-0 inclusive scans of 2^28-element row-major u32 matrices, one
    per column count; "ms" is their mean."""
    from hephaestus_amd import Layout, StridedView

    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=3, lo=0, hi=255)
    out = dev.alloc_uninitialized(np.uint32, n)
    per, nbytes = {}, []
    for c in widths:
        lay = Layout.c_contiguous([n // c, c])
        plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0,
                                                  hx.ScanDirection.Forward, StridedView(out, lay))
        per[c] = time_plan(dev, plan.dispatch, args.steps, args.warmup)
        nbytes.append(8 * (n // c) * c)
        log(f"{name}: {c} columns {per[c]:.4f} ms/launch")
    return {"n": n, "ms": statistics.mean(per.values()), "bytes": statistics.mean(nbytes)}


def bench_colscan_narrow_u32(hx, dev, args):
    """32, 64 and 128 columns: the narrow-column form (three passes)."""
    return _colscans_u32(hx, dev, args, "colscan_narrow_u32", (32, 64, 128))


def bench_colscan_rowtile_u32(hx, dev, args):
    """3, 4, 12 and 16 columns: single-pass row tiles (look-back over
    C-wide carries)."""
    return _colscans_u32(hx, dev, args, "colscan_rowtile_u32", (3, 4, 12, 16))


def bench_colscan_rowtile_wide_u32(hx, dev, args):
    """100 and 255 columns: three-pass row tiles."""
    return _colscans_u32(hx, dev, args, "colscan_rowtile_wide_u32", (100, 255))


def bench_colsum_period_f32(hx, dev, args):
    """Axis-0 sums of 2^28-element row-major f32 matrices with 3, 5, 12 and
    24 columns (the period form); "ms" is their mean."""
    from hephaestus_amd import Layout, StridedView

    n = 1 << 28
    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=6, lo=-1.0, hi=1.0)
    out = dev.alloc_uninitialized(np.float32, 32)
    per, nbytes = {}, []
    for c in (3, 5, 12, 24):
        m = (n // c) * c
        plan = hx.RocmAxisReductionOps().prepare_reduce_axis_into(
            dev, hx.SumOp, StridedView(x, Layout.c_contiguous([n // c, c])), 0,
            StridedView(out, Layout.c_contiguous([1, c])))
        per[c] = time_plan(dev, plan.dispatch, args.steps, args.warmup)
        nbytes.append(4 * m + 4 * c)
        log(f"colsum_period_f32: {c} columns {per[c]:.4f} ms/launch")
    return {"n": n, "ms": statistics.mean(per.values()), "bytes": statistics.mean(nbytes)}


def bench_rows_short_f32(hx, dev, args):
    """The fused row reduce (sum, max and argmax of fmaf(.5, x, .25) per
    row, cfg3's statistics) over 2^28 f32 in back-to-back rows of 1, 3, 12
    and 100 elements (the LDS row tiles); "ms" is their mean."""
    n = 1 << 28
    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=7, lo=-1.0, hi=1.0)
    per, nbytes = {}, []
    for c in (1, 3, 12, 100):
        rows = n // c
        s = dev.alloc_uninitialized(np.float32, rows)
        m = dev.alloc_uninitialized(np.float32, rows)
        i = dev.alloc_uninitialized(np.uint32, rows)
        plan = hx.RocmAxisReductionOps().prepare_reduce_rows_fused(dev, x, rows, c, prologue=(0.5, 0.25), out_sum=s,
                                                                   out_max=m, out_argmax=i)
        per[c] = time_plan(dev, plan.dispatch, args.steps, args.warmup)
        nbytes.append(4 * rows * c + 12 * rows)
        plan.destroy()
        for b in (s, m, i):
            b.free()
        log(f"rows_short_f32: {c} elements a row {per[c]:.4f} ms/launch")
    return {"n": n, "ms": statistics.mean(per.values()), "bytes": statistics.mean(nbytes)}


def bench_segmented_long_i32(hx, dev, args):
    """Segmented sums of 2^27 i32 values with geometric segment lengths of
    mean 3000, 10^5, 10^6 and 10^7 (long segments: tiles without a segment
    start, whose carries come from look-backs); "ms" is their mean."""
    from oracle import oracle  # geometric offsets are generated on the host

    n = 1 << 27
    x = dev.alloc_uninitialized(np.int32, n)
    dev.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    per, nbytes = {}, []
    for mean in (3000.0, 1e5, 1e6, 1e7):
        off = oracle.geometric_offsets(n, mean, seed=5)
        ob = dev.upload(off)
        out = dev.alloc_uninitialized(np.int32, off.size - 1)
        plan = hx.RocmSegmentedReductionOps().prepare_segmented_sum(dev, x, ob, out)
        per[mean] = time_plan(dev, plan.dispatch, args.steps, args.warmup)
        nbytes.append(4 * n + 4 * off.size + 4 * (off.size - 1))
        log(f"segmented_long_i32: mean {mean:g}, {off.size - 1} segments, {per[mean]:.4f} ms/launch")
    return {"n": n, "ms": statistics.mean(per.values()), "bytes": statistics.mean(nbytes)}


def bench_copy_u32(hx, dev, args):
    """The copy kernel behind copy_buffer over 2^28 u32, queued back to back
    (hx_copy_async): the yardstick (read B + write B) for the HBM byte
    counters, and the read+write stream ceiling."""
    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=7, lo=0, hi=255)
    y = dev.alloc_uninitialized(np.uint32, n)
    ms = time_plan(dev, lambda: dev.copy_buffer_async(x, y), args.steps, args.warmup)
    return {"n": n, "ms": ms, "bytes": 8 * n}


def _counter_csv(path: Path, counter: str | None = None) -> dict:
    """{kernel name: [per-dispatch values]} of one counter (or of the only
    counter) from one rocprofv3 --pmc run (CSV)."""
    import csv

    files = sorted(path.rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {path}")
    out: dict = {}
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if counter is None or row["Counter_Name"] == counter:
                    out.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return out


def _lds_summary(root: Path) -> dict:
    """LDS instructions and bank-conflict cycles per dispatch of each
    workload's kernel, from root/<workload>/lds runs of
    `rocprofv3 --pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT`."""
    import statistics

    out = {}
    for w in WORKLOADS:
        d = root / w / "lds"
        if not d.exists():
            continue
        entry = {"kernel": KERNEL_OF[w]}
        for c in ("SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT"):
            vals = [v for k, vs in _counter_csv(d, c).items() if KERNEL_OF[w] in k for v in vs]
            entry[c] = statistics.median(vals) if vals else None
        out[w] = entry
    return out


def pmc_summary(root: Path) -> int:
    """Turn rocprofv3 --pmc runs into profiles/pmc_traffic.json.

    Expects root/<workload>/fetch and root/<workload>/write, each the output
    directory of `rocprofv3 --pmc FETCH_SIZE` (resp. WRITE_SIZE) over
    `bench.py --workload <workload>`; optional root/<workload>/lds runs of
    `--pmc SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT` go to profiles/pmc_lds.json.  Counters are KiB per dispatch; each
    is scaled by the factor that maps the copy kernel's reading to its known
    traffic (read 4n, write 4n bytes)."""
    import statistics

    raw = {}
    for w in WORKLOADS:
        if not (root / w).exists():
            continue
        entry = {}
        for which in ("fetch", "write"):
            rows = _counter_csv(root / w / which)
            vals = [v for k, vs in rows.items() if KERNEL_OF[w] in k for v in vs]
            if not vals:
                raise SystemExit(f"{w}/{which}: no dispatch of {KERNEL_OF[w]}")
            entry[which + "_kib"] = statistics.median(vals)
            entry["dispatches"] = len(vals)
        raw[w] = entry
    if "copy_u32" not in raw:
        raise SystemExit("copy_u32 calibration run missing")
    copy_bytes = 4 * (1 << 28)
    f_fetch = copy_bytes / (raw["copy_u32"]["fetch_kib"] * 1024)
    f_write = copy_bytes / (raw["copy_u32"]["write_kib"] * 1024)
    out = {"_calibration": {"kernel": "copy_tiles_kernel, 2^28 u32 (read 1 GiB, write 1 GiB)",
                            "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4)}}
    for w, e in raw.items():
        fetch = e["fetch_kib"] * 1024 * f_fetch
        write = e["write_kib"] * 1024 * f_write
        out[w] = {"kernel": KERNEL_OF[w], "fetch_kib": e["fetch_kib"], "write_kib": e["write_kib"],
                  "dispatches": e["dispatches"], "hbm_bytes_per_launch": round(fetch + write)}
    lds = _lds_summary(root)
    if lds:
        (REPO / "profiles" / "pmc_lds.json").write_text(json.dumps(lds, indent=1) + "\n")
    dst = REPO / "profiles" / "pmc_traffic.json"
    dst.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out, indent=1))
    return 0


# Kernels of each default configuration, as (name substring, launch grid
# in threads) pairs of the kernel trace; one step runs each once.
TRACE_CONFIGS = [
    ("scan_u32", "u32 exclusive scan 2^28 (headline)", [("scan_tiles_kernel<unsigned int", 8192 * 512)], 8 << 28),
    ("sum_f32", "f32 sum 2^28", [("full_reduce_kernel<float", 768 * 256)], (4 << 28) + 4),
    # f32: one 256-thread block per 8192 elements below 768 blocks
    ("sum_f32_2_20", "f32 sum 2^20 (cfg1)", [("full_reduce_kernel<float", (1 << 20) // 8192 * 256)], (4 << 20) + 4),
    ("rows_f32", "rows 65536 x 4096 (cfg3)", [("rows_kernel<float", 65536 * 256)], (4 << 28) + 12 * 65536),
    ("segmented_i32", "segmented 2^27 (cfg4)", [("seg_tile_map_kernel", None), ("segmented_sum_kernel", None)], None),
    ("scan_f32_2_30", "f32 inclusive scan 2^30 (cfg5)", [("scan_tiles_kernel<float", None)], 8 << 30),
    ("copy_u32", "copy 1 GiB (ceiling yardstick)", [("copy_tiles_kernel", 4096 * 512)], 8 << 28),
    ("blit", "hipMemcpyAsync 1 GiB (ceiling)", [("__amd_rocclr_copyBuffer", 131072)], 8 << 28),
]


def trace_summary(root: Path, bench_json: Path | None) -> int:
    """Markdown summary of a `rocprofv3 --kernel-trace --stats` run of the
    default bench: per kernel and launch grid, calls and the mean, median,
    minimum and maximum duration, then per configuration the step time (its
    kernels' means added, over the launches the bench timed) beside the
    bench's own event-timed mean."""
    import csv

    files = sorted(root.rglob("*kernel_trace.csv"))
    if not files:
        raise SystemExit(f"no *kernel_trace.csv under {root}")
    starts: dict = {}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                key = (r["Kernel_Name"], int(r["Grid_Size_X"]))
                t0, t1 = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
                starts.setdefault(key, []).append((t0, (t1 - t0) / 1e3))
    # Every group's durations in launch order.
    groups = {k: [d for _, d in sorted(v)] for k, v in starts.items()}
    bench = json.loads(bench_json.read_text()) if bench_json else None
    sec = (bench or {}).get("secondary", {})
    ceil = (bench or {}).get("ceiling", {})
    warm = int((bench or {}).get("warmup", 0))
    # Untimed launches at the start of each configuration (settle, then
    # warm-up): the step times below skip them, so they cover the launches
    # the bench's events timed.
    untimed = {"scan_u32": (bench or {}).get("timing", {}).get("settle_launches", 0),
               "sum_f32": sec.get("f32_sum_reduce_2_28", {}).get("settle_launches", 0),
               "sum_f32_2_20": sec.get("cfg1_f32_sum_2_20", {}).get("settle_launches", 0),
               "rows_f32": sec.get("cfg3_rows_f32_65536x4096", {}).get("settle_launches", 0),
               "segmented_i32": sec.get("cfg4_segmented_i32_2_27", {}).get("settle_launches", 0),
               "scan_f32_2_30": sec.get("cfg5_scan_f32_2_30", {}).get("settle_launches", 0),
               "copy_u32": ceil.get("copy_kernel", {}).get("settle_launches", 0),
               "blit": ceil.get("runtime_blit_hipMemcpyAsync", {}).get("settle_launches", 0)}
    untimed = {k: int(v or 0) + warm for k, v in untimed.items()} if bench else {}
    # The launches each configuration's event-timed mean covers, right after
    # its untimed ones.  A kernel+grid group can hold later launches of
    # another leg (the ceiling's one-tile-per-row scan runs the headline's
    # kernel on the headline's grid), so only this window is taken.
    top_steps = int((bench or {}).get("steps", 0))
    timed = {"scan_u32": top_steps,
             "sum_f32": sec.get("f32_sum_reduce_2_28", {}).get("steps", 0),
             "sum_f32_2_20": sec.get("cfg1_f32_sum_2_20", {}).get("steps", 0),
             "rows_f32": sec.get("cfg3_rows_f32_65536x4096", {}).get("steps", 0),
             "segmented_i32": sec.get("cfg4_segmented_i32_2_27", {}).get("steps", 0),
             "scan_f32_2_30": sec.get("cfg5_scan_f32_2_30", {}).get("steps", 0),
             "copy_u32": top_steps, "blit": top_steps}
    bench_ms = {"scan_u32": (bench or {}).get("ms_per_step"),
                "sum_f32": sec.get("f32_sum_reduce_2_28", {}).get("ms_per_launch"),
                "sum_f32_2_20": sec.get("cfg1_f32_sum_2_20", {}).get("ms_per_launch"),
                "rows_f32": sec.get("cfg3_rows_f32_65536x4096", {}).get("ms_per_launch"),
                "segmented_i32": sec.get("cfg4_segmented_i32_2_27", {}).get("ms_per_launch"),
                "scan_f32_2_30": sec.get("cfg5_scan_f32_2_30", {}).get("ms_per_launch"),
                "copy_u32": (bench or {}).get("ceiling", {}).get("copy_kernel", {}).get("mean_ms"),
                "blit": (bench or {}).get("ceiling", {}).get("runtime_blit_hipMemcpyAsync", {}).get("mean_ms")}
    seg_bytes = (sec.get("cfg4_segmented_i32_2_27") or {}).get("algorithmic_bytes_per_launch")
    lines = ["| kernel | grid (threads) | calls | mean us | median us | min us | max us |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        short = name.replace("hx::(anonymous namespace)::", "").replace("hx::", "").replace("|", "\\|")
        short = short if len(short) <= 110 else short[:110] + "..."
        lines.append(f"| `{short}` | {grid} | {len(d)} | {statistics.mean(d):.1f} | {statistics.median(d):.1f} | "
                     f"{min(d):.1f} | {max(d):.1f} |")
    lines += ["", "| configuration | kernels per step | untimed launches skipped | timed launches taken "
                  "| trace: step us (means added) | trace: step us (medians added) "
                  "| bench: event-timed us per step | trace frac | bench frac |",
              "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for key, label, kernels, nbytes in TRACE_CONFIGS:
        nbytes = seg_bytes if key == "segmented_i32" else nbytes
        mean_sum = med_sum = 0.0
        found = True
        for sub, grid in kernels:
            ds = [d for (name, g), d in groups.items() if sub in name and (grid is None or g == grid)]
            if not ds:
                found = False
                break
            skip = untimed.get(key, 0)
            take = int(timed.get(key) or 0) if bench else 0
            d = [x for lst in ds for x in (lst[skip:skip + take] if take else lst[skip:])]
            if not d:
                found = False
                break
            mean_sum += statistics.mean(d)
            med_sum += statistics.median(d)
        if not found:
            continue
        b = bench_ms.get(key)
        tf = f"{nbytes / (mean_sum * 1e-6) / 8e12:.4f}" if nbytes else "-"
        bf = f"{nbytes / (b * 1e-3) / 8e12:.4f}" if (nbytes and b) else "-"
        lines.append(f"| {label} | {len(kernels)} | {untimed.get(key, 0)} | {timed.get(key, 0) if bench else '-'} | "
                     f"{mean_sum:.1f} | {med_sum:.1f} | "
                     f"{b * 1e3 if b else float('nan'):.1f} | {tf} | {bf} |")
    print("\n".join(lines))
    return 0


def _raw(fn_name: str, *args):
    """A closure calling one C-ABI entry point with prebuilt ctypes arguments,
    so that per-call host cost is one ctypes dispatch, as close as Python gets
    to the reference's direct Rust calls."""
    from hephaestus_amd import _ffi

    fn = getattr(_ffi.lib(), fn_name)

    def call():
        status = fn(*args)
        if status != 0:
            _ffi.check(status)
    return call


def latency_suite(hx, dev, args) -> dict:
    """The reference's only published timings for this path are small
    problems on its WGPU backend (RTX 5080, Windows 11; benchmark_results.md:
    151-158, harness crates/hephaestus-wgpu/benches/comparative.rs: 50
    back-to-back calls, one device poll, wall time / 50).  The same shapes,
    timed the same way on this path (`us_per_call`), plus the HIP-event time
    per launch on the device stream (`gpu_us_per_launch`).  Different
    hardware and backend: a reference point, not `vs_baseline`."""
    import ctypes

    from hephaestus_amd import Layout, _ffi
    from hephaestus_amd.device import hx_dtype

    def lay(layout):
        return ctypes.byref(_ffi.layout_struct(layout))

    def wall_us(call, iters=50, warm=5) -> float:
        for _ in range(warm):
            call()
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            call()
        dev.synchronize()
        return (time.perf_counter() - t0) / iters * 1e6

    out = {}

    def record(name, call, ref_us, source):
        out[name] = {"us_per_call": round(wall_us(call), 2),
                     "gpu_us_per_launch": round(time_plan(dev, call, 200, 20) * 1e3, 2),
                     "reference_wgpu_rtx5080_us": ref_us, "reference_source": source}

    n = 1 << 20
    xs = dev.upload((np.arange(n) % 17).astype(np.uint32))
    o1 = dev.alloc_zeroed(np.uint32, 1)
    plan = hx.RocmFullReductionOps().prepare_reduce_full(
        dev, hx.SumOp, hx.StridedView(xs, Layout.c_contiguous([n])), hx.StridedView(o1, Layout.c_contiguous([1])))
    record("sum_u32_2_20_prepared", _raw("hx_plan_dispatch", plan.handle, None), 42.70, "benchmark_results.md:151")

    m = 256
    a = dev.upload(np.arange(m * m, dtype=np.float32) / 1000.0)
    row = dev.alloc_zeroed(np.float32, m)
    li, lo = Layout.c_contiguous([m, m]), Layout.c_contiguous([1, m])
    ops = {"sum": (hx.SumOp, 22.14, 152), "min": (hx.MinOp, 20.73, 153), "max": (hx.MaxOp, 11.78, 154),
           "mean": (hx.MeanOp, 18.05, 155)}
    plans = []  # the reference rows are "axis-0 tiled prepared": prepared plans here too
    for name, (op, ref, line) in ops.items():
        plans.append(hx.RocmAxisReductionOps().prepare_reduce_axis_into(
            dev, op, hx.StridedView(a, li), 0, hx.StridedView(row, lo)))
        record(f"axis0_{name}_256x256", _raw("hx_plan_dispatch", plans[-1].handle, None), ref,
               f"benchmark_results.md:{line}")
    full = dev.alloc_zeroed(np.float32, m * m)
    record("cumsum_axis1_256x256", _raw("hx_scan", dev.handle, hx.CumSumOp.code, hx_dtype(np.float32),
                                        _ffi.SCAN_INCLUSIVE, _ffi.SCAN_FORWARD, a.ptr, m * m, lay(li), 1,
                                        full.ptr, m * m, lay(li), None),
           46.53, "benchmark_results.md:158")
    k = 65536
    u, v = dev.upload(np.ones(k, np.float32)), dev.upload(np.full(k, 0.5, np.float32))
    o2 = dev.alloc_zeroed(np.float32, 1)
    lk = Layout.c_contiguous([k])
    record("dot_f32_65536", _raw("hx_map_reduce", dev.handle, _ffi.MAP_DOT, hx_dtype(np.float32), u.ptr, k, lay(lk),
                                 v.ptr, k, lay(lk), o2.ptr, 1, None),
           97.42, "benchmark_results.md:161")
    record("trace_f32_256x256", _raw("hx_trace", dev.handle, hx_dtype(np.float32), a.ptr, m * m, lay(li), o2.ptr, 1,
                                     None),
           42.72, "benchmark_results.md:162")
    return out


def device_record(dev) -> dict:
    """CU count and architecture from the library; current and peak clocks
    from amd-smi when the tool answers within a few seconds."""
    import shutil
    import subprocess

    topo = dev.topology()
    rec = {"name": topo.name, "arch": topo.arch, "compute_units": topo.compute_units}
    tool = shutil.which("amd-smi")
    if tool:
        try:
            r = subprocess.run([tool, "metric", "--clock", "--json"], capture_output=True, text=True, timeout=15)
            if r.returncode == 0:
                data = json.loads(r.stdout)
                if isinstance(data, dict):
                    data = data.get("gpu_data", [data])
                clock = data[0].get("clock", {}) if data else {}
                picked = {}
                for key in ("gfx_0", "mem_0"):
                    c = clock.get(key)
                    if isinstance(c, dict):
                        picked[key] = {k: (c[k] or {}).get("value") for k in ("clk", "max_clk")
                                       if isinstance(c.get(k), dict)}
                # sampled after the timed runs, so "clk" is usually the idle clock
                rec["clocks_mhz"] = picked or None
        except (OSError, ValueError, AttributeError, TypeError, IndexError, subprocess.SubprocessError):
            rec["clocks_mhz"] = None
    return rec


def run_config(name, hx, dev, args, cpu_seconds):
    """Time one configuration; returns (record, workload dict)."""
    w = globals()[f"wl_{name}"](hx, dev)
    # The 2^30 scan takes 1.4 ms a launch: a quarter of the steps.  The 2^20
    # sum is cache-resident and launch-bound (5 us a launch): ten times the
    # steps, so its timed pass lasts milliseconds like the others' (over 100
    # launches, 0.5 ms, the mean came out 6.7 us against batch medians of
    # 5.0).
    steps = {"scan_f32_2_30": max(5, args.steps // 4), "sum_f32_2_20": max(1000, 10 * args.steps)}.get(name, args.steps)
    t = time_launches(dev, w["run"], steps, args.warmup)
    rec = {"value": round(gbs(w["bytes"], t["mean_ms"]), 1), "unit": "GB/s", "dtype": w["dtype"],
           "workload": w["workload"], "n": w["n"], "algorithmic_bytes_per_launch": w["bytes"], "steps": steps,
           "ms_per_launch": round(t["mean_ms"], 5), "median_ms": round(t["median_ms"], 5),
           "min_ms": round(t["min_ms"], 5), "settle_launches": t["settle_launches"],
           "elements_per_s": round(w["n"] / (t["mean_ms"] * 1e-3), 1),
           "roofline": roofline(w["bytes"], t["mean_ms"], name)}
    if w["verify"] is not None:
        rec["gpu_output_check"] = w["verify"]()
    if cpu_seconds > 0:
        rec["cpu_baseline"] = w["cpu"](cpu_seconds)
    log(f"{name}: {t['mean_ms']:.4f} ms/launch (median {t['median_ms']:.4f}, min {t['min_ms']:.4f}) "
        f"{rec['value']:.1f} GB/s")
    return rec, w


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=("default", "all") + WORKLOADS, default="default")
    ap.add_argument("--cpu-seconds", type=float, default=6.0,
                    help="CPU time for the headline's baseline (each other configuration gets a third)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-summary", metavar="DIR", help="summarise rocprofv3 --pmc runs under DIR and exit")
    ap.add_argument("--trace-summary", metavar="DIR",
                    help="summarise a rocprofv3 --kernel-trace run of the default bench under DIR and exit")
    ap.add_argument("--bench-json", metavar="FILE", help="with --trace-summary: that run's bench JSON line")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed device time per configuration before its warm-up steps")
    args = ap.parse_args()
    globals()["SETTLE_MS"] = args.settle_ms
    if args.pmc_summary:
        return pmc_summary(Path(args.pmc_summary))
    if args.trace_summary:
        return trace_summary(Path(args.trace_summary), Path(args.bench_json) if args.bench_json else None)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world}).", file=sys.stderr)
        return 2

    import hephaestus_amd as hx

    dev = hx.RocmDevice.try_default()
    topo = dev.topology()
    log(f"device {topo.name} {topo.arch} CUs={topo.compute_units} lib={hx.native_library_path()} "
        f"host cores={os.cpu_count()}")

    if args.workload not in ("default", "all"):
        if args.workload in ("scan_u32", "sum_f32", "sum_f32_2_20", "rows_f32", "segmented_i32", "scan_f32_2_30"):
            w = globals()[f"wl_{args.workload}"](hx, dev)
            ms = time_plan(dev, w["run"], args.steps, args.warmup)
            n, nbytes = w["n"], w["bytes"]
        else:
            r = globals()[f"bench_{args.workload}"](hx, dev, args)
            ms, n, nbytes = r["ms"], r["n"], r["bytes"]
        g = gbs(nbytes, ms)
        print(json.dumps({"workload": args.workload, "n": n, "ms": round(ms, 5), "GB/s": round(g, 1),
                          "frac": round(g / PEAK_GBS, 4), "elements_per_s": round(n / (ms * 1e-3), 1)}))
        return 0

    cpu_head = 0.0 if args.no_cpu_baseline else args.cpu_seconds
    cpu_other = cpu_head / 3.0
    # Every configuration's buffers stay resident until the end, as a
    # caller's would: a 1 GiB input allocated into memory that an earlier
    # configuration had freed streamed 4% slower (the f32 sum at 2^28: 154.5
    # us in a fresh process, 161 after the scan's buffers were freed).
    head, w = run_config("scan_u32", hx, dev, args, cpu_head)
    resident = [w]
    secondary = {}
    for key, name in (("f32_sum_reduce_2_28", "sum_f32"), ("cfg1_f32_sum_2_20", "sum_f32_2_20"),
                      ("cfg3_rows_f32_65536x4096", "rows_f32"), ("cfg4_segmented_i32_2_27", "segmented_i32"),
                      ("cfg5_scan_f32_2_30", "scan_f32_2_30")):
        secondary[key], w = run_config(name, hx, dev, args, cpu_other)
        resident.append(w)
    ceil = ceiling(hx, dev, args.steps, args.warmup)
    del resident
    best = max(ceil["copy_kernel"]["GB/s"], ceil["runtime_blit_hipMemcpyAsync"]["GB/s"])
    ceil["best_GB/s"] = best
    ceil["headline_scan_over_best"] = round(head["value"] / best, 4)
    ceil["headline_scan_over_in_order_copy"] = round(head["value"] / ceil["copy_scan_shape_block_order"]["GB/s"], 4)
    ceil["headline_scan_over_lookback_free"] = round(
        head["value"] / ceil["scan_rows_one_tile_no_lookback"]["GB/s"], 4)
    log(f"ceiling: copy kernel {ceil['copy_kernel']['GB/s']} GB/s, runtime blit "
        f"{ceil['runtime_blit_hipMemcpyAsync']['GB/s']} GB/s, scan-shaped copy in block order "
        f"{ceil['copy_scan_shape_block_order']['GB/s']} GB/s, same scan kernel without look-back "
        f"{ceil['scan_rows_one_tile_no_lookback']['GB/s']} GB/s; scan at {ceil['headline_scan_over_best']:.3f} "
        f"of best, {ceil['headline_scan_over_in_order_copy']:.3f} of the in-order copy, "
        f"{ceil['headline_scan_over_lookback_free']:.3f} of itself without look-back")

    line = {
        "metric": "achieved HBM GB/s (% of peak) for f32 sum-reduce and u32 scan at 2^28 elems",
        "value": head["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_launch"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (SplitMix64 seeds, generated in HBM; the BASELINE.json distributions)",
        "config": {"workload": head["workload"], "n": head["n"],
                   "algorithmic_bytes_per_step": head["algorithmic_bytes_per_launch"],
                   "elements_per_s": head["elements_per_s"]},
        "timing": {"mean_ms": head["ms_per_launch"], "median_ms": head["median_ms"], "min_ms": head["min_ms"],
                   "settle_ms": SETTLE_MS, "settle_launches": head["settle_launches"]},
        "roofline": head["roofline"],
    }
    if "cpu_baseline" in head:
        line["cpu_baseline"] = head["cpu_baseline"]
    line["secondary"] = secondary
    line["ceiling"] = ceil
    if args.workload == "all":
        extra = {}
        for name in ("segmented_short_i32", "copy_u32", "dot_f32", "axpy_f32", "colsum_f32", "colscan_u32",
                     "colscan_narrow_u32", "segmented_long_i32", "colscan_rowtile_u32",
                     "colscan_rowtile_wide_u32", "colsum_period_f32", "rows_short_f32"):
            r = globals()[f"bench_{name}"](hx, dev, args)
            g = gbs(r["bytes"], r["ms"])
            extra[name] = {"value": round(g, 1), "unit": "GB/s", "ms_per_launch": round(r["ms"], 5),
                           "roofline": roofline(r["bytes"], r["ms"], name)}
            log(f"{name}: {r['ms']:.4f} ms/launch {g:.1f} GB/s")
        line["extra"] = extra
        line["latency"] = latency_suite(hx, dev, args)
    line["host"] = {"cpu_count": os.cpu_count()}
    line["device"] = device_record(dev)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
