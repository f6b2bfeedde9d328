#!/usr/bin/env python3
"""Throughput of the reduction / scan hot path on one MI355X.

Metric: achieved HBM GB/s (and fraction of the 8 TB/s peak)
for the u32 exclusive scan and the f32 sum-reduce at 2^28 elements.  A step
is one exclusive scan of the 2^28-element u32 operand (the headline configuration); inputs
are generated in HBM before timing, and every step is one launch of the
single-pass look-back scan kernel.  The f32 sum-reduce at 2^28 is timed the
same way and reported under "secondary".

`value` and `roofline.achieved` are algorithmic bytes (read 4n + write 4n
for the scan) divided by the mean launch time, measured with HIP events on
the stream the kernels run on.  `cpu_baseline` times the CPU oracle (a
sequential port of the same semantics) on this host over the same input.

Usage: python bench.py [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

PEAK_GBS = 8000.0  # MI355X HBM3E
WORKLOADS = ("scan_u32", "sum_f32", "rows_f32", "segmented_i32", "segmented_short_i32", "scan_f32_2_30",
             "copy_u32", "dot_f32", "axpy_f32", "colsum_f32", "colscan_u32")
# Dominant kernel of each workload (substring of its name in rocprofv3 output).
KERNEL_OF = {"scan_u32": "scan_tiles_kernel", "sum_f32": "full_reduce_kernel<", "rows_f32": "rows_kernel",
             "segmented_i32": "segmented_sum_kernel", "segmented_short_i32": "seg_short_kernel",
             "scan_f32_2_30": "scan_tiles_kernel",
             "copy_u32": "copy_tiles_kernel", "dot_f32": "map_reduce_kernel<", "axpy_f32": "vector_tiles_kernel<1",
             "colsum_f32": "cols_tiles_kernel", "colscan_u32": "col_lookback_kernel"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_plan(dev, run, steps: int, warmup: int) -> float:
    """Mean milliseconds per launch of `run` over `steps` back-to-back launches."""
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
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if any."""
    f = REPO / "profiles" / "pmc_traffic.json"
    if not f.exists():
        return None
    data = json.loads(f.read_text())
    entry = data.get(name)
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def roofline(bytes_per_launch: float, ms: float, name: str) -> dict:
    achieved = bytes_per_launch / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_for(name)}


def bench_scan_u32(hx, dev, args):
    from hephaestus_amd import Layout, StridedView

    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=2, lo=0, hi=255)
    out = dev.alloc_uninitialized(np.uint32, n)
    lay = Layout.c_contiguous([n])
    plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                              StridedView(out, lay), hx.ScanKind.Exclusive)
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    nbytes = 2 * 4 * n
    return {"n": n, "ms": ms, "bytes": nbytes, "x": x, "out": out}


def bench_sum_f32(hx, dev, args):
    from hephaestus_amd import Layout, StridedView

    n = 1 << 28
    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=1, lo=-1.0, hi=1.0)
    out = dev.alloc_zeroed(np.float32, 1)
    plan = hx.RocmFullReductionOps().prepare_reduce_full(dev, hx.SumOp, StridedView(x, Layout.c_contiguous([n])),
                                                         StridedView(out, Layout.c_contiguous([1])))
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    return {"n": n, "ms": ms, "bytes": 4 * n + 4, "x": x, "out": out}


def bench_rows_f32(hx, dev, args):
    rows, cols = 65536, 4096
    x = dev.alloc_uninitialized(np.float32, rows * cols)
    dev.fill_normal(x, seed=3)
    s = dev.alloc_uninitialized(np.float32, rows)
    m = dev.alloc_uninitialized(np.float32, rows)
    i = dev.alloc_uninitialized(np.uint32, rows)
    ops = hx.RocmAxisReductionOps()
    run = lambda: ops.reduce_rows_fused(dev, x, rows, cols, prologue=(0.5, 0.25), out_sum=s, out_max=m, out_argmax=i)
    ms = time_plan(dev, run, args.steps, args.warmup)
    return {"n": rows * cols, "ms": ms, "bytes": 4 * rows * cols + 12 * rows}


def bench_segmented_i32(hx, dev, args):
    from oracle import oracle  # geometric offsets are generated on the host

    n = 1 << 27
    x = dev.alloc_uninitialized(np.int32, n)
    dev.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    off = oracle.geometric_offsets(n, 300.0, seed=5)
    ob = dev.upload(off)
    out = dev.alloc_uninitialized(np.int32, off.size - 1)
    plan = hx.RocmSegmentedReductionOps().prepare_segmented_sum(dev, x, ob, out)
    ms = time_plan(dev, plan.dispatch, args.steps, args.warmup)
    s = off.size - 1
    return {"n": n, "ms": ms, "bytes": 4 * n + 4 * (s + 1) + 4 * s}


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


def bench_scan_f32_2_30(hx, dev, args):
    from hephaestus_amd import Layout, StridedView

    n = 1 << 30
    x = dev.alloc_uninitialized(np.float32, n)
    dev.fill_uniform_real(x, seed=6, lo=0.0, hi=1.0)
    out = dev.alloc_uninitialized(np.float32, n)
    lay = Layout.c_contiguous([n])
    plan = hx.RocmScanOps().prepare_scan_axis(dev, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                              StridedView(out, lay))
    ms = time_plan(dev, plan.dispatch, max(1, args.steps // 4), max(1, args.warmup // 2))
    return {"n": n, "ms": ms, "bytes": 8 * n}


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


def bench_copy_u32(hx, dev, args):
    """The device copy kernel behind copy_buffer over 2^28 u32: the yardstick
    (read B + write B) for the HBM byte counters, and the streaming ceiling."""
    n = 1 << 28
    x = dev.alloc_uninitialized(np.uint32, n)
    dev.fill_uniform_int(x, seed=7, lo=0, hi=255)
    y = dev.alloc_uninitialized(np.uint32, n)
    ms = time_plan(dev, lambda: dev.copy_buffer(x, y), args.steps, args.warmup)
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


def cpu_baseline(dev, scan, seconds: float) -> dict:
    """Time the oracle's sequential exclusive scan on this host's cores over
    the same 2^28-element input; verify the GPU output against it."""
    from oracle import oracle

    x = dev.download_owned(scan["x"])
    got = dev.download_owned(scan["out"])
    n = x.size
    out = np.empty_like(x)
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.lib().hxo_scan_sum_u32(x.ctypes.data, n, 1, 0, out.ctypes.data)
        reps += 1
        el = time.perf_counter() - t0
        if el >= seconds or reps >= 50:
            break
    per = el / reps
    verified = bool(np.array_equal(got, out))
    threads = min(16, os.cpu_count() or 1)
    t1 = time.perf_counter()
    oracle.scan_excl_u32_threads(x, out, threads)
    tt = time.perf_counter() - t1
    return {
        "value": round(8 * n / per / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"the full 2^28-element u32 exclusive scan, {reps} sequential passes of the C oracle "
                  f"(oracle/hx_oracle.c hxo_scan_sum_u32), {per * 1e3:.1f} ms per pass",
        "multithread": {"value": round(8 * n / tt / 1e9, 3), "cores": threads,
                        "sample": "one pass of the two-pass pthread scan hxo_scan_excl_u32_threads"},
        "gpu_output_verified": verified,
    }


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


def _cpu_rate(run, bytes_per_pass: float, seconds: float = 2.0, max_reps: int = 20):
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


def cpu_secondary(name: str, seconds: float) -> dict | None:
    """The oracle (one host core, kind "port") on a bounded host-generated
    sample of a secondary workload; rates are per algorithmic byte like the
    GPU figure.  None for workloads the oracle has no function for."""
    from oracle import oracle

    def line(gbs, reps, ms, sample):
        return {"value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"{sample}; {reps} passes, {ms:.1f} ms per pass"}

    if name == "sum_f32":
        n = 1 << 26
        x = oracle.uniform_real(n, 1, -1.0, 1.0)
        r = _cpu_rate(lambda: oracle.full_sum(x), 4.0 * n, seconds)
        return line(*r, "2^26 f32 (a quarter of the GPU input), oracle full_sum (f64 accumulation)")
    if name == "rows_f32":
        rows, cols = 4096, 4096
        x = oracle.normal(rows * cols, 3)
        r = _cpu_rate(lambda: oracle.rows(x, rows, cols, prologue=(0.5, 0.25)), 4.0 * rows * cols + 12.0 * rows,
                      seconds)
        return line(*r, "4096 x 4096 f32 (1/16 of the GPU rows), oracle rows (sum, max, argmax of fmaf(.5,x,.25))")
    if name == "segmented_i32":
        n = 1 << 25
        x = oracle.uniform_int(n, 4, -1000, 1000, dtype=np.int32)
        off = oracle.geometric_offsets(n, 300.0, seed=5)
        s = off.size - 1
        r = _cpu_rate(lambda: oracle.segmented_sum(x, off), 4.0 * n + 8.0 * s + 4, seconds)
        return line(*r, f"2^25 i32 values, {s} geometric(300) segments, oracle segmented_sum")
    if name == "segmented_short_i32":
        n = 1 << 25
        x = oracle.uniform_int(n, 4, -1000, 1000, dtype=np.int32)
        off = oracle.geometric_offsets(n, 4.0, seed=5)
        s = off.size - 1
        r = _cpu_rate(lambda: oracle.segmented_sum(x, off), 4.0 * n + 8.0 * s + 4, seconds)
        return line(*r, f"2^25 i32 values, {s} geometric(4) segments, oracle segmented_sum")
    if name == "scan_f32_2_30":
        n = 1 << 23
        x = oracle.uniform_real(n, 6, 0.0, 1.0)
        r = _cpu_rate(lambda: oracle.scan_sum(x), 8.0 * n, seconds)
        return line(*r, "2^23 f32 (1/128 of the GPU input), oracle scan_sum (compensated f64 prefix and |prefix|)")
    if name == "dot_f32":
        n = 1 << 26
        a, b = oracle.uniform_real(n, 1, -1.0, 1.0), oracle.uniform_real(n, 2, -1.0, 1.0)
        r = _cpu_rate(lambda: oracle.dot(a, b), 8.0 * n, seconds)
        return line(*r, "2^26 f32 pairs, oracle dot (exact products, f64 accumulation)")
    if name == "axpy_f32":
        n = 1 << 24
        a, b = oracle.uniform_real(n, 1, -1.0, 1.0), oracle.uniform_real(n, 2, -1.0, 1.0)
        r = _cpu_rate(lambda: oracle.fma_arrays(a, b, 0.5), 12.0 * n, seconds)
        return line(*r, "2^24 f32, oracle fma_arrays (libm fmaf per element)")
    return None


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


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=("default", "all") + WORKLOADS, default="default")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-summary", metavar="DIR", help="summarise rocprofv3 --pmc runs under DIR and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        return pmc_summary(Path(args.pmc_summary))

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE={world}).", file=sys.stderr)
        return 2

    import hephaestus_amd as hx

    dev = hx.RocmDevice.try_default()
    topo = dev.topology()
    log(f"device {topo.name} {topo.arch} CUs={topo.compute_units} lib={hx.native_library_path()}")

    if args.workload not in ("default", "all"):
        fn = globals()[f"bench_{args.workload}"]
        r = fn(hx, dev, args)
        gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
        print(json.dumps({"workload": args.workload, "n": r["n"], "ms": round(r["ms"], 5),
                          "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4),
                          "elements_per_s": round(r["n"] / (r["ms"] * 1e-3), 1)}))
        return 0

    scan = bench_scan_u32(hx, dev, args)
    log(f"scan u32 2^28: {scan['ms']:.4f} ms/launch")
    ssum = bench_sum_f32(hx, dev, args)
    log(f"sum f32 2^28: {ssum['ms']:.4f} ms/launch")

    value = scan["bytes"] / (scan["ms"] * 1e-3) / 1e9
    line = {
        "metric": "achieved HBM GB/s (% of peak) for f32 sum-reduce and u32 scan at 2^28 elems",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(scan["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic (SplitMix64 seed 2, uniform integers in [0,256), generated in HBM)",
        "config": {"workload": "u32 exclusive prefix scan, n=2^28 (the headline configuration)",
                   "n": scan["n"], "algorithmic_bytes_per_step": scan["bytes"],
                   "elements_per_s": round(scan["n"] / (scan["ms"] * 1e-3), 1)},
        "roofline": roofline(scan["bytes"], scan["ms"], "scan_u32"),
        "secondary": {
            "f32_sum_reduce_2_28": {
                "value": round(ssum["bytes"] / (ssum["ms"] * 1e-3) / 1e9, 1), "unit": "GB/s",
                "ms_per_launch": round(ssum["ms"], 5),
                "elements_per_s": round(ssum["n"] / (ssum["ms"] * 1e-3), 1),
                "roofline": roofline(ssum["bytes"], ssum["ms"], "sum_f32"),
            }
        },
    }
    if args.workload == "all":
        for name in ("rows_f32", "segmented_i32", "segmented_short_i32", "scan_f32_2_30", "copy_u32", "dot_f32",
                     "axpy_f32", "colsum_f32", "colscan_u32"):
            r = globals()[f"bench_{name}"](hx, dev, args)
            gbs = r["bytes"] / (r["ms"] * 1e-3) / 1e9
            line["secondary"][name] = {"value": round(gbs, 1), "unit": "GB/s", "ms_per_launch": round(r["ms"], 5),
                                       "elements_per_s": round(r["n"] / (r["ms"] * 1e-3), 1),
                                       "roofline": roofline(r["bytes"], r["ms"], name)}
            if not args.no_cpu_baseline:
                cb = cpu_secondary(name, 2.0)
                if cb is not None:
                    line["secondary"][name]["cpu_baseline"] = cb
            log(f"{name}: {r['ms']:.4f} ms/launch {gbs:.1f} GB/s")
    if args.workload == "all":
        line["latency"] = latency_suite(hx, dev, args)
        for name, r in line["latency"].items():
            log(f"{name}: {r['us_per_call']} us per call, {r['gpu_us_per_launch']} us per launch "
                f"(reference WGPU RTX 5080: {r['reference_wgpu_rtx5080_us']} us)")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(dev, scan, args.cpu_seconds)
        line["secondary"]["f32_sum_reduce_2_28"]["cpu_baseline"] = cpu_secondary("sum_f32", 2.0)
    line["device"] = device_record(dev)
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
