"""CPU tests of bench.py's offline helpers (no GPU needed).

The trace summary must price each configuration over the launches the bench
timed: the settle and warm-up launches at the start of a configuration are
skipped, so the trace step time compares with the event-timed mean.
"""
from __future__ import annotations

import csv
import json

import bench


def _write_trace(path, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, grid, t0, us in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size_X": grid, "Start_Timestamp": t0,
                        "End_Timestamp": t0 + int(us * 1000)})


def test_trace_summary_skips_untimed_launches(tmp_path, capsys):
    scan = "void scan_tiles_kernel<unsigned int, OpSum, PackedStatus, true, true, false, 16, true, 8>(ScanParams)"
    grid = 8192 * 512
    # 2 settle + 1 warm-up launches at 1000 us, then 5 timed at 350 us, then
    # 4 launches of a later leg on the same kernel and grid (the ceiling's
    # one-tile-per-row scan) at 341 us; the rows are written out of order to
    # check the sort by start time.
    durations = [1000.0, 1000.0, 1000.0] + [350.0] * 5 + [341.0] * 4
    rows = [(scan, grid, 1_000_000 * (i + 1), d) for i, d in enumerate(durations)]
    trace_dir = tmp_path / "stats"
    trace_dir.mkdir()
    _write_trace(trace_dir / "x_kernel_trace.csv", list(reversed(rows)))
    bj = tmp_path / "bench.json"
    bj.write_text(json.dumps({"warmup": 1, "steps": 5, "ms_per_step": 0.35,
                              "timing": {"settle_launches": 2}, "secondary": {}, "ceiling": {}}))
    assert bench.trace_summary(trace_dir, bj) == 0
    out = capsys.readouterr().out
    line = next(ln for ln in out.splitlines() if ln.startswith("| u32 exclusive scan 2^28"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    # label, kernels, skipped, taken, mean sum, median sum, bench us, trace frac, bench frac
    assert cells[2] == "3" and cells[3] == "5"
    assert cells[4] == "350.0" and cells[5] == "350.0"
    assert cells[6] == "350.0"
    assert abs(float(cells[7]) - (8 << 28) / 350e-6 / 8e12) < 1e-4
    # The per-kernel table still lists every dispatch.
    kline = next(ln for ln in out.splitlines() if ln.startswith("| `void scan_tiles_kernel"))
    assert f"| {grid} | 12 |" in kline


def test_trace_summary_without_bench_json_keeps_every_launch(tmp_path, capsys):
    scan = "void scan_tiles_kernel<unsigned int, OpSum>(ScanParams)"
    rows = [(scan, 8192 * 512, 1000 * (i + 1), d) for i, d in enumerate([100.0, 300.0])]
    trace_dir = tmp_path / "stats"
    trace_dir.mkdir()
    _write_trace(trace_dir / "y_kernel_trace.csv", rows)
    assert bench.trace_summary(trace_dir, None) == 0
    out = capsys.readouterr().out
    line = next(ln for ln in out.splitlines() if ln.startswith("| u32 exclusive scan 2^28"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[2] == "0" and cells[3] == "-" and cells[4] == "200.0"


class _FakeEvent:
    def __init__(self, clock):
        self.clock = clock
        self.t = 0.0

    def record(self):
        self.t = self.clock["ms"]

    def synchronize(self):
        self.clock["syncs"] += 1

    def elapsed_ms(self, other):
        return other.t - self.t


class _FakeDevice:
    """Each launch advances a fake device clock by `ms_per_launch`."""

    def __init__(self, ms_per_launch):
        self.clock = {"ms": 0.0, "syncs": 0}
        self.ms = ms_per_launch
        self.launches = 0

    @property
    def syncs(self):
        return self.clock["syncs"]

    def event(self):
        return _FakeEvent(self.clock)

    def synchronize(self):
        pass

    def launch(self):
        self.launches += 1
        self.clock["ms"] += self.ms


def test_settle_runs_until_its_device_time_has_passed():
    dev = _FakeDevice(0.35)
    n = bench.settle(dev, dev.launch, 100.0)
    assert n == dev.launches
    # just past 100 ms of device time, in two batches: the 10-launch
    # calibration, then the rest back to back
    assert 100.0 <= n * 0.35 <= 100.0 + 2 * 0.35
    assert dev.syncs == 2
    assert bench.settle(dev, dev.launch, 0.0) == 0


def test_time_launches_reports_settle_and_times_exactly_the_steps():
    dev = _FakeDevice(2.0)
    bench.SETTLE_MS, saved = 20.0, bench.SETTLE_MS
    try:
        t = bench.time_launches(dev, dev.launch, steps=10, warmup=3)
    finally:
        bench.SETTLE_MS = saved
    assert t["settle_launches"] == 10
    assert t["mean_ms"] == 2.0 and t["median_ms"] == 2.0 and t["min_ms"] == 2.0
    # settle + warm-up + timed pass + five batches of two
    assert dev.launches == 10 + 3 + 10 + 10
