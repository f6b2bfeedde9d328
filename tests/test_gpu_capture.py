"""HIP graph capture, the look-back tag range and the tagged-word formats.

* Prepared plans dispatched on a capturing stream record a clear of their
  status words and run with the tag reserved for captured work, so the
  instantiated graph replays correctly any number of times with new inputs
  (prepared plans observe writes to their bound buffers:
  crates/hephaestus-conformance/src/full_reduction.rs:173-208).  Replays are
  interleaved with eager dispatches of the same plans and eager immediate
  calls, with synchronisations between them, and every result is checked
  against the oracle.
* Immediate entry points refuse a capturing stream before queueing anything.
* The eager tag range wraps after 2^30 - 2 launches on one workspace; the
  wrapping launch clears the status words first (driven here with
  hx_debug_set_launch_count).
* Partial slots of the one-launch reductions never read a scan's status
  words as current partials (the two formats share a workspace region and a
  tag counter).
"""
from __future__ import annotations

import ctypes
import gc

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView, _ffi

pytestmark = pytest.mark.gpu

FULL = hx.RocmFullReductionOps()
SCAN = hx.RocmScanOps()
SEG = hx.RocmSegmentedReductionOps()
EPS = 2.0 ** -23
CAPTURE_MODE_GLOBAL = 0
LAST_EAGER_TAG = (1 << 14) - 2  # eager tags cycle through [1, 2^14 - 1)


def _hip():
    return ctypes.CDLL("libamdhip64.so")


class Stream:
    """A caller-owned default-priority stream."""

    def __init__(self):
        self.handle = ctypes.c_void_p()
        assert _hip().hipStreamCreate(ctypes.byref(self.handle)) == 0

    @property
    def value(self):
        return self.handle.value

    def sync(self):
        assert _hip().hipStreamSynchronize(self.handle) == 0

    def close(self, device):
        self.sync()
        _ffi.check(_ffi.lib().hx_stream_release(device.handle, self.handle))
        _hip().hipStreamDestroy(self.handle)


class Capture:
    """hipStreamBeginCapture .. hipStreamEndCapture, then an instantiated graph."""

    def __init__(self, stream: Stream):
        self.stream = stream
        self.graph = ctypes.c_void_p()
        self.exec = ctypes.c_void_p()

    def __enter__(self):
        gc.disable()  # no buffer may be freed (an unsafe call) during a global-mode capture
        assert _hip().hipStreamBeginCapture(self.stream.handle, CAPTURE_MODE_GLOBAL) == 0
        return self

    def __exit__(self, *exc):
        err = _hip().hipStreamEndCapture(self.stream.handle, ctypes.byref(self.graph))
        gc.enable()
        assert err == 0, f"hipStreamEndCapture failed: {err}"
        if exc[0] is None:
            assert _hip().hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0) == 0
        return False

    def replay(self):
        assert _hip().hipGraphLaunch(self.exec, self.stream.handle) == 0
        self.stream.sync()

    def destroy(self):
        if self.exec:
            _hip().hipGraphExecDestroy(self.exec)
        if self.graph:
            _hip().hipGraphDestroy(self.graph)


def _flat(buf):
    return StridedView(buf, Layout.c_contiguous([len(buf)]))


def _one(buf):
    return StridedView(buf, Layout.c_contiguous([1]))


def _f32_sum_ok(got, x, oracle):
    ref, ab = oracle.full_sum(x)
    n = x.size
    return abs(float(got) - ref) <= 2 * max(1, (n - 1).bit_length()) * EPS * ab


class Workloads:
    """Plans of every tagged kind over buffers that the test rewrites."""

    def __init__(self, device, oracle):
        self.device, self.oracle = device, oracle
        self.n_scan = 70 * 32768 + 123          # 71 u32 tiles: two superblocks, a ragged last tile
        self.n_fscan = 5 * 49152 + 77           # f32 tiles carry f64 statuses
        self.n_sum = 3_000_001                  # 733 blocks of partial slots
        self.n_seg = 1_000_003
        self.xs = device.alloc_zeroed(np.uint32, self.n_scan)
        self.ys = device.alloc_zeroed(np.uint32, self.n_scan)
        self.xf = device.alloc_zeroed(np.float32, self.n_fscan)
        self.yf = device.alloc_zeroed(np.float32, self.n_fscan)
        self.xr = device.alloc_zeroed(np.float32, self.n_sum)
        self.out_sum = device.alloc_zeroed(np.float32, 1)
        self.xm = device.alloc_zeroed(np.uint32, self.n_sum)
        self.out_max = device.alloc_zeroed(np.uint32, 1)
        self.vals = device.alloc_zeroed(np.int32, self.n_seg)
        self.offsets = oracle.geometric_offsets(self.n_seg, 300.0, seed=7)
        self.offs = device.upload(self.offsets)
        self.out_seg = device.alloc_zeroed(np.int32, self.offsets.size - 1)
        # Axis-0 scans of narrow matrices: the row-tile look-back over C-wide
        # carries (u32: 7 tiles of 5440 rows; f32, mirrored and exclusive:
        # 6 tiles of 1360 rows with f64 carries).
        self.rc = (6 * 5440 + 7, 3)
        self.fc = (5 * 1360 + 3, 12)
        self.xc = device.alloc_zeroed(np.uint32, self.rc[0] * self.rc[1])
        self.yc = device.alloc_zeroed(np.uint32, self.rc[0] * self.rc[1])
        self.xfc = device.alloc_zeroed(np.float32, self.fc[0] * self.fc[1])
        self.yfc = device.alloc_zeroed(np.float32, self.fc[0] * self.fc[1])
        lay_c, lay_f = Layout.c_contiguous(list(self.rc)), Layout.c_contiguous(list(self.fc))
        self.plans = [
            SCAN.prepare_scan_axis(device, hx.CumSumOp, _flat(self.xs), 0, hx.ScanDirection.Forward,
                                   _flat(self.ys), hx.ScanKind.Exclusive),
            SCAN.prepare_scan_axis(device, hx.CumSumOp, _flat(self.xf), 0, hx.ScanDirection.Forward,
                                   _flat(self.yf), hx.ScanKind.Inclusive),
            FULL.prepare_reduce_full(device, hx.SumOp, _flat(self.xr), _one(self.out_sum)),
            FULL.prepare_reduce_full(device, hx.MaxOp, _flat(self.xm), _one(self.out_max)),
            SEG.prepare_segmented_sum(device, self.vals, self.offs, self.out_seg),
            SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(self.xc, lay_c), 0, hx.ScanDirection.Forward,
                                   StridedView(self.yc, lay_c), hx.ScanKind.Inclusive),
            SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(self.xfc, lay_f), 0, hx.ScanDirection.Reverse,
                                   StridedView(self.yfc, lay_f), hx.ScanKind.Exclusive),
        ]

    def refill(self, seed):
        o, d = self.oracle, self.device
        self.h_xs = o.uniform_int(self.n_scan, seed=seed, lo=0, hi=255)
        self.h_xf = o.uniform_real(self.n_fscan, seed=seed + 1, lo=0.0, hi=1.0)
        self.h_xr = o.uniform_real(self.n_sum, seed=seed + 2, lo=-1.0, hi=1.0)
        self.h_xm = o.uniform_int(self.n_sum, seed=seed + 3, lo=0, hi=2**32 - 1)
        self.h_vals = o.uniform_int(self.n_seg, seed=seed + 4, lo=-1000, hi=1000, dtype=np.int32)
        self.h_xc = o.uniform_int(self.rc[0] * self.rc[1], seed=seed + 5, lo=0, hi=2**32 - 1)
        self.h_xfc = o.uniform_real(self.fc[0] * self.fc[1], seed=seed + 6, lo=-1.0, hi=1.0)
        for buf, host in ((self.xs, self.h_xs), (self.xf, self.h_xf), (self.xr, self.h_xr),
                          (self.xm, self.h_xm), (self.vals, self.h_vals), (self.xc, self.h_xc),
                          (self.xfc, self.h_xfc)):
            d.write_buffer(buf, host)
        for buf in (self.ys, self.yf, self.out_sum, self.out_max, self.out_seg, self.yc, self.yfc):
            d.write_buffer(buf, np.zeros(len(buf), buf.dtype))

    def check(self, what):
        o, d = self.oracle, self.device
        assert np.array_equal(d.download_owned(self.ys), o.scan_sum(self.h_xs, exclusive=True)), f"{what}: u32 scan"
        ref, absref = o.scan_sum(self.h_xf)
        bad, _ = o.check_f32_bound(d.download_owned(self.yf), ref, absref, self.n_fscan)
        assert bad == 0, f"{what}: f32 scan"
        assert _f32_sum_ok(d.download_owned(self.out_sum)[0], self.h_xr, o), f"{what}: f32 sum"
        assert d.download_owned(self.out_max)[0] == self.h_xm.max(), f"{what}: u32 max"
        assert np.array_equal(d.download_owned(self.out_seg), o.segmented_sum(self.h_vals, self.offsets)), \
            f"{what}: segmented sum"
        r, c = self.rc
        want = np.cumsum(self.h_xc.reshape(r, c), axis=0, dtype=np.uint32)
        assert np.array_equal(d.download_owned(self.yc).reshape(r, c), want), f"{what}: u32 column scan"
        r, c = self.fc
        got = d.download_owned(self.yfc).reshape(r, c)
        cols = self.h_xfc.reshape(r, c)
        for j in range(c):
            ref, absref = o.scan_sum(np.ascontiguousarray(cols[:, j]), exclusive=True, reverse=True)
            bad, _ = o.check_f32_bound(np.ascontiguousarray(got[:, j]), ref, absref, r)
            assert bad == 0, f"{what}: f32 column scan, column {j}"


def test_captured_plans_replay_with_new_inputs(device, oracle):
    w = Workloads(device, oracle)
    s = Stream()
    try:
        w.refill(seed=100)
        cap = Capture(s)
        with cap:
            for p in w.plans:
                p.dispatch(s.value)
        try:
            for rep in range(3):
                w.refill(seed=200 + 10 * rep)
                cap.replay()
                w.check(f"replay {rep}")
                # Eager dispatches of the same plans on the device stream
                # between replays, then an eager immediate call.
                w.refill(seed=300 + 10 * rep)
                for p in w.plans:
                    p.dispatch()
                w.check(f"eager dispatch after replay {rep}")
                ys = device.alloc_zeroed(np.uint32, w.n_scan)
                SCAN.exclusive_scan_into(device, w.xs, ys)
                assert np.array_equal(device.download_owned(ys), oracle.scan_sum(w.h_xs, exclusive=True))
        finally:
            cap.destroy()
    finally:
        s.close(device)


def test_captured_batch_replays(device, oracle):
    """hx_plan_dispatch_batch on a capturing stream, replayed twice."""
    w = Workloads(device, oracle)
    s = Stream()
    try:
        w.refill(seed=400)
        arr = (ctypes.c_void_p * len(w.plans))(*[p.handle for p in w.plans])
        cap = Capture(s)
        with cap:
            _ffi.check(_ffi.lib().hx_plan_dispatch_batch(arr, len(w.plans), s.value))
        try:
            for rep in range(2):
                w.refill(seed=500 + 10 * rep)
                cap.replay()
                w.check(f"batch replay {rep}")
        finally:
            cap.destroy()
    finally:
        s.close(device)


def test_immediate_calls_refuse_a_capturing_stream(device, oracle):
    """Immediate entry points fail with DispatchFailed before queueing
    anything, and leave their outputs untouched."""
    n = 3 * 32768 + 5
    x = device.upload(oracle.uniform_int(n, seed=9, lo=0, hi=255))
    sentinel = np.full(n, 0xA5A5A5A5, np.uint32)
    y = device.upload(sentinel)
    out = device.upload(np.array([7], np.uint32))
    vals = device.upload(oracle.uniform_int(n, seed=10, lo=-5, hi=5, dtype=np.int32))
    offsets = oracle.geometric_offsets(n, 30.0, seed=11)
    offs = device.upload(offsets)
    seg = device.upload(np.full(offsets.size - 1, 3, np.int32))
    s = Stream()
    try:
        cap = Capture(s)
        with cap:
            with pytest.raises(hx.DispatchFailed, match="HIP graph"):
                SCAN.exclusive_scan_into(device, x, y, stream=s.value)
            with pytest.raises(hx.DispatchFailed, match="HIP graph"):
                FULL.reduce_full_into(device, hx.SumOp, _flat(x), _one(out), stream=s.value)
            with pytest.raises(hx.DispatchFailed, match="HIP graph"):
                SEG.segmented_sum_into(device, vals, offs, seg, stream=s.value)
        cap.replay()  # an empty graph
        cap.destroy()
        assert np.array_equal(device.download_owned(y), sentinel)
        assert device.download_owned(out)[0] == 7
        assert np.all(device.download_owned(seg) == 3)
    finally:
        s.close(device)


def test_captured_noalloc_scan_replays(device, oracle):
    """hx_scan_noalloc (the entry point for callers that cannot allocate)
    recorded into a graph: clear kernel + scan, replayed with new inputs."""
    n = 40 * 32768 + 999
    x = device.alloc_zeroed(np.uint32, n)
    y = device.alloc_zeroed(np.uint32, n)
    s = Stream()
    try:
        cap = Capture(s)
        with cap:
            SCAN.scan_axis_into_noalloc(device, hx.CumSumOp, _flat(x), 0, hx.ScanDirection.Forward, _flat(y),
                                        hx.ScanKind.Exclusive, s.value)
        try:
            for rep in range(3):
                h = oracle.uniform_int(n, seed=600 + rep, lo=0, hi=2**32 - 1)
                device.write_buffer(x, h)
                cap.replay()
                assert np.array_equal(device.download_owned(y), oracle.scan_sum(h, exclusive=True)), rep
        finally:
            cap.destroy()
    finally:
        s.close(device)


def _set_launches(device, plan=None, stream=None, launches=0):
    _ffi.check(_ffi.lib().hx_debug_set_launch_count(device.handle, plan.handle if plan else None, stream,
                                                    launches))


def test_tag_wrap_on_a_plan(device, oracle):
    """A plan's launch that wraps the eager tag range clears its status words
    and still scans, reduces and sums correctly."""
    w = Workloads(device, oracle)
    w.refill(seed=700)
    for p in w.plans:
        p.dispatch()              # tag 1
    w.check("tag 1")
    for p in w.plans:
        _set_launches(device, plan=p, launches=LAST_EAGER_TAG - 1)
    w.refill(seed=710)
    for p in w.plans:
        p.dispatch()              # the last eager tag
    w.check("last tag")
    w.refill(seed=720)
    for p in w.plans:
        p.dispatch()              # wraps: clear, then tag 1 again
    w.check("wrapped")
    w.refill(seed=730)
    for p in w.plans:
        p.dispatch()              # tag 2
    w.check("after the wrap")


def test_tag_wrap_on_a_stream(device, oracle):
    """The same wrap on a stream's immediate workspace."""
    n = 70 * 32768 + 3
    s = Stream()
    try:
        x = device.upload(oracle.uniform_int(n, seed=800, lo=0, hi=255))
        y = device.alloc_zeroed(np.uint32, n)
        SCAN.exclusive_scan_into(device, x, y, stream=s.value)
        _set_launches(device, stream=s.value, launches=LAST_EAGER_TAG - 1)
        for seed in (801, 802, 803):
            h = oracle.uniform_int(n, seed=seed, lo=0, hi=255)
            device.write_buffer(x, h)
            SCAN.exclusive_scan_into(device, x, y, stream=s.value)
            s.sync()
            assert np.array_equal(device.download_owned(y), oracle.scan_sum(h, exclusive=True)), seed
            hf = oracle.uniform_real(n, seed=seed, lo=-1.0, hi=1.0)
            xf = device.upload(hf)
            o = device.alloc_zeroed(np.float32, 1)
            FULL.reduce_full_into(device, hx.SumOp, _flat(xf), _one(o), stream=s.value)
            s.sync()
            assert _f32_sum_ok(device.download_owned(o)[0], hf, oracle), seed
    finally:
        s.close(device)


def test_debug_launch_count_needs_a_known_stream(device):
    s = Stream()
    try:
        with pytest.raises(hx.InvalidConfiguration, match="no immediate workspace"):
            _set_launches(device, stream=s.value, launches=5)
    finally:
        s.close(device)


def test_full_reduce_after_a_scan_on_a_fresh_stream(device, oracle):
    """A scan at tag t leaves status words whose high half is 4t + flag; the
    full reduction at tag 4t + 2 (and the dot at 4t + 1) that follows on the
    same stream must not take them for its partial slots."""
    s = Stream()
    try:
        n_scan = 40 * 32768                       # 40 tiles of status words
        hs = oracle.uniform_int(n_scan, seed=900, lo=0, hi=255)
        x = device.upload(hs)
        y = device.alloc_zeroed(np.uint32, n_scan)
        SCAN.exclusive_scan_into(device, x, y, stream=s.value)          # tag 1: words 5 / 6
        tiny = device.upload(np.ones(16, np.uint32))
        o = device.alloc_zeroed(np.uint32, 1)
        for _ in range(3):                                            # tags 2..4, one block each
            FULL.reduce_full_into(device, hx.SumOp, _flat(tiny), _one(o), stream=s.value)
        n = 1 << 24
        hu = oracle.uniform_int(n, seed=901, lo=0, hi=2**32 - 1)
        xu = device.upload(hu)
        hf = oracle.uniform_real(n, seed=902, lo=-1.0, hi=1.0)
        xf = device.upload(hf)
        ou = device.alloc_zeroed(np.uint32, 1)
        of = device.alloc_zeroed(np.float32, 1)
        FULL.reduce_full_into(device, hx.SumOp, _flat(xu), _one(ou), stream=s.value)  # tag 5 = 4*1 + 1
        FULL.reduce_full_into(device, hx.SumOp, _flat(xf), _one(of), stream=s.value)  # tag 6 = 4*1 + 2
        s.sync()
        assert int(device.download_owned(ou)[0]) == int(hu.astype(np.uint64).sum() % (1 << 32))
        assert _f32_sum_ok(device.download_owned(of)[0], hf, oracle)
        assert np.array_equal(device.download_owned(y), oracle.scan_sum(hs, exclusive=True))
    finally:
        s.close(device)


def test_stream_release_frees_and_recreates(device, oracle):
    """hx_stream_release drops a stream's immediate buffers; a later call on
    the same stream builds new ones; releasing twice, or NULL, is a no-op."""
    n = 5 * 32768 + 1
    h = oracle.uniform_int(n, seed=950, lo=0, hi=255)
    x = device.upload(h)
    y = device.alloc_zeroed(np.uint32, n)
    s = Stream()
    try:
        for _ in range(2):
            SCAN.exclusive_scan_into(device, x, y, stream=s.value)
            s.sync()
            assert np.array_equal(device.download_owned(y), oracle.scan_sum(h, exclusive=True))
            _ffi.check(_ffi.lib().hx_stream_release(device.handle, s.handle))
            _ffi.check(_ffi.lib().hx_stream_release(device.handle, s.handle))
            device.write_buffer(y, np.zeros(n, np.uint32))
        _ffi.check(_ffi.lib().hx_stream_release(device.handle, None))
    finally:
        s.close(device)
