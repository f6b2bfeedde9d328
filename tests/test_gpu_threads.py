"""Immediate entry points shared by host threads and streams.

The reference device is Send + Sync and every call gets its own partials
(crates/hephaestus-rocm/src/application/pipeline.rs:88,101-108,343).  Here
several host threads issue immediate scans and sums on the device stream and
on two caller-created streams at once; every result must equal the oracle's.
ctypes releases the GIL around each C call, so the threads really overlap
inside the library.
"""
from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ITERS = 50
THREADS = 4
N_SCAN = (1 << 20) + 12345  # 33 look-back tiles, the last one ragged
N_SUM = (1 << 20) + 777
INPUTS = 5  # distinct seeded inputs per thread


def _hip():
    return ctypes.CDLL("libamdhip64.so")


class _Stream:
    """A caller-owned default-priority stream (hipStreamCreate)."""

    def __init__(self):
        self.handle = ctypes.c_void_p()
        err = _hip().hipStreamCreate(ctypes.byref(self.handle))
        assert err == 0, f"hipStreamCreate failed: {err}"

    def close(self):
        if self.handle:
            _hip().hipStreamSynchronize(self.handle)
            _hip().hipStreamDestroy(self.handle)
            self.handle = ctypes.c_void_p()


def test_immediate_calls_from_threads_and_streams(device, oracle):
    import hephaestus_amd as hx
    from hephaestus_amd import Layout, StridedView

    print(f"[threads] {THREADS} threads x {ITERS} scans of {N_SCAN} u32 and sums of {N_SUM} f32", flush=True)
    streams = [_Stream(), _Stream()]
    per_thread_stream = [None, streams[0].handle.value, streams[1].handle.value, None]
    scan_ops, red_ops = hx.RocmScanOps(), hx.RocmFullReductionOps()

    jobs = []
    for t in range(THREADS):
        xs = [oracle.uniform_int(N_SCAN, seed=100 + 10 * t + k, lo=0, hi=2**32 - 1) for k in range(INPUTS)]
        fs = [oracle.uniform_real(N_SUM, seed=200 + 10 * t + k, lo=-1.0, hi=1.0) for k in range(INPUTS)]
        jobs.append({
            "xs": xs, "fs": fs,
            "xb": [device.upload(x) for x in xs], "fb": [device.upload(f) for f in fs],
            "scan_out": [device.alloc_zeroed(np.uint32, N_SCAN) for _ in range(ITERS)],
            "sum_out": [device.alloc_zeroed(np.float32, 1) for _ in range(ITERS)],
            "stream": per_thread_stream[t], "error": None,
        })
    device.synchronize()
    start = threading.Barrier(THREADS)

    def work(job):
        try:
            start.wait()
            lin_s, lin_1 = Layout.c_contiguous([N_SUM]), Layout.c_contiguous([1])
            for i in range(ITERS):
                k = i % INPUTS
                scan_ops.exclusive_scan_into(device, job["xb"][k], job["scan_out"][i], stream=job["stream"])
                red_ops.reduce_full_into(device, hx.SumOp, StridedView(job["fb"][k], lin_s),
                                         StridedView(job["sum_out"][i], lin_1), stream=job["stream"])
        except Exception as exc:  # reported by the main thread
            job["error"] = exc

    threads = [threading.Thread(target=work, args=(job,)) for job in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
        assert not th.is_alive(), "a host thread did not finish"
    device.synchronize()
    for s in streams:
        s.close()

    tol_log = 2 * oracle.ceil_log2(N_SUM) * 2.0**-23
    for t, job in enumerate(jobs):
        assert job["error"] is None, f"thread {t}: {job['error']}"
        want_scan = [oracle.scan_sum(x, exclusive=True) for x in job["xs"]]
        want_sum = [oracle.full_sum(f) for f in job["fs"]]
        for i in range(ITERS):
            k = i % INPUTS
            got = device.download_owned(job["scan_out"][i])
            assert np.array_equal(got, want_scan[k]), f"thread {t} iteration {i}: scan differs"
            s = float(device.download_owned(job["sum_out"][i])[0])
            ref, ab = want_sum[k]
            assert abs(s - ref) <= tol_log * ab, f"thread {t} iteration {i}: sum {s} vs {ref}"


def test_immediate_scratch_grows_under_queued_work(device, oracle):
    """A larger call on a stream grows that stream's buffers while launches
    queued on it may still read the old ones: the old buffer must not be
    freed under them.  Chunked column scans (fewer than 256 lines) stage
    their chunk totals in the stream's scratch: small ones are queued, a
    large one forces the scratch past its first 1 MiB, then small ones run
    again, all without a host synchronisation in between."""
    import hephaestus_amd as hx
    from hephaestus_amd import Layout, StridedView

    ops = hx.RocmScanOps()
    stream = _Stream()
    try:
        cols = 252  # a multiple of 4 below 256 lines: the chunked column scan
        small_rows, big_rows = 4096, 1 << 17  # 128 and 4096 chunks: 0.13 MB and 4.1 MB of totals
        rng = np.random.default_rng(11)
        small = [rng.integers(0, 2**32, small_rows * cols, dtype=np.uint32) for _ in range(3)]
        big = rng.integers(0, 2**32, big_rows * cols, dtype=np.uint32)
        ls, lb = Layout.c_contiguous([small_rows, cols]), Layout.c_contiguous([big_rows, cols])
        sb = [device.upload(x) for x in small]
        bb = device.upload(big)
        outs = [device.alloc_zeroed(np.uint32, small_rows * cols) for _ in range(6)]
        big_out = device.alloc_zeroed(np.uint32, big_rows * cols)
        s = stream.handle.value
        print(f"[threads] chunked column scans [{small_rows},{cols}] x3, [{big_rows},{cols}], x3", flush=True)
        for k in range(3):
            ops.scan_axis_into(device, hx.CumSumOp, StridedView(sb[k], ls), 0, hx.ScanDirection.Forward,
                               StridedView(outs[k], ls), stream=s)
        ops.scan_axis_into(device, hx.CumSumOp, StridedView(bb, lb), 0, hx.ScanDirection.Forward,
                           StridedView(big_out, lb), stream=s)
        for k in range(3):
            ops.scan_axis_into(device, hx.CumSumOp, StridedView(sb[k], ls), 0, hx.ScanDirection.Forward,
                               StridedView(outs[3 + k], ls), stream=s)
        device.synchronize()
        for k in range(6):
            want = np.cumsum(small[k % 3].reshape(small_rows, cols), axis=0, dtype=np.uint32).ravel()
            assert np.array_equal(device.download_owned(outs[k]), want), k
        want = np.cumsum(big.reshape(big_rows, cols), axis=0, dtype=np.uint32).ravel()
        assert np.array_equal(device.download_owned(big_out), want)
    finally:
        stream.close()
