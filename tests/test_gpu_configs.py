"""The five benchmark configurations at their full sizes on one MI355X.

Inputs are generated in HBM by the library's SplitMix64 fill kernels (whose
bits tests/test_gpu_parity.py pins to the oracle's), downloaded, and checked
against the oracle on the host: integer results bit-exact, f32 results
within 2*ceil(log2 n)*eps_f32*sum|y| of a compensated f64 accumulation.
Size-independent properties (determinism, exclusive = inclusive shifted,
scan differences, a checksum of the segment sums) are checked as well."""
from __future__ import annotations

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

pytestmark = pytest.mark.gpu

FULL = hx.RocmFullReductionOps()
AXIS = hx.RocmAxisReductionOps()
SCAN = hx.RocmScanOps()
SEG = hx.RocmSegmentedReductionOps()
EPS = 2.0**-23


def bound(n, abs_sum):
    return 2 * (int(n) - 1).bit_length() * EPS * abs_sum


def note(msg):
    print(f"[config] {msg}", flush=True)


@pytest.mark.parametrize("log2n", [20, 28])
def test_f32_full_sum(device, oracle, log2n):
    """Config 1 (n = 2^20) and the metric's f32 sum-reduce (n = 2^28)."""
    n = 1 << log2n
    note(f"f32 sum n=2^{log2n}")
    x = device.alloc_uninitialized(np.float32, n)
    device.fill_uniform_real(x, seed=1, lo=-1.0, hi=1.0)
    out = device.alloc_zeroed(np.float32, 1)
    plan = FULL.prepare_reduce_full(device, hx.SumOp, StridedView(x, Layout.c_contiguous([n])),
                                    StridedView(out, Layout.c_contiguous([1])))
    plan.dispatch()
    first = device.download_owned(out)
    plan.dispatch()
    second = device.download_owned(out)
    assert first.view(np.uint32)[0] == second.view(np.uint32)[0]  # deterministic
    host = device.download_owned(x)
    ref, ab = oracle.full_sum(host)
    assert abs(float(first[0]) - ref) <= bound(n, ab)
    # with f64 accumulation the result is the correctly rounded sum
    assert abs(float(first[0]) - ref) <= abs(ref) * 2.0**-24 + 1e-30


def test_u32_exclusive_scan_2_28(device, oracle):
    """Config 2: u32 exclusive scan of 2^28 values in [0, 256)."""
    n = 1 << 28
    note("u32 exclusive scan n=2^28")
    x = device.alloc_uninitialized(np.uint32, n)
    device.fill_uniform_int(x, seed=2, lo=0, hi=255)
    out = device.alloc_uninitialized(np.uint32, n)
    lay = Layout.c_contiguous([n])
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                                  StridedView(out, lay), hx.ScanKind.Exclusive)
    plan.dispatch()
    plan.dispatch()  # second launch on the same workspace (tag rollover path)
    host = device.download_owned(x)
    got = device.download_owned(out)
    assert got[0] == 0
    assert np.array_equal(np.diff(got), host[:-1])  # out[i+1] - out[i] = x[i] mod 2^32
    assert np.array_equal(got, oracle.scan_sum(host, exclusive=True))


def test_f32_rows_sum_max_argmax_with_prologue(device, oracle):
    """Config 3: [65536 x 4096] N(0,1), y = fmaf(0.5, x, 0.25), per-row
    sum, max and argmax from one read."""
    rows, cols = 65536, 4096
    note("rows 65536x4096")
    x = device.alloc_uninitialized(np.float32, rows * cols)
    device.fill_normal(x, seed=3)
    s = device.alloc_uninitialized(np.float32, rows)
    m = device.alloc_uninitialized(np.float32, rows)
    i = device.alloc_uninitialized(np.uint32, rows)
    AXIS.reduce_rows_fused(device, x, rows, cols, prologue=(0.5, 0.25), out_sum=s, out_max=m, out_argmax=i)
    host = device.download_owned(x)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host, rows, cols, prologue=(0.5, 0.25))
    assert np.array_equal(device.download_owned(i), i_ref)
    assert np.array_equal(device.download_owned(m).view(np.uint32), m_ref.view(np.uint32))
    err = np.abs(device.download_owned(s).astype(np.float64) - s_ref)
    assert np.all(err <= bound(cols, a_ref))


def test_i32_segmented_sum_2_27(device, oracle):
    """Config 4: 2^27 values in [-1000, 1000], geometric segments (mean
    300, min 1), u32 offsets."""
    n = 1 << 27
    note("segmented n=2^27")
    x = device.alloc_uninitialized(np.int32, n)
    device.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    off = oracle.geometric_offsets(n, 300.0, seed=5)
    ob = device.upload(off)
    out = device.alloc_uninitialized(np.int32, off.size - 1)
    SEG.validate_offsets(device, ob, n)
    SEG.segmented_sum_into(device, x, ob, out)
    got = device.download_owned(out)
    host = device.download_owned(x)
    assert abs(off.size - 1 - n / 300) < 0.02 * n / 300
    # checksum of checksums: the segment sums add up to the total (mod 2^32)
    assert np.sum(got, dtype=np.int32) == oracle.full_sum(host)
    assert np.array_equal(got, oracle.segmented_sum(host, off))


@pytest.mark.parametrize("mean", [1.0, 4.0, 1e6])
def test_i32_segmented_sum_2_27_short_segments(device, oracle, mean):
    """Config 4's 2^27 values with other geometric segment lengths: means 1
    and 4 take the segment-parallel path, mean 10^6 the 16384-value tiles;
    bit-exact, plus the checksum of checksums."""
    n = 1 << 27
    note(f"segmented n=2^27 mean {mean:g}")
    x = device.alloc_uninitialized(np.int32, n)
    device.fill_uniform_int(x, seed=4, lo=-1000, hi=1000)
    off = oracle.geometric_offsets(n, mean, seed=5)
    ob = device.upload(off)
    out = device.alloc_uninitialized(np.int32, off.size - 1)
    SEG.segmented_sum_into(device, x, ob, out)
    got = device.download_owned(out)
    host = device.download_owned(x)
    assert np.sum(got, dtype=np.int32) == oracle.full_sum(host)
    assert np.array_equal(got, oracle.segmented_sum(host, off))


def test_f32_inclusive_scan_2_30(device, oracle):
    """Config 5: f32 inclusive scan of 2^30 uniform[0,1) values (4 GiB in,
    4 GiB out), every output within the bound."""
    n = 1 << 30
    note("f32 inclusive scan n=2^30")
    x = device.alloc_uninitialized(np.float32, n)
    device.fill_uniform_real(x, seed=6, lo=0.0, hi=1.0)
    out = device.alloc_uninitialized(np.float32, n)
    lay = Layout.c_contiguous([n])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward, StridedView(out, lay))
    got = device.download_owned(out)
    note("f32 scan downloaded; checking")
    host = device.download_owned(x)
    bad, worst = oracle.check_scan_f32(host, got)
    note(f"f32 scan worst |err|/(eps*sum|x|) = {worst:.3f} (bound {2 * 30})")
    assert bad == 0, worst
    assert np.all(np.diff(got[:: 1 << 16]) >= 0)  # monotone for non-negative inputs


def test_f32_column_sum_65536x4096(device, oracle):
    """The column-tile path at the bench shape: axis-0 sum of 65536 x 4096
    N(0,1) f32, every column against the oracle's f64 fold of that column,
    and bitwise equal on a second dispatch (fixed fold order)."""
    r, c = 65536, 4096
    note("f32 axis-0 sum 65536x4096")
    x = device.alloc_uninitialized(np.float32, r * c)
    device.fill_normal(x, seed=7)
    out = device.alloc_zeroed(np.float32, c)
    plan = AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(x, Layout.c_contiguous([r, c])), 0,
                                         StridedView(out, Layout.c_contiguous([1, c])))
    plan.dispatch()
    first = device.download_owned(out)
    plan.dispatch()
    assert np.array_equal(first.view(np.uint32), device.download_owned(out).view(np.uint32))
    cols = np.ascontiguousarray(device.download_owned(x).reshape(r, c).T)
    for j in range(c):
        ref, ab = oracle.full_sum(cols[j])
        assert abs(float(first[j]) - ref) <= bound(r, ab), j


def test_u32_column_scan_65536x4096(device, oracle):
    """The chunked column scan at the bench shape, inclusive and exclusive:
    every element bit-exact against the wrapped cumulative sum of its
    column."""
    r, c = 65536, 4096
    note("u32 axis-0 scan 65536x4096")
    x = device.alloc_uninitialized(np.uint32, r * c)
    device.fill_uniform_int(x, seed=8, lo=0, hi=255)
    out = device.alloc_uninitialized(np.uint32, r * c)
    lay = Layout.c_contiguous([r, c])
    host = device.download_owned(x).reshape(r, c)
    want = np.cumsum(host, axis=0, dtype=np.uint32)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward, StridedView(out, lay))
    assert np.array_equal(device.download_owned(out).reshape(r, c), want)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive)
    assert np.array_equal(device.download_owned(out).reshape(r, c), want - host)
