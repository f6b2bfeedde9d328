"""The forward-progress fallbacks, forced from the host.

Every bounded wait in the library has a fallback that makes progress without
the block it waits for. A look-back (scans, column scans, segmented sums)
computes a missing predecessor from the input. The gathering block of a
one-launch reduction (full reduce, map-reductions) recomputes a missing
partial from the operand. In normal runs these almost never fire, so
hx_debug_set_wait_limits sets the limits to 0 and to 1 here:

- look-back 0: every unpublished predecessor is computed at once;
- gather 0: every partial is recomputed by the gathering block.

Each result is compared with the same call at the default limits and with
the oracle. Integer results and f32 reductions must be bit-identical. f32
scans must stay within their bound. A superblock rebuilt by a fallback may
differ from its owner's value in the last bits, so the f32 scans are not
compared bit for bit."""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView, _ffi

from test_gpu_axis import run_column_scan

pytestmark = pytest.mark.gpu

FULL = hx.RocmFullReductionOps()
SCAN = hx.RocmScanOps()
SEG = hx.RocmSegmentedReductionOps()
DEFAULT_LIMITS = (64, 1 << 14)
FORCED = [(0, 0), (1, 1)]


@contextlib.contextmanager
def wait_limits(lookback, gather):
    lib = _ffi.lib()
    _ffi.check(lib.hx_debug_set_wait_limits(lookback, gather))
    try:
        yield
    finally:
        _ffi.check(lib.hx_debug_set_wait_limits(*DEFAULT_LIMITS))


def _full_results(device, xf, xu):
    """Every full-reduction kind on an f32 and a u32 operand, plus the
    map-reductions, as one list of scalars."""
    n = xf.size
    lay = Layout.c_contiguous([n])
    one = Layout.c_contiguous([1])
    fb, ub = device.upload(xf), device.upload(xu)
    res = []
    for op, buf, dt in [(hx.SumOp, fb, np.float32), (hx.SumOp, ub, np.uint32), (hx.MaxOp, fb, np.float32),
                        (hx.MinOp, ub, np.uint32), (hx.ProdOp, ub, np.uint32), (hx.MeanOp, fb, np.float32)]:
        out = device.alloc_zeroed(dt, 1)
        FULL.reduce_full_into(device, op, StridedView(buf, lay), StridedView(out, one))
        res.append(device.download_owned(out)[0])
    idx, val = device.alloc_zeroed(np.uint32, 1), device.alloc_zeroed(np.float32, 1)
    FULL.argmax_full_into(device, StridedView(fb, lay), idx, val)
    res += [device.download_owned(idx)[0], device.download_owned(val)[0]]
    for fn in (hx.norm_l1, hx.norm_l2, hx.norm_max):
        res.append(device.download_owned(fn(device, StridedView(fb, lay)))[0])
    res.append(device.download_owned(hx.dot(device, StridedView(fb, lay), StridedView(fb, lay)))[0])
    res.append(device.download_owned(hx.dot(device, StridedView(ub, lay), StridedView(ub, lay)))[0])
    return [np.asarray(r).tobytes() for r in res]


@pytest.mark.parametrize("limits", FORCED)
@pytest.mark.parametrize("n", [1, 5000, (1 << 20) + 3])
def test_full_and_map_reductions_bit_identical_under_forced_fallbacks(device, oracle, limits, n):
    xf = oracle.uniform_real(n, seed=n + 11, lo=-1.0, hi=1.0)
    xu = oracle.uniform_int(n, seed=n + 12, lo=0, hi=2**32 - 1)
    normal = _full_results(device, xf, xu)
    with wait_limits(*limits):
        forced = _full_results(device, xf, xu)
    assert forced == normal
    ref, ab = oracle.full_sum(xf)
    got = np.frombuffer(forced[0], np.float32)[0]
    assert abs(float(got) - ref) <= 2 * (n - 1).bit_length() * 2.0**-23 * ab + abs(ref) * 2.0**-24


def _scan(device, x, exclusive, reverse, out_off=0):
    n = x.size
    buf = device.upload(x)
    out = device.alloc_zeroed(x.dtype, n + out_off)
    lay = Layout.c_contiguous([n])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 0,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward,
                        StridedView(out, Layout.try_new([n], [1], out_off)),
                        hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive)
    return device.download_owned(out)[out_off:]


# 2^21 + 5 u32: 65 tiles of 32768, so both look-back levels (superblocks of
# 64 tiles) and the ragged last tile run; f32 lines take the same tiles.
@pytest.mark.parametrize("limits", FORCED)
@pytest.mark.parametrize("exclusive,reverse", [(True, False), (False, True)])
def test_scans_under_forced_fallbacks(device, oracle, limits, exclusive, reverse):
    n = (1 << 21) + 5
    xu = oracle.uniform_int(n, seed=5, lo=0, hi=2**32 - 1)
    xf = oracle.uniform_real(n, seed=6, lo=0.0, hi=1.0)
    normal_u = _scan(device, xu, exclusive, reverse)
    with wait_limits(*limits):
        forced_u = _scan(device, xu, exclusive, reverse)
        forced_f = _scan(device, xf, exclusive, reverse)
        # an output off a 16-byte boundary: lines then run on the output's
        # grid, their first tile partial (rebuilt with its bounds)
        shifted_u = _scan(device, xu, exclusive, reverse, out_off=3)
    assert np.array_equal(forced_u, normal_u)
    assert np.array_equal(shifted_u, normal_u)
    assert np.array_equal(forced_u, oracle.scan_sum(xu, exclusive=exclusive, reverse=reverse))
    ref, ab = oracle.scan_sum(xf, exclusive=exclusive, reverse=reverse)
    bad, worst = oracle.check_f32_bound(forced_f, ref, ab, n)
    assert bad == 0, worst


# Single-pass column look-back (256 lines and more): integer and f32 lines,
# sums and products, forward and reverse; 1003 lines leave a partial last
# group, whose rebuilt aggregates read only the lines that exist.
@pytest.mark.parametrize("limits", FORCED)
@pytest.mark.parametrize("dtype", [np.uint32, np.float32])
@pytest.mark.parametrize("reverse", [False, True])
def test_column_lookback_scans_under_forced_fallbacks(device, oracle, limits, dtype, reverse):
    with wait_limits(*limits):
        run_column_scan(device, oracle, "sum", dtype, (4099, 1000), (1000, 1), 0, 0, False, reverse, seed=17)
        run_column_scan(device, oracle, "prod", dtype, (3001, 512), (512, 1), 0, 0, True, reverse, seed=19)
        run_column_scan(device, oracle, "sum", dtype, (2001, 1003), (1003, 1), 0, 0, True, reverse, seed=21)


# Row-tile column look-back (axis 0 of dense matrices with 2 to 255 columns
# outside the narrow form): a missing predecessor's column aggregate is
# rebuilt from the input by the waiting thread.  13, 15 and 47 tiles.
@pytest.mark.parametrize("limits", FORCED)
@pytest.mark.parametrize("dtype", [np.uint32, np.float32])
@pytest.mark.parametrize("reverse", [False, True])
def test_row_tile_lookback_scans_under_forced_fallbacks(device, oracle, limits, dtype, reverse):
    with wait_limits(*limits):
        run_column_scan(device, oracle, "sum", dtype, (70001, 3), (3, 1), 0, 0, False, reverse, seed=23)
        run_column_scan(device, oracle, "prod", dtype, (20001, 12), (12, 1), 0, 0, True, reverse, seed=29)
        run_column_scan(device, oracle, "sum", dtype, (3001, 255), (255, 1), 0, 0, True, reverse, seed=31)


def _segmented(device, values, offsets):
    vb = device.upload(values)
    ob = device.upload(offsets.astype(np.uint32))
    out = device.upload(np.full(offsets.size - 1, 0x5A5A5A5A, np.uint32).view(values.dtype))
    SEG.segmented_sum_into(device, vb, ob, out)
    return device.download_owned(out)


# Element tiles of 8192 values (mean 300) and 16384 values (mean 50000,
# where nearly no tile holds a segment start, so look-backs chain far).  At
# 2^24 values (1024 tiles, 16 superblocks) mean 50000 takes the two-level
# look-back, which folds missing superblocks from their tiles, and mean 10^6
# the one-level walk over tiles.
@pytest.mark.parametrize("limits", FORCED)
@pytest.mark.parametrize("n,mean", [(1 << 21, 300.0), (1 << 21, 50000.0), (1 << 24, 50000.0), (1 << 24, 1e6)])
def test_segmented_sums_under_forced_fallbacks(device, oracle, limits, n, mean):
    x = oracle.uniform_int(n, seed=23, lo=-1000, hi=1000, dtype=np.int32)
    off = oracle.geometric_offsets(n, mean, seed=29)
    normal = _segmented(device, x, off)
    with wait_limits(*limits):
        forced = _segmented(device, x, off)
    assert np.array_equal(forced, normal)
    assert np.array_equal(forced, oracle.segmented_sum(x, off))


def test_default_wait_limits_are_restored(device, oracle):
    """A scan after the forced runs is still the default path (bit-exact)."""
    x = oracle.uniform_int(1 << 20, seed=31, lo=0, hi=255)
    assert np.array_equal(_scan(device, x, True, False), oracle.scan_sum(x, exclusive=True))
