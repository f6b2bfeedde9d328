"""Scans along short dense lines (scan_short_lines_kernel): lines of fewer
than 256 elements packed back to back, scanned as one flat range with a
segmented scan that restarts at each line start.  Every line length from 1
up to 255 that changes the arithmetic (remainders of the 256-element step,
lines of one, two and three elements, lines crossing vector, step, wave and
tile edges), inclusive and exclusive, forward and reverse, sums and
products.  Integers are compared bit for bit with numpy's scan of each row;
f32 sums are held to 2*ceil(log2 len)*eps*sum|x| per output against an f64
scan of each row (a line's own elements only)."""
from __future__ import annotations

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

pytestmark = pytest.mark.gpu

SCAN = hx.RocmScanOps()
TILE = 8 * 64 * 4 * 16  # elements per tile of the short-line kernel
LENS = [1, 2, 3, 4, 5, 7, 8, 13, 16, 31, 32, 33, 64, 100, 127, 128, 129, 200, 255]
KINDS = [(hx.ScanKind.Inclusive, hx.ScanDirection.Forward), (hx.ScanKind.Exclusive, hx.ScanDirection.Forward),
         (hx.ScanKind.Inclusive, hx.ScanDirection.Reverse), (hx.ScanKind.Exclusive, hx.ScanDirection.Reverse)]


def _rows_scan(m, op, kind, direction, dtype):
    """numpy's scan of each row (u32 wraps mod 2^32; f32 in f64)."""
    v = m[:, ::-1] if direction == hx.ScanDirection.Reverse else m
    acc = np.uint32 if dtype == np.uint32 else np.float64
    with np.errstate(over="ignore"):
        s = np.cumsum(v, axis=1, dtype=acc) if op == "sum" else np.cumprod(v, axis=1, dtype=acc)
    if kind == hx.ScanKind.Exclusive:
        first = np.zeros if op == "sum" else np.ones
        s = np.concatenate([first((m.shape[0], 1), acc), s[:, :-1]], axis=1)
    return s[:, ::-1] if direction == hx.ScanDirection.Reverse else s


def _lines_for(length):
    # three tiles and a ragged fourth, whatever the line length
    return (3 * TILE + 1000) // length + 1


def _run(device, host, rows, length, op, kind, direction, offset_rows=0):
    buf = device.upload(host)
    out = device.alloc_zeroed(host.dtype, host.size)
    lay = Layout.try_new([rows, length], [length, 1], offset_rows * length)
    opcls = hx.CumSumOp if op == "sum" else hx.CumProdOp
    SCAN.scan_axis_into(device, opcls, StridedView(buf, lay), 1, direction, StridedView(out, lay), kind)
    got = device.download_owned(out)[offset_rows * length:(offset_rows + rows) * length]
    return got.reshape(rows, length)


@pytest.mark.parametrize("kind,direction", KINDS)
@pytest.mark.parametrize("length", LENS)
def test_u32_short_line_sums_bit_exact(device, oracle, length, kind, direction):
    rows = _lines_for(length)
    host = oracle.uniform_int(rows * length, seed=length, lo=0, hi=2**32 - 1)
    got = _run(device, host, rows, length, "sum", kind, direction)
    assert np.array_equal(got, _rows_scan(host.reshape(rows, length), "sum", kind, direction, np.uint32))


@pytest.mark.parametrize("kind,direction", KINDS)
@pytest.mark.parametrize("length", [3, 8, 100, 255])
def test_u32_short_line_products_bit_exact(device, oracle, length, kind, direction):
    rows = _lines_for(length)
    host = (oracle.uniform_int(rows * length, seed=length + 7, lo=0, hi=2**32 - 1) | 1).astype(np.uint32)
    got = _run(device, host, rows, length, "prod", kind, direction)
    assert np.array_equal(got, _rows_scan(host.reshape(rows, length), "prod", kind, direction, np.uint32))


@pytest.mark.parametrize("kind,direction", KINDS)
@pytest.mark.parametrize("length", [1, 2, 5, 16, 33, 128, 200, 255])
def test_f32_short_line_sums_within_bound(device, oracle, length, kind, direction):
    rows = _lines_for(length)
    host = oracle.uniform_real(rows * length, seed=length + 3, lo=-1.0, hi=1.0)
    got = _run(device, host, rows, length, "sum", kind, direction).astype(np.float64)
    m = host.reshape(rows, length)
    want = _rows_scan(m, "sum", kind, direction, np.float32)
    ab = _rows_scan(np.abs(m), "sum", kind, direction, np.float32)
    k = 2 * max(1, oracle.ceil_log2(length)) * 2.0**-23
    assert np.all(np.abs(got - want) <= k * ab)


@pytest.mark.parametrize("length", [3, 100])
def test_f32_short_line_products_within_gamma(device, oracle, length):
    rows = _lines_for(length)
    host = oracle.uniform_real(rows * length, seed=length + 9, lo=0.99, hi=1.01)
    got = _run(device, host, rows, length, "prod", hx.ScanKind.Inclusive, hx.ScanDirection.Forward)
    want = _rows_scan(host.reshape(rows, length), "prod", hx.ScanKind.Inclusive, hx.ScanDirection.Forward,
                      np.float32)
    g = length * 2.0**-24
    assert np.all(np.abs(got.astype(np.float64) - want) <= g / (1 - g) * np.abs(want))


@pytest.mark.parametrize("length", [5, 100])
def test_short_lines_of_a_row_range(device, oracle, length):
    """Rows r0 .. r0 + rows of a larger matrix: the view starts mid-buffer
    (element offset r0 * len, any 4-byte alignment) and the rows around it
    stay untouched."""
    total_rows, r0 = _lines_for(length) + 50, 17
    rows = total_rows - r0 - 9
    host = oracle.uniform_int(total_rows * length, seed=length + 11, lo=0, hi=1000)
    buf = device.upload(host)
    out = device.upload(np.full(host.size, 7, np.uint32))
    lay = Layout.try_new([rows, length], [length, 1], r0 * length)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 1, hx.ScanDirection.Forward,
                        StridedView(out, lay), hx.ScanKind.Inclusive)
    got = device.download_owned(out)
    want = np.cumsum(host.reshape(total_rows, length)[r0:r0 + rows], axis=1, dtype=np.uint32)
    assert np.array_equal(got[r0 * length:(r0 + rows) * length].reshape(rows, length), want)
    assert np.all(got[:r0 * length] == 7) and np.all(got[(r0 + rows) * length:] == 7)


def test_short_line_plans_need_no_workspace(device):
    x = device.alloc_zeroed(np.uint32, 1000 * 100)
    y = device.alloc_zeroed(np.uint32, 1000 * 100)
    lay = Layout.c_contiguous([1000, 100])
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(x, lay), 1, hx.ScanDirection.Forward,
                                  StridedView(y, lay), hx.ScanKind.Inclusive)
    assert plan.workspace_bytes() == 0
    plan.dispatch()
    plan.destroy()
