"""Axis reductions and axis scans on the shapes that need the split forms:
tall matrices reduced or scanned along axis 0 (column tiles over chunks of
the axis), few long rows reduced along axis 1 (split rows), transposed and
negative-stride views, every op and dtype.  Each output line is checked
against the oracle's fold of the same line: bit-exact for integers, max, min
and argmax; f32 sums within 2*ceil(log2 n)*eps_f32*sum|y| of the oracle's
f64 accumulation; f32 products (no oracle function) against numpy's f64
product."""
from __future__ import annotations

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

pytestmark = pytest.mark.gpu

AXIS = hx.RocmAxisReductionOps()
SCAN = hx.RocmScanOps()
EPS = 2.0**-23
OPS = {"sum": hx.SumOp, "mean": hx.MeanOp, "prod": hx.ProdOp, "min": hx.MinOp, "max": hx.MaxOp,
       "argmax": hx.ArgMaxOp}


def f32_bound(n, abs_sum):
    return 2 * (int(n) - 1).bit_length() * EPS * abs_sum


def prod_bound(n):
    """gamma_{n-1} = (n-1)u / (1 - (n-1)u), u = 2^-24: the relative error
    bound of any evaluation order of a product of n f32 factors.  It exists
    only while (n-1)u < 1; from 2^24 + 1 factors no relative bound holds,
    and the result is inf (a check against it then rejects only NaN; the
    tests' factors lie near 1, so the reference is never 0)."""
    k = (int(n) - 1) * 2.0**-24
    return k / (1.0 - k) if k < 1.0 else float("inf")


def lines_of(host, shape, strides, offset, axis):
    """The reduced lines of a rank-2 view, in output order."""
    idx = offset + np.indices(shape)[0] * strides[0] + np.indices(shape)[1] * strides[1]
    sel = host[idx]
    return np.ascontiguousarray(sel if axis == 1 else sel.T)


def expect(oracle, op, lines):
    if op == "sum":
        return [oracle.full_sum(l) for l in lines]
    if op == "mean":
        return [oracle.full_sum(l) for l in lines]
    if op == "prod":
        if lines.dtype == np.float32:  # no f32 product in the oracle: numpy's f64 product, rtol below
            return [np.prod(l.astype(np.float64)) for l in lines]
        return [oracle.full_prod(l) for l in lines]
    if op == "min":
        return [oracle.full_min(l) for l in lines]
    if op == "max":
        return [oracle.full_max(l) for l in lines]
    return [oracle.full_argmax(l) for l in lines]


def run_axis(device, op, dtype, host, shape, strides, offset, axis):
    buf = device.upload(host)
    nout = shape[1 - axis]
    out_dtype = np.uint32 if op == "argmax" else dtype
    out = device.upload(np.full(nout, 7, out_dtype))
    out_shape = [shape[0], 1] if axis == 1 else [1, shape[1]]
    AXIS.reduce_axis_into(device, OPS[op], StridedView(buf, Layout.try_new(list(shape), list(strides), offset)),
                          axis, StridedView(out, Layout.c_contiguous(out_shape)))
    return device.download_owned(out)


def check(oracle, op, dtype, got, lines):
    want = expect(oracle, op, lines)
    n = lines.shape[1]
    if dtype == np.float32 and op in ("sum", "mean"):
        for g, (ref, ab) in zip(got, want):
            if op == "sum":
                assert abs(float(g) - ref) <= f32_bound(n, ab)
            else:
                assert abs(float(g) - ref / n) <= f32_bound(n, ab) / n + EPS * abs(ref / n)
        return
    if dtype == np.float32 and op == "prod":
        for g, ref in zip(got, want):
            assert abs(float(g) - ref) <= EPS * abs(ref)
        return
    if op == "mean":
        if dtype == np.int32:
            want = [np.int32(int(np.int32(w)) // n if int(np.int32(w)) >= 0 else -((-int(np.int32(w))) // n))
                    for w in want]
        else:
            want = [np.uint32(int(w) // n) for w in want]
    assert np.array_equal(np.asarray(got), np.asarray(want, dtype=got.dtype))


def host_for(oracle, dtype, n, seed, op):
    if dtype == np.float32:
        if op == "prod":
            return oracle.uniform_real(n, seed, 0.999, 1.001)
        return oracle.normal(n, seed)
    if op == "argmax":
        return (oracle.uniform_int(n, seed, 0, 50)).astype(dtype)  # many ties
    if dtype == np.int32:
        return oracle.uniform_int(n, seed, -1000, 1000, dtype=np.int32)
    return oracle.uniform_int(n, seed, 0, 2**32 - 1)


# (rows, cols), axis: tall column tiles (vector and scalar lanes), a single
# chunk, few long rows (vector and scalar), and a [N,1] column.
SHAPES = [((4099, 1000), 0), ((3001, 999), 0), ((20, 256), 0), ((3, 100003), 1), ((5, 65536), 1),
          ((100000, 1), 0),
          # narrow columns, 2 to 95, past 1024 lines (the period form: the
          # dense range in 1 KiB blocks, every P-th block per wave,
          # P = C / gcd(C, 256)): powers of two (P = 1), ranges that end
          # inside a vector or a block, many waves per residue, C = 95
          # (P = 95), 1025 lines; below 1025 lines the one-launch block form,
          # from 96 columns the column tiles again
          ((1048577, 4), 0), ((70001, 8), 0), ((5000, 16), 0), ((3001, 32), 0), ((4096, 2), 0), ((4097, 2), 0),
          ((1, 4), 0),
          ((1048577, 3), 0), ((70001, 5), 0), ((30001, 6), 0), ((20000, 90), 0), ((4099, 95), 0),
          ((9000, 64), 0), ((1025, 7), 0), ((20000, 100), 0), ((4099, 255), 0)]


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("shape,axis", SHAPES)
def test_split_axis_reduce(device, oracle, shape, axis, dtype, op):
    r, c = shape
    host = host_for(oracle, dtype, r * c, seed=r + 3 * c + axis, op=op)
    strides = (c, 1)
    got = run_axis(device, op, dtype, host, shape, strides, 0, axis)
    check(oracle, op, dtype, got, lines_of(host, shape, strides, 0, axis))


@pytest.mark.parametrize("op", ["sum", "max", "argmax"])
def test_axis_reduce_transposed_and_reversed_views(device, oracle, op):
    r, c = 2000, 516
    host = host_for(oracle, np.float32, r * c, seed=91, op=op)
    # column-major view of a [c, r] buffer: axis 1 is strided, outputs adjacent
    shape, strides = (c, r), (1, c)
    got = run_axis(device, op, np.float32, host, shape, strides, 0, 1)
    check(oracle, op, np.float32, got, lines_of(host, shape, strides, 0, 1))
    # outputs walk backwards (stride -1) while the axis is strided
    shape, strides, offset = (r, c), (c, -1), c - 1
    got = run_axis(device, op, np.float32, host, shape, strides, offset, 0)
    check(oracle, op, np.float32, got, lines_of(host, shape, strides, offset, 0))
    # rows read from their ends (axis 1 at stride -1): every op but argmax
    # reads them forwards; then rows in reverse order as well
    for strides, offset in (((c, -1), c - 1), ((-c, -1), r * c - 1)):
        got = run_axis(device, op, np.float32, host, (r, c), strides, offset, 1)
        check(oracle, op, np.float32, got, lines_of(host, (r, c), strides, offset, 1))


# Axis-0 reductions of small matrices (at most 1024 lines and 2^20 elements,
# more than 32 lines) take one launch: a block of 16 waves per group of
# outputs, each wave walking a slice of the axis, the slices folded in LDS.
# [1000, 300] and [1024, 1024] have 16-byte lanes (outputs a multiple of 4),
# [999, 1049] and [77, 5] one output per lane; [1025, 1000] is past the line
# limit and takes the two-launch split.
SMALL_COLUMN_SHAPES = [(256, 256), (1000, 300), (1024, 1024), (999, 1049), (77, 5), (33, 64), (1025, 1000)]


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("shape", SMALL_COLUMN_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_small_column_reductions(device, oracle, shape, dtype, op):
    r, c = shape
    host = host_for(oracle, dtype, r * c, seed=7 * r + c, op=op)
    got = run_axis(device, op, dtype, host, shape, (c, 1), 0, 0)
    check(oracle, op, dtype, got, lines_of(host, shape, (c, 1), 0, 0))


@pytest.mark.parametrize("op", ["sum", "max", "argmax", "min"])
def test_small_column_reductions_of_strided_views(device, oracle, op):
    r, c = 200, 516
    host = host_for(oracle, np.float32, r * c + 3, seed=17, op=op)
    # axis 1 of a column-major view: the outputs are adjacent, the axis strided
    shape, strides = (c, r), (1, c)
    got = run_axis(device, op, np.float32, host, shape, strides, 0, 1)
    check(oracle, op, np.float32, got, lines_of(host, shape, strides, 0, 1))
    # outputs walking backwards, and a view that starts 3 elements in
    for shape, strides, offset in (((r, c), (c, -1), c - 1), ((r, c), (c, 1), 3)):
        got = run_axis(device, op, np.float32, host, shape, strides, offset, 0)
        check(oracle, op, np.float32, got, lines_of(host, shape, strides, offset, 0))


def test_small_column_f32_sums_are_deterministic(device, oracle):
    host = oracle.normal(1000 * 300, seed=23)
    a = run_axis(device, "sum", np.float32, host, (1000, 300), (300, 1), 0, 0)
    b = run_axis(device, "sum", np.float32, host, (1000, 300), (300, 1), 0, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("op", ["sum", "argmax", "min"])
@pytest.mark.parametrize("offset", [4, 1])
@pytest.mark.parametrize("c", [8, 3, 90])
def test_narrow_columns_offset_views(device, oracle, op, offset, c):
    # offset 4 keeps the range 16-byte aligned, offset 1 does not (16-byte
    # vectors need only 4-byte alignment)
    r = 30001
    host = host_for(oracle, np.float32, offset + r * c, seed=offset, op=op)
    got = run_axis(device, op, np.float32, host, (r, c), (c, 1), offset, 0)
    check(oracle, op, np.float32, got, lines_of(host, (r, c), (c, 1), offset, 0))


@pytest.mark.parametrize("r,c", [(8192, 1024), (1 << 20, 3), (40000, 95)])
def test_split_f32_sums_are_deterministic(device, oracle, r, c):
    host = oracle.normal(r * c, seed=5)
    a = run_axis(device, "sum", np.float32, host, (r, c), (c, 1), 0, 0)
    b = run_axis(device, "sum", np.float32, host, (r, c), (c, 1), 0, 0)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# Short dense rows along axis 1 (1 to 255 elements a row, rows back to
# back): tiles of (8192 // C) & ~3 whole rows staged in LDS, a row per
# thread up to 63 elements and groups of 2, 4 or 8 lanes a row beyond
# (64: 2, 127-200: 4, 255: 8).  Row counts give several tiles and a ragged
# last one; offsets 1-3 start the matrix off a 16-byte boundary.  (256,
# 100) is the first length past the tiles (lane groups again).
SHORT_ROWS = [(1, 3 * 8192 + 5, 0), (2, 3 * 4096 + 1, 1), (3, 2 * 2728 + 7, 2), (4, 5 * 2048 + 3, 3),
              (5, 2 * 1636 + 1, 0), (6, 3000, 1), (7, 5000, 2), (8, 2049, 0), (12, 1366, 3), (15, 2 * 544 + 9, 1),
              (16, 1000, 0), (33, 3 * 248 + 5, 1), (64, 3 * 128 + 1, 0), (100, 2 * 80 + 3, 2), (127, 3 * 64 + 1, 3),
              (128, 300, 1), (160, 2 * 48 + 5, 2), (255, 3 * 32 + 1, 3), (256, 100, 0)]


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("c,rows,offset", SHORT_ROWS)
def test_short_row_axis_reduce(device, oracle, c, rows, offset, dtype, op):
    host = host_for(oracle, dtype, offset + rows * c + 3, seed=7 * c + rows, op=op)
    got = run_axis(device, op, dtype, host, (rows, c), (c, 1), offset, 1)
    check(oracle, op, dtype, got, lines_of(host, (rows, c), (c, 1), offset, 1))


# Short rows a little apart (row stride L > C, within 2C or 32 elements):
# the tiles load the padding with the rows, ((8192 - C) // L + 1) & ~3 rows a
# tile.  Odd and even distances (scalar and vector LDS reads), one-element
# rows of a wider matrix, groups of lanes a row (100 of 130, 200 of 203),
# and past the limits (L = 40 for 4 elements, L = 260 for 150): the lane
# groups again.
PADDED_ROWS = [(4, 5, 5000, 1), (3, 4, 7000, 0), (1, 7, 9000, 2), (12, 16, 2000, 3), (2, 32, 1000, 1),
               (7, 9, 3000, 0), (100, 120, 300, 2), (100, 130, 100, 1), (200, 203, 100, 3), (4, 40, 500, 0),
               (150, 260, 100, 1)]


@pytest.mark.parametrize("op", ["sum", "max", "argmax", "prod"])
@pytest.mark.parametrize("dtype", [np.float32, np.int32])
@pytest.mark.parametrize("c,ld,rows,offset", PADDED_ROWS)
def test_padded_short_row_axis_reduce(device, oracle, c, ld, rows, offset, dtype, op):
    host = host_for(oracle, dtype, offset + rows * ld + 3, seed=11 * c + ld, op=op)
    got = run_axis(device, op, dtype, host, (rows, c), (ld, 1), offset, 1)
    check(oracle, op, dtype, got, lines_of(host, (rows, c), (ld, 1), offset, 1))


def test_single_column_rows_of_any_column_stride(device, oracle):
    """[N, 1] views reduced along axis 1: the column stride of a one-element
    row is never used, so every stride takes the short-row tiles."""
    rows = 3 * 8192 + 11
    host = oracle.normal(rows + 5, seed=3)
    for strides in [(1, 1), (1, 5), (1, 0), (1, -3)]:
        got = run_axis(device, "max", np.float32, host, (rows, 1), strides, 2, 1)
        assert np.array_equal(got.view(np.uint32), host[2:2 + rows].view(np.uint32))


@pytest.mark.parametrize("c", [1, 2, 3, 5, 8, 15, 24, 64, 127, 192, 255])
@pytest.mark.parametrize("offset", [0, 1])
def test_fused_short_rows_many_tiles(device, oracle, c, offset):
    rows = 3 * ((8192 // c) & ~3) + 77
    host = oracle.normal(offset + rows * c, seed=c + 40 * offset)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host[offset:], rows, c, prologue=(0.5, 0.25))
    buf = device.upload(host)
    s = device.alloc_zeroed(np.float32, rows)
    m = device.alloc_zeroed(np.float32, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    AXIS.reduce_rows_fused(device, buf, rows, c, c, offset, (0.5, 0.25), s, m, i)
    assert np.array_equal(device.download_owned(i), i_ref)
    assert np.array_equal(device.download_owned(m).view(np.uint32), m_ref.view(np.uint32))
    bound = np.array([f32_bound(c, a) for a in a_ref])
    assert np.all(np.abs(device.download_owned(s).astype(np.float64) - s_ref) <= bound)


@pytest.mark.parametrize("subset", ["sum+max+argmax", "sum", "argmax"])
def test_fused_rows_with_few_long_rows(device, oracle, subset):
    rows, cols = 3, (1 << 20) + 12
    host = oracle.normal(rows * cols, seed=17)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host, rows, cols, prologue=(0.5, 0.25))
    buf = device.upload(host)
    want = subset.split("+")
    s = device.upload(np.full(rows, 7.0, np.float32)) if "sum" in want else None
    m = device.upload(np.full(rows, 7.0, np.float32)) if "max" in want else None
    i = device.upload(np.full(rows, 7, np.uint32)) if "argmax" in want else None
    AXIS.reduce_rows_fused(device, buf, rows, cols, out_sum=s, out_max=m, out_argmax=i, prologue=(0.5, 0.25))
    if s is not None:
        assert np.all(np.abs(device.download_owned(s) - s_ref) <= [f32_bound(cols, a) for a in a_ref])
    if m is not None:
        assert np.array_equal(device.download_owned(m), m_ref)
    if i is not None:
        assert np.array_equal(device.download_owned(i), i_ref)


def test_prepared_split_axis_reduce_rebinds(device, oracle):
    r, c = 4096, 512
    x = oracle.uniform_int(r * c, seed=2, lo=0, hi=1000)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, c)
    plan = AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(buf, Layout.c_contiguous([r, c])), 0,
                                    StridedView(out, Layout.c_contiguous([1, c])))
    assert plan.workspace_bytes() > 0
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), x.reshape(r, c).sum(axis=0, dtype=np.uint32))
    y = oracle.uniform_int(r * c, seed=3, lo=0, hi=1000)
    device.write_buffer(buf, y)
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), y.reshape(r, c).sum(axis=0, dtype=np.uint32))


# ------------------------------------------------------------ column scans
def scan_lines_want(oracle, op, lines, exclusive, reverse):
    """Per line: the oracle's scan (ints: bit-exact; f32 sum: (ref, |prefix|))."""
    if op == "sum":
        return [oracle.scan_sum(l, exclusive=exclusive, reverse=reverse) for l in lines]
    if lines.dtype == np.float32:  # no f32 product scan in the oracle: numpy's f64 product, rtol below
        out = []
        for l in lines:
            v = l.astype(np.float64)[::-1] if reverse else l.astype(np.float64)
            c = np.cumprod(v)
            if exclusive:
                c = np.concatenate([[1.0], c[:-1]])
            out.append(c[::-1] if reverse else c)
        return out
    return [oracle.scan_prod(l, exclusive=exclusive, reverse=reverse) for l in lines]


def run_column_scan(device, oracle, op, dtype, shape, strides, offset, axis, exclusive, reverse, seed):
    r, c = shape
    size = offset + 1 + sum((shape[d] - 1) * abs(strides[d]) for d in range(2))
    if dtype == np.float32:
        host = (oracle.uniform_real(size, seed, 0.999, 1.001) if op == "prod"
                else oracle.uniform_real(size, seed, -1.0, 1.0))
    elif dtype == np.int32:
        host = oracle.uniform_int(size, seed, -1000, 1000, dtype=np.int32)
    else:
        host = oracle.uniform_int(size, seed, 0, 2**32 - 1)
    buf = device.upload(host)
    out = device.upload(np.full(size, 7, dtype))
    lay = Layout.try_new(list(shape), list(strides), offset)  # the output mirrors the input's layout
    SCAN.scan_axis_into(device, hx.CumSumOp if op == "sum" else hx.CumProdOp, StridedView(buf, lay), axis,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive)
    got_host = device.download_owned(out)
    got_lines = lines_of(got_host, shape, strides, offset, axis)
    touched = np.zeros(size, bool)
    touched[offset + np.indices(shape)[0] * strides[0] + np.indices(shape)[1] * strides[1]] = True
    assert np.all(got_host[~touched] == 7)
    lines = lines_of(host, shape, strides, offset, axis)
    want = scan_lines_want(oracle, op, lines, exclusive, reverse)
    n = lines.shape[1]
    for g, w in zip(got_lines, want):
        if dtype == np.float32 and op == "sum":
            bad, worst = oracle.check_f32_bound(g, w[0], w[1], n)
            assert bad == 0, worst
        elif dtype == np.float32:
            # Products: relative rounding errors compound along the line (the
            # reference's serial f32 products behave the same way), so the
            # bound is the textbook one for a product of n floats, gamma_{n-1}
            # relative (Higham, Accuracy and Stability, sec. 3.1).
            assert np.all(np.abs(g.astype(np.float64) - w) <= prod_bound(n) * np.abs(w))
        else:
            assert np.array_equal(g, w)


# (rows, cols) scanned along axis 0.  Single-pass look-back (256 lines and
# more): 16-byte lanes over many chunks, line counts 3, 1 and 2 past a
# multiple of 4 (the last group's lane moves its lines one by one), one tile
# only; the chunked form with 130 lines.
COLUMN_SHAPES = [(4099, 1000), (3001, 999), (3001, 1001), (2000, 1022), (20, 256), (5000, 130),
                 # narrow columns (32, 64, 128): the dense range scanned with
                 # strided lane scans, one or many chunks
                 (4097, 32), (1000, 64), (3001, 128),
                 # other columns below 256: row tiles of up to 16384 elements
                 # staged through LDS, a thread per column and row group.  Up
                 # to 24 columns one pass with a look-back over C-wide carries
                 # (257 tiles for 2 and 4 columns), wider three passes; many
                 # tiles with a partial last one, a single tile, one row
                 ((1 << 20) + 1, 2), ((1 << 20) + 3, 4), (70001, 3), (30001, 5), (4099, 7), (70001, 8),
                 (20001, 12), (65536, 16), (5000, 24), (3000, 100), (1000, 200), (3001, 255), (5, 3), (5, 4),
                 (1, 6)]


@pytest.mark.parametrize("kind", ["inclusive", "exclusive"])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("op", ["sum", "prod"])
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("shape", COLUMN_SHAPES)
def test_column_scan(device, oracle, shape, dtype, op, reverse, kind):
    r, c = shape
    run_column_scan(device, oracle, op, dtype, shape, (c, 1), 0, 0, kind == "exclusive", reverse,
                    seed=r * 7 + c)


# Many short lines in the column layout (lines adjacent, steps far apart):
# up to 64 steps over at least 1024 line groups take one read-and-write pass
# with no carries.  Axis 0 of row-major [L, M] with vector lanes (M a
# multiple of 4) and scalar lanes, and axis 1 of a column-major [M, 3].
# Expected values: numpy's wrapped integer scans, and for f32 sums an f64
# scan with the usual bound.
SHORT_COLUMN_SCANS = [((4, 1 << 20), (1 << 20, 1), 0), ((3, (1 << 18) + 1), ((1 << 18) + 1, 1), 0),
                      ((32, 1 << 18), (1 << 18, 1), 0), (((1 << 18) + 3, 3), (1, (1 << 18) + 3), 1)]


@pytest.mark.parametrize("kind", ["inclusive", "exclusive"])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("op,dtype", [("sum", np.uint32), ("sum", np.int32), ("prod", np.uint32),
                                      ("sum", np.float32)])
@pytest.mark.parametrize("shape,strides,axis", SHORT_COLUMN_SCANS)
def test_column_scan_of_many_short_lines(device, oracle, shape, strides, axis, op, dtype, reverse, kind):
    size = shape[0] * shape[1]
    if dtype == np.float32:
        host = oracle.uniform_real(size, 41, -1.0, 1.0)
    elif dtype == np.int32:
        host = oracle.uniform_int(size, 42, -1000, 1000, dtype=np.int32)
    else:
        host = oracle.uniform_int(size, 43, 0, 2**32 - 1)
    buf = device.upload(host)
    out = device.upload(np.full(size, 7, dtype))
    lay = Layout.try_new(list(shape), list(strides), 0)
    SCAN.scan_axis_into(device, hx.CumSumOp if op == "sum" else hx.CumProdOp, StridedView(buf, lay), axis,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive if kind == "exclusive" else hx.ScanKind.Inclusive)
    lines = lines_of(host, shape, strides, 0, axis).T  # steps along axis 0
    got = lines_of(device.download_owned(out), shape, strides, 0, axis).T
    v = lines[::-1] if reverse else lines
    acc = np.float64 if dtype == np.float32 else np.uint32
    with np.errstate(over="ignore"):
        want = np.cumsum(v, axis=0, dtype=acc) if op == "sum" else np.cumprod(v, axis=0, dtype=acc)
        ab = np.cumsum(np.abs(v.astype(np.float64)), axis=0)
    if kind == "exclusive":
        first = np.zeros if op == "sum" else np.ones
        want = np.concatenate([first((1, v.shape[1]), acc), want[:-1]])
        ab = np.concatenate([np.zeros((1, v.shape[1])), ab[:-1]])
    if reverse:
        want, ab = want[::-1], ab[::-1]
    if dtype == np.float32:
        n = lines.shape[0]
        bad, worst = oracle.check_f32_bound(np.ascontiguousarray(got).ravel(), np.ascontiguousarray(want).ravel(),
                                            np.ascontiguousarray(ab).ravel(), n)
        assert bad == 0, worst
    else:
        assert np.array_equal(got.view(np.uint32), want.astype(np.uint32))


# Row-wise (axis 1) scans of many lines: a line of up to 32768 elements is one
# tile of the smallest shape that holds it (256, 512, 1024, 2048, 4096, 8192,
# 16384 or 32768 elements), longer lines chain 32768-element tiles.  Lengths either
# side of every boundary; "misaligned" rows (stride cols + 1, offset 1) take
# the scalar path of each shape.
ROW_SCAN_SHAPES = [(300, 256), (300, 257), (130, 512), (130, 513), (67, 1024), (67, 1025), (33, 2048),
                   (33, 2049), (17, 4096), (17, 4100), (9, 8192), (9, 8193), (5, 16384), (5, 16385), (3, 32769),
                   (130, 3)]
ROW_SCAN_VARIANTS = [("sum", False, False, True), ("sum", True, True, True), ("prod", False, False, True),
                     ("sum", False, True, False), ("sum", True, False, False)]


@pytest.mark.parametrize("variant", ROW_SCAN_VARIANTS, ids=lambda v: "-".join(map(str, v)))
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("shape", ROW_SCAN_SHAPES)
def test_row_scan_tile_shapes(device, oracle, shape, dtype, variant):
    op, exclusive, reverse, aligned = variant
    r, c = shape
    strides, offset = ((c, 1), 0) if aligned else ((c + 1, 1), 1)
    run_column_scan(device, oracle, op, dtype, shape, strides, offset, 1, exclusive, reverse, seed=r * 5 + c)


@pytest.mark.parametrize("dtype", [np.float32, np.uint32])
@pytest.mark.parametrize("shape", [(3001, 1000), (3000, 100), (100003, 8), (100003, 3), (30001, 6)])
def test_column_scan_off_16_byte_boundaries(device, oracle, shape, dtype):
    # offset 1: every line's vectors start 4 bytes past a 16-byte boundary
    # (single pass for 1000 lines, row tiles for the others); vectors need only 4-byte
    # alignment, so both keep one 16-byte access per lane and step
    r, c = shape
    run_column_scan(device, oracle, "sum", dtype, shape, (c, 1), 1, 0, False, False, seed=r + c)
    run_column_scan(device, oracle, "sum", dtype, shape, (c, 1), 1, 0, True, True, seed=r + c + 1)


@pytest.mark.parametrize("kind", ["inclusive", "exclusive"])
@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("op", ["sum", "prod"])
@pytest.mark.parametrize("dtype", [np.float32, np.uint32])
@pytest.mark.parametrize("shape,ld", [((3000, 100), 104), ((65536, 16), 17)])
def test_chunked_column_scan_of_padded_rows(device, oracle, shape, ld, dtype, op, reverse, kind):
    # rows padded past their width (line stride 1, element stride ld > C):
    # not the dense range of the row-tile or narrow forms, so fewer than 256
    # lines take the chunked reduce-then-scan
    r, c = shape
    run_column_scan(device, oracle, op, dtype, shape, (ld, 1), 0, 0, kind == "exclusive", reverse, seed=r + ld)


@pytest.mark.parametrize("op", ["sum", "prod"])
def test_column_scan_transposed_and_reversed_lines(device, oracle, op):
    # column-major view: axis 1 strided, lines adjacent
    run_column_scan(device, oracle, op, np.int32, (516, 2000), (1, 516), 0, 1, False, False, seed=1)
    # lines walk backwards in memory (stride -1)
    run_column_scan(device, oracle, op, np.int32, (2000, 516), (516, -1), 515, 0, True, True, seed=2)
    run_column_scan(device, oracle, op, np.float32, (2000, 516), (516, -1), 515, 0, False, False, seed=3)


def test_prepared_column_scan_rebinds(device, oracle):
    r, c = 8192, 256
    x = oracle.uniform_int(r * c, seed=4, lo=0, hi=1000)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, r * c)
    lay = Layout.c_contiguous([r, c])
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(buf, lay), 0, hx.ScanDirection.Forward,
                                  StridedView(out, lay), hx.ScanKind.Exclusive)
    assert plan.workspace_bytes() > 0
    for _ in range(2):
        plan.dispatch()
    want = np.cumsum(x.reshape(r, c), axis=0, dtype=np.uint32) - x.reshape(r, c)
    assert np.array_equal(device.download_owned(out).reshape(r, c), want)
    y = oracle.uniform_int(r * c, seed=5, lo=0, hi=1000)
    device.write_buffer(buf, y)
    plan.dispatch()
    want = np.cumsum(y.reshape(r, c), axis=0, dtype=np.uint32) - y.reshape(r, c)
    assert np.array_equal(device.download_owned(out).reshape(r, c), want)


def test_prepared_axis_reduction_batch(device, oracle):
    """submit_prepared_axis_reduction_batch (prepared_axis_reduction.rs:84-92):
    eight prepared axis-0 sums of one input, as the reference's comparative
    bench batches them, then a rebind."""
    r, c = 4096, 256
    x = oracle.uniform_int(r * c, seed=9, lo=0, hi=1000)
    buf = device.upload(x)
    outs = [device.alloc_zeroed(np.uint32, c) for _ in range(8)]
    plans = [AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(buf, Layout.c_contiguous([r, c])), 0,
                                           StridedView(o, Layout.c_contiguous([1, c]))) for o in outs]
    hx.submit_prepared_axis_reduction_batch(device, plans)
    want = x.reshape(r, c).sum(axis=0, dtype=np.uint32)
    for o in outs:
        assert np.array_equal(device.download_owned(o), want)
    y = oracle.uniform_int(r * c, seed=10, lo=0, hi=1000)
    device.write_buffer(buf, y)
    hx.submit_prepared_axis_reduction_batch(device, plans)
    assert np.array_equal(device.download_owned(outs[-1]), y.reshape(r, c).sum(axis=0, dtype=np.uint32))


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("c", [32, 8, 100])
def test_prepared_narrow_column_scan_rebinds(device, oracle, reverse, c):
    # narrow-column scans through a prepared plan (narrow form, one-pass and
    # three-pass row tiles): the workspace for the carries or look-back
    # statuses comes with the plan; later writes to the input are observed
    r = 300001
    lay = Layout.c_contiguous([r, c])
    x = oracle.uniform_int(r * c, seed=4, lo=0, hi=1000)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, r * c)
    direction = hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(buf, lay), 0, direction, StridedView(out, lay))

    def want(v):
        m = v.reshape(r, c)
        if reverse:
            return np.cumsum(m[::-1], axis=0, dtype=np.uint32)[::-1]
        return np.cumsum(m, axis=0, dtype=np.uint32)

    plan.dispatch()
    assert np.array_equal(device.download_owned(out).reshape(r, c), want(x))
    y = oracle.uniform_int(r * c, seed=5, lo=0, hi=1000)
    device.write_buffer(buf, y)
    plan.dispatch()
    assert np.array_equal(device.download_owned(out).reshape(r, c), want(y))


@pytest.mark.parametrize("shape,axis", [((500001, 8), 0), ((300001, 3), 1)])
def test_prepared_narrow_axis_reduce_rebinds(device, oracle, shape, axis):
    # narrow columns (axis 0) and rows of 3 elements (a thread per row, axis 1)
    r, c = shape
    x = oracle.uniform_int(r * c, seed=6, lo=0, hi=1000)
    buf = device.upload(x)
    nout = c if axis == 0 else r
    out = device.alloc_zeroed(np.uint32, nout)
    out_shape = [1, c] if axis == 0 else [r, 1]
    plan = AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(buf, Layout.c_contiguous([r, c])), axis,
                                         StridedView(out, Layout.c_contiguous(out_shape)))
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), x.reshape(r, c).sum(axis=axis, dtype=np.uint32))
    y = oracle.uniform_int(r * c, seed=7, lo=0, hi=1000)
    device.write_buffer(buf, y)
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), y.reshape(r, c).sum(axis=axis, dtype=np.uint32))
