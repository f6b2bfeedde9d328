"""Seeded random sweep of rank-2 axis reductions and axis scans.

The other axis tests pick shapes at each planning boundary by hand; this one
draws 120 cases from a fixed seed -- shapes from 1 to 4096 per side (narrow,
tall, wide and square), every layout the view type allows (row-major,
column-major, padded lines, either axis walking backwards, offsets), every op,
dtype, direction and kind -- and checks each against the oracle line by line
to the same bar as the hand-picked tests: bit-exact for integers, min, max
and argmax; f32 sums within 2*ceil(log2 n)*eps*sum|x|; f32 products within
gamma_{n-1} (any evaluation order).  Scans write through the input's own
layout, so every element outside the view must keep its fill value.
"""
from __future__ import annotations

import contextlib

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

import test_gpu_axis
from test_gpu_axis import EPS, OPS, check, f32_bound, host_for, lines_of, prod_bound, run_column_scan

AXIS = hx.RocmAxisReductionOps()
DTYPES = [np.float32, np.uint32, np.int32]
LAYOUTS = ["row", "col", "padded", "rev_cols", "rev_rows", "rev_both"]


def _side(rng):
    """1 to 4096, log-uniform, with the narrow widths 1-8 and powers of two
    (and their neighbours) drawn more often than chance would."""
    pick = rng.integers(0, 4)
    if pick == 0:
        return int(rng.integers(1, 9))
    if pick == 1:
        p = 1 << int(rng.integers(2, 13))
        return max(1, p + int(rng.integers(-1, 2)))
    return int(np.exp(rng.uniform(0.0, np.log(4096.0))))


def _shape(rng):
    r, c = _side(rng), _side(rng)
    if rng.integers(0, 4) == 0:  # tall: many rows of few columns
        r = int(rng.integers(4096, 70000))
        c = int(rng.integers(1, 33))
    while r * c > (1 << 21):
        r = max(1, r // 2)
    return r, c


def _layout(rng, shape, kind):
    """(strides, offset) for a view of `shape`; offsets keep every index
    non-negative."""
    r, c = shape
    pad = int(rng.integers(1, 4))
    extra = int(rng.integers(0, 5))
    if kind == "row":
        strides = (c, 1)
    elif kind == "col":
        strides = (1, r)
    elif kind == "padded":
        strides = (c + pad, 1)
    elif kind == "rev_cols":
        strides = (c + pad, -1)
    elif kind == "rev_rows":
        strides = (-(c + pad), 1)
    else:
        strides = (-(c + pad), -1)
    offset = extra + sum((shape[d] - 1) * -strides[d] for d in range(2) if strides[d] < 0)
    return strides, offset


def _cases(seed, count, scan):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        shape = _shape(rng)
        layout = LAYOUTS[int(rng.integers(0, len(LAYOUTS)))]
        strides, offset = _layout(rng, shape, layout)
        axis = int(rng.integers(0, 2))
        dtype = DTYPES[int(rng.integers(0, 3))]
        if scan:
            op = ["sum", "prod"][int(rng.integers(0, 2))]
            extra = (bool(rng.integers(0, 2)), bool(rng.integers(0, 2)))  # exclusive, reverse
        else:
            op = list(OPS)[int(rng.integers(0, len(OPS)))]
            extra = ()
        out.append(pytest.param(shape, strides, offset, axis, dtype, op, extra, 1000 * seed + i,
                                id=f"{i}-{shape[0]}x{shape[1]}-{layout}-ax{axis}-{np.dtype(dtype).name}-{op}"))
    return out


class _PreparedScan:
    """scan_axis_into through hx_prepare_scan: one plan, two dispatches."""

    def scan_axis_into(self, device, op, input, axis, direction, output, kind):
        plan = hx.RocmScanOps().prepare_scan_axis(device, op, input, axis, direction, output, kind)
        try:
            plan.dispatch()
            plan.dispatch()
        finally:
            plan.destroy()


def _buffer_size(shape, strides, offset):
    return offset + 1 + sum((shape[d] - 1) * max(strides[d], 0) for d in range(2))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,strides,offset,axis,dtype,op,extra,seed", _cases(11, 60, scan=False))
def test_random_axis_reduce(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed):
    size = _buffer_size(shape, strides, offset)
    host = host_for(oracle, dtype, size, seed=seed, op=op)
    buf = device.upload(host)
    nout = shape[1 - axis]
    out_dtype = np.uint32 if op == "argmax" else dtype
    out = device.upload(np.full(nout + 1, 7, out_dtype))  # one element past the outputs
    out_shape = [shape[0], 1] if axis == 1 else [1, shape[1]]
    view = StridedView(buf, Layout.try_new(list(shape), list(strides), offset))
    outputs = StridedView(out, Layout.c_contiguous(out_shape))
    if seed % 2:  # odd seeds: the prepared plan, dispatched twice
        plan = AXIS.prepare_reduce_axis_into(device, OPS[op], view, axis, outputs)
        try:
            plan.dispatch()
            plan.dispatch()
        finally:
            plan.destroy()
    else:
        AXIS.reduce_axis_into(device, OPS[op], view, axis, outputs)
    got = device.download_owned(out)
    assert got[nout] == 7
    lines = lines_of(host, shape, strides, offset, axis)
    if dtype == np.float32 and op == "prod":
        n = lines.shape[1]
        want = [np.prod(l.astype(np.float64)) for l in lines]
        assert np.all(np.abs(got[:nout].astype(np.float64) - want) <= prod_bound(n) * np.abs(want))
        return
    check(oracle, op, dtype, got[:nout], lines)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,strides,offset,axis,dtype,op,extra,seed", _cases(12, 60, scan=True))
def test_random_axis_scan(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed, monkeypatch):
    exclusive, reverse = extra
    if seed % 2:  # odd seeds: the prepared plan, dispatched twice
        monkeypatch.setattr(test_gpu_axis, "SCAN", _PreparedScan())
    run_column_scan(device, oracle, op, dtype, shape, strides, offset, axis, exclusive, reverse, seed)


def _narrow_cases(seed, count, scan):
    """Axis 0 of dense row-major matrices with 2 to 255 columns and more
    than 1024 rows, at element offsets 0-4: the period-form sums (up to 95
    columns), the column tiles beyond, and the row-tile scans (one pass up
    to 24 columns, three beyond)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        c = min(255, int(np.exp(rng.uniform(np.log(2.0), np.log(256.0)))))  # log-uniform widths
        r = int(rng.integers(1025, max(1026, (1 << 21) // c)))
        offset = int(rng.integers(0, 5))
        dtype = DTYPES[int(rng.integers(0, 3))]
        if scan:
            op = ["sum", "prod"][int(rng.integers(0, 2))]
            extra = (bool(rng.integers(0, 2)), bool(rng.integers(0, 2)))  # exclusive, reverse
        else:
            op = list(OPS)[int(rng.integers(0, len(OPS)))]
            extra = ()
        out.append(pytest.param((r, c), (c, 1), offset, 0, dtype, op, extra, 1000 * seed + i,
                                id=f"n{i}-{r}x{c}-off{offset}-{np.dtype(dtype).name}-{op}"))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("shape,strides,offset,axis,dtype,op,extra,seed", _narrow_cases(13, 40, scan=False))
def test_random_narrow_axis_reduce(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed):
    test_random_axis_reduce(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed)


@pytest.mark.gpu
@pytest.mark.parametrize("shape,strides,offset,axis,dtype,op,extra,seed", _narrow_cases(14, 40, scan=True))
def test_random_narrow_axis_scan(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed,
                                 monkeypatch):
    test_random_axis_scan(device, oracle, shape, strides, offset, axis, dtype, op, extra, seed, monkeypatch)


def test_case_lists_cover_the_layouts_and_paths():
    """The fixed seeds reach every layout, both axes, narrow (at most 8
    columns) and tall (more than 4096 rows) shapes (CPU only)."""
    for scan, seed in ((False, 11), (True, 12)):
        cases = [p.values for p in _cases(seed, 60, scan)]
        ids = [p.id for p in _cases(seed, 60, scan)]
        assert {i.split("-")[2] for i in ids} == set(LAYOUTS)
        assert {c[3] for c in cases} == {0, 1}
        assert any(c[0][1] <= 8 for c in cases) and any(c[0][0] > 4096 for c in cases)
        assert all(c[0][0] * c[0][1] <= (1 << 21) for c in cases)
    # The narrow sweeps reach each form: period sums (<= 95 columns) and
    # column tiles, one-pass (<= 24) and three-pass row-tile scans.
    widths = [p.values[0][1] for p in _narrow_cases(13, 40, False)]
    assert any(c <= 95 for c in widths) and any(c >= 96 for c in widths)
    widths = [p.values[0][1] for p in _narrow_cases(14, 40, True)]
    assert any(c <= 24 for c in widths) and any(c > 24 and c not in (32, 64, 128) for c in widths)
    assert all(p.values[0][0] > 1024 for p in _narrow_cases(14, 40, True) + _narrow_cases(13, 40, False))


# ------------------------------------------------------------ 1-D forms
FULL = hx.RocmFullReductionOps()
SCAN = hx.RocmScanOps()
SEG = hx.RocmSegmentedReductionOps()


@contextlib.contextmanager
def _prefix(device, buf, count):
    """The first `count` elements of `buf` as a buffer of their own; the
    memory stays `buf`'s (the alias never frees it)."""
    alias = hx.RocmBuffer(device, buf.ptr, count, buf.dtype)
    try:
        yield alias
    finally:
        alias.ptr = None


def _length(rng, top):
    """1 to 2^top, log-uniform, with powers of two and their neighbours
    drawn more often than chance would."""
    if rng.integers(0, 3) == 0:
        return max(1, (1 << int(rng.integers(0, top + 1))) + int(rng.integers(-1, 2)))
    return int(np.exp(rng.uniform(0.0, top * np.log(2.0))))


def _cases_1d(seed, count, scan):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = _length(rng, 24)
        stride = [1, 1, 1, 2, 3, -1, -2][int(rng.integers(0, 7))]
        offset = int(rng.integers(0, 5)) + (n - 1) * max(-stride, 0)
        dtype = DTYPES[int(rng.integers(0, 3))]
        if scan:
            op = ["sum", "sum", "prod"][int(rng.integers(0, 3))]
            extra = (bool(rng.integers(0, 2)), bool(rng.integers(0, 2)))  # exclusive, reverse
        else:
            op = list(OPS)[int(rng.integers(0, len(OPS)))]
            extra = ()
        out.append(pytest.param(n, stride, offset, dtype, op, extra, 1000 * seed + i,
                                id=f"{i}-n{n}-s{stride}-o{offset}-{np.dtype(dtype).name}-{op}"))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n,stride,offset,dtype,op,extra,seed", _cases_1d(13, 60, scan=False))
def test_random_full_reduce(device, oracle, n, stride, offset, dtype, op, extra, seed):
    size = offset + 1 + (n - 1) * max(stride, 0)
    host = host_for(oracle, dtype, size, seed=seed, op=op)
    sel = np.ascontiguousarray(host[offset + np.arange(n, dtype=np.int64) * stride])
    buf = device.upload(host)
    view = StridedView(buf, Layout.try_new([n], [stride], offset))
    if op == "argmax":
        idx = device.upload(np.full(2, 7, np.uint32))
        with _prefix(device, idx, 1) as first:
            FULL.argmax_full_into(device, view, first, None)
        got = device.download_owned(idx)
        assert got[1] == 7
        assert int(got[0]) == oracle.full_argmax(sel)
        return
    out = device.upload(np.full(2, 7, dtype))
    FULL.reduce_full_into(device, OPS[op], view, StridedView(out, Layout.c_contiguous([1])))
    got = device.download_owned(out)
    assert got[1] == 7
    if dtype == np.float32 and op == "prod":
        want = np.prod(sel.astype(np.float64))
        assert abs(float(got[0]) - want) <= prod_bound(n) * abs(want)
        return
    check(oracle, op, dtype, got[:1], sel[None, :])


@pytest.mark.gpu
@pytest.mark.parametrize("n,stride,offset,dtype,op,extra,seed", _cases_1d(14, 60, scan=True))
def test_random_scan(device, oracle, n, stride, offset, dtype, op, extra, seed):
    """Scans of 1-D views, written through the input's own layout."""
    exclusive, reverse = extra
    size = offset + 1 + (n - 1) * max(stride, 0)
    if dtype == np.float32:
        host = (oracle.uniform_real(size, seed, 0.999, 1.001) if op == "prod"
                else oracle.uniform_real(size, seed, -1.0, 1.0))
    else:
        host = oracle.uniform_int(size, seed, -1000, 1000, dtype=np.int32).view(dtype)
    where = offset + np.arange(n, dtype=np.int64) * stride
    sel = np.ascontiguousarray(host[where])
    buf = device.upload(host)
    out = device.upload(np.full(size, 7, dtype))
    lay = Layout.try_new([n], [stride], offset)
    SCAN.scan_axis_into(device, hx.CumSumOp if op == "sum" else hx.CumProdOp, StridedView(buf, lay), 0,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive)
    got_host = device.download_owned(out)
    touched = np.zeros(size, bool)
    touched[where] = True
    assert np.all(got_host[~touched] == 7)
    got = got_host[where]
    if op == "sum":
        want = oracle.scan_sum(sel, exclusive=exclusive, reverse=reverse)
        if dtype == np.float32:
            bad, worst = oracle.check_f32_bound(got, want[0], want[1], n)
            assert bad == 0, worst
        else:
            assert np.array_equal(got, want)
    elif dtype == np.float32:
        v = sel.astype(np.float64)[::-1] if reverse else sel.astype(np.float64)
        c = np.cumprod(v)
        if exclusive:
            c = np.concatenate([[1.0], c[:-1]])
        want = c[::-1] if reverse else c
        assert np.all(np.abs(got.astype(np.float64) - want) <= prod_bound(n) * np.abs(want))
    else:
        assert np.array_equal(got, oracle.scan_prod(sel, exclusive=exclusive, reverse=reverse))


def _random_offsets(rng, n):
    """CSR offsets over n values mixing segment regimes: geometric lengths of
    a per-run mean from 0.5 to 70000, runs of empty segments, one long
    segment; the first offset is 0 and the last n."""
    lengths = []
    total = 0
    while total < n:
        kind = int(rng.integers(0, 10))
        if kind == 0:
            run = [0] * int(rng.integers(1, 6000))  # empty segments
        elif kind == 1:
            run = [int(rng.integers(1, max(2, n // 2 + 1)))]  # one long segment
        else:
            mean = [0.5, 2.0, 8.0, 15.0, 40.0, 300.0, 5000.0, 70000.0][int(rng.integers(0, 8))]
            count = int(rng.integers(1, 4000))
            run = list(rng.geometric(1.0 / (mean + 1.0), size=count) - 1)
        lengths += run
        total += int(sum(run))
    off = np.concatenate([[0], np.minimum(np.cumsum(lengths, dtype=np.int64), n)]).astype(np.uint32)
    if rng.integers(0, 4) == 0:  # trailing empty segments
        off = np.concatenate([off, np.full(int(rng.integers(1, 3000)), n, np.uint32)])
    return off


def _cases_segmented(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = _length(rng, 22)
        off = _random_offsets(rng, n)
        dtype = [np.int32, np.uint32][int(rng.integers(0, 2))]
        out.append(pytest.param(n, off, dtype, 1000 * seed + i,
                                id=f"{i}-n{n}-S{off.size - 1}-{np.dtype(dtype).name}"))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n,offsets,dtype,seed", _cases_segmented(15, 40))
def test_random_segmented_sum(device, oracle, n, offsets, dtype, seed):
    x = oracle.uniform_int(n, seed, lo=0, hi=1 << 31, dtype=np.uint32).view(dtype)
    vb = device.upload(x)
    ob = device.upload(offsets)
    out = device.upload(np.full(offsets.size, 0x5A5A5A5A, np.uint32).view(dtype))  # one past the outputs
    with _prefix(device, out, offsets.size - 1) as outputs:
        SEG.segmented_sum_into(device, vb, ob, outputs)
    got = device.download_owned(out)
    assert got.view(np.uint32)[-1] == 0x5A5A5A5A
    assert np.array_equal(got[:-1], oracle.segmented_sum(x, offsets))


# ------------------------------------------------------------ fused rows
AXIS_ROWS = hx.RocmAxisReductionOps()


def _cases_rows(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        if rng.integers(0, 4) == 0:  # few long rows (split rows)
            rows, cols = int(rng.integers(1, 6)), _length(rng, 18)
        else:
            rows, cols = _side(rng), _length(rng, 13)
        pad = [0, 0, 1, 3, 4][int(rng.integers(0, 5))]
        offset = int(rng.integers(0, 5))
        dtype = DTYPES[int(rng.integers(0, 3))]
        prologue = None
        if dtype == np.float32 and rng.integers(0, 3) > 0:
            prologue = ([0.5, -0.5, 1.0, -2.0][int(rng.integers(0, 4))], float(rng.uniform(-1.0, 1.0)))
        wanted = int(rng.integers(1, 8))  # bits: sum, max, argmax
        prepared = bool(rng.integers(0, 2))
        out.append(pytest.param(rows, cols, cols + pad, offset, dtype, prologue, wanted, prepared, 1000 * seed + i,
                                id=f"{i}-{rows}x{cols}-ld{cols + pad}-o{offset}-{np.dtype(dtype).name}"
                                   f"-{'aff' if prologue else 'id'}-w{wanted}-{'prep' if prepared else 'imm'}"))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,ld,offset,dtype,prologue,wanted,prepared,seed", _cases_rows(16, 60))
def test_random_rows_fused(device, oracle, rows, cols, ld, offset, dtype, prologue, wanted, prepared, seed):
    """Sum, max and argmax of fmaf(a, x, b) per row (any subset of the three
    outputs), immediate or prepared, against the oracle's row fold."""
    size = offset + (rows - 1) * ld + cols + 2
    if dtype == np.float32:
        host = oracle.normal(size, seed=seed)
    else:
        host = (oracle.uniform_int(size, seed, 0, 50)).astype(dtype)  # ties for argmax
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host[offset:], rows, cols, ld, prologue=prologue)
    buf = device.upload(host)
    bufs = [device.upload(np.full(rows + 1, 7, dt)) for dt in (dtype, dtype, np.uint32)]
    with contextlib.ExitStack() as stack:
        views = [stack.enter_context(_prefix(device, b, rows)) if wanted >> k & 1 else None
                 for k, b in enumerate(bufs)]
        if prepared:
            plan = AXIS_ROWS.prepare_reduce_rows_fused(device, buf, rows, cols, ld, offset, prologue, *views)
            try:
                plan.dispatch()
                plan.dispatch()  # a second dispatch rewrites the same outputs
            finally:
                plan.destroy()
        else:
            AXIS_ROWS.reduce_rows_fused(device, buf, rows, cols, ld, offset, prologue, *views)
    got = [device.download_owned(b) for b in bufs]
    for k, g in enumerate(got):
        if not wanted >> k & 1:
            assert np.all(g == 7)
            continue
        assert g[rows] == 7
        g = g[:rows]
        if k == 2:
            assert np.array_equal(g, i_ref)
        elif k == 1:
            assert np.array_equal(g.view(np.uint32), m_ref.view(np.uint32))
        elif dtype == np.float32:
            bound = np.array([f32_bound(cols, a) for a in a_ref])
            assert np.all(np.abs(g.astype(np.float64) - s_ref) <= bound)
        else:
            assert np.array_equal(g, s_ref)


# ------------------------------------------------------------ dot and norms
def _cases_vector(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        n = _length(rng, 22) if rng.integers(0, 10) else 0
        views = []
        for _ in range(2):
            stride = [1, 1, 1, 2, 3, -1, -2][int(rng.integers(0, 7))]
            views.append((stride, int(rng.integers(0, 5)) + max(n - 1, 0) * max(-stride, 0)))
        dtype = DTYPES[int(rng.integers(0, 3))]
        out.append(pytest.param(n, views, dtype, 1000 * seed + i,
                                id=f"{i}-n{n}-a{views[0][0]}o{views[0][1]}-b{views[1][0]}o{views[1][1]}"
                                   f"-{np.dtype(dtype).name}"))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("n,views,dtype,seed", _cases_vector(17, 40))
def test_random_dot_and_norms(device, oracle, n, views, dtype, seed):
    """dot(a, b) of two independently strided and offset views, and the L1,
    L2 and max norms of the first."""
    from test_gpu_vector import one

    hosts, sels, svs = [], [], []
    for k, (stride, offset) in enumerate(views):
        size = offset + 1 + max(n - 1, 0) * max(stride, 0)
        if dtype == np.float32:
            host = oracle.uniform_real(size, seed + k, -2.0, 2.0)
        else:
            host = oracle.uniform_int(size, seed + k, 0, 2**32 - 1).view(dtype)
        sels.append(np.ascontiguousarray(host[offset + np.arange(n, dtype=np.int64) * stride]))
        svs.append(StridedView(device.upload(host), Layout.try_new([n], [stride], offset)))
        hosts.append(host)
    a, b = sels
    got_dot = one(device, hx.dot(device, svs[0], svs[1]))
    got_l1 = one(device, hx.norm_l1(device, svs[0]))
    assert one(device, hx.norm_max(device, svs[0])) == oracle.norm_max(a)
    if dtype != np.float32:
        assert got_dot == oracle.dot(a, b)
        assert got_l1 == oracle.norm_l1(a)
        return
    want, mags = oracle.dot(a, b)
    assert abs(float(got_dot) - want) <= f32_bound(max(n, 1), mags) + abs(want) * EPS / 2
    l1 = oracle.norm_l1(a)
    assert abs(float(got_l1) - l1) <= f32_bound(max(n, 1), l1) + l1 * EPS
    l2 = oracle.norm_l2(a)
    assert abs(float(one(device, hx.norm_l2(device, svs[0]))) - l2) <= l2 * 2 * EPS
