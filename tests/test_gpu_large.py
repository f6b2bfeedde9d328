"""Maximum sizes: full reductions, argmax and a scan over 2^32 elements and
more, and segmented sums over 2^32 - 1 values (the most u32 offsets
address) -- 16 GiB operands, where element counts, offsets and logical
indices no longer fit in 31 or 32 bits. Inputs are generated on the device with constant
or planted values, so every result has a closed form. The reference checks
no size this large; the oracle would take minutes here, and the closed
forms pin the same arithmetic (u32 sums and products wrap mod 2^32, f32
sums accumulate in f64, argmax ties go to the lowest index)."""
from __future__ import annotations

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView, _ffi

pytestmark = pytest.mark.gpu

FULL = hx.RocmFullReductionOps()
SCAN = hx.RocmScanOps()
N = (1 << 32) + 1029  # past 2^32, not a multiple of any tile or vector width
ONE = Layout.c_contiguous([1])


def _slice(device, buf, start, count):
    out = device.alloc_zeroed(buf.dtype, count)
    _ffi.check(_ffi.lib().hx_copy(device.handle, buf.ptr + start * buf.itemsize, count, out.ptr, count,
                                  buf.itemsize))
    return device.download_owned(out)


def _full(device, op, buf, n, dtype):
    out = device.alloc_zeroed(dtype, 1)
    FULL.reduce_full_into(device, op, StridedView(buf, Layout.c_contiguous([n])), StridedView(out, ONE))
    return device.download_owned(out)[0]


def test_u32_full_reductions_past_2_32_elements(device):
    buf = device.alloc_uninitialized(np.uint32, N)
    device.fill_uniform_int(buf, seed=1, lo=3, hi=3)
    assert _slice(device, buf, N - 4, 4).tolist() == [3, 3, 3, 3]
    assert _full(device, hx.SumOp, buf, N, np.uint32) == (3 * N) % 2**32
    assert _full(device, hx.ProdOp, buf, N, np.uint32) == pow(3, N, 2**32)
    assert _full(device, hx.MaxOp, buf, N, np.uint32) == 3
    assert _full(device, hx.MinOp, buf, N, np.uint32) == 3
    # A view of the last 2^32 + 5 elements starting past element 2^10: the
    # head peel and the 64-bit offset arithmetic of the flat path.
    n2 = (1 << 32) + 5
    out = device.alloc_zeroed(np.uint32, 1)
    FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, Layout.try_new([n2], [1], N - n2)),
                          StridedView(out, ONE))
    assert device.download_owned(out)[0] == (3 * n2) % 2**32
    buf.free()


def test_f32_sum_and_mean_past_2_32_elements(device):
    buf = device.alloc_uninitialized(np.float32, N)
    device.fill_uniform_real(buf, seed=2, lo=1.0, hi=1.0)  # fmaf(0, u, 1) = 1 everywhere
    assert _slice(device, buf, 0, 2).tolist() == [1.0, 1.0]
    # The f64 sum is exact (N < 2^53); one rounding to f32.
    assert _full(device, hx.SumOp, buf, N, np.float32) == np.float32(float(N))
    assert _full(device, hx.MeanOp, buf, N, np.float32) == np.float32(1.0)
    # Rows of a 65537-wide matrix: the row walker with offsets past 2^32.
    rows, ld, cols = (N - 1029) // 65537, 65537, 65530
    out = device.alloc_zeroed(np.float32, 1)
    FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, Layout.try_new([rows, cols], [ld, 1], 1029)),
                          StridedView(out, ONE))
    assert device.download_owned(out)[0] == np.float32(float(rows * cols))
    buf.free()


def test_argmax_at_the_largest_count(device):
    """The largest argmax operand (2^32 - 2 elements: index 0xFFFFFFFF is the
    no-index sentinel): a planted maximum past 2^31 wins over an equal one at
    the last index, and after it is removed the last index wins."""
    n = (1 << 32) - 2
    buf = device.alloc_uninitialized(np.uint32, n)
    device.fill_uniform_int(buf, seed=3, lo=5, hi=5)
    device.write_sub_buffer(buf, n - 1, np.array([7], np.uint32))
    device.write_sub_buffer(buf, (1 << 31) + 3, np.array([7], np.uint32))
    idx = device.alloc_zeroed(np.uint32, 1)
    val = device.alloc_zeroed(np.uint32, 1)
    lay = Layout.c_contiguous([n])
    FULL.argmax_full_into(device, StridedView(buf, lay), idx, val)
    assert int(device.download_owned(idx)[0]) == (1 << 31) + 3
    assert int(device.download_owned(val)[0]) == 7
    device.write_sub_buffer(buf, (1 << 31) + 3, np.array([5], np.uint32))
    FULL.argmax_full_into(device, StridedView(buf, lay), idx, val)
    assert int(device.download_owned(idx)[0]) == n - 1
    buf.free()


def test_exclusive_scan_past_2_32_elements(device):
    """All-ones u32: out[i] = i mod 2^32, so the prefix wraps once (at
    element 2^32) and the last tile is ragged."""
    x = device.alloc_uninitialized(np.uint32, N)
    device.fill_uniform_int(x, seed=4, lo=1, hi=1)
    out = device.alloc_uninitialized(np.uint32, N)
    lay = Layout.c_contiguous([N])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                        StridedView(out, lay), hx.ScanKind.Exclusive)
    for start in (0, (1 << 31) - 4, (1 << 32) - 4, N - 8):
        want = [(start + i) % 2**32 for i in range(8)]
        assert _slice(device, out, start, 8).tolist() == want, start
    x.free()
    out.free()


SEG = hx.RocmSegmentedReductionOps()


@pytest.mark.parametrize("case", ["geometric-300", "geometric-50000", "extremes"])
def test_segmented_sum_at_the_largest_count(device, case):
    """n = 2^32 - 1 values (the most u32 offsets address), all ones, so
    every segment's sum is its length. Element tiles of 8192 values (mean
    300, about 14.3 million segments) and of 16384 values (mean 50000),
    and hand-placed segments: empty ones at both ends, one of a single
    value, one ending at 2^31 and one spanning past 2^31 to the end."""
    n = 2**32 - 1
    if case == "extremes":
        offsets = np.array([0, 0, 1, 2**31, 2**32 - 2, n, n], np.uint64)
    else:
        mean = 300.0 if case == "geometric-300" else 50000.0
        rng = np.random.default_rng(7)
        lengths = rng.geometric(1.0 / mean, size=int(n / mean * 1.05) + 64).astype(np.uint64)
        ends = np.cumsum(lengths)
        offsets = np.concatenate([[0], ends[ends < n], [n]]).astype(np.uint64)
    values = device.alloc_uninitialized(np.int32, n)
    device.fill_uniform_int(values, seed=8, lo=1, hi=1)
    off = device.upload(offsets.astype(np.uint32))
    out = device.upload(np.full(offsets.size - 1, -7, np.int32))
    SEG.segmented_sum_into(device, values, off, out)
    want = np.diff(offsets.astype(np.int64))
    got = device.download_owned(out).view(np.uint32).astype(np.int64)
    assert np.array_equal(got, want)
    values.free()


def test_f32_scan_past_2_32_elements(device):
    """All-ones f32, inclusive: within a tile the f32 prefixes are exact
    integers (< 2^24) and the inter-tile carry is f64, so out[i] is the
    f32 rounding of i + 1 exactly, far inside the 2*ceil(log2 n)*eps*i
    bound, across the 2^24, 2^31 and 2^32 boundaries."""
    x = device.alloc_uninitialized(np.float32, N)
    device.fill_uniform_real(x, seed=5, lo=1.0, hi=1.0)
    out = device.alloc_uninitialized(np.float32, N)
    lay = Layout.c_contiguous([N])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0, hx.ScanDirection.Forward,
                        StridedView(out, lay), hx.ScanKind.Inclusive)
    for start in (0, (1 << 24) - 4, (1 << 31) - 4, (1 << 32) - 4, N - 8):
        want = np.array([float(start + i + 1) for i in range(8)], np.float64).astype(np.float32)
        assert np.array_equal(_slice(device, out, start, 8), want), start
    x.free()
    out.free()


def test_rows_past_2_31_rows(device):
    """2^31 + 3 rows of 2 f32 (one thread per row): row indices past 2^31
    and outputs of 2^31 + 3 entries. Every row is (1, 1) except planted
    rows whose second element is 5."""
    rows, cols = (1 << 31) + 3, 2
    x = device.alloc_uninitialized(np.float32, rows * cols)
    device.fill_uniform_real(x, seed=6, lo=1.0, hi=1.0)
    planted = [0, (1 << 31) - 1, 1 << 31, rows - 1]
    for r in planted:
        device.write_sub_buffer(x, r * cols + 1, np.array([5.0], np.float32))
    s = device.alloc_zeroed(np.float32, rows)
    m = device.alloc_zeroed(np.float32, rows)
    a = device.alloc_zeroed(np.uint32, rows)
    hx.RocmAxisReductionOps().reduce_rows_fused(device, x, rows, cols, out_sum=s, out_max=m, out_argmax=a)
    for start in (0, (1 << 31) - 2, rows - 4):
        want_s = [6.0 if start + i in planted else 2.0 for i in range(4)]
        want_m = [5.0 if start + i in planted else 1.0 for i in range(4)]
        want_a = [1 if start + i in planted else 0 for i in range(4)]
        assert _slice(device, s, start, 4).tolist() == want_s, start
        assert _slice(device, m, start, 4).tolist() == want_m, start
        assert _slice(device, a, start, 4).tolist() == want_a, start
    for b in (x, s, m, a):
        b.free()


@pytest.mark.parametrize("kind,reverse", [("inclusive", False), ("exclusive", True)])
def test_narrow_column_scan_with_many_tiles(device, kind, reverse):
    """[2^23 + 5, 64] u32 along axis 0: 10923 tiles of 12288 vectors, so
    each thread of the carry pass owns 11 tiles (past its one-batch case).
    Every element is 1 except x[r0][c0] = 1000, so column c gets out[r][c] =
    r + 1 (inclusive forward) or R - 1 - r (exclusive reverse), plus 999 in
    column c0 from row r0 on (forward) or before row r0 (reverse)."""
    R, C = (1 << 23) + 5, 64
    r0, c0 = (1 << 22) + 7, 37
    x = device.alloc_uninitialized(np.uint32, R * C)
    device.fill_uniform_int(x, seed=9, lo=1, hi=1)
    device.write_sub_buffer(x, r0 * C + c0, np.array([1000], np.uint32))
    out = device.alloc_uninitialized(np.uint32, R * C)
    lay = Layout.c_contiguous([R, C])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive if kind == "exclusive" else hx.ScanKind.Inclusive)
    for r in (0, 1, 767, 768, r0 - 1, r0, r0 + 1, (1 << 23) - 1, R - 1):  # 768 rows per tile
        got = _slice(device, out, r * C, C)
        want = np.full(C, (R - 1 - r) if reverse else (r + 1), np.uint64)
        if (r < r0) if reverse else (r >= r0):
            want[c0] += 999
        assert np.array_equal(got, want.astype(np.uint32)), r
    x.free()
    out.free()


@pytest.mark.parametrize("kind,reverse", [("inclusive", False), ("exclusive", True)])
@pytest.mark.parametrize("C,R,tile_rows", [(3, 3 * (1 << 24) + 5, 5440), (100, 1500007, 160)])
def test_row_tile_column_scan_with_many_tiles(device, kind, reverse, C, R, tile_rows):
    """Row tiles along axis 0, u32, with about 9200 tiles: [3 * 2^24 + 5, 3]
    (tiles of 5440 rows, whole 128-byte lines) looks back in one pass over
    9253 tiles;
    [1500007, 100] (tiles of 160 rows, 9376 tiles) takes three passes, and
    each thread of its carry pass owns 10 tiles (past its one-batch case).
    Every element is 1 except x[r0][c0] = 1000, as in the narrow case
    above."""
    r0, c0 = R // 3 + 7, C - 1
    x = device.alloc_uninitialized(np.uint32, R * C)
    device.fill_uniform_int(x, seed=9, lo=1, hi=1)
    device.write_sub_buffer(x, r0 * C + c0, np.array([1000], np.uint32))
    out = device.alloc_uninitialized(np.uint32, R * C)
    lay = Layout.c_contiguous([R, C])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, lay), 0,
                        hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward, StridedView(out, lay),
                        hx.ScanKind.Exclusive if kind == "exclusive" else hx.ScanKind.Inclusive)
    tr = tile_rows
    for r in (0, 1, tr - 1, tr, r0 - 1, r0, r0 + 1, R - tr - 1, R - tr, R - 1):
        got = _slice(device, out, r * C, C)
        want = np.full(C, (R - 1 - r) if reverse else (r + 1), np.uint64)
        if (r < r0) if reverse else (r >= r0):
            want[c0] += 999
        assert np.array_equal(got, want.astype(np.uint32)), r
    x.free()
    out.free()


def test_row_scans_of_2_26_lines(device):
    """[2^26 + 5, 4] u32 scanned along axis 1: every line is one 64-lane
    tile, so one launch would need 2^32 + 320 work-items, past the 32-bit
    grid size; the tiles go out in several launches.  Lines of one tile
    never look back and publish no status, so the plan's workspace is the
    256-byte header alone (not a status line per tile).  Every element is 1
    except planted x[r][2] = 7, so out[r] = (1, 2, 9, 10) there and
    (1, 2, 3, 4) elsewhere."""
    R, C = (1 << 26) + 5, 4
    x = device.alloc_uninitialized(np.uint32, R * C)
    device.fill_uniform_int(x, seed=11, lo=1, hi=1)
    planted = [0, (1 << 26) - 1, 1 << 26, R - 1]
    for r in planted:
        device.write_sub_buffer(x, r * C + 2, np.array([7], np.uint32))
    out = device.alloc_zeroed(np.uint32, R * C)
    lay = Layout.c_contiguous([R, C])
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(x, lay), 1, hx.ScanDirection.Forward,
                                  StridedView(out, lay), hx.ScanKind.Inclusive)
    assert plan.workspace_bytes() <= 256
    plan.dispatch()
    for r in (0, 1, (1 << 26) - 2, (1 << 26) - 1, 1 << 26, (1 << 26) + 1, R - 1):
        want = [1, 2, 9, 10] if r in planted else [1, 2, 3, 4]
        assert _slice(device, out, r * C, C).tolist() == want, r
    plan.destroy()
    x.free()
    out.free()


def test_strided_row_sums_of_2_26_rows(device):
    """Sums along axis 1 of the [2^26 + 3, 2] view with strides (4, 2) of a
    u32 buffer: neither stride is 1, so each row gets a 64-lane group and
    one launch would need 2^32 + 192 work-items; the rows go out in several
    launches.  Every element is 1 except planted x[4 r + 2] = 9 (the second
    element of row r), so out[r] = 10 there and 2 elsewhere."""
    R = (1 << 26) + 3
    x = device.alloc_uninitialized(np.uint32, 4 * R)
    device.fill_uniform_int(x, seed=12, lo=1, hi=1)
    planted = [0, (1 << 26) - 1, 1 << 26, R - 1]
    for r in planted:
        device.write_sub_buffer(x, 4 * r + 2, np.array([9], np.uint32))
    out = device.alloc_zeroed(np.uint32, R)
    view = StridedView(x, Layout.try_new([R, 2], [4, 2], 0))
    hx.RocmAxisReductionOps().reduce_axis_into(device, hx.SumOp, view, 1,
                                               StridedView(out, Layout.c_contiguous([R, 1])))
    for start in (0, (1 << 26) - 2, R - 4):
        want = [10 if start + i in planted else 2 for i in range(4)]
        assert _slice(device, out, start, 4).tolist() == want, start
    x.free()
    out.free()


def test_single_element_rows_past_2_32_rows(device):
    """[2^32 + 1029, 1] u32 summed along axis 1 takes the short-row LDS tiles
    (8192 rows a tile, row indices past 2^32): out[r] = x[r].  Every element
    is 1 except planted 7s either side of 2^32."""
    x = device.alloc_uninitialized(np.uint32, N)
    device.fill_uniform_int(x, seed=13, lo=1, hi=1)
    planted = [0, (1 << 32) - 1, 1 << 32, N - 1]
    for r in planted:
        device.write_sub_buffer(x, r, np.array([7], np.uint32))
    out = device.alloc_zeroed(np.uint32, N)
    hx.RocmAxisReductionOps().reduce_axis_into(device, hx.SumOp, StridedView(x, Layout.c_contiguous([N, 1])), 1,
                                               StridedView(out, Layout.c_contiguous([N, 1])))
    for start in (0, (1 << 32) - 4, N - 4):
        want = [7 if start + i in planted else 1 for i in range(4)]
        assert _slice(device, out, start, 4).tolist() == want, start
    x.free()
    out.free()


def test_reversed_view_reductions_past_2_32_elements(device):
    """A stride -1 view of N u32 streamed as the dense range it covers: sum
    3N mod 2^32 of all-3s, and the max of one planted value."""
    x = device.alloc_uninitialized(np.uint32, N)
    device.fill_uniform_int(x, seed=14, lo=3, hi=3)
    view = StridedView(x, Layout.try_new([N], [-1], N - 1))
    out = device.alloc_zeroed(np.uint32, 1)
    FULL.reduce_full_into(device, hx.SumOp, view, StridedView(out, ONE))
    assert int(device.download_owned(out)[0]) == (3 * N) % 2**32
    device.write_sub_buffer(x, (1 << 32) + 3, np.array([11], np.uint32))
    FULL.reduce_full_into(device, hx.MaxOp, view, StridedView(out, ONE))
    assert int(device.download_owned(out)[0]) == 11
    x.free()
    out.free()


def test_exclusive_scan_off_the_line_grid_past_2_32_elements(device):
    """All-ones u32 scanned into an output 5 elements past a 128-byte
    boundary: the line runs on a virtual line 5 longer, tiles on the
    output's grid; out[5 + i] = i mod 2^32 and the 5 elements before it stay
    untouched."""
    x = device.alloc_uninitialized(np.uint32, N)
    device.fill_uniform_int(x, seed=15, lo=1, hi=1)
    out = device.alloc_uninitialized(np.uint32, N + 5)
    device.write_sub_buffer(out, 0, np.full(5, 0xABCD, np.uint32))
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(x, Layout.c_contiguous([N])), 0, hx.ScanDirection.Forward,
                        StridedView(out, Layout.try_new([N], [1], 5)), hx.ScanKind.Exclusive)
    assert _slice(device, out, 0, 5).tolist() == [0xABCD] * 5
    for start in (0, (1 << 31) - 4, (1 << 32) - 4, N - 8):
        want = [(start + i) % 2**32 for i in range(8)]
        assert _slice(device, out, 5 + start, 8).tolist() == want, start
    x.free()
    out.free()
