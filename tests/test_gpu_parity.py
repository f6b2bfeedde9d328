"""Parity of every kernel family with the CPU oracle on the same seeded
inputs, at sizes the oracle checks in seconds: ragged lengths around the
tile and vector boundaries, misaligned views, every dtype, the prologue,
special values and empty operands.  Integer results must be bit-exact; f32
sums and scans must satisfy |err| <= 2*ceil(log2 n)*eps_f32*sum|y| against
the oracle's f64 accumulation."""
from __future__ import annotations

import ctypes

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
SIZES = [1, 2, 3, 4, 5, 63, 64, 65, 255, 256, 257, 1023, 1024, 1025, 4095, 4096, 4097,
         8191, 8192, 8193, 12345, 65536 + 17, 1 << 20, (1 << 20) + 3]


def f32_bound(n, abs_sum):
    """North-star bound 2*ceil(log2 n)*eps_f32*sum|y| (0 for n <= 1: exact)."""
    return 2 * (int(n) - 1).bit_length() * EPS * abs_sum


def inputs(oracle, dtype, n, seed):
    if dtype == np.float32:
        return oracle.uniform_real(n, seed, -1.0, 1.0)
    if dtype == np.int32:
        return oracle.uniform_int(n, seed, -1000, 1000, dtype=np.int32)
    return oracle.uniform_int(n, seed, 0, 2**32 - 1)


def full(device, op, host, layout=None, prologue=None):
    buf = device.upload(host)
    out = device.alloc_zeroed(host.dtype, 1)
    lay = layout or Layout.c_contiguous([host.size])
    FULL.reduce_full_into(device, op, StridedView(buf, lay), StridedView(out, Layout.c_contiguous([1])),
                          prologue=prologue)
    return device.download_owned(out)[0]


# ------------------------------------------------------------ generator
@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_device_generator_matches_oracle_bits(device, oracle, n):
    u = device.alloc_uninitialized(np.uint32, n)
    device.fill_uniform_int(u, seed=42, lo=0, hi=255)
    assert np.array_equal(device.download_owned(u), oracle.uniform_int(n, 42, 0, 255))
    i = device.alloc_uninitialized(np.int32, n)
    device.fill_uniform_int(i, seed=7, lo=-1000, hi=1000)
    assert np.array_equal(device.download_owned(i), oracle.uniform_int(n, 7, -1000, 1000, dtype=np.int32))
    f = device.alloc_uninitialized(np.float32, n)
    device.fill_uniform_real(f, seed=1, lo=-1.0, hi=1.0)
    assert np.array_equal(device.download_owned(f).view(np.uint32),
                          oracle.uniform_real(n, 1, -1.0, 1.0).view(np.uint32))


def test_device_normal_generator_is_close_to_oracle(device, oracle):
    n = 1 << 16
    f = device.alloc_uninitialized(np.float32, n)
    device.fill_normal(f, seed=3)
    got = device.download_owned(f)
    want = oracle.normal(n, 3)
    # device and host libm may differ in the last f64 ulp of log/cos/sqrt
    assert np.max(np.abs(got - want)) <= 4e-7 * np.max(np.abs(want))


# ------------------------------------------------------------ full reduce
@pytest.mark.parametrize("n", SIZES)
def test_full_sum_f32_within_bound(device, oracle, n):
    x = inputs(oracle, np.float32, n, seed=n)
    ref, ab = oracle.full_sum(x)
    got = float(full(device, hx.SumOp, x))
    assert abs(got - ref) <= f32_bound(n, ab), (n, got, ref)


@pytest.mark.parametrize("dtype", [np.uint32, np.int32])
@pytest.mark.parametrize("n", SIZES)
def test_full_integer_reductions_bit_exact(device, oracle, dtype, n):
    x = inputs(oracle, dtype, n, seed=n + 1)
    assert full(device, hx.SumOp, x) == oracle.full_sum(x)
    assert full(device, hx.ProdOp, x) == oracle.full_prod(x)
    assert full(device, hx.MaxOp, x) == oracle.full_max(x)
    assert full(device, hx.MinOp, x) == oracle.full_min(x)


@pytest.mark.parametrize("n", [1, 3, 4097, 1 << 20])
def test_full_max_min_f32_bit_exact(device, oracle, n):
    x = oracle.normal(n, seed=n)
    assert full(device, hx.MaxOp, x).view(np.uint32) == oracle.full_max(x).view(np.uint32)
    assert full(device, hx.MinOp, x).view(np.uint32) == oracle.full_min(x).view(np.uint32)


@pytest.mark.parametrize("offset", [0, 1, 2, 3, 5])
def test_full_reduce_misaligned_views(device, oracle, offset):
    n = 100003
    host = inputs(oracle, np.uint32, n + offset + 7, seed=9)
    buf = device.upload(host)
    out = device.alloc_zeroed(np.uint32, 1)
    lay = Layout.try_new([n], [1], offset)
    FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, lay), StridedView(out, Layout.c_contiguous([1])))
    assert device.download_owned(out)[0] == oracle.full_sum(host[offset:offset + n])


def test_full_reduce_strided_views(device, oracle):
    host = inputs(oracle, np.int32, 3000, seed=4)
    for shape, strides, offset in (([10, 30], [1, 100], 5), ([1000], [3], 0), ([50, 20], [20, 1], 0),
                                   ([7, 11], [-11, 1], 66), ([2, 3, 4, 5], [60, 20, 5, 1], 0)):
        lay = Layout.try_new(shape, strides, offset)
        idx = offset + sum(np.indices(shape)[d] * strides[d] for d in range(len(shape)))
        sel = host[idx.ravel()]
        buf = device.upload(host)
        out = device.alloc_zeroed(np.int32, 1)
        FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, lay), StridedView(out, Layout.c_contiguous([1])))
        assert device.download_owned(out)[0] == oracle.full_sum(np.ascontiguousarray(sel))
        FULL.reduce_full_into(device, hx.MaxOp, StridedView(buf, lay), StridedView(out, Layout.c_contiguous([1])))
        assert device.download_owned(out)[0] == oracle.full_max(np.ascontiguousarray(sel))


# Non-dense views walked as rows: contiguous rows of every length either side
# of the 4-element vector (16-byte loads at 4-byte alignment), row starts off
# 16-byte boundaries, merged row-major dimensions, rank 3 and 4 outer walks,
# negative outer strides, and element walks (inner stride != 1, transposes).
ROW_VIEWS = [
    ([300, 1], [7, 1], 0),                     # one column: element walk
    ([300, 3], [7, 1], 1),                     # rows of 3: element walk
    ([300, 4], [7, 1], 2),                     # one vector per row
    ([300, 5], [7, 1], 3),                     # vector + 1-element tail
    ([123, 9], [11, 1], 1),
    ([64, 1000], [1003, 1], 5),                # a slice of wider rows
    ([7, 9, 13], [200, 20, 1], 3),             # rank 3, two outer digits
    ([3, 4, 5, 6], [400, 90, 15, 1], 2),       # rank 4, three outer digits
    ([3, 4, 5, 6], [360, 90, 18, 1], 0),       # dims 1 and 2 merge (90 = 18 * 5)
    ([40, 33], [-40, 1], 1560 + 3),            # rows in reverse order
    ([500], [3], 4),                           # stride 3
    ([50, 40], [1, 50], 0),                    # transposed (dense, permuted: argmax in memory order)
    ([6, 7, 8], [1, 48, 6], 0),                # rank-3 permutation
    ([9, 5, 4], [20, 1, 5], 3),                # rank-3 permutation, offset
    ([20, 30], [2, 60], 1),                    # inner stride 60
    ([33, 17], [-1, 40], 32),                  # negative inner stride
    # dense ranges read backwards: streamed flat from the lowest element
    # (argmax keeps the row walk, whose indices follow the view)
    ([5000], [-1], 4999),                      # reversed
    ([40, 33], [-33, -1], 1319),               # fully reversed
    ([33, 40], [-1, 33], 32),                  # reversed transpose
]


def _view_elems(host, shape, strides, offset):
    idx = offset + sum(np.indices(shape)[d] * strides[d] for d in range(len(shape)))
    return np.ascontiguousarray(host[idx.ravel()])


@pytest.mark.parametrize("view", ROW_VIEWS, ids=lambda v: "x".join(map(str, v[0])) + "_" + "_".join(map(str, v[1])))
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
def test_full_reduce_row_walks(device, oracle, view, dtype):
    shape, strides, offset = view
    span = offset + 1 + sum((e - 1) * st for e, st in zip(shape, strides) if st > 0)
    host = inputs(oracle, dtype, span + 3, seed=sum(shape) + 7)
    if dtype != np.float32:
        host = (host % 977).astype(dtype)  # ties for argmax
    lay = Layout.try_new(shape, strides, offset)
    sel = _view_elems(host, shape, strides, offset)
    buf = device.upload(host)
    one = Layout.c_contiguous([1])
    out = device.alloc_zeroed(dtype, 1)

    def run(op):
        FULL.reduce_full_into(device, op, StridedView(buf, lay), StridedView(out, one))
        return device.download_owned(out)[0]

    if dtype == np.float32:
        ref, ab = oracle.full_sum(sel)
        assert abs(float(run(hx.SumOp)) - ref) <= f32_bound(sel.size, ab)
    else:
        assert run(hx.SumOp) == oracle.full_sum(sel)
        assert run(hx.ProdOp) == oracle.full_prod(sel)
    assert run(hx.MaxOp) == oracle.full_max(sel)
    assert run(hx.MinOp) == oracle.full_min(sel)
    idx = device.alloc_zeroed(np.uint32, 1)
    val = device.alloc_zeroed(dtype, 1)
    FULL.argmax_full_into(device, StridedView(buf, lay), idx, val)
    want = oracle.full_argmax(sel)
    assert int(device.download_owned(idx)[0]) == want
    assert device.download_owned(val)[0] == sel[want]


@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
def test_full_reduce_of_a_long_reversed_view(device, oracle, dtype):
    """A reversed dense view of 2^20 + 3 elements (many blocks, a ragged
    end) reduced by every kind: the flat stream from its lowest element."""
    n = (1 << 20) + 3
    host = inputs(oracle, dtype, n + 2, seed=23)
    if dtype != np.float32:
        host = (host % 977).astype(dtype)
    lay = Layout.try_new([n], [-1], n)  # elements n .. 1 of the buffer
    sel = np.ascontiguousarray(host[1:n + 1][::-1])
    buf = device.upload(host)
    one = Layout.c_contiguous([1])
    out = device.alloc_zeroed(dtype, 1)

    def run(op, prologue=None):
        FULL.reduce_full_into(device, op, StridedView(buf, lay), StridedView(out, one), prologue=prologue)
        return device.download_owned(out)[0]

    if dtype == np.float32:
        ref, ab = oracle.full_sum(sel)
        assert abs(float(run(hx.SumOp)) - ref) <= f32_bound(n, ab)
        assert abs(float(run(hx.MeanOp)) - ref / n) <= f32_bound(n, ab) / n + EPS * abs(ref / n)
        ref, ab = oracle.full_sum(sel, prologue=(0.5, 0.25))
        assert abs(float(run(hx.SumOp, (0.5, 0.25))) - ref) <= f32_bound(n, ab)
    else:
        assert run(hx.SumOp) == oracle.full_sum(sel)
        assert run(hx.ProdOp) == oracle.full_prod(sel)
    assert run(hx.MaxOp) == oracle.full_max(sel)
    assert run(hx.MinOp) == oracle.full_min(sel)
    idx = device.alloc_zeroed(np.uint32, 1)
    val = device.alloc_zeroed(dtype, 1)
    FULL.argmax_full_into(device, StridedView(buf, lay), idx, val)
    assert int(device.download_owned(idx)[0]) == oracle.full_argmax(sel)


def test_full_reduce_row_walk_with_prologue(device, oracle):
    host = inputs(oracle, np.float32, 70000, seed=3)
    shape, strides, offset = [250, 255], [257, 1], 2
    lay = Layout.try_new(shape, strides, offset)
    sel = _view_elems(host, shape, strides, offset)
    buf = device.upload(host)
    one = Layout.c_contiguous([1])
    out = device.alloc_zeroed(np.float32, 1)
    FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, lay), StridedView(out, one), prologue=(0.5, 0.25))
    ref, ab = oracle.full_sum(sel, prologue=(0.5, 0.25))
    assert abs(float(device.download_owned(out)[0]) - ref) <= f32_bound(sel.size, ab)
    idx = device.alloc_zeroed(np.uint32, 1)
    FULL.argmax_full_into(device, StridedView(buf, lay), idx, None, prologue=(-0.5, 0.25))
    assert int(device.download_owned(idx)[0]) == oracle.full_argmax(sel, prologue=(-0.5, 0.25))


def test_full_reduce_row_walk_at_scale(device, oracle):
    """A 4096 x 4000 slice of 4096-wide rows (the walker's multi-row steps,
    the fallback-free path at full grid) and its stride-2 columns."""
    rows, cols, ld = 4096, 4000, 4096
    host = inputs(oracle, np.uint32, rows * ld, seed=21)
    buf = device.upload(host)
    one = Layout.c_contiguous([1])
    out = device.alloc_zeroed(np.uint32, 1)
    for shape, strides in (([rows, cols], [ld, 1]), ([rows, cols // 2], [ld, 2])):
        lay = Layout.try_new(shape, strides, 0)
        sel = _view_elems(host, shape, strides, 0)
        FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, lay), StridedView(out, one))
        assert device.download_owned(out)[0] == oracle.full_sum(sel)
        idx = device.alloc_zeroed(np.uint32, 1)
        FULL.argmax_full_into(device, StridedView(buf, lay), idx, None)
        assert int(device.download_owned(idx)[0]) == oracle.full_argmax(sel)


def test_full_reduce_output_offset(device):
    buf = device.upload(np.arange(10, dtype=np.uint32))
    out = device.upload(np.full(4, 99, np.uint32))
    FULL.reduce_full_into(device, hx.SumOp, StridedView(buf, Layout.c_contiguous([10])),
                          StridedView(out, Layout.try_new([1], [1], 2)))
    assert list(device.download_owned(out)) == [99, 99, 45, 99]


def test_integer_mean_at_the_largest_counts(device):
    """Integer means at counts beyond 2^31: the wrapped sum divided by the
    count in the element type.  A constant input gives the sum in closed
    form (c*n mod 2^32); an i32 count of 2^31 is rejected before launch and
    leaves the output untouched."""
    n_u = (1 << 31) + 3  # 8 GiB of u32
    print(f"[mean] u32 mean over {n_u} elements, i32 over {2**31 - 1}", flush=True)
    buf = device.alloc_uninitialized(np.uint32, n_u)
    out = device.upload(np.full(1, 99, np.uint32))
    one = Layout.c_contiguous([1])
    for c in (1, 3, 0xFFFFFFFF):
        device.fill_uniform_int(buf, seed=1, lo=c, hi=c)
        FULL.reduce_full_into(device, hx.MeanOp, StridedView(buf, Layout.c_contiguous([n_u])), StridedView(out, one))
        assert int(device.download_owned(out)[0]) == ((c * n_u) % 2**32) // n_u, c
    ibuf = hx.RocmBuffer(device, buf.ptr, n_u, np.int32)  # the same memory viewed as i32
    try:
        iout = device.upload(np.full(1, 99, np.int32))
        n_i = (1 << 31) - 1
        for c in (1, -1, 3):
            device.fill_uniform_int(ibuf, seed=1, lo=c, hi=c)
            FULL.reduce_full_into(device, hx.MeanOp, StridedView(ibuf, Layout.c_contiguous([n_i])),
                                  StridedView(iout, one))
            wrapped = ((c * n_i + 2**31) % 2**32) - 2**31
            assert int(device.download_owned(iout)[0]) == int(wrapped / n_i), c  # C division truncates
        device.write_buffer(iout, np.full(1, 99, np.int32))
        with pytest.raises(hx.DispatchFailed, match="i32 divisor range"):
            FULL.reduce_full_into(device, hx.MeanOp, StridedView(ibuf, Layout.c_contiguous([1 << 31])),
                                  StridedView(iout, one))
        assert int(device.download_owned(iout)[0]) == 99
    finally:
        ibuf.ptr = None  # the memory belongs to `buf`


def test_full_sum_with_prologue(device, oracle):
    x = oracle.uniform_real((1 << 20) + 5, seed=2, lo=-1.0, hi=1.0)
    ref, ab = oracle.full_sum(x, prologue=(0.5, 0.25))
    got = float(full(device, hx.SumOp, x, prologue=(0.5, 0.25)))
    assert abs(got - ref) <= f32_bound(x.size, ab)
    assert full(device, hx.MaxOp, x, prologue=(0.5, 0.25)) == oracle.full_max(x, prologue=(0.5, 0.25))


def test_full_special_values(device):
    nan, inf = np.float32("nan"), np.float32("inf")
    assert full(device, hx.MaxOp, np.array([nan, 1.0, nan, -2.0], np.float32)) == 1.0
    assert full(device, hx.MaxOp, np.array([nan, nan], np.float32)) == np.float32(-3.4028235e38)
    assert full(device, hx.MaxOp, np.array([-inf, -inf], np.float32)) == np.float32(-3.4028235e38)
    assert full(device, hx.MinOp, np.array([inf], np.float32)) == np.float32(3.4028235e38)
    z = np.array([-0.0, 0.0, -0.0], np.float32)
    assert full(device, hx.MaxOp, z).view(np.uint32) == 0
    assert full(device, hx.MinOp, z).view(np.uint32) == 0x80000000
    assert full(device, hx.MaxOp, np.zeros(0, np.int32)) == np.iinfo(np.int32).min
    assert full(device, hx.ProdOp, np.zeros(0, np.uint32)) == 1
    assert full(device, hx.MinOp, np.zeros(0, np.uint32)) == 0xFFFFFFFF


# ------------------------------------------------------------ argmax
@pytest.mark.parametrize("dtype", [np.float32, np.uint32, np.int32])
@pytest.mark.parametrize("n", [1, 2, 65, 4097, 1 << 20])
def test_full_argmax_matches_oracle(device, oracle, dtype, n):
    x = inputs(oracle, dtype, n, seed=n + 3)
    if dtype != np.float32:
        x = (x % 97).astype(dtype)  # many ties: lowest index must win
    buf = device.upload(x)
    idx = device.alloc_zeroed(np.uint32, 1)
    val = device.alloc_zeroed(dtype, 1)
    FULL.argmax_full_into(device, StridedView(buf, Layout.c_contiguous([n])), idx, val)
    want = oracle.full_argmax(x)
    assert int(device.download_owned(idx)[0]) == want
    assert device.download_owned(val)[0] == x[want]


def test_argmax_special_cases(device):
    def am(host, prologue=None):
        buf = device.upload(host)
        idx = device.alloc_zeroed(np.uint32, 1)
        FULL.argmax_full_into(device, StridedView(buf, Layout.c_contiguous([host.size])), idx, prologue=prologue)
        return int(device.download_owned(idx)[0])

    nan = np.float32("nan")
    assert am(np.array([nan, 1.0, 5.0, 5.0], np.float32)) == 2
    assert am(np.array([nan, nan], np.float32)) == 0xFFFFFFFF
    assert am(np.array([-0.0, 0.0], np.float32)) == 1
    assert am(np.zeros(0, np.float32)) == 0xFFFFFFFF
    assert am(np.array([3.0, -1.0], np.float32), prologue=(-1.0, 0.0)) == 1


# ------------------------------------------------------------ rows
@pytest.mark.parametrize("rows,cols,ld,offset", [
    (1, 1, 1, 0), (3, 4, 4, 0), (7, 63, 63, 0), (5, 64, 68, 4), (33, 4096, 4096, 0),
    (17, 4099, 4103, 1), (256, 1000, 1000, 0), (1000, 257, 260, 8), (2, 70000, 70000, 0),
    # row starts off 16-byte boundaries: 0-3 element heads and tails per row
    (300, 4095, 4095, 0), (129, 4093, 4093, 3), (77, 4097, 4097, 2), (64, 3, 5, 1), (5, 6, 7, 3),
    # few long rows off 16-byte boundaries (split rows)
    (3, 70001, 70003, 1), (1, 200003, 200003, 2)])
def test_rows_fused_f32(device, oracle, rows, cols, ld, offset):
    host = oracle.normal(offset + (rows - 1) * ld + cols + 3, seed=rows * cols)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host[offset:], rows, cols, ld, prologue=(0.5, 0.25))
    buf = device.upload(host)
    s = device.alloc_zeroed(np.float32, rows)
    m = device.alloc_zeroed(np.float32, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    AXIS.reduce_rows_fused(device, buf, rows, cols, ld, offset, (0.5, 0.25), s, m, i)
    gs, gm, gi = device.download_owned(s), device.download_owned(m), device.download_owned(i)
    assert np.array_equal(gi, i_ref)
    assert np.array_equal(gm.view(np.uint32), m_ref.view(np.uint32))
    bound = np.array([f32_bound(cols, a) for a in a_ref])
    assert np.all(np.abs(gs.astype(np.float64) - s_ref) <= bound)


# Row lengths either side of every lanes-per-row threshold (4, 16, 64, 128 and
# 256 lanes, about four 16-byte vectors per lane), with 67 rows so the last
# block of the 4- and 16-lane forms is partly empty, and starts off 16-byte
# boundaries (offset 1, row stride cols + 1).
@pytest.mark.parametrize("cols", [1, 2, 3, 15, 16, 17, 63, 64, 65, 127, 128, 255, 256, 257, 1023, 1024, 1025,
                                  2047, 2048, 2049, 4095, 4096, 4097, 8191])
@pytest.mark.parametrize("aligned", [True, False])
def test_rows_fused_across_group_sizes(device, oracle, cols, aligned):
    rows = 67
    ld, offset = (cols, 0) if aligned else (cols + 1, 1)
    host = oracle.normal(offset + (rows - 1) * ld + cols, seed=cols + 7)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host[offset:], rows, cols, ld, prologue=(0.5, 0.25))
    buf = device.upload(host)
    s = device.alloc_zeroed(np.float32, rows)
    m = device.alloc_zeroed(np.float32, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    AXIS.reduce_rows_fused(device, buf, rows, cols, ld, offset, (0.5, 0.25), s, m, i)
    assert np.array_equal(device.download_owned(i), i_ref)
    assert np.array_equal(device.download_owned(m).view(np.uint32), m_ref.view(np.uint32))
    bound = np.array([f32_bound(cols, a) for a in a_ref])
    assert np.all(np.abs(device.download_owned(s).astype(np.float64) - s_ref) <= bound)


@pytest.mark.parametrize("dtype", [np.uint32, np.int32])
def test_rows_fused_integers(device, oracle, dtype):
    rows, cols = 300, 777
    host = (inputs(oracle, dtype, rows * cols, seed=5) % 50).astype(dtype)
    s_ref, _, m_ref, i_ref = oracle.rows(host, rows, cols)
    buf = device.upload(host)
    s = device.alloc_zeroed(dtype, rows)
    m = device.alloc_zeroed(dtype, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    AXIS.reduce_rows_fused(device, buf, rows, cols, out_sum=s, out_max=m, out_argmax=i)
    assert np.array_equal(device.download_owned(s), s_ref)
    assert np.array_equal(device.download_owned(m), m_ref)
    assert np.array_equal(device.download_owned(i), i_ref)


@pytest.mark.parametrize("subset", ["sum", "max", "argmax", "sum+argmax", "max+argmax"])
def test_rows_output_subsets(device, oracle, subset):
    rows, cols = 40, 300
    host = oracle.normal(rows * cols, seed=8)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host, rows, cols)
    buf = device.upload(host)
    want = subset.split("+")
    s = device.upload(np.full(rows, 7.0, np.float32)) if "sum" in want else None
    m = device.upload(np.full(rows, 7.0, np.float32)) if "max" in want else None
    i = device.upload(np.full(rows, 7, np.uint32)) if "argmax" in want else None
    AXIS.reduce_rows_fused(device, buf, rows, cols, out_sum=s, out_max=m, out_argmax=i)
    if s is not None:
        assert np.all(np.abs(device.download_owned(s) - s_ref) <= [f32_bound(cols, a) for a in a_ref])
    if m is not None:
        assert np.array_equal(device.download_owned(m), m_ref)
    if i is not None:
        assert np.array_equal(device.download_owned(i), i_ref)


def _special_rows(rng, rows, cols):
    """Rows drawn from small pools of special values, so NaNs of both signs,
    signed zeros, infinities, f32 extremes and ties fall inside every 16-value
    stretch a lane reads: each row family stresses one rule of the max/argmax
    order (NaN ignored, -0 < +0, the first of equal maxima)."""
    qnan, nqnan, snan = (np.array([b], np.uint32).view(np.float32) for b in (0x7FC00000, 0xFFC00000, 0x7F800001))
    inf, fmax = np.float32(np.inf), np.float32(3.4028235e38)
    pools = [
        np.concatenate([qnan, nqnan, snan, np.float32([-0.0, 0.0, 1.0, -1.0])]),  # max 1, ties
        np.concatenate([qnan, nqnan, np.float32([-0.0, -0.0, -0.0, 0.0])]),       # zeros only
        np.concatenate([qnan, nqnan, snan]),                                       # NaN only: no max
        np.concatenate([nqnan, np.float32([-inf, -inf])]),                         # below f32::MIN
        np.concatenate([qnan, np.float32([inf, -inf, fmax, -fmax, 2.0])]),         # infinities
        np.float32([fmax, -fmax, 1.0, -1.0]),                                      # extremes, sums overflow f32
    ]
    x = np.empty((rows, cols), np.float32)
    for r in range(rows):
        pool = pools[r % len(pools)]
        x[r] = pool[rng.integers(0, pool.size, cols)]
        if r % 7 == 3:  # a single winner placed late in the row
            x[r, (r * 131) % cols] = np.float32(8.0) if r % len(pools) in (0, 4, 5) else x[r, 0]
    return x


@pytest.mark.parametrize("rows,cols", [(96, 4096), (48, 16384), (60, 1000), (64, 64), (6, 70001), (9000, 3),
                                       (20000, 1), (5000, 8)])
@pytest.mark.parametrize("prologue", [None, (0.5, 0.25)])
def test_rows_special_values(device, oracle, rows, cols, prologue):
    """Max and argmax bit-exact with the oracle on NaNs, signed zeros,
    infinities and ties; sums equal in NaN/inf pattern and within the bound
    where finite (including rows whose partial sums pass f32's range)."""
    x = _special_rows(np.random.default_rng(rows * 10 + cols), rows, cols)
    s_ref, a_ref, m_ref, i_ref = oracle.rows(x.ravel(), rows, cols, prologue=prologue)
    buf = device.upload(x.ravel())
    s = device.alloc_zeroed(np.float32, rows)
    m = device.alloc_zeroed(np.float32, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    AXIS.reduce_rows_fused(device, buf, rows, cols, prologue=prologue, out_sum=s, out_max=m, out_argmax=i)
    gi, gm = device.download_owned(i), device.download_owned(m)
    bad = np.nonzero(gi != i_ref)[0]
    assert bad.size == 0, f"argmax rows {bad[:8]}: got {gi[bad[:8]]}, want {i_ref[bad[:8]]}"
    assert np.array_equal(gm.view(np.uint32), m_ref.view(np.uint32))
    gs = device.download_owned(s).astype(np.float64)
    with np.errstate(over="ignore"):  # sums past f32's range round to inf, as on the device
        ref32 = s_ref.astype(np.float32).astype(np.float64)  # the f32 the row sum rounds to
    nonfinite = ~np.isfinite(ref32)
    assert np.array_equal(np.isnan(gs), np.isnan(ref32))
    assert np.array_equal(gs[nonfinite & ~np.isnan(ref32)], ref32[nonfinite & ~np.isnan(ref32)])
    fin = ~nonfinite
    bound = np.array([f32_bound(cols, a) for a in a_ref])
    assert np.all(np.abs(gs[fin] - s_ref[fin]) <= bound[fin])


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("op", ["sum", "max", "min", "prod", "argmax"])
def test_axis_reduce_matches_oracle(device, oracle, axis, op):
    r, c = 123, 517
    host = (oracle.uniform_int(r * c, seed=11, lo=0, hi=9)).astype(np.uint32)
    mat = host.reshape(r, c)
    lines = mat if axis == 1 else np.ascontiguousarray(mat.T)
    if op == "sum":
        want = np.array([oracle.full_sum(l) for l in lines], np.uint32)
    elif op == "max":
        want = np.array([oracle.full_max(l) for l in lines], np.uint32)
    elif op == "min":
        want = np.array([oracle.full_min(l) for l in lines], np.uint32)
    elif op == "prod":
        want = np.array([oracle.full_prod(l) for l in lines], np.uint32)
    else:
        want = np.array([oracle.full_argmax(l) for l in lines], np.uint32)
    opcls = {"sum": hx.SumOp, "max": hx.MaxOp, "min": hx.MinOp, "prod": hx.ProdOp, "argmax": hx.ArgMaxOp}[op]
    buf = device.upload(host)
    out_shape = [r, 1] if axis == 1 else [1, c]
    out = device.alloc_zeroed(np.uint32, want.size)
    AXIS.reduce_axis_into(device, opcls, StridedView(buf, Layout.c_contiguous([r, c])), axis,
                          StridedView(out, Layout.c_contiguous(out_shape)))
    assert np.array_equal(device.download_owned(out), want)


# ------------------------------------------------------------ scans
@pytest.mark.parametrize("exclusive", [False, True])
@pytest.mark.parametrize("n", SIZES)
def test_scan_u32_bit_exact(device, oracle, n, exclusive):
    x = inputs(oracle, np.uint32, n, seed=n + 5)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, n)
    kind = hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.c_contiguous([n])), 0,
                        hx.ScanDirection.Forward, StridedView(out, Layout.c_contiguous([n])), kind)
    assert np.array_equal(device.download_owned(out), oracle.scan_sum(x, exclusive=exclusive))


# Scan tiles are 32768 elements and superblocks 64 tiles (2^21 elements):
# sizes on either side of both edges, and several superblocks with a
# ragged tail, in every direction and kind.
SCAN_EDGES = [32767, 32768, 32769, 3 * 32768 + 1, (1 << 21) - 1, 1 << 21, (1 << 21) + 1,
              3 * (1 << 21) + 32768 + 7]


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
@pytest.mark.parametrize("n", SCAN_EDGES)
def test_scan_u32_tile_and_superblock_edges(device, oracle, n, kind, direction):
    x = oracle.uniform_int(n, seed=n ^ 0x5A, lo=0, hi=2**32 - 1)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, n)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.c_contiguous([n])), 0, direction,
                        StridedView(out, Layout.c_contiguous([n])), kind)
    want = oracle.scan_sum(x, exclusive=kind == hx.ScanKind.Exclusive,
                           reverse=direction == hx.ScanDirection.Reverse)
    assert np.array_equal(device.download_owned(out), want)


# Reverse scans of lengths that are multiples of 4 take the mirrored
# 16-byte path for whole tiles and the scalar path for the ragged one.
REV_VEC = [4, 32768, 32772, 3 * 32768 + 100, (1 << 21) + 4, 64 * 32768 * 2 + 32768 + 12]


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("n", REV_VEC)
def test_reverse_scans_vector_path(device, oracle, n, kind):
    excl = kind == hx.ScanKind.Exclusive
    x = oracle.uniform_int(n, seed=n ^ 0x77, lo=0, hi=2**32 - 1)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, n)
    lay = Layout.c_contiguous([n])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 0, hx.ScanDirection.Reverse,
                        StridedView(out, lay), kind)
    assert np.array_equal(device.download_owned(out), oracle.scan_sum(x, exclusive=excl, reverse=True))
    xf = oracle.uniform_real(n, seed=n + 9, lo=-1.0, hi=1.0)
    fb = device.upload(xf)
    of = device.alloc_zeroed(np.float32, n)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(fb, lay), 0, hx.ScanDirection.Reverse,
                        StridedView(of, lay), kind)
    ref, ab = oracle.scan_sum(xf, exclusive=excl, reverse=True)
    bad, worst = oracle.check_f32_bound(device.download_owned(of), ref, ab, n)
    assert bad == 0, worst


@pytest.mark.parametrize("shape", [(3, 65540), (5, 32768), (2, 100004)])
def test_reverse_scans_of_rank2_lines(device, oracle, shape):
    r, c = shape
    x = oracle.uniform_int(r * c, seed=r * c, lo=-1000, hi=1000, dtype=np.int32)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.int32, r * c)
    lay = Layout.c_contiguous([r, c])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 1, hx.ScanDirection.Reverse,
                        StridedView(out, lay))
    want = np.cumsum(x.reshape(r, c)[:, ::-1], axis=1, dtype=np.int32)[:, ::-1]
    assert np.array_equal(device.download_owned(out).reshape(r, c), want)


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
def test_scans_of_views_read_backwards(device, oracle, kind, direction):
    """Lines that run backwards in both operands (stride -1): the planner
    scans the mirrored lines the other way, with ascending addresses, which
    must equal the view's own scan.  A long 1-D line (look-back tiles, a
    ragged end) of u32 and f32, and every row of a matrix read from its
    end."""
    excl = kind == hx.ScanKind.Exclusive
    rev = direction == hx.ScanDirection.Reverse
    n = (1 << 21) + 5
    x = oracle.uniform_int(n + 1, seed=51, lo=0, hi=2**32 - 1)
    buf = device.upload(x)
    out = device.upload(np.full(n + 1, 7, np.uint32))
    lay = Layout.try_new([n], [-1], n)  # elements n .. 1
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 0, direction, StridedView(out, lay), kind)
    got = device.download_owned(out)
    assert got[0] == 7
    assert np.array_equal(got[1:][::-1], oracle.scan_sum(np.ascontiguousarray(x[1:][::-1]), exclusive=excl,
                                                           reverse=rev))
    xf = oracle.uniform_real(n + 1, seed=52, lo=-1.0, hi=1.0)
    fb = device.upload(xf)
    fo = device.upload(np.full(n + 1, 7.0, np.float32))
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(fb, lay), 0, direction, StridedView(fo, lay), kind)
    ref, ab = oracle.scan_sum(np.ascontiguousarray(xf[1:][::-1]), exclusive=excl, reverse=rev)
    gf = device.download_owned(fo)
    assert gf[0] == 7.0
    bad, worst = oracle.check_f32_bound(np.ascontiguousarray(gf[1:][::-1]), ref, ab, n)
    assert bad == 0, worst
    r, c = 300, 1001
    xi = oracle.uniform_int(r * c, seed=53, lo=-1000, hi=1000, dtype=np.int32)
    ib = device.upload(xi)
    ob = device.alloc_zeroed(np.int32, r * c)
    rl = Layout.try_new([r, c], [c, -1], c - 1)  # every row read from its end
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(ib, rl), 1, direction, StridedView(ob, rl), kind)
    m = xi.reshape(r, c)[:, ::-1]
    v = m[:, ::-1] if rev else m
    want = np.cumsum(v, axis=1, dtype=np.int32)
    if excl:
        want = np.concatenate([np.zeros((r, 1), np.int32), want[:, :-1]], axis=1)
    if rev:
        want = want[:, ::-1]
    assert np.array_equal(device.download_owned(ob).reshape(r, c)[:, ::-1], want)


@pytest.mark.parametrize("dtype", [np.uint32, np.float32])
@pytest.mark.parametrize("in_off,out_off", [(1, 1), (0, 3), (2, 1), (3, 0), (8, 8), (0, 17), (31, 5)])
@pytest.mark.parametrize("kind,direction", [(hx.ScanKind.Inclusive, hx.ScanDirection.Forward),
                                            (hx.ScanKind.Exclusive, hx.ScanDirection.Forward),
                                            (hx.ScanKind.Exclusive, hx.ScanDirection.Reverse)])
def test_scans_of_views_off_16_byte_boundaries(device, oracle, dtype, in_off, out_off, kind, direction):
    """Long lines whose output starts off a 128-byte boundary run on a
    virtual line 1-31 elements longer, tiles on the output's 128-byte grid:
    the virtual elements (before a forward line, past a reverse line's end)
    are never read or stored, and every other element is.  Input offsets
    independent of the output's; a second pass scans rows whose starts share
    one misalignment (row stride a multiple of 32)."""
    excl = kind == hx.ScanKind.Exclusive
    rev = direction == hx.ScanDirection.Reverse
    n = (1 << 21) + 7
    if dtype == np.uint32:
        x = oracle.uniform_int(n + 32, seed=61, lo=0, hi=2**32 - 1)
    else:
        x = oracle.uniform_real(n + 32, seed=62, lo=-1.0, hi=1.0)
    buf = device.upload(x)
    out = device.upload(np.full(n + 32, 7, dtype))
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.try_new([n], [1], in_off)), 0,
                        direction, StridedView(out, Layout.try_new([n], [1], out_off)), kind)
    got = device.download_owned(out)
    assert np.all(got[:out_off] == 7) and np.all(got[out_off + n:] == 7)
    xs = np.ascontiguousarray(x[in_off:in_off + n])
    if dtype == np.uint32:
        assert np.array_equal(got[out_off:out_off + n], oracle.scan_sum(xs, exclusive=excl, reverse=rev))
    else:
        ref, ab = oracle.scan_sum(xs, exclusive=excl, reverse=rev)
        bad, worst = oracle.check_f32_bound(np.ascontiguousarray(got[out_off:out_off + n]), ref, ab, n)
        assert bad == 0, worst
    if dtype == np.uint32:
        r, c, ld = 3, 70001, 70016
        xi = oracle.uniform_int(r * ld + 32, seed=63, lo=0, hi=2**32 - 1)
        ib = device.upload(xi)
        ob = device.upload(np.full(r * ld + 32, 7, np.uint32))
        SCAN.scan_axis_into(device, hx.CumProdOp, StridedView(ib, Layout.try_new([r, c], [ld, 1], in_off)), 1,
                            direction, StridedView(ob, Layout.try_new([r, c], [ld, 1], out_off)), kind)
        g = device.download_owned(ob)
        for k in range(r):
            want = oracle.scan_prod(np.ascontiguousarray(xi[in_off + k * ld:in_off + k * ld + c]), exclusive=excl,
                                    reverse=rev)
            assert np.array_equal(g[out_off + k * ld:out_off + k * ld + c], want), k
            assert np.all(g[out_off + k * ld + c:out_off + (k + 1) * ld] == 7), k


@pytest.mark.parametrize("n", SCAN_EDGES)
def test_scan_f32_tile_and_superblock_edges(device, oracle, n):
    x = oracle.uniform_real(n, seed=n + 3, lo=-1.0, hi=1.0)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.float32, n)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.c_contiguous([n])), 0,
                        hx.ScanDirection.Forward, StridedView(out, Layout.c_contiguous([n])))
    ref, ab = oracle.scan_sum(x)
    bad, worst = oracle.check_f32_bound(device.download_owned(out), ref, ab, n)
    assert bad == 0, worst


# f32 lines longer than 32768 elements take 8-wave x 16-step tiles of 32768
# elements: lengths either side of one, two and 64 tiles (a superblock), the
# mirrored reverse path, and lengths of the former 49152-element f32 tiles.
F32_LONG = [32769, 65535, 65536, 65537, 2 * 32768 + 4, 49152, 49153, 64 * 32768, 64 * 32768 + 32768 + 12,
            65 * 32768 + 3, 65 * 49152 + 3]


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
@pytest.mark.parametrize("n", F32_LONG)
def test_scan_f32_long_tile_edges(device, oracle, n, direction, kind):
    rev = direction == hx.ScanDirection.Reverse
    excl = kind == hx.ScanKind.Exclusive
    x = oracle.uniform_real(n, seed=n + 21, lo=-1.0, hi=1.0)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.float32, n)
    lay = Layout.c_contiguous([n])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 0, direction, StridedView(out, lay), kind)
    ref, ab = oracle.scan_sum(x, exclusive=excl, reverse=rev)
    bad, worst = oracle.check_f32_bound(device.download_owned(out), ref, ab, n)
    assert bad == 0, worst


# Special values in early tiles reach later tiles through the f64 tile carry
# (applied as an f32 hi + lo pair): infinities, NaN and, for products, zeros.
# Lines of five 32768-element tiles and a ragged sixth, one launch for all
# lines.  Non-finite and zero outputs must match numpy's f64 scan in kind;
# finite ones stay within the bound (sums) or gamma_{n-1} relative
# (products).  A carry beyond f32's range gives +-inf, as the reference's
# f32 accumulation does (crates/hephaestus-core/src/domain/accelerator/
# scan.rs:90-150), so the values stay far from it.
SPECIAL_LEN = 5 * 32768 + 77


def _special_lines(op):
    rng = np.random.default_rng(4242 if op == "sum" else 4343)
    lo, hi = (0.0, 1.0) if op == "sum" else (0.999, 1.001)
    x = rng.uniform(lo, hi, (6, SPECIAL_LEN)).astype(np.float32)
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    x[0, 40000] = inf                           # +inf from tile 1 on
    x[1, 70000] = nan                           # NaN from tile 2 on
    x[2, 100] = 0.0 if op == "prod" else inf    # prod: 0, then 0 * inf = NaN; sum: inf, then inf - inf
    x[2, 100000] = inf if op == "prod" else -inf
    x[3, 32768] = -inf                          # first element of tile 1
    x[5, 50000] = 0.0 if op == "prod" else x[5, 50000]  # prod: exact zeros from tile 1 on
    x[5, SPECIAL_LEN - 1] = nan                 # the ragged last tile
    return x


@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("op", ["sum", "prod"])
def test_scan_f32_special_values_across_tiles(device, oracle, op, kind, direction):
    x = _special_lines(op)
    rows, cols = x.shape
    buf = device.upload(x.reshape(-1))
    out = device.alloc_zeroed(np.float32, rows * cols)
    lay = Layout.c_contiguous([rows, cols])
    SCAN.scan_axis_into(device, hx.CumSumOp if op == "sum" else hx.CumProdOp, StridedView(buf, lay), 1,
                        direction, StridedView(out, lay), kind)
    got = device.download_owned(out).reshape(rows, cols).astype(np.float64)
    rev = direction == hx.ScanDirection.Reverse
    k = 2 * oracle.ceil_log2(cols) * 2.0**-23
    g = (cols - 1) * 2.0**-24
    for r in range(rows):
        v = x[r].astype(np.float64)[::-1] if rev else x[r].astype(np.float64)
        with np.errstate(invalid="ignore"):
            want = np.cumsum(v) if op == "sum" else np.cumprod(v)
            ab = np.cumsum(np.abs(v))
        if kind == hx.ScanKind.Exclusive:
            want = np.concatenate([[0.0 if op == "sum" else 1.0], want[:-1]])
            ab = np.concatenate([[0.0], ab[:-1]])
        if rev:
            want, ab = want[::-1], ab[::-1]
        g_r = got[r]
        assert np.array_equal(np.isnan(g_r), np.isnan(want)), (r, "NaN pattern")
        assert np.array_equal(np.isposinf(g_r), np.isposinf(want)), (r, "+inf pattern")
        assert np.array_equal(np.isneginf(g_r), np.isneginf(want)), (r, "-inf pattern")
        fin = np.isfinite(want)
        if op == "sum":
            assert np.all(np.abs(g_r[fin] - want[fin]) <= k * ab[fin]), r
        else:
            assert np.array_equal(g_r[fin] == 0.0, want[fin] == 0.0), (r, "zeros")
            assert np.all(np.abs(g_r[fin] - want[fin]) <= g / (1.0 - g) * np.abs(want[fin])), r


@pytest.mark.parametrize("shape", [(3, 49153), (2, 64 * 49152 + 5)])
def test_scan_f32_long_rank2_lines(device, oracle, shape):
    """Several long f32 lines in one launch: tiles and superblocks per line."""
    r, c = shape
    x = oracle.uniform_real(r * c, seed=r + c, lo=0.0, hi=1.0)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.float32, r * c)
    lay = Layout.c_contiguous([r, c])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), 1, hx.ScanDirection.Forward,
                        StridedView(out, lay))
    got = device.download_owned(out).reshape(r, c)
    for i in range(r):
        ref, ab = oracle.scan_sum(x[i * c:(i + 1) * c])
        assert oracle.check_f32_bound(got[i], ref, ab, c)[0] == 0, i


@pytest.mark.parametrize("exclusive", [False, True])
@pytest.mark.parametrize("n", [1, 2, 5, 4096, 4097, 65536 + 17, (1 << 20) + 3])
def test_scan_f32_within_bound(device, oracle, n, exclusive):
    x = oracle.uniform_real(n, seed=n, lo=0.0, hi=1.0)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.float32, n)
    kind = hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.c_contiguous([n])), 0,
                        hx.ScanDirection.Forward, StridedView(out, Layout.c_contiguous([n])), kind)
    ref, ab = oracle.scan_sum(x, exclusive=exclusive)
    bad, worst = oracle.check_f32_bound(device.download_owned(out), ref, ab, n)
    assert bad == 0, worst


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
@pytest.mark.parametrize("op", ["sum", "prod"])
def test_scan_directions_kinds_and_ops(device, oracle, kind, direction, op):
    n = 50001
    x = (oracle.uniform_int(n, seed=12, lo=0, hi=2**32 - 1) | 1).astype(np.uint32)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, n)
    opcls = hx.CumSumOp if op == "sum" else hx.CumProdOp
    SCAN.scan_axis_into(device, opcls, StridedView(buf, Layout.c_contiguous([n])), 0, direction,
                        StridedView(out, Layout.c_contiguous([n])), kind)
    fn = oracle.scan_sum if op == "sum" else oracle.scan_prod
    want = fn(x, exclusive=kind == hx.ScanKind.Exclusive, reverse=direction == hx.ScanDirection.Reverse)
    assert np.array_equal(device.download_owned(out), want)


@pytest.mark.parametrize("kind", [hx.ScanKind.Inclusive, hx.ScanKind.Exclusive])
@pytest.mark.parametrize("direction", [hx.ScanDirection.Forward, hx.ScanDirection.Reverse])
@pytest.mark.parametrize("n", [5, 4097, 100003])
def test_scan_f32_products_within_gamma(device, oracle, n, direction, kind):
    """f32 cumprod: no oracle function, so numpy's f64 product is the check,
    within gamma_{n-1} = (n-1)u/(1-(n-1)u) relative (u = 2^-24), the bound for
    a product of n f32 factors in any evaluation order."""
    x = oracle.uniform_real(n, seed=n + 21, lo=0.999, hi=1.001)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.float32, n)
    SCAN.scan_axis_into(device, hx.CumProdOp, StridedView(buf, Layout.c_contiguous([n])), 0, direction,
                        StridedView(out, Layout.c_contiguous([n])), kind)
    v = x.astype(np.float64)[::-1] if direction == hx.ScanDirection.Reverse else x.astype(np.float64)
    want = np.cumprod(v)
    if kind == hx.ScanKind.Exclusive:
        want = np.concatenate([[1.0], want[:-1]])
    if direction == hx.ScanDirection.Reverse:
        want = want[::-1]
    k = (n - 1) * 2.0**-24
    got = device.download_owned(out).astype(np.float64)
    assert np.all(np.abs(got - want) <= k / (1.0 - k) * np.abs(want))


@pytest.mark.parametrize("shape,axis", [((512, 4096), 1), ((3, 10000), 1), ((4096, 300), 0), ((40, 7), 0),
                                        ((1000, 1001), 1), ((257, 5), 1),
                                        # one line along axis 0 (line stride 1, unused): vector path
                                        ((100000, 1), 0), ((100003, 1), 0)])
def test_scan_rank2_lines(device, oracle, shape, axis):
    r, c = shape
    host = oracle.uniform_int(r * c, seed=r + c, lo=-1000, hi=1000, dtype=np.int32)
    mat = host.reshape(r, c)
    buf = device.upload(host)
    out = device.alloc_zeroed(np.int32, r * c)
    lay = Layout.c_contiguous([r, c])
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, lay), axis, hx.ScanDirection.Forward,
                        StridedView(out, lay))
    want = np.cumsum(mat, axis=axis, dtype=np.int32)
    assert np.array_equal(device.download_owned(out).reshape(r, c), want)


def test_scan_strided_rank1_views(device, oracle):
    n = 20000
    host = oracle.uniform_int(3 * n + 10, seed=13, lo=0, hi=100)
    buf = device.upload(host)
    out = device.alloc_zeroed(np.uint32, 2 * n + 1)
    SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(buf, Layout.try_new([n], [3], 1)), 0,
                        hx.ScanDirection.Forward, StridedView(out, Layout.try_new([n], [2], 1)))
    got = device.download_owned(out)
    assert np.array_equal(got[1::2][:n], oracle.scan_sum(np.ascontiguousarray(host[1:3 * n:3])))
    assert np.all(got[0::2] == 0)  # untouched gaps


def test_scan_repeated_launches_reuse_workspace(device, oracle):
    """The look-back status words are tagged per launch: many launches in a
    row, switching sizes and dtypes, must each be exact."""
    for rep in range(6):
        n = [5000000, 4097, 1 << 20, 123457, 5000000, 7][rep]
        x = oracle.uniform_int(n, seed=rep, lo=0, hi=255)
        buf = device.upload(x)
        out = device.alloc_zeroed(np.uint32, n)
        SCAN.exclusive_scan_into(device, buf, out)
        assert np.array_equal(device.download_owned(out), oracle.scan_sum(x, exclusive=True)), rep
        xf = oracle.uniform_real(n, seed=rep, lo=0.0, hi=1.0)
        fb = device.upload(xf)
        fo = device.alloc_zeroed(np.float32, n)
        SCAN.inclusive_scan_into(device, fb, fo)
        bad, _ = oracle.check_scan_f32(xf, device.download_owned(fo))
        assert bad == 0, rep


# ------------------------------------------------------------ segmented
def _segmented(device, values, offsets):
    vb = device.upload(values)
    ob = device.upload(offsets.astype(np.uint32))
    out = device.upload(np.full(offsets.size - 1, 0x5A5A5A5A, np.uint32).view(values.dtype))
    SEG.segmented_sum_into(device, vb, ob, out)
    return device.download_owned(out)


def test_segmented_sum_edge_offsets(device, oracle):
    x = oracle.uniform_int(20000, seed=14, lo=-1000, hi=1000, dtype=np.int32)
    cases = [
        [0, 20000],
        [0, 0, 0, 20000, 20000],
        [0, 1, 2, 3, 4096, 4096, 4097, 8191, 8192, 8193, 20000],
        list(range(0, 20001, 1)),  # every element its own segment
        [0] + list(range(4096, 20000, 4096)) + [20000],  # boundaries on tile edges
        [0, 3, 3, 3, 19999, 20000],
    ]
    for off in cases:
        off = np.array(off, np.uint32)
        assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off)), off[:8]


@pytest.mark.parametrize("n,mean", [(1, 300.0), (4096, 300.0), (1 << 20, 300.0), ((1 << 20) + 9, 3.0),
                                    (1 << 20, 50000.0)])
def test_segmented_sum_geometric(device, oracle, n, mean):
    x = oracle.uniform_int(n, seed=n, lo=-1000, hi=1000, dtype=np.int32)
    off = oracle.geometric_offsets(n, mean, seed=n + 1)
    assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off))


# Mean segment lengths up to 29 take the segment-parallel path: blocks of
# up to 7424 S / n consecutive segments (at most 4096, 16 a thread), whole
# groups of 256 where that keeps 80% of them (3584, 1792, 768, 512 at
# means 2, 4, 8, 14, 256 at 28) and a partly filled last group otherwise (464
# at 16, 371 at 20); a span of up to 8192 values per block, longer spans
# deferred to a chunk worklist; means 31 and 40 take the element-tile path.
@pytest.mark.parametrize("mean", [0.5, 1.0, 2.0, 4.0, 8.0, 14.0, 16.0, 20.0, 28.0, 31.0, 40.0])
@pytest.mark.parametrize("dtype", [np.int32, np.uint32])
def test_segmented_sum_short_segments(device, oracle, mean, dtype):
    n = (1 << 20) + 13
    x = oracle.uniform_int(n, seed=int(mean * 10), lo=0, hi=1 << 31, dtype=np.uint32).view(dtype)
    off = oracle.geometric_offsets(n, mean, seed=int(mean * 10) + 1)
    assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off))


def _short_with_long(n, mean, longs, seed):
    """Geometric offsets of the given mean with the cuts inside each
    [start, start + length) of `longs` removed: long segments among short
    ones, so a block's span exceeds one 8192-value chunk."""
    rng = np.random.default_rng(seed)
    cuts = np.flatnonzero(rng.random(n - 1) < 1.0 / mean) + 1
    keep = np.ones(cuts.size, bool)
    for start, length in longs:
        keep &= ~((cuts > start) & (cuts < start + length))
    extra = [v for start, length in longs for v in (start, start + length) if 0 < v < n]
    cuts = np.unique(np.concatenate([cuts[keep], np.array(extra, np.int64)]))
    return np.concatenate([[0], cuts, [n]]).astype(np.uint32)


SHORT_LONG_CASES = [
    ((1 << 21) + 5, 2.0, [(1 << 20, 1 << 19)]),                      # one long segment mid-stream
    ((1 << 21) + 5, 4.0, [(100, 8192 - 100), (20000, 8193), (40000, 16384 * 3 + 1)]),
    ((1 << 20), 1.0, [(0, 8192), (8192, 8192), (16384, 1)]),         # exact chunk-sized segments at 0
    ((1 << 20), 3.0, [(5000, 9000), (14001, 9000), (23002, 9000)]),  # several long ones in one block
    ((1 << 20) + 1, 1.0, [(0, 1 << 19)]),                            # half of everything in one segment
]


@pytest.mark.parametrize("n,mean,longs", SHORT_LONG_CASES)
def test_segmented_sum_short_with_long_segments(device, oracle, n, mean, longs):
    x = oracle.uniform_int(n, seed=n % 1000, lo=-1 << 30, hi=1 << 30, dtype=np.int32)
    off = _short_with_long(n, mean, longs, seed=n % 997)
    assert 256 * n <= 7424 * (off.size - 1), "case must take the short path"
    assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off))


def test_segmented_short_path_empty_segments_around_one_long(device, oracle):
    """All values in one segment between 2^17 empty segments on each side:
    the mean is 8, so the short path takes it, and the one block holding
    the long segment defers 255 chunks, written by its wave together."""
    n = 1 << 21
    x = oracle.uniform_int(n, seed=35, lo=0, hi=1 << 20)
    off = np.concatenate([np.zeros(1 << 17, np.uint32), np.full(1 << 17, n, np.uint32)])
    got = _segmented(device, x, off)
    assert np.array_equal(got, oracle.segmented_sum(x, off))
    assert got[(1 << 17) - 1] == np.uint32(oracle.segmented_sum(x, np.array([0, n], np.uint32))[0])


def test_segmented_short_path_repeated_calls(device, oracle):
    """The deferred-chunk count is cleared by every call: back-to-back calls
    with different inputs, the second smaller, on the shared scratch."""
    for seed, n in ((1, (1 << 21) + 5), (2, (1 << 19) + 3), (3, (1 << 21) + 5)):
        x = oracle.uniform_int(n, seed=seed, lo=-1000, hi=1000, dtype=np.int32)
        off = _short_with_long(n, 2.0, [(n // 3, n // 4), (n // 2, 20000)], seed=seed)
        assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off)), seed


def test_prepared_segmented_sum_short_path(device, oracle):
    n = (1 << 20) + 7
    x = oracle.uniform_int(n, seed=31, lo=-1000, hi=1000, dtype=np.int32)
    off = _short_with_long(n, 4.0, [(7000, 50000)], seed=31)
    vb, ob = device.upload(x), device.upload(off)
    out = device.alloc_zeroed(np.int32, off.size - 1)
    plan = SEG.prepare_segmented_sum(device, vb, ob, out)
    assert plan.workspace_bytes() > 0
    for _ in range(3):
        plan.dispatch()
    assert np.array_equal(device.download_owned(out), oracle.segmented_sum(x, off))
    y = oracle.uniform_int(n, seed=32, lo=-1000, hi=1000, dtype=np.int32)
    device.write_buffer(vb, y)
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), oracle.segmented_sum(y, off))


def test_segmented_short_path_malformed_offsets_stay_in_bounds(device, oracle):
    """Decreasing offsets and offsets beyond n on the short path: the call
    completes without a fault, and a well-formed call afterwards is exact."""
    n = 100000
    x = oracle.uniform_int(n, seed=33, lo=0, hi=10)
    off = np.arange(0, n + 1, 2, dtype=np.uint32)
    off[100:5000:7] = 3
    off[6000:9000:5] = 4000000000
    off[20000] = n + 12345
    _segmented(device, x, off)
    good = oracle.geometric_offsets(n, 2.0, seed=34)
    assert np.array_equal(_segmented(device, x, good), oracle.segmented_sum(x, good))


def _crowded(n, mean, clusters, seed):
    """Geometric offsets of the given mean plus runs of empty segments:
    `clusters` holds (position, count) pairs; after each run, 200 short
    segments of 1..150 values start at the position (summed by the excess
    kernel when the run crowds their tile)."""
    rng = np.random.default_rng(seed)
    cuts = list(np.flatnonzero(rng.random(n - 1) < 1.0 / mean) + 1)
    for pos, count in clusters:
        cuts += [pos] * count
        cuts += list(pos + np.cumsum(rng.integers(1, 151, 200)))
    cuts = np.sort(np.array([c for c in cuts if 0 <= c <= n], np.int64))
    return np.concatenate([[0], cuts, [n]]).astype(np.uint32)


CROWDED_CASES = [
    ("trailing empties", [((1 << 22) + 5, 1 << 16)]),
    ("leading empties", [(0, 1 << 16)]),
    ("mid-tile run", [(3 * 8192 + 1000, 50000)]),
    ("runs at a tile edge and mid-tile", [(5 * 8192, 9000), (9 * 8192 + 77, 4097), (20 * 8192 + 5, 4095)]),
]


@pytest.mark.parametrize("name,clusters", CROWDED_CASES, ids=[c[0] for c in CROWDED_CASES])
def test_segmented_sum_crowded_tiles(device, oracle, name, clusters):
    """Tiles with more than 4096 segment ends (runs of empty segments) at a
    mean above the short-path limit: the element-tile path hands the excess
    ends to seg_excess_kernel, and empties at offset 0 are written by the
    tile map kernel."""
    n = (1 << 22) + 5
    x = oracle.uniform_int(n, seed=len(name), lo=-1 << 30, hi=1 << 30, dtype=np.int32)
    off = _crowded(n, 300.0, clusters, seed=len(name))
    assert 256 * n > 7424 * (off.size - 1), "case must take the element-tile path"
    assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off))


def test_prepared_segmented_sum_crowded_tile(device, oracle):
    n = (1 << 22) + 5
    x = oracle.uniform_int(n, seed=41, lo=-1000, hi=1000, dtype=np.int32)
    off = _crowded(n, 300.0, [(7 * 8192 + 3, 30000)], seed=41)
    vb, ob = device.upload(x), device.upload(off)
    out = device.alloc_zeroed(np.int32, off.size - 1)
    plan = SEG.prepare_segmented_sum(device, vb, ob, out)
    for _ in range(3):
        plan.dispatch()
    assert np.array_equal(device.download_owned(out), oracle.segmented_sum(x, off))


def test_segmented_crowded_malformed_offsets_stay_in_bounds(device, oracle):
    """A crowded tile whose offsets decrease: the call completes without a
    fault, and a well-formed call afterwards is exact."""
    n = 1 << 20
    x = oracle.uniform_int(n, seed=42, lo=0, hi=10)
    off = np.concatenate([[0], np.full(10000, 5000), np.full(10000, 3000), [n]]).astype(np.uint32)
    _segmented(device, x, off)
    good = oracle.geometric_offsets(n, 300.0, seed=43)
    assert np.array_equal(_segmented(device, x, good), oracle.segmented_sum(x, good))


def test_segmented_sum_16k_tile_edges(device, oracle):
    """Segmented tiles hold 16384 values: boundaries on and beside tile
    edges, empty segments at an edge, a segment spanning several tiles (the
    carry crosses tiles without a head), and runs of one-element segments
    across an edge."""
    t = 16384
    n = 4 * t + 77
    x = oracle.uniform_int(n, seed=16, lo=-1000, hi=1000, dtype=np.int32)
    cases = [
        [0, t - 1, t, t + 1, 2 * t, 2 * t, 2 * t, n],
        [0, 5, n - 3, n],                                   # spans every tile
        [0] + list(range(t - 40, t + 40)) + [3 * t, n],      # unit segments across an edge
        [0, t, 2 * t, 3 * t, 4 * t, n, n, n],               # exact tile edges, empties at n
        [0, 0, 0, 1, 2 * t + 3, 2 * t + 3, 4 * t, 4 * t + 1, n],
    ]
    for off in cases:
        off = np.array(off, np.uint32)
        assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off)), off[:8]


def test_segmented_sum_long_segment_tiles(device, oracle):
    """Means of 4096 values or more take 16384-value tiles: boundaries on
    and beside their edges, a segment spanning every tile, empties at an
    edge and at n."""
    t = 16384
    n = (1 << 20) + 77
    x = oracle.uniform_int(n, seed=44, lo=-1 << 30, hi=1 << 30, dtype=np.int32)
    cases = [
        [0, t - 1, t, t + 1, 3 * t, n],
        [0, 5, n - 3, n],
        [0, 2 * t, 2 * t, 2 * t, 40 * t + 3, n, n],
        [0, t // 2 + 1, 17 * t - 1, 33 * t, n],
    ]
    for off in cases:
        off = np.array(off, np.uint32)
        assert n >= 4096 * (off.size - 1), "case must take the long-segment tiles"
        assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off)), off[:8]


# 2^25 + 13 values: 4097 tiles of 8192 values (mean 3000) or 2049 of 16384
# (the rest), i.e. 32 to 64 superblocks of 64 tiles.  Means below 2^18 take
# the two-level look-back (superblock prefixes, missing superblocks folded
# from their tiles), the others the walk over tiles; "spanning" puts one
# segment of 2.1e7 values (20 superblocks of 16384-value tiles) among
# mean-3000 ones.
@pytest.mark.parametrize("mean", [3000.0, 50000.0, 200000.0, 300000.0, 1e7, "spanning"])
def test_segmented_sum_many_superblocks(device, oracle, mean):
    n = (1 << 25) + 13
    x = oracle.uniform_int(n, seed=51, lo=-1000, hi=1000, dtype=np.int32)
    if mean == "spanning":
        off = oracle.geometric_offsets(n, 3000.0, seed=52).astype(np.int64)
        a, b = 100 * 8192 + 7, 2660 * 8192 + 3
        off = np.concatenate([off[off < a], [a, b], off[off > b]]).astype(np.uint32)
    else:
        off = oracle.geometric_offsets(n, mean, seed=53)
    assert np.array_equal(_segmented(device, x, off), oracle.segmented_sum(x, off))


def _crowded_long(n, seed):
    """Geometric(20000) segments plus: 5000 empty segments mid-tile, 4097 at
    a 16384-value tile edge, and 3000 segments of 1..4 values packed into one
    tile -- crowded tiles (more than 2048 and more than 4096 ends) on the
    16384-value tile route."""
    rng = np.random.default_rng(seed)
    t = 16384
    cuts = list(np.flatnonzero(rng.random(n - 1) < 1.0 / 20000.0) + 1)
    cuts += [37 * t + 5000] * 5000
    cuts += [90 * t] * 4097
    cuts += list(150 * t + 11 + np.cumsum(rng.integers(1, 5, 3000)))
    cuts = np.sort(np.array([c for c in cuts if 0 <= c <= n], np.int64))
    return np.concatenate([[0], cuts, [n]]).astype(np.uint32)


def test_segmented_crowded_long_segment_tiles(device, oracle):
    """Crowded tiles on the long-segment route (mean n/S >= 4096 selects
    16384-value tiles): several mask rounds, and ends beyond the tile's
    first 4096 summed by the map kernel; immediate and prepared forms."""
    n = 1 << 26
    x = oracle.uniform_int(n, seed=45, lo=-1 << 30, hi=1 << 30, dtype=np.int32)
    off = _crowded_long(n, seed=45)
    s = off.size - 1
    assert n >= 4096 * s, "case must take the long-segment tiles"
    t = 16384
    ends_per_tile = np.bincount(np.minimum((off[1:].astype(np.int64) - 1) // t, n // t - 1), minlength=n // t)
    assert ends_per_tile.max() > 4096 and ((ends_per_tile > 2048) & (ends_per_tile <= 4096)).any()
    want = oracle.segmented_sum(x, off)
    assert np.array_equal(_segmented(device, x, off), want)
    vb, ob = device.upload(x), device.upload(off)
    out = device.alloc_zeroed(np.int32, s)
    plan = SEG.prepare_segmented_sum(device, vb, ob, out)
    for _ in range(2):
        plan.dispatch()
    assert np.array_equal(device.download_owned(out), want)


@pytest.mark.parametrize("cuts_n", [300, 12000])
@pytest.mark.parametrize("skew", [1, 2, 3])
def test_segmented_sum_values_off_16_byte_boundaries(device, oracle, skew, cuts_n):
    """Values handed over as a raw pointer at an element offset: the tile loads
    are 16-byte vectors that need only 4-byte alignment (300 cuts: the
    element-tile path; 12000: the short-segment path)."""
    from hephaestus_amd import _ffi

    n = 3 * 8192 + 77
    x = oracle.uniform_int(n + skew, seed=skew, lo=-1000, hi=1000, dtype=np.int32)
    rng = np.random.default_rng(skew)
    cuts = np.sort(rng.choice(np.arange(1, n), size=cuts_n, replace=False))
    offsets = np.concatenate([[0], cuts, [n]]).astype(np.uint32)
    vb = device.upload(x)
    ob = device.upload(offsets)
    out = device.upload(np.full(offsets.size - 1, 0x5A5A5A5A, np.uint32).view(np.int32))
    _ffi.check(_ffi.lib().hx_segmented_reduce(device.handle, _ffi.OP_SUM, _ffi.DTYPE_I32, vb.ptr + 4 * skew, n,
                                              ob.ptr, offsets.size, out.ptr, offsets.size - 1, None))
    assert np.array_equal(device.download_owned(out), oracle.segmented_sum(x[skew:], offsets))


def test_segmented_sum_empty_values(device):
    vb = device.alloc_zeroed(np.int32, 16)  # aligned allocation, but n = 0 values
    ob = device.upload(np.zeros(4, np.uint32))
    out = device.upload(np.full(3, 9, np.int32))
    from hephaestus_amd import _ffi
    _ffi.check(_ffi.lib().hx_segmented_reduce(device.handle, _ffi.OP_SUM, _ffi.DTYPE_I32, vb.ptr, 0,
                                              ob.ptr, 4, out.ptr, 3, None))
    assert list(device.download_owned(out)) == [0, 0, 0]


def test_segment_offsets_validation(device):
    ob = device.upload(np.array([0, 5, 3, 10], np.uint32))
    with pytest.raises(hx.DispatchFailed) as e:
        SEG.validate_offsets(device, ob, 10)
    assert e.value.message == "invalid segment offsets: offsets must be non-decreasing"
    ob = device.upload(np.array([0, 5, 9], np.uint32))
    with pytest.raises(hx.DispatchFailed) as e:
        SEG.validate_offsets(device, ob, 10)
    assert "start at 0 and end at the element count" in e.value.message
    SEG.validate_offsets(device, device.upload(np.array([0, 5, 10], np.uint32)), 10)


def test_segmented_malformed_offsets_stay_in_bounds(device, oracle):
    """Offsets beyond n are clamped; the call completes and never faults."""
    x = oracle.uniform_int(10000, seed=15, lo=0, hi=10)
    off = np.array([0, 5000, 20000, 30000], np.uint32)
    got = _segmented(device, x, off)
    assert got[0] == oracle.full_sum(x[:5000])
    assert got[1] == oracle.full_sum(x[5000:])
    assert got[2] == 0


# ------------------------------------------------------------ prepared plans
def test_prepared_plans_allocate_once_and_rebind(device, oracle):
    n = 1 << 20
    x = oracle.uniform_int(n, seed=16, lo=0, hi=255)
    buf = device.upload(x)
    out = device.alloc_zeroed(np.uint32, n)
    lay = Layout.c_contiguous([n])
    plan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(buf, lay), 0, hx.ScanDirection.Forward,
                                  StridedView(out, lay), hx.ScanKind.Exclusive)
    assert plan.workspace_bytes() > 0
    for _ in range(3):
        plan.dispatch()
    assert np.array_equal(device.download_owned(out), oracle.scan_sum(x, exclusive=True))
    y = oracle.uniform_int(n, seed=17, lo=0, hi=255)
    device.write_buffer(buf, y)
    plan.dispatch()
    assert np.array_equal(device.download_owned(out), oracle.scan_sum(y, exclusive=True))


def test_prepared_batch_submission(device, oracle):
    """submit_prepared_reduction_batch (prepared_reduction.rs:164-174): the
    min/max clause of the CUDA contract (tests/contract.rs:717-726) plus a
    map-reduction and a scan in the same batch, then a rebind."""
    n = 1027
    x = (np.arange(n) % 17).astype(np.uint32)
    buf = device.upload(x)
    one = Layout.c_contiguous([1])
    lay = Layout.c_contiguous([n])
    outs = [device.alloc_zeroed(np.uint32, 1) for _ in range(2)]
    pmin = FULL.prepare_reduce_full(device, hx.MinOp, StridedView(buf, lay), StridedView(outs[0], one))
    pmax = FULL.prepare_reduce_full(device, hx.MaxOp, StridedView(buf, lay), StridedView(outs[1], one))
    scan_out = device.alloc_zeroed(np.uint32, n)
    pscan = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(buf, lay), 0, hx.ScanDirection.Forward,
                                   StridedView(scan_out, lay), hx.ScanKind.Inclusive)
    pl1 = hx.PreparedMapReduction(device, hx._ffi.MAP_NORM_L1, StridedView(buf, lay), None)
    hx.submit_prepared_reduction_batch([pmin, pmax, pscan, pl1])
    assert device.download_owned(outs[0])[0] == 0
    assert device.download_owned(outs[1])[0] == 16
    assert np.array_equal(device.download_owned(scan_out), oracle.scan_sum(x))
    assert device.download_owned(pl1.output)[0] == oracle.full_sum(x)
    y = (x + 3).astype(np.uint32)
    device.write_buffer(buf, y)
    hx.submit_prepared_reduction_batch([pmin, pmax, pscan, pl1])
    assert device.download_owned(outs[0])[0] == 3
    assert device.download_owned(outs[1])[0] == 19
    assert np.array_equal(device.download_owned(scan_out), oracle.scan_sum(y))
    assert device.download_owned(pl1.output)[0] == oracle.full_sum(y)
    hx.submit_prepared_reduction_batch([])


def _check_rows(device, oracle, host, rows, cols, ld, offset, pro, s, m, i):
    s_ref, a_ref, m_ref, i_ref = oracle.rows(host[offset:], rows, cols, ld, prologue=pro)
    assert np.array_equal(device.download_owned(i), i_ref)
    assert np.array_equal(device.download_owned(m), m_ref)
    got = device.download_owned(s).astype(np.float64)
    if host.dtype == np.float32:
        assert np.all(np.abs(got - s_ref) <= f32_bound(cols, a_ref))
    else:
        assert np.array_equal(device.download_owned(s), s_ref)


@pytest.mark.parametrize("rows,cols,ld,offset", [(4096, 1000, 1000, 0), (300, 4099, 4101, 3), (8, 1 << 20, 1 << 20, 0)])
def test_prepared_rows_allocate_once_and_rebind(device, oracle, rows, cols, ld, offset):
    """hx_prepare_reduce_rows (prepared_axis_reduction.rs:20-222): dispatches
    re-read the bound input (rebind contract), and the few-long-rows split
    form keeps its partials in the plan's own workspace."""
    n = offset + (rows - 1) * ld + cols
    pro = (0.5, 0.25)
    x = oracle.normal(n, seed=31)
    buf = device.upload(x)
    s, m = device.alloc_zeroed(np.float32, rows), device.alloc_zeroed(np.float32, rows)
    i = device.alloc_zeroed(np.uint32, rows)
    plan = AXIS.prepare_reduce_rows_fused(device, buf, rows, cols, row_stride=ld, offset=offset, prologue=pro,
                                          out_sum=s, out_max=m, out_argmax=i)
    if cols >= 1 << 20:
        assert plan.workspace_bytes() > 0  # split rows stage chunk partials in the plan
    for _ in range(2):
        plan.dispatch()
    _check_rows(device, oracle, x, rows, cols, ld, offset, pro, s, m, i)
    y = oracle.normal(n, seed=32)
    device.write_buffer(buf, y)
    plan.dispatch()
    _check_rows(device, oracle, y, rows, cols, ld, offset, pro, s, m, i)


def test_prepared_rows_batch_submission(device, oracle):
    """Prepared fused-rows plans go through submit_prepared_axis_reduction_batch
    (prepared_axis_reduction.rs:84-92) with an axis plan, then rebind."""
    rows, cols = 1000, 777
    xf = oracle.normal(rows * cols, seed=33)
    xi = oracle.uniform_int(rows * cols, seed=34, lo=-1000, hi=1000, dtype=np.int32)
    bf, bi = device.upload(xf), device.upload(xi)
    sf, mf, af = (device.alloc_zeroed(np.float32, rows), device.alloc_zeroed(np.float32, rows),
                  device.alloc_zeroed(np.uint32, rows))
    si, mi, ai = (device.alloc_zeroed(np.int32, rows), device.alloc_zeroed(np.int32, rows),
                  device.alloc_zeroed(np.uint32, rows))
    colsum = device.alloc_zeroed(np.int32, cols)
    pf = AXIS.prepare_reduce_rows_fused(device, bf, rows, cols, prologue=(0.5, 0.25), out_sum=sf, out_max=mf,
                                        out_argmax=af)
    pi = AXIS.prepare_reduce_rows_fused(device, bi, rows, cols, out_sum=si, out_max=mi, out_argmax=ai)
    pc = AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(bi, Layout.c_contiguous([rows, cols])), 0,
                                       StridedView(colsum, Layout.c_contiguous([1, cols])))
    for _ in range(2):
        hx.submit_prepared_axis_reduction_batch(device, [pf, pi, pc])
        _check_rows(device, oracle, xf, rows, cols, cols, 0, (0.5, 0.25), sf, mf, af)
        _check_rows(device, oracle, xi, rows, cols, cols, 0, None, si, mi, ai)
        want = xi.reshape(rows, cols).astype(np.int64).sum(axis=0).astype(np.int32)
        assert np.array_equal(device.download_owned(colsum), want)
        xf = oracle.normal(rows * cols, seed=35)
        xi = oracle.uniform_int(rows * cols, seed=36, lo=-1000, hi=1000, dtype=np.int32)
        device.write_buffer(bf, xf)
        device.write_buffer(bi, xi)


def test_prepared_rows_validate_at_prepare(device):
    """Invalid operands are rejected when the plan is prepared, with the
    immediate form's messages, and no plan is returned."""
    buf = device.alloc_zeroed(np.float32, 100)
    m = device.alloc_zeroed(np.float32, 10)
    with pytest.raises(hx.DispatchFailed, match="layout rejected"):
        AXIS.prepare_reduce_rows_fused(device, buf, 10, 11, out_max=m)
    with pytest.raises(hx.DispatchFailed, match="max_axis is undefined for empty axis 1"):
        AXIS.prepare_reduce_rows_fused(device, buf, 10, 0, out_max=m)
    with pytest.raises(hx.DispatchFailed, match="row stride 9 is shorter"):
        AXIS.prepare_reduce_rows_fused(device, buf, 10, 10, row_stride=9, out_max=m)


def test_batch_rejects_null_plan_before_running_any(device):
    from hephaestus_amd import _ffi

    n = 64
    buf = device.upload(np.ones(n, np.uint32))
    out = device.alloc_zeroed(np.uint32, 1)
    plan = FULL.prepare_reduce_full(device, hx.SumOp, StridedView(buf, Layout.c_contiguous([n])),
                                    StridedView(out, Layout.c_contiguous([1])))
    arr = (ctypes.c_void_p * 2)(plan.handle, None)
    with pytest.raises(hx.InvalidConfiguration, match="null plan at batch index 1"):
        _ffi.check(_ffi.lib().hx_plan_dispatch_batch(arr, 2, None))
    assert device.download_owned(out)[0] == 0


# ------------------------------------------------------------ copy_buffer
@pytest.mark.parametrize("n", [1, 3, 4, 5, 65535, 65536, 65537, 3 * 65536 + 5, (1 << 20) + 3])
def test_copy_buffer_bit_exact(device, oracle, n):
    """copy_buffer runs a streaming kernel: 256 KiB tiles, a 16-byte body for
    the remainder and a byte tail."""
    x = oracle.uniform_int(n, seed=n + 77, lo=0, hi=2**32 - 1)
    src = device.upload(x)
    dst = device.alloc_zeroed(np.uint32, n)
    device.copy_buffer(src, dst)
    assert np.array_equal(device.download_owned(dst), x)
    again = device.alloc_zeroed(np.uint32, n)
    device.copy_buffer_async(dst, again)  # stream-ordered before the download
    assert np.array_equal(device.download_owned(again), x)


@pytest.mark.parametrize("skew,nbytes", [(1, 1), (1, 17), (3, 4099), (4, 262144 + 20), (8, 3 * 262144), (0, 262144 + 15)])
def test_copy_unaligned_ranges(device, oracle, skew, nbytes):
    """hx_copy on raw byte ranges: misaligned starts take the bytewise kernel,
    aligned ones the tiles plus a remainder; bytes outside the range stay."""
    from hephaestus_amd import _ffi

    total = nbytes + 64
    x = oracle.uniform_int((total + 3) // 4, seed=nbytes, lo=0, hi=2**32 - 1).view(np.uint8)[:total].copy()
    src = device.upload(x)
    dst = device.alloc_zeroed(np.uint8, total)
    _ffi.check(_ffi.lib().hx_copy(device.handle, src.ptr + skew, nbytes, dst.ptr + skew, nbytes, 1))
    got = device.download_owned(dst)
    want = np.zeros(total, np.uint8)
    want[skew:skew + nbytes] = x[skew:skew + nbytes]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("tiles", [1, 3, 257])
def test_copy_in_scan_shape_bit_exact(device, oracle, tiles):
    """hx_debug_copy_scan_shape (the bench's in-order yardstick) moves whole
    128 KiB tiles bit-exactly and rejects partial tiles."""
    from hephaestus_amd import _ffi

    n = tiles * 32768
    x = oracle.uniform_int(n, seed=tiles, lo=0, hi=2**32 - 1)
    src = device.upload(x)
    dst = device.alloc_zeroed(np.uint32, n + 1)
    _ffi.check(_ffi.lib().hx_debug_copy_scan_shape(device.handle, src.ptr, dst.ptr, 4 * n, None))
    got = device.download_owned(dst)
    assert np.array_equal(got[:n], x) and got[n] == 0
    with pytest.raises(hx.DispatchFailed, match="whole 131072-byte tiles"):
        _ffi.check(_ffi.lib().hx_debug_copy_scan_shape(device.handle, src.ptr, dst.ptr, 4 * n - 16, None))
