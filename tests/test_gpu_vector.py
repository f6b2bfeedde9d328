"""Map-reductions (dot, trace, norms) and the dense vector forms on the GPU.

Clauses restated from crates/hephaestus-conformance/src/dense_vector.rs:36-184
and crates/hephaestus-rocm/tests/contract.rs:2615-2737 (fixtures in
tests/golden/reference_kats.json), then parity with the oracle at sizes that
exercise the vectorised and strided paths.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
EPS = 2.0**-23
OPS = hx.RocmDenseVectorOps()


def one(device, buf):
    return device.download_owned(buf)[0]


def f32_bound(n, mags):
    return 2 * max(1, (int(n) - 1).bit_length()) * EPS * mags


# ---------------------------------------------------------- dense_vector.rs
def test_dense_vector_contract(device):
    k = KATS["dense_vector"]
    f = lambda v: np.array(v, np.float32)
    source = device.upload(f(k["copy"]))
    target = device.alloc_zeroed(np.float32, 4)
    OPS.copy_vector(device, source, target)
    assert list(device.download_owned(target)) == k["copy"]
    with pytest.raises(hx.LengthMismatch):
        OPS.copy_vector(device, source, device.alloc_zeroed(np.float32, 3))
    OPS.scale_vector(device, target, 2.0)
    assert list(device.download_owned(target)) == k["scale_by_2"]
    y = device.upload(f(k["axpy_target"]))
    OPS.axpy(device, y, source, k["axpy_factor"])
    assert list(device.download_owned(y)) == k["axpy"]
    y = device.upload(f(k["axpy_target"]))
    OPS.xpay(device, y, source, k["axpy_factor"])
    assert list(device.download_owned(y)) == k["xpay"]
    left, right = device.upload(f(k["left"])), device.upload(f(k["right"]))
    out = device.alloc_zeroed(np.float32, 4)
    for fn, key in ((OPS.subtract_into, "subtract"), (OPS.add_into, "add"), (OPS.multiply_into, "multiply"),
                    (OPS.divide_into, "divide")):
        fn(device, left, right, out)
        assert list(device.download_owned(out)) == k[key], key
    a, b = device.upload(f(k["dot_a"])), device.upload(f(k["dot_b"]))
    prepared = OPS.prepare_dot(device, a, b)
    assert OPS.dot_prepared(device, prepared, a, b) == k["dot"]
    assert OPS.dot_prepared(device, prepared, a, b) == k["dot"]  # idempotent
    device.write_buffer(a, np.full(4, 2.0, np.float32))
    assert OPS.dot_prepared(device, prepared, a, b) == k["dot_after_a_all_twos"]  # rebind observed
    with pytest.raises(hx.DispatchFailed, match="prepared dot received different device allocations"):
        OPS.dot_prepared(device, prepared, device.upload(np.ones(4, np.float32)), b)
    v = device.upload(f(k["norm_vector"]))
    assert OPS.norm_l1(device, v) == k["norm_l1"]
    assert OPS.norm_max(device, v) == k["norm_max"]
    pn = OPS.prepare_norm_l2(device, v)
    assert abs(OPS.norm_l2_prepared(device, pn, v) - k["norm_l2"]) <= k["norm_l2"] * EPS
    device.write_buffer(v, f(k["norm_vector_rebound"]))
    assert abs(OPS.norm_l2_prepared(device, pn, v) - k["norm_l2_rebound"]) <= k["norm_l2_rebound"] * EPS


def test_vector_length_mismatches_are_rejected_untouched(device):
    t = device.upload(np.arange(4, dtype=np.float32))
    s = device.upload(np.ones(5, np.float32))
    with pytest.raises(hx.LengthMismatch) as e:
        OPS.axpy(device, t, s, 2.0)
    assert (e.value.host_len, e.value.device_len) == (4, 5)
    with pytest.raises(hx.LengthMismatch):
        OPS.add_into(device, t, t, device.alloc_zeroed(np.float32, 3))
    assert list(device.download_owned(t)) == [0.0, 1.0, 2.0, 3.0]
    with pytest.raises(hx.InvalidConfiguration):
        OPS.scale_vector(device, device.upload(np.ones(4, np.int32)), 2.0)


# ------------------------------------------------- rocm contract.rs:2615-2737
def test_map_reduction_contract(device):
    k = KATS["map_reduction"]
    m = device.upload(np.array(k["matrix_i32"], np.int32))
    lm = Layout.c_contiguous(k["matrix_shape"])
    assert one(device, hx.norm_l1(device, StridedView(m, lm))) == k["norm_l1"]
    assert one(device, hx.norm_max(device, StridedView(m, lm))) == k["norm_max"]
    lhs = device.upload(np.array(k["dot_lhs_i32"], np.int32))
    rhs = device.upload(np.array(k["dot_rhs_i32"], np.int32))
    ll = Layout.try_new(k["dot_lhs_shape"], k["dot_lhs_strides"], k["dot_lhs_offset"])
    lr = Layout.c_contiguous([5])
    assert one(device, hx.dot(device, StridedView(lhs, ll), StridedView(rhs, lr))) == k["dot"]
    tr = device.upload(np.array(k["trace_i32"], np.int32))
    assert one(device, hx.trace(device, StridedView(tr, Layout.c_contiguous(k["trace_shape"])))) == k["trace"]
    l2 = device.upload(np.array(k["l2_f32"], np.float32))
    assert one(device, hx.norm_l2(device, StridedView(l2, Layout.c_contiguous([2])))) == k["norm_l2"]
    # The reference matches the DispatchFailed message field (contract.rs:2717-2736).
    with pytest.raises(hx.DispatchFailed) as e:
        hx.dot(device, StridedView(lhs, ll), StridedView(rhs, Layout.c_contiguous([4])))
    assert e.value.message.startswith(k["dot_mismatch_prefix"]), e.value.message
    with pytest.raises(hx.DispatchFailed) as e:
        hx.trace(device, StridedView(m, lm))
    assert e.value.message.startswith(k["trace_rect_prefix"]), e.value.message


# ------------------------------------------------------- parity at sizes
SIZES = [0, 1, 3, 4, 5, 1023, 4097, 65536 + 17, (1 << 20) + 3]


@pytest.mark.parametrize("n", SIZES)
def test_dot_and_norms_f32(device, oracle, n):
    a = oracle.uniform_real(n, seed=n + 1, lo=-2.0, hi=2.0)
    b = oracle.uniform_real(n, seed=n + 2, lo=-2.0, hi=2.0)
    da, db = device.upload(a), device.upload(b)
    lay = Layout.c_contiguous([n])
    want, mags = oracle.dot(a, b)
    got = float(one(device, hx.dot(device, StridedView(da, lay), StridedView(db, lay))))
    assert abs(got - want) <= f32_bound(n, mags) + abs(want) * EPS / 2, (got, want)
    l1 = oracle.norm_l1(a)
    assert abs(float(one(device, hx.norm_l1(device, StridedView(da, lay)))) - l1) <= f32_bound(n, l1) + l1 * EPS
    l2 = oracle.norm_l2(a)
    got2 = float(one(device, hx.norm_l2(device, StridedView(da, lay))))
    assert abs(got2 - l2) <= l2 * 2 * EPS + 1e-30, (got2, l2)
    assert one(device, hx.norm_max(device, StridedView(da, lay))) == oracle.norm_max(a)


@pytest.mark.parametrize("dtype", [np.int32, np.uint32])
@pytest.mark.parametrize("n", [0, 7, 4099, (1 << 20) + 5])
def test_dot_and_norms_integers_bit_exact(device, oracle, n, dtype):
    a = oracle.uniform_int(n, seed=n + 3, lo=0, hi=2**32 - 1).view(dtype)
    b = oracle.uniform_int(n, seed=n + 4, lo=0, hi=2**32 - 1).view(dtype)
    da, db = device.upload(a), device.upload(b)
    lay = Layout.c_contiguous([n])
    assert one(device, hx.dot(device, StridedView(da, lay), StridedView(db, lay))) == oracle.dot(a, b)
    assert one(device, hx.norm_l1(device, StridedView(da, lay))) == oracle.norm_l1(a)
    assert one(device, hx.norm_max(device, StridedView(da, lay))) == oracle.norm_max(a)


def test_int_min_and_nan_semantics(device, oracle):
    i = np.array([-2**31, 5, -7, -2**31], np.int32)
    di = device.upload(i)
    lay = Layout.c_contiguous([4])
    assert one(device, hx.norm_max(device, StridedView(di, lay))) == 7
    assert one(device, hx.norm_l1(device, StridedView(di, lay))) == oracle.norm_l1(i)
    only = device.upload(np.array([-2**31], np.int32))
    assert one(device, hx.norm_max(device, StridedView(only, Layout.c_contiguous([1])))) == -2**31
    f = np.array([1.0, np.nan, -3.0, -0.0], np.float32)
    df = device.upload(f)
    assert one(device, hx.norm_max(device, StridedView(df, lay))) == 3.0
    empty = device.alloc_zeroed(np.float32, 0)
    assert one(device, hx.norm_max(device, StridedView(empty, Layout.c_contiguous([0])))) == np.float32(-3.4028235e38)
    assert one(device, hx.norm_l2(device, StridedView(empty, Layout.c_contiguous([0])))) == 0.0


def test_strided_and_misaligned_views(device, oracle):
    """Transposed and offset views take the strided path; a dot whose
    operands disagree in 16-byte phase must match too."""
    r, c = 300, 257
    host = oracle.uniform_real(r * c + 3, seed=9, lo=-1.0, hi=1.0)
    buf = device.upload(host)
    t = Layout.try_new([c, r], [1, c], 0)  # transpose of [r, c]
    ref = host[: r * c].reshape(r, c).T.copy()
    assert one(device, hx.norm_max(device, StridedView(buf, t))) == np.max(np.abs(ref))
    l1 = oracle.norm_l1(ref.ravel())
    assert abs(float(one(device, hx.norm_l1(device, StridedView(buf, t)))) - l1) <= f32_bound(r * c, l1) + l1 * EPS
    n = 70001
    a = Layout.try_new([n], [1], 1)  # offset 1: 4 bytes out of 16-byte phase with b
    b = Layout.try_new([n], [1], 2)
    want, mags = oracle.dot(host[1:1 + n], host[2:2 + n])
    got = float(one(device, hx.dot(device, StridedView(buf, a), StridedView(buf, b))))
    assert abs(got - want) <= f32_bound(n, mags) + abs(want) * EPS / 2
    neg = Layout.try_new([1000], [-3], 2999)  # reversed, stride 3
    want = oracle.norm_l1(np.ascontiguousarray(host[2999::-3][:1000]))
    assert abs(float(one(device, hx.norm_l1(device, StridedView(buf, neg)))) - want) <= f32_bound(1000, want) + want * EPS


def test_trace_views(device, oracle):
    n = 513
    m = oracle.uniform_int(n * n, seed=10, lo=-1000, hi=1000, dtype=np.int32)
    buf = device.upload(m)
    assert one(device, hx.trace(device, StridedView(buf, Layout.c_contiguous([n, n])))) == np.trace(m.reshape(n, n))
    t = Layout.try_new([n, n], [1, n], 0)
    assert one(device, hx.trace(device, StridedView(buf, t))) == np.trace(m.reshape(n, n))
    empty = device.alloc_zeroed(np.int32, 0)
    out = hx.trace(device, StridedView(empty, Layout.c_contiguous([0, 0])))
    assert one(device, out) == 0


@pytest.mark.parametrize("n", [1, 3, 4, 4096, 4096 * 3 + 5, 1000003])
def test_vector_forms_bit_exact(device, oracle, n):
    # 4096 elements is one whole tile of the tiled kernel; the other sizes
    # exercise the tile/remainder split and the remainder-only path.
    t = oracle.uniform_real(n, seed=n + 5, lo=-3.0, hi=3.0)
    s = oracle.uniform_real(n, seed=n + 6, lo=0.5, hi=3.0)
    f = np.float32(0.7)
    dt, ds = device.upload(t), device.upload(s)
    OPS.axpy(device, dt, ds, float(f))
    assert np.array_equal(device.download_owned(dt), oracle.fma_arrays(s, t, f))
    dt = device.upload(t)
    OPS.xpay(device, dt, ds, float(f))
    assert np.array_equal(device.download_owned(dt), oracle.fma_arrays(t, s, f))
    dt = device.upload(t)
    OPS.scale_vector(device, dt, float(f))
    assert np.array_equal(device.download_owned(dt), t * f)
    out = device.alloc_zeroed(np.float32, n)
    for fn, ref in ((OPS.add_into, t + s), (OPS.subtract_into, t - s), (OPS.multiply_into, t * s),
                    (OPS.divide_into, t / s)):
        fn(device, device.upload(t), ds, out)
        assert np.array_equal(device.download_owned(out), ref.astype(np.float32))


@pytest.mark.parametrize("offsets", [(1, 2, 3), (3, 0, 1), (2, 2, 2)])
@pytest.mark.parametrize("n", [5, 4096 * 3 + 7, 1000003])
def test_vector_forms_at_element_offsets(device, oracle, n, offsets):
    """Operands that start off 16-byte boundaries (raw pointers into larger
    buffers): the 16-byte vector paths need only 4-byte alignment; the
    elements around each range stay untouched."""
    from hephaestus_amd import _ffi

    ot, os_, oo = offsets
    pad = 8
    t = oracle.uniform_real(n + pad, seed=n + 11, lo=-3.0, hi=3.0)
    s = oracle.uniform_real(n + pad, seed=n + 12, lo=0.5, hi=3.0)
    f = np.float32(0.7)
    dt, ds = device.upload(t), device.upload(s)
    lib = _ffi.lib()
    _ffi.check(lib.hx_vector_update(device.handle, 1, _ffi.DTYPE_F32, dt.ptr + 4 * ot, n, ds.ptr + 4 * os_, n,
                                    float(f), None))  # axpy
    want = t.copy()
    want[ot:ot + n] = oracle.fma_arrays(s[os_:os_ + n], t[ot:ot + n], f)
    assert np.array_equal(device.download_owned(dt), want)
    out = device.upload(np.full(n + pad, 9.0, np.float32))
    _ffi.check(lib.hx_vector_binary(device.handle, 5, _ffi.DTYPE_F32, ds.ptr + 4 * os_, n, ds.ptr + 4 * ot, n,
                                    out.ptr + 4 * oo, n, None))  # mul
    want = np.full(n + pad, 9.0, np.float32)
    want[oo:oo + n] = s[os_:os_ + n] * s[ot:ot + n]
    assert np.array_equal(device.download_owned(out), want)


# Pairs of same-shape views walked as rows (layout_rows_pair): dimensions
# merge only where both operands allow it; 16-byte units only where both
# have contiguous rows.  (a layout, b layout) as (shape, a strides, a offset,
# b strides, b offset).
PAIR_VIEWS = [
    ([64, 1000], [1003, 1], 5, [1000, 1], 0),        # slice . dense: vector units
    ([64, 1001], [1003, 1], 1, [1001, 1], 2),        # ragged rows, both contiguous
    ([7, 9, 13], [200, 20, 1], 3, [117, 13, 1], 0),  # rank 3: a slice, b dense (merges for b only)
    ([3, 4, 5, 6], [400, 90, 15, 1], 2, [360, 90, 18, 1], 1),
    ([50, 40], [1, 50], 0, [40, 1], 0),              # transposed . dense: element walk
    ([40, 33], [-40, 1], 1563, [33, 1], 0),          # reversed rows
    ([500], [3], 4, [-2, ], 1200),                   # stride 3 . stride -2
    ([300, 3], [7, 1], 1, [3, 1], 0),                # rows of 3
    # views that cover a dense range, reversed or transposed, with the same
    # strides: streamed as flat ranges from their lowest elements
    ([5000], [-1], 4999, [-1], 9999),                # both reversed
    ([40, 33], [-33, -1], 1319, [-33, -1], 6319),    # both fully reversed
    ([33, 40], [-1, 33], 32, [-1, 33], 2032),        # reversed transpose
    ([5000], [-1], 4999, [1], 7),                    # reversed . forward: element walk
    # a transposed matrix paired with a row-major one: 64 x 64 tiles, the
    # transposed tile turned through LDS (edge tiles ragged in both
    # directions, padded leading dimensions, any element offsets)
    ([130, 70], [1, 131], 3, [75, 1], 17),
    ([64, 128], [128, 1], 0, [1, 64], 0),            # row-major . transposed
    ([256, 256], [1, 256], 0, [256, 1], 1000),       # full tiles only
    ([16, 200], [1, 16], 5, [200, 1], 9),            # smallest tiled extent
    ([200, 15], [1, 200], 0, [15, 1], 0),            # below it: element walk
    ([1, 96, 80], [9999, 1, 96], 2, [7680, 80, 1], 1),  # a unit dimension
    # three extents: a batch of transposed . row-major pairs, the batch
    # extent in any position and its strides of any sign
    ([97, 3, 33], [1, 97, 291], 0, [99, 33, 1], 0),
    ([5, 40, 70], [2800, 1, 40], 7, [2800, 70, 1], 3),
    ([4, 30, 20], [-600, 1, 30], 1805, [600, 20, 1], 0),
    ([20, 6, 30], [30, 600, 1], 2, [1, 20, 600], 11),  # the batch in the middle
    ([3, 17, 15], [255, 1, 17], 0, [255, 15, 1], 0),   # below the tiled extent
]


def _elems(host, shape, strides, offset):
    idx = offset + sum(np.indices(shape)[d] * strides[d] for d in range(len(shape)))
    return np.ascontiguousarray(host[idx.ravel()])


@pytest.mark.parametrize("view", PAIR_VIEWS, ids=lambda v: "x".join(map(str, v[0])) + f"_{v[1]}_{v[3]}")
@pytest.mark.parametrize("dtype", [np.float32, np.int32])
def test_map_reductions_of_strided_views(device, oracle, view, dtype):
    shape, sa, oa, sb, ob = view
    size = 70000
    if dtype == np.float32:
        host = oracle.uniform_real(size, seed=sum(shape), lo=-2.0, hi=2.0)
    else:
        host = oracle.uniform_int(size, seed=sum(shape), lo=-1000, hi=1000, dtype=np.int32)
    buf = device.upload(host)
    la, lb = Layout.try_new(shape, sa, oa), Layout.try_new(shape, sb, ob)
    xa, xb = _elems(host, shape, sa, oa), _elems(host, shape, sb, ob)
    n = xa.size
    va, vb = StridedView(buf, la), StridedView(buf, lb)
    if dtype == np.float32:
        want, mags = oracle.dot(xa, xb)
        got = float(one(device, hx.dot(device, va, vb)))
        assert abs(got - want) <= f32_bound(n, mags) + abs(want) * EPS / 2, (got, want)
        l1 = oracle.norm_l1(xa)
        assert abs(float(one(device, hx.norm_l1(device, va))) - l1) <= f32_bound(n, l1) + l1 * EPS
        l2 = oracle.norm_l2(xa)
        assert abs(float(one(device, hx.norm_l2(device, va))) - l2) <= l2 * 2 * EPS + 1e-30
    else:
        assert one(device, hx.dot(device, va, vb)) == oracle.dot(xa, xb)
        assert one(device, hx.norm_l1(device, va)) == oracle.norm_l1(xa)
    assert one(device, hx.norm_max(device, va)) == oracle.norm_max(xa)


@pytest.mark.parametrize("shape", [(2048, 3000), (3001, 2047), (40000, 17)])
@pytest.mark.parametrize("dtype", [np.float32, np.int32])
def test_dot_of_a_transpose_with_a_row_major_matrix(device, oracle, shape, dtype):
    """Many tiles per block and both operand orders."""
    r, c = shape
    if dtype == np.float32:
        ha = oracle.uniform_real(r * c + 3, seed=r, lo=-2.0, hi=2.0)
        hb = oracle.uniform_real(r * c + 5, seed=c, lo=-2.0, hi=2.0)
    else:
        ha = oracle.uniform_int(r * c + 3, seed=r, lo=-70000, hi=70000, dtype=np.int32)
        hb = oracle.uniform_int(r * c + 5, seed=c, lo=-70000, hi=70000, dtype=np.int32)
    ba, bb = device.upload(ha), device.upload(hb)
    la = Layout.try_new([r, c], [1, r], 3)  # column-major
    lb = Layout.try_new([r, c], [c, 1], 5)  # row-major
    xa = ha[3:3 + r * c].reshape(c, r).T.ravel()
    xb = hb[5:5 + r * c]
    for va, vb, pa, pb in ((StridedView(ba, la), StridedView(bb, lb), xa, xb),
                           (StridedView(bb, lb), StridedView(ba, la), xb, xa)):
        if dtype == np.float32:
            want, mags = oracle.dot(pa, pb)
            got = float(one(device, hx.dot(device, va, vb)))
            assert abs(got - want) <= f32_bound(r * c, mags) + abs(want) * EPS / 2, (got, want)
        else:
            assert one(device, hx.dot(device, va, vb)) == oracle.dot(pa, pb)


def test_dot_of_transposed_pairs_random_geometry(device, oracle):
    """Seeded sweep of the tiled pairing: extents 16-300, padded leading
    dimensions, element offsets and either operand transposed, bit-exact in
    i32."""
    rng = np.random.default_rng(2029)
    host = oracle.uniform_int(400000, seed=77, lo=-5000, hi=5000, dtype=np.int32)
    buf = device.upload(host)
    for _ in range(60):
        r, c = (int(v) for v in rng.integers(16, 301, size=2))
        cld = r + int(rng.integers(0, 9))
        rld = c + int(rng.integers(0, 9))
        oa = int(rng.integers(0, 400000 - cld * c))
        ob = int(rng.integers(0, 400000 - rld * r))
        la = Layout.try_new([r, c], [1, cld], oa)
        lb = Layout.try_new([r, c], [rld, 1], ob)
        xa, xb = _elems(host, [r, c], [1, cld], oa), _elems(host, [r, c], [rld, 1], ob)
        va, vb = StridedView(buf, la), StridedView(buf, lb)
        if rng.integers(0, 2):
            va, vb, xa, xb = vb, va, xb, xa
        assert one(device, hx.dot(device, va, vb)) == oracle.dot(xa, xb), (r, c, cld, rld, oa, ob)


def test_dot_of_batched_transposed_pairs_random_geometry(device, oracle):
    """Seeded sweep of batches of transposed . row-major pairs: the batch
    extent in any position, batch strides of either sign, bit-exact in i32."""
    rng = np.random.default_rng(2030)
    size = 400000
    host = oracle.uniform_int(size, seed=78, lo=-5000, hi=5000, dtype=np.int32)
    buf = device.upload(host)
    for _ in range(40):
        nb = int(rng.integers(2, 5))
        r, c = (int(v) for v in rng.integers(16, 121, size=2))
        cld, rld = r + int(rng.integers(0, 5)), c + int(rng.integers(0, 5))
        abs_, bbs = cld * c, rld * r
        sa = [1, cld]   # (i, j) strides of the transposed operand
        sb = [rld, 1]   # (i, j) strides of the row-major one
        sga = abs_ if rng.integers(0, 2) else -abs_
        sgb = bbs if rng.integers(0, 2) else -bbs
        pos = int(rng.integers(0, 3))  # where the batch extent sits
        shape, stra, strb = [r, c], list(sa), list(sb)
        shape.insert(pos, nb)
        stra.insert(pos, sga)
        strb.insert(pos, sgb)
        oa = int(rng.integers(0, size - nb * abs_)) + (abs_ * (nb - 1) if sga < 0 else 0)
        ob = int(rng.integers(0, size - nb * bbs)) + (bbs * (nb - 1) if sgb < 0 else 0)
        la, lb = Layout.try_new(shape, stra, oa), Layout.try_new(shape, strb, ob)
        xa, xb = _elems(host, shape, stra, oa), _elems(host, shape, strb, ob)
        va, vb = StridedView(buf, la), StridedView(buf, lb)
        if rng.integers(0, 2):
            va, vb, xa, xb = vb, va, xb, xa
        assert one(device, hx.dot(device, va, vb)) == oracle.dot(xa, xb), (shape, stra, strb, oa, ob)
