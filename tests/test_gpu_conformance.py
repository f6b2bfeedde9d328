"""The reference's conformance clauses, run on the MI355X through the C ABI.

Each test restates one clause module of crates/hephaestus-conformance/src
(transfer.rs, full_reduction.rs, axis_reduction.rs, scan.rs) with the same
fixtures and exact expectations, so a reader can hold the two side by side.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import Layout, StridedView

pytestmark = pytest.mark.gpu

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
FULL = hx.RocmFullReductionOps()
AXIS = hx.RocmAxisReductionOps()
SCAN = hx.RocmScanOps()


def fixture_rows():
    return np.array([1.0, 2.0, 3.0, 2.0] * 3, dtype=np.float32)


# ------------------------------------------------------------- transfer.rs
def test_transfer_contract(device):
    bits = [int(b, 16) for b in KATS["transfer"]["pattern_bits"]]
    pattern = np.array(bits, dtype=np.uint32).view(np.float32)
    buf = device.upload(pattern)
    assert len(buf) == 5
    got = np.zeros(5, np.float32)
    device.download(buf, got)
    assert list(got.view(np.uint32)) == bits
    assert list(device.download_owned(buf).view(np.uint32)) == bits

    zeros = device.alloc_zeroed(np.float32, 4)
    assert list(device.download_owned(zeros)) == [0.0] * 4
    device.write_buffer(zeros, np.array(KATS["transfer"]["write_buffer"], np.float32))
    assert list(device.download_owned(zeros)) == KATS["transfer"]["write_buffer"]
    device.write_sub_buffer(zeros, 1, np.array(KATS["transfer"]["write_sub_at_1"], np.float32))
    after = KATS["transfer"]["after_write_sub"]
    assert list(device.download_owned(zeros)) == after

    copy = device.alloc_zeroed(np.float32, 4)
    device.copy_buffer(zeros, copy)
    assert list(device.download_owned(copy)) == after

    with pytest.raises(hx.LengthMismatch):
        device.download(copy, np.zeros(3, np.float32))
    long = device.alloc_zeroed(np.float32, 6)
    with pytest.raises(hx.LengthMismatch):
        device.copy_buffer(copy, long)
    with pytest.raises(hx.LengthMismatch):
        device.write_buffer(copy, np.ones(2, np.float32))
    with pytest.raises(hx.LengthMismatch):
        device.write_sub_buffer(copy, 3, np.ones(2, np.float32))
    assert list(device.download_owned(copy)) == after  # rejections did not write

    topo = device.topology()
    assert topo.warp_width & (topo.warp_width - 1) == 0
    assert topo.max_threads_per_unit >= topo.warp_width

    empty = device.upload(np.zeros(0, np.float32))
    assert len(empty) == 0 and empty.ptr is None
    device.download(empty, np.zeros(0, np.float32))
    assert device.download_owned(empty).size == 0


def test_large_transfer_round_trip_is_bitwise(device):
    # Crosses the pinned staging chunk (32 MiB) several times, ragged end.
    n = (80 << 20) // 4 + 7
    host = np.random.default_rng(0).integers(0, 2**32, n, dtype=np.uint32)
    buf = device.upload(host)
    back = device.download_owned(buf)
    assert np.array_equal(back, host)
    device.write_sub_buffer(buf, n - 5, np.arange(5, dtype=np.uint32))
    assert np.array_equal(device.download_owned(buf)[-5:], np.arange(5, dtype=np.uint32))


# ------------------------------------------------------- full_reduction.rs
def _reduce(device, op, source, layout):
    out = device.alloc_zeroed(np.float32, 1)
    FULL.reduce_full_into(device, op, StridedView(source, layout), StridedView(out, Layout.c_contiguous([1])))
    return float(device.download_owned(out)[0])


def test_full_reduction_contract(device):
    k = KATS["full_reduction"]
    source = device.upload(fixture_rows())
    dense = Layout.c_contiguous([3, 4])
    assert _reduce(device, hx.SumOp, source, dense) == k["sum"]
    assert _reduce(device, hx.ProdOp, source, dense) == k["prod"]
    assert _reduce(device, hx.MinOp, source, dense) == k["min"]
    assert _reduce(device, hx.MaxOp, source, dense) == k["max"]

    transposed = Layout.try_new([4, 3], [1, 4], 0)
    assert _reduce(device, hx.SumOp, source, transposed) == k["transposed"]["sum"]
    assert _reduce(device, hx.ProdOp, source, transposed) == k["transposed"]["prod"]

    square = device.upload(np.arange(1, 10, dtype=np.float32))
    assert _reduce(device, hx.SumOp, square, Layout.try_new([3], [4], 0)) == k["diagonal"]["sum"]

    out1 = device.alloc_zeroed(np.float32, 1)
    scalar = Layout.c_contiguous([1])
    prepared = FULL.prepare_reduce_full(device, hx.ProdOp, StridedView(source, dense), StridedView(out1, scalar))
    FULL.dispatch_full(device, prepared)
    assert list(device.download_owned(out1)) == [1728.0]
    FULL.dispatch_full(device, prepared)
    assert list(device.download_owned(out1)) == [1728.0]
    device.write_buffer(source, np.full(12, 2.0, np.float32))
    FULL.dispatch_full(device, prepared)
    assert list(device.download_owned(out1)) == [4096.0]
    device.write_buffer(source, fixture_rows())

    out = device.upload(np.array([9.0, 9.0], np.float32))
    with pytest.raises(hx.HephaestusError):
        FULL.reduce_full_into(device, hx.SumOp, StridedView(source, dense), StridedView(out, Layout.c_contiguous([2])))
    assert list(device.download_owned(out)) == [9.0, 9.0]


def test_rocm_reduction_kats(device):
    # crates/hephaestus-rocm/tests/contract.rs:811-933 (u32 i % 17)
    for n in KATS["rocm_reduce_u32"]["sizes"]:
        host = np.array([i % 17 for i in range(n)], dtype=np.uint32)
        buf = device.upload(host)
        lay = Layout.c_contiguous([n])
        for op, want in ((hx.SumOp, host.sum()), (hx.MinOp, host.min()), (hx.MaxOp, host.max())):
            out = device.alloc_zeroed(np.uint32, 1)
            FULL.reduce_full_into(device, op, StridedView(buf, lay), StridedView(out, Layout.c_contiguous([1])))
            assert int(device.download_owned(out)[0]) == int(want)
    empty = device.upload(np.zeros(0, np.uint32))
    out = device.upload(np.array([0xFFFFFFFF], np.uint32))
    FULL.reduce_full_into(device, hx.SumOp, StridedView(empty, Layout.c_contiguous([0])),
                          StridedView(out, Layout.c_contiguous([1])))
    assert int(device.download_owned(out)[0]) == 0


# ------------------------------------------------------- axis_reduction.rs
def _axis(device, op, buf, layout, axis, out_shape, dtype=np.float32):
    out = device.alloc_zeroed(dtype, int(np.prod(out_shape)))
    AXIS.reduce_axis_into(device, op, StridedView(buf, layout), axis, StridedView(out, Layout.c_contiguous(out_shape)))
    return list(device.download_owned(out))


def test_axis_reduction_contract(device):
    k = KATS["axis_reduction"]
    buf = device.upload(np.arange(1, 13, dtype=np.float32))
    lay = Layout.c_contiguous([3, 4])
    assert _axis(device, hx.ProdOp, buf, lay, 0, [1, 4]) == k["prod_axis0"]
    assert _axis(device, hx.ProdOp, buf, lay, 1, [3, 1]) == k["prod_axis1"]
    assert _axis(device, hx.MinOp, buf, lay, 0, [1, 4]) == k["min_axis0"]
    assert _axis(device, hx.MaxOp, buf, lay, 0, [1, 4]) == k["max_axis0"]
    assert _axis(device, hx.MinOp, buf, lay, 1, [3, 1]) == k["min_axis1"]
    assert _axis(device, hx.MaxOp, buf, lay, 1, [3, 1]) == k["max_axis1"]
    assert _axis(device, hx.MeanOp, buf, lay, 0, [1, 4]) == k["mean_axis0"]
    assert _axis(device, hx.MeanOp, buf, lay, 1, [3, 1]) == k["mean_axis1"]
    t = k["transposed_prod_axis1"]
    assert _axis(device, hx.ProdOp, buf, Layout.try_new(t["shape"], t["strides"]), 1, [4, 1]) == t["expect"]

    out = device.alloc_zeroed(np.float32, 4)
    with pytest.raises(hx.HephaestusError):
        AXIS.prod_axis_into(device, StridedView(buf, lay), 2, StridedView(out, Layout.c_contiguous([1, 4])))

    out = device.alloc_zeroed(np.float32, 4)
    ol = Layout.c_contiguous([1, 4])
    prepared = AXIS.prepare_reduce_axis_into(device, hx.ProdOp, StridedView(buf, lay), 0, StridedView(out, ol))
    AXIS.dispatch_prepared(device, prepared)
    assert list(device.download_owned(out)) == k["prod_axis0"]
    AXIS.dispatch_prepared(device, prepared)
    assert list(device.download_owned(out)) == k["prod_axis0"]
    device.write_buffer(buf, np.full(12, 2.0, np.float32))
    AXIS.dispatch_prepared(device, prepared)
    assert list(device.download_owned(out)) == k["rebind_all_twos_prod_axis0"]
    device.write_buffer(buf, np.arange(1, 13, dtype=np.float32))

    sum_out = device.alloc_zeroed(np.float32, 4)
    p_sum = AXIS.prepare_reduce_axis_into(device, hx.SumOp, StridedView(buf, lay), 0, StridedView(sum_out, ol))
    AXIS.dispatch_prepared(device, p_sum)
    got_sum = list(device.download_owned(sum_out))
    assert got_sum == k["sum_axis0"]
    assert got_sum != k["prod_axis0"]

    wrong = device.alloc_zeroed(np.float32, 3)
    with pytest.raises(hx.HephaestusError):
        AXIS.prepare_reduce_axis_into(device, hx.ProdOp, StridedView(buf, lay), 0,
                                      StridedView(wrong, Layout.c_contiguous([1, 3])))


def test_rocm_axis_u32_kats(device):
    k = KATS["rocm_axis_u32"]
    buf = device.upload(np.array(k["input"], np.uint32))
    lay = Layout.c_contiguous([3, 4])
    u = np.uint32
    assert _axis(device, hx.SumOp, buf, lay, 1, [3, 1], u) == k["sum_rows"]
    assert _axis(device, hx.SumOp, buf, lay, 0, [1, 4], u) == k["sum_cols"]
    assert _axis(device, hx.MinOp, buf, lay, 1, [3, 1], u) == k["min_rows"]
    assert _axis(device, hx.MaxOp, buf, lay, 1, [3, 1], u) == k["max_rows"]
    assert _axis(device, hx.ProdOp, buf, lay, 1, [3, 1], u) == k["prod_rows"]
    assert _axis(device, hx.ProdOp, buf, lay, 0, [1, 4], u) == k["prod_cols"]
    assert _axis(device, hx.ProdOp, buf, Layout.try_new([4, 3], [1, 4]), 1, [4, 1], u) == k["prod_cols"]

    wrong = device.alloc_zeroed(np.uint32, 6)
    with pytest.raises(hx.DispatchFailed) as e:
        AXIS.reduce_axis_into(device, hx.SumOp, StridedView(buf, lay), 1, StridedView(wrong, Layout.c_contiguous([3, 2])))
    assert e.value.message.startswith(KATS["messages"]["axis_shape_prefix"])
    with pytest.raises(hx.DispatchFailed) as e:
        AXIS.reduce_axis_into(device, hx.SumOp, StridedView(buf, lay), 1, StridedView(buf, Layout.c_contiguous([3, 1])))
    assert e.value.message == KATS["messages"]["axis_alias"]
    empty = device.upload(np.zeros(0, np.uint32))
    out3 = device.alloc_zeroed(np.uint32, 3)
    with pytest.raises(hx.DispatchFailed) as e:
        AXIS.mean_axis_into(device, StridedView(empty, Layout.c_contiguous([3, 0])), 1,
                            StridedView(out3, Layout.c_contiguous([3, 1])))
    assert e.value.message == KATS["messages"]["mean_empty_axis1"]
    assert _axis(device, hx.ProdOp, empty, Layout.c_contiguous([0, 3]), 0, [1, 3], u) == [1, 1, 1]


# ----------------------------------------------------------------- scan.rs
def _scan(device, op, axis, direction, host=None, kind=hx.ScanKind.Inclusive, shape=(3, 4), dtype=np.float32):
    host = fixture_rows() if host is None else host
    src = device.upload(host.astype(dtype))
    out = device.alloc_zeroed(dtype, host.size)
    lay = Layout.c_contiguous(list(shape))
    SCAN.scan_axis_into(device, op, StridedView(src, lay), axis, direction, StridedView(out, lay), kind)
    return list(device.download_owned(out))


def test_scan_contract(device):
    k = KATS["scan"]
    # prepared rebind clause (scan.rs:155-205)
    src = device.upload(fixture_rows())
    out = device.alloc_zeroed(np.float32, 12)
    lay = Layout.c_contiguous([3, 4])
    prepared = SCAN.prepare_scan_axis(device, hx.CumSumOp, StridedView(src, lay), 1, hx.ScanDirection.Forward,
                                      StridedView(out, lay))
    SCAN.dispatch_scan(device, prepared)
    assert list(device.download_owned(out)) == k["cumsum_axis1_forward"]
    SCAN.dispatch_scan(device, prepared)
    assert list(device.download_owned(out)) == k["cumsum_axis1_forward"]
    device.write_buffer(src, np.ones(12, np.float32))
    SCAN.dispatch_scan(device, prepared)
    assert list(device.download_owned(out)) == k["rebind_all_ones_cumsum_axis1"]

    F, R = hx.ScanDirection.Forward, hx.ScanDirection.Reverse
    assert _scan(device, hx.CumSumOp, 1, F) == k["cumsum_axis1_forward"]
    assert _scan(device, hx.CumSumOp, 1, R) == k["cumsum_axis1_reverse"]
    assert _scan(device, hx.CumProdOp, 1, F) == k["cumprod_axis1_forward"]
    assert _scan(device, hx.CumSumOp, 0, F) == k["cumsum_axis0_forward"]

    src = device.upload(fixture_rows())
    out = device.upload(np.full(12, 9.0, np.float32))
    with pytest.raises(hx.HephaestusError):
        SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(src, lay), 2, F, StridedView(out, lay))
    assert list(device.download_owned(out)) == [9.0] * 12


def test_rocm_scan_i32_kats(device):
    k = KATS["rocm_scan_i32"]
    x = np.array(k["input"], np.int32)
    F, R = hx.ScanDirection.Forward, hx.ScanDirection.Reverse
    args = dict(host=x, shape=(2, 4), dtype=np.int32)
    assert _scan(device, hx.CumSumOp, 1, F, **args) == k["cumsum_axis1"]
    assert _scan(device, hx.CumSumOp, 1, R, **args) == k["reverse_axis1"]
    assert _scan(device, hx.CumSumOp, 0, R, **args) == k["suffix_axis0"]
    assert _scan(device, hx.CumSumOp, 0, F, **args) == k["cumsum_axis0"]
    assert _scan(device, hx.CumProdOp, 1, F, **args) == k["cumprod_axis1"]
    assert _scan(device, hx.CumProdOp, 0, F, **args) == k["cumprod_axis0"]
    assert _scan(device, hx.CumProdOp, 1, R, **args) == k["suffix_prod_axis1"]
    assert _scan(device, hx.CumProdOp, 0, R, **args) == k["suffix_prod_axis0"]
    long = np.array([i % 7 - 3 for i in range(1025)], np.int32)
    assert _scan(device, hx.CumSumOp, 1, F, host=long, shape=(1, 1025), dtype=np.int32) == list(
        np.cumsum(long, dtype=np.int32))
    src = device.upload(x)
    lay = Layout.c_contiguous([2, 4])
    wrong = device.alloc_zeroed(np.int32, 8)
    with pytest.raises(hx.DispatchFailed) as e:
        SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(src, lay), 1, F, StridedView(wrong, Layout.c_contiguous([4, 2])))
    assert e.value.message.startswith(KATS["messages"]["scan_shape_prefix"])
    with pytest.raises(hx.DispatchFailed) as e:
        SCAN.scan_axis_into(device, hx.CumSumOp, StridedView(src, lay), 1, F, StridedView(src, lay))
    assert e.value.message == KATS["messages"]["scan_alias"]
