"""hx_scan_noalloc (the scan whose workspace is a fixed device array) against
hx_scan, the entry point it is a variant of: two calls in a row on each
shape, the second smaller, so the second runs over status words the first
left behind.  Integer results are bit-exact against hx_scan and the oracle;
f32 results are held to the oracle's bound 2*ceil(log2 n)*eps_f32*sum|x|, as
are their differences from hx_scan.  Oversized scans are rejected before
any launch and leave the output untouched."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _scan_both(device, op_kind, x, shape, axis, direction, kind):
    import hephaestus_amd as hx
    from hephaestus_amd import Layout, StridedView

    ops = hx.RocmScanOps()
    lay = Layout.c_contiguous(list(shape))
    xb = device.upload(x)
    ref_out = device.alloc_zeroed(x.dtype, x.size)
    got_out = device.alloc_zeroed(x.dtype, x.size)
    print(f"[no-alloc] {x.dtype} shape {shape} axis {axis} {direction} {kind}", flush=True)
    ops.scan_axis_into(device, op_kind, StridedView(xb, lay), axis, direction, StridedView(ref_out, lay), kind)
    ops.scan_axis_into_noalloc(device, op_kind, StridedView(xb, lay), axis, direction, StridedView(got_out, lay),
                               kind)
    device.synchronize()
    return device.download_owned(ref_out), device.download_owned(got_out)


def _lines(x, shape, axis):
    """The scan lines of a C-contiguous array in (line, element) order."""
    a = x.reshape(shape)
    return np.ascontiguousarray(a if axis == len(shape) - 1 else np.moveaxis(a, 0, -1)).reshape(-1, shape[axis])


CASES = [
    # (dtype, [first shape, second smaller shape], axis, reverse, exclusive)
    (np.uint32, [(1 << 24) + 12345], [(1 << 20) + 7], 0, False, True),
    (np.int32, [(3 << 20) + 1], [65536 * 3 + 5], 0, True, False),
    (np.uint32, [1000, 4099], [300, 77], 1, True, False),
    (np.int32, [2048, 256], [500, 256], 0, False, True),
    (np.uint32, [4096, 252], [1000, 252], 0, False, False),
    (np.float32, [(1 << 22) + 3], [100003], 0, False, False),
    (np.float32, [2000, 3000], [64, 33], 1, True, True),
]


@pytest.mark.parametrize("dtype,first,second,axis,reverse,exclusive", CASES)
def test_noalloc_scan_matches_hx_scan_twice(device, oracle, dtype, first, second, axis, reverse, exclusive):
    import hephaestus_amd as hx

    direction = hx.ScanDirection.Reverse if reverse else hx.ScanDirection.Forward
    kind = hx.ScanKind.Exclusive if exclusive else hx.ScanKind.Inclusive
    for call, shape in enumerate((first, second)):
        n = int(np.prod(shape))
        if dtype == np.float32:
            x = oracle.uniform_real(n, seed=40 + call, lo=-1.0, hi=1.0)
        else:
            x = oracle.uniform_int(n, seed=40 + call, lo=0, hi=2**32 - 1).view(dtype)
        ref, got = _scan_both(device, hx.CumSumOp, x, shape, axis, direction, kind)
        line_len = shape[axis]
        if dtype != np.float32:
            assert np.array_equal(got, ref), (call, shape)
            want = np.concatenate([oracle.scan_sum(l, exclusive=exclusive, reverse=reverse)
                                   for l in _lines(x, shape, axis)])
            assert np.array_equal(_lines(got, shape, axis).ravel(), want), (call, shape)
            continue
        tol_k = 2 * oracle.ceil_log2(line_len) * 2.0**-23
        for lx, lg, lr in zip(_lines(x, shape, axis), _lines(got, shape, axis), _lines(ref, shape, axis)):
            r, ab = oracle.scan_sum(lx, exclusive=exclusive, reverse=reverse)
            assert oracle.check_f32_bound(lg, r, ab, line_len)[0] == 0, (call, shape)
            assert oracle.check_f32_bound(lr, r, ab, line_len)[0] == 0, (call, shape)
            assert np.all(np.abs(lg.astype(np.float64) - lr) <= tol_k * ab), (call, shape)


def test_noalloc_scan_rejects_oversized_workspace(device):
    """A single-pass column scan of 65536 x 4096 u32 needs about 9 MiB of
    status words, more than the fixed array: DispatchFailed, nothing
    launched, output untouched."""
    import hephaestus_amd as hx
    from hephaestus_amd import Layout, StridedView, _ffi

    assert _ffi.lib().hx_noalloc_scratch_bytes() == 8 << 20
    rows, cols = 65536, 4096
    lay = Layout.c_contiguous([rows, cols])
    x = device.alloc_zeroed(np.uint32, rows * cols)
    out = device.upload(np.full(rows * cols, 7, np.uint32))
    with pytest.raises(hx.DispatchFailed, match="no-allocation scratch holds 8388608"):
        hx.RocmScanOps().scan_axis_into_noalloc(device, hx.CumSumOp, StridedView(x, lay), 0,
                                                hx.ScanDirection.Forward, StridedView(out, lay))
    device.synchronize()
    assert np.all(device.download_owned(out) == 7)
