"""The reduction / scan seams over the C ABI.

Names and argument meaning follow the reference's traits so code written
against them reads the same:

* `RocmFullReductionOps`  FullReductionOps  (core reduction.rs:243-309)
* `RocmAxisReductionOps`  AxisReductionOps  (core reduction.rs:74-223)
* `RocmScanOps`           ScanOps           (core scan.rs:197-264)

plus operations the reference does not have: full and row
argmax, the fused row reduce with the `y = fmaf(a, x, b)` prologue,
exclusive scans and the segmented sum.  Operators are passed as the marker
classes below instead of type parameters.  Every call validates in the
native planners first and raises the matching HephaestusError, leaving the
outputs untouched.
"""
from __future__ import annotations

import ctypes
import enum

import numpy as np

from . import _ffi, errors
from .device import RocmBuffer, RocmDevice, hx_dtype
from .layout import Layout, StridedView


# --- operator markers (core ops.rs:735-803) --------------------------------
class SumOp:
    code = _ffi.OP_SUM


class ProdOp:
    code = _ffi.OP_PROD


class MinOp:
    code = _ffi.OP_MIN


class MaxOp:
    code = _ffi.OP_MAX


class MeanOp:
    code = _ffi.OP_MEAN


class ArgMaxOp:
    code = _ffi.OP_ARGMAX


class CumSumOp:
    code = _ffi.OP_SUM


class CumProdOp:
    code = _ffi.OP_PROD


class ScanDirection(enum.IntEnum):
    """core scan.rs:36-43"""

    Forward = _ffi.SCAN_FORWARD
    Reverse = _ffi.SCAN_REVERSE


class ScanKind(enum.IntEnum):
    Inclusive = _ffi.SCAN_INCLUSIVE
    Exclusive = _ffi.SCAN_EXCLUSIVE


def _lp(layout: Layout):
    return ctypes.byref(_ffi.layout_struct(layout))


class PreparedPlan:
    """A prepared dispatch bound to its operands; owns its workspace."""

    def __init__(self, device: RocmDevice, handle: int, keep: tuple):
        self.device = device
        self.handle = handle
        self._keep = keep  # operands stay alive as long as the plan

    def dispatch(self, stream=None) -> None:
        _ffi.check(_ffi.lib().hx_plan_dispatch(self.handle, stream))

    def workspace_bytes(self) -> int:
        b = ctypes.c_uint64()
        _ffi.check(_ffi.lib().hx_plan_workspace_bytes(self.handle, ctypes.byref(b)))
        return b.value

    def destroy(self) -> None:
        if self.handle:
            _ffi.lib().hx_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def submit_prepared_reduction_batch(plans) -> None:
    """Dispatch prepared plans in order on the device stream with no host
    synchronisation between them (rocm application/prepared_reduction.rs:
    164-174).  Accepts PreparedPlan and PreparedMapReduction handles."""
    plans = list(plans)
    if not plans:
        return
    arr = (ctypes.c_void_p * len(plans))(*[p.handle for p in plans])
    _ffi.check(_ffi.lib().hx_plan_dispatch_batch(arr, len(plans), None))


def submit_prepared_axis_reduction_batch(device: RocmDevice, plans) -> None:
    """Prepared axis reductions dispatched in order on the device stream
    (rocm application/prepared_axis_reduction.rs:84-92)."""
    plans = list(plans)
    for p in plans:
        if p.device is not device:
            raise errors.DispatchFailed("prepared axis reduction belongs to a different device")
    submit_prepared_reduction_batch(plans)


class RocmFullReductionOps:
    """FullReductionOps<RocmDevice, T> (rocm full_reduction_seam.rs:28-120)."""

    def reduce_full_into(self, device: RocmDevice, op, input: StridedView, output: StridedView,
                         prologue=None, stream=None) -> None:
        aff = _ffi.affine_struct(prologue)
        _ffi.check(
            _ffi.lib().hx_reduce_full(
                device.handle, op.code, hx_dtype(input.buffer.dtype), input.buffer.ptr,
                len(input.buffer), _lp(input.layout), output.buffer.ptr, len(output.buffer),
                _lp(output.layout), ctypes.byref(aff) if aff else None, stream,
            )
        )

    def prepare_reduce_full(self, device: RocmDevice, op, input: StridedView, output: StridedView,
                            prologue=None) -> PreparedPlan:
        plan = ctypes.c_void_p()
        aff = _ffi.affine_struct(prologue)
        _ffi.check(
            _ffi.lib().hx_prepare_reduce_full(
                device.handle, op.code, hx_dtype(input.buffer.dtype), input.buffer.ptr,
                len(input.buffer), _lp(input.layout), output.buffer.ptr, len(output.buffer),
                _lp(output.layout), ctypes.byref(aff) if aff else None, ctypes.byref(plan),
            )
        )
        return PreparedPlan(device, plan.value, (input, output))

    def dispatch_full(self, device: RocmDevice, prepared: PreparedPlan, stream=None) -> None:
        prepared.dispatch(stream)

    def argmax_full_into(self, device: RocmDevice, input: StridedView, index: RocmBuffer,
                         value: RocmBuffer | None = None, prologue=None, stream=None) -> None:
        """Index (u32) of the maximum, ties to the lowest index; NaN ignored."""
        if index.dtype != np.uint32 or len(index) != 1:
            raise errors.DispatchFailed("argmax index output must be a 1-element u32 buffer")
        if value is not None and (value.dtype != input.buffer.dtype or len(value) != 1):
            raise errors.DispatchFailed("argmax value output must be a 1-element buffer of the input dtype")
        aff = _ffi.affine_struct(prologue)
        _ffi.check(
            _ffi.lib().hx_argmax_full(
                device.handle, hx_dtype(input.buffer.dtype), input.buffer.ptr, len(input.buffer),
                _lp(input.layout), value.ptr if value is not None else None, index.ptr,
                ctypes.byref(aff) if aff else None, stream,
            )
        )


class RocmAxisReductionOps:
    """AxisReductionOps<RocmDevice, T> (rank-2 views, one axis collapsed)."""

    def reduce_axis_into(self, device: RocmDevice, op, input: StridedView, axis: int,
                         output: StridedView, stream=None) -> None:
        _ffi.check(
            _ffi.lib().hx_reduce_axis(
                device.handle, op.code, hx_dtype(input.buffer.dtype), input.buffer.ptr,
                len(input.buffer), _lp(input.layout), int(axis), output.buffer.ptr,
                len(output.buffer), _lp(output.layout), stream,
            )
        )

    def prod_axis_into(self, device, input, axis, output, stream=None):
        self.reduce_axis_into(device, ProdOp, input, axis, output, stream)

    def mean_axis_into(self, device, input, axis, output, stream=None):
        self.reduce_axis_into(device, MeanOp, input, axis, output, stream)

    def min_axis_into(self, device, input, axis, output, stream=None):
        self.reduce_axis_into(device, MinOp, input, axis, output, stream)

    def max_axis_into(self, device, input, axis, output, stream=None):
        self.reduce_axis_into(device, MaxOp, input, axis, output, stream)

    def argmax_axis_into(self, device, input, axis, output, stream=None):
        """`output` is a u32 view holding the index along `axis`."""
        self.reduce_axis_into(device, ArgMaxOp, input, axis, output, stream)

    def prepare_reduce_axis_into(self, device: RocmDevice, op, input: StridedView, axis: int,
                                 output: StridedView) -> PreparedPlan:
        plan = ctypes.c_void_p()
        _ffi.check(
            _ffi.lib().hx_prepare_reduce_axis(
                device.handle, op.code, hx_dtype(input.buffer.dtype), input.buffer.ptr,
                len(input.buffer), _lp(input.layout), int(axis), output.buffer.ptr,
                len(output.buffer), _lp(output.layout), ctypes.byref(plan),
            )
        )
        return PreparedPlan(device, plan.value, (input, output))

    def dispatch_prepared(self, device: RocmDevice, prepared: PreparedPlan, stream=None) -> None:
        prepared.dispatch(stream)

    @staticmethod
    def _rows_args(input, rows, cols, row_stride, offset, prologue, out_sum, out_max, out_argmax):
        row_stride = cols if row_stride is None else row_stride
        outs = [b for b in (out_sum, out_max, out_argmax) if b is not None]
        out_len = len(outs[0]) if outs else rows
        for b in outs:
            if len(b) != out_len:
                raise errors.LengthMismatch(len(b), out_len)
        if out_argmax is not None and out_argmax.dtype != np.uint32:
            raise errors.DispatchFailed("argmax output must be u32")
        for b in (out_sum, out_max):
            if b is not None and b.dtype != input.dtype:
                raise errors.DispatchFailed("sum/max outputs must have the input dtype")
        aff = _ffi.affine_struct(prologue)
        return (hx_dtype(input.dtype), input.ptr, len(input), int(rows), int(cols), int(row_stride), int(offset),
                ctypes.byref(aff) if aff else None, out_sum.ptr if out_sum is not None else None,
                out_max.ptr if out_max is not None else None,
                out_argmax.ptr if out_argmax is not None else None, out_len)

    def reduce_rows_fused(self, device: RocmDevice, input: RocmBuffer, rows: int, cols: int,
                          row_stride: int | None = None, offset: int = 0, prologue=None,
                          out_sum: RocmBuffer | None = None, out_max: RocmBuffer | None = None,
                          out_argmax: RocmBuffer | None = None, stream=None) -> None:
        """Sum, max and argmax of y = fmaf(a, x, b) per row, from one read."""
        args = self._rows_args(input, rows, cols, row_stride, offset, prologue, out_sum, out_max, out_argmax)
        _ffi.check(_ffi.lib().hx_reduce_rows(device.handle, *args, stream))

    def prepare_reduce_rows_fused(self, device: RocmDevice, input: RocmBuffer, rows: int, cols: int,
                                  row_stride: int | None = None, offset: int = 0, prologue=None,
                                  out_sum: RocmBuffer | None = None, out_max: RocmBuffer | None = None,
                                  out_argmax: RocmBuffer | None = None) -> PreparedPlan:
        """Prepared reduce_rows_fused (hx_prepare_reduce_rows): validated
        once, dispatched without allocation, batchable."""
        args = self._rows_args(input, rows, cols, row_stride, offset, prologue, out_sum, out_max, out_argmax)
        plan = ctypes.c_void_p()
        _ffi.check(_ffi.lib().hx_prepare_reduce_rows(device.handle, *args, ctypes.byref(plan)))
        return PreparedPlan(device, plan.value, (input, out_sum, out_max, out_argmax))


class RocmScanOps:
    """ScanOps<RocmDevice, T> over rank-1 and rank-2 views."""

    def scan_axis_into(self, device: RocmDevice, op, input: StridedView, axis: int,
                       direction: ScanDirection, output: StridedView,
                       kind: ScanKind = ScanKind.Inclusive, stream=None) -> None:
        _ffi.check(
            _ffi.lib().hx_scan(
                device.handle, op.code, hx_dtype(input.buffer.dtype), int(kind), int(direction),
                input.buffer.ptr, len(input.buffer), _lp(input.layout), int(axis),
                output.buffer.ptr, len(output.buffer), _lp(output.layout), stream,
            )
        )

    def scan_axis_into_noalloc(self, device: RocmDevice, op, input: StridedView, axis: int,
                               direction: ScanDirection, output: StridedView,
                               kind: ScanKind = ScanKind.Inclusive, stream=None) -> None:
        """scan_axis_into through hx_scan_noalloc: no device allocation; the
        workspace is the device's fixed scratch array."""
        _ffi.check(
            _ffi.lib().hx_scan_noalloc(
                device.handle, op.code, hx_dtype(input.buffer.dtype), int(kind), int(direction),
                input.buffer.ptr, len(input.buffer), _lp(input.layout), int(axis),
                output.buffer.ptr, len(output.buffer), _lp(output.layout), stream,
            )
        )

    def prepare_scan_axis(self, device: RocmDevice, op, input: StridedView, axis: int,
                          direction: ScanDirection, output: StridedView,
                          kind: ScanKind = ScanKind.Inclusive) -> PreparedPlan:
        plan = ctypes.c_void_p()
        _ffi.check(
            _ffi.lib().hx_prepare_scan(
                device.handle, op.code, hx_dtype(input.buffer.dtype), int(kind), int(direction),
                input.buffer.ptr, len(input.buffer), _lp(input.layout), int(axis),
                output.buffer.ptr, len(output.buffer), _lp(output.layout), ctypes.byref(plan),
            )
        )
        return PreparedPlan(device, plan.value, (input, output))

    def dispatch_scan(self, device: RocmDevice, prepared: PreparedPlan, stream=None) -> None:
        prepared.dispatch(stream)

    # Flat 1-D conveniences.
    def exclusive_scan_into(self, device, input: RocmBuffer, output: RocmBuffer, stream=None):
        lay = Layout.c_contiguous([len(input)])
        self.scan_axis_into(device, CumSumOp, StridedView(input, lay), 0, ScanDirection.Forward,
                            StridedView(output, Layout.c_contiguous([len(output)])),
                            ScanKind.Exclusive, stream)

    def inclusive_scan_into(self, device, input: RocmBuffer, output: RocmBuffer, stream=None):
        lay = Layout.c_contiguous([len(input)])
        self.scan_axis_into(device, CumSumOp, StridedView(input, lay), 0, ScanDirection.Forward,
                            StridedView(output, Layout.c_contiguous([len(output)])),
                            ScanKind.Inclusive, stream)


class RocmSegmentedReductionOps:
    """Segmented sum over CSR-style offsets."""

    def segmented_sum_into(self, device: RocmDevice, values: RocmBuffer, offsets: RocmBuffer,
                           output: RocmBuffer, stream=None) -> None:
        if offsets.dtype != np.uint32:
            raise errors.DispatchFailed("segment offsets must be u32")
        if output.dtype != values.dtype:
            raise errors.DispatchFailed("segmented sum output must have the values dtype")
        _ffi.check(
            _ffi.lib().hx_segmented_reduce(
                device.handle, _ffi.OP_SUM, hx_dtype(values.dtype), values.ptr, len(values),
                offsets.ptr, len(offsets), output.ptr, len(output), stream,
            )
        )

    def prepare_segmented_sum(self, device: RocmDevice, values: RocmBuffer, offsets: RocmBuffer,
                              output: RocmBuffer) -> PreparedPlan:
        if offsets.dtype != np.uint32:
            raise errors.DispatchFailed("segment offsets must be u32")
        plan = ctypes.c_void_p()
        _ffi.check(
            _ffi.lib().hx_prepare_segmented_reduce(
                device.handle, _ffi.OP_SUM, hx_dtype(values.dtype), values.ptr, len(values),
                offsets.ptr, len(offsets), output.ptr, len(output), ctypes.byref(plan),
            )
        )
        return PreparedPlan(device, plan.value, (values, offsets, output))

    def validate_offsets(self, device: RocmDevice, offsets: RocmBuffer, n: int) -> None:
        _ffi.check(_ffi.lib().hx_validate_segment_offsets(device.handle, offsets.ptr, len(offsets), int(n)))


# --- host planners (no device needed) ---------------------------------------
def validate_reduction_width(width: int) -> None:
    _ffi.check(_ffi.lib().hx_validate_reduction_width(int(width)))


def reduction_pass_count(length: int, width: int) -> int:
    return int(_ffi.lib().hx_reduction_pass_count(int(length), int(width)))


def plan_axis_reduction(input: Layout, input_buf_len: int, output: Layout, output_buf_len: int,
                        axis: int, width: int = 256, buffers_alias: bool = False):
    """core reduction.rs:410-500: returns (output_len, axis_len); output_len
    0 is the empty no-op."""
    out_len = ctypes.c_uint64()
    axis_len = ctypes.c_uint64()
    _ffi.check(
        _ffi.lib().hx_plan_axis_reduction(
            _lp(input), int(input_buf_len), _lp(output), int(output_buf_len), int(axis), int(width),
            1 if buffers_alias else 0, ctypes.byref(out_len), ctypes.byref(axis_len),
        )
    )
    return out_len.value, axis_len.value


def plan_axis_scan(input: Layout, input_buf_len: int, output: Layout, output_buf_len: int,
                   axis: int, width: int = 256, buffers_alias: bool = False):
    """core scan.rs:87-178: returns (lines, line_len); lines 0 is the no-op."""
    lines = ctypes.c_uint64()
    line_len = ctypes.c_uint64()
    _ffi.check(
        _ffi.lib().hx_plan_axis_scan(
            _lp(input), int(input_buf_len), _lp(output), int(output_buf_len), int(axis), int(width),
            1 if buffers_alias else 0, ctypes.byref(lines), ctypes.byref(line_len),
        )
    )
    return lines.value, line_len.value
