"""Map-reductions and dense vector operations over the C ABI.

* `dot`, `trace`, `norm_l1`, `norm_l2`, `norm_max` mirror the ROCm
  reference's free functions (crates/hephaestus-rocm/src/application/linalg/
  norms.rs:394-490): strided views in, a new one-element device buffer out.
* `prepare_dot`, `prepare_norm_l2` mirror prepared_map_reduction.rs:63-213:
  the operands are bound, each dispatch re-reads them.
* `RocmDenseVectorOps` mirrors DenseVectorOps<RocmDevice, f32>
  (crates/hephaestus-core/src/domain/vector.rs:57-200; ROCm implementation
  crates/hephaestus-rocm/src/application/vector.rs:141-373): whole buffers
  as vectors, scalar results returned to the host.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _ffi, errors
from .device import RocmBuffer, RocmDevice, hx_dtype
from .layout import Layout, StridedView


def _lp(layout: Layout):
    return ctypes.byref(_ffi.layout_struct(layout))


def _map(device: RocmDevice, kind: int, a: StridedView, b: StridedView | None, out: RocmBuffer, stream=None):
    _ffi.check(
        _ffi.lib().hx_map_reduce(
            device.handle, kind, hx_dtype(a.buffer.dtype), a.buffer.ptr, len(a.buffer), _lp(a.layout),
            b.buffer.ptr if b is not None else None, len(b.buffer) if b is not None else 0,
            _lp(b.layout) if b is not None else None, out.ptr, len(out), stream,
        )
    )


def _scalar_out(device: RocmDevice, like: RocmBuffer) -> RocmBuffer:
    return device.alloc_uninitialized(like.dtype, 1)


def dot(device: RocmDevice, a: StridedView, b: StridedView, stream=None) -> RocmBuffer:
    """Σᵢ a[i]·b[i] over views of equal logical shape (norms.rs:396-412)."""
    if a.buffer.dtype != b.buffer.dtype:
        raise errors.DispatchFailed("dot product operands must share an element type")
    out = _scalar_out(device, a.buffer)
    _map(device, _ffi.MAP_DOT, a, b, out, stream)
    return out


def trace(device: RocmDevice, matrix: StridedView, stream=None) -> RocmBuffer:
    """Σᵢ aᵢᵢ of a square rank-2 view (norms.rs:414-444)."""
    out = _scalar_out(device, matrix.buffer)
    _ffi.check(
        _ffi.lib().hx_trace(
            device.handle, hx_dtype(matrix.buffer.dtype), matrix.buffer.ptr, len(matrix.buffer),
            _lp(matrix.layout), out.ptr, len(out), stream,
        )
    )
    return out


def norm_l1(device: RocmDevice, view: StridedView, stream=None) -> RocmBuffer:
    """Σ|x| (norms.rs:446-455)."""
    out = _scalar_out(device, view.buffer)
    _map(device, _ffi.MAP_NORM_L1, view, None, out, stream)
    return out


def norm_l2(device: RocmDevice, view: StridedView, stream=None) -> RocmBuffer:
    """sqrt(Σx²), f32 only (norms.rs:457-478)."""
    out = _scalar_out(device, view.buffer)
    _map(device, _ffi.MAP_NORM_L2, view, None, out, stream)
    return out


def norm_max(device: RocmDevice, view: StridedView, stream=None) -> RocmBuffer:
    """max|x| with the MaxOp identity for an empty view (norms.rs:480-490)."""
    out = _scalar_out(device, view.buffer)
    _map(device, _ffi.MAP_NORM_MAX, view, None, out, stream)
    return out


class PreparedMapReduction:
    """A bound map-reduction: its plan, its one-element output buffer, and the
    allocations it was prepared against (prepared_map_reduction.rs)."""

    def __init__(self, device: RocmDevice, kind: int, a: StridedView, b: StridedView | None):
        self.device = device
        self.output = _scalar_out(device, a.buffer)
        self._operands = (a, b)
        self._ptrs = (a.buffer.ptr, b.buffer.ptr if b is not None else None)
        plan = ctypes.c_void_p()
        _ffi.check(
            _ffi.lib().hx_prepare_map_reduce(
                device.handle, kind, hx_dtype(a.buffer.dtype), a.buffer.ptr, len(a.buffer), _lp(a.layout),
                b.buffer.ptr if b is not None else None, len(b.buffer) if b is not None else 0,
                _lp(b.layout) if b is not None else None, self.output.ptr, len(self.output), ctypes.byref(plan),
            )
        )
        self.handle = plan.value

    def matches(self, a: RocmBuffer, b: RocmBuffer | None = None) -> bool:
        return a.ptr == self._ptrs[0] and (b is None or b.ptr == self._ptrs[1])

    def dispatch(self, stream=None) -> None:
        _ffi.check(_ffi.lib().hx_plan_dispatch(self.handle, stream))

    def destroy(self) -> None:
        if self.handle:
            _ffi.lib().hx_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def prepare_dot(device: RocmDevice, a: StridedView, b: StridedView) -> PreparedMapReduction:
    return PreparedMapReduction(device, _ffi.MAP_DOT, a, b)


def prepare_norm_l2(device: RocmDevice, view: StridedView) -> PreparedMapReduction:
    return PreparedMapReduction(device, _ffi.MAP_NORM_L2, view, None)


def _flat(buf: RocmBuffer) -> StridedView:
    return StridedView(buf, Layout.c_contiguous([len(buf)]))


class RocmDenseVectorOps:
    """DenseVectorOps<RocmDevice, f32>."""

    @staticmethod
    def _scalar(device: RocmDevice, buf: RocmBuffer) -> float:
        return float(device.download_owned(buf)[0])

    def copy_vector(self, device: RocmDevice, source: RocmBuffer, target: RocmBuffer) -> None:
        if len(source) != len(target):
            raise errors.LengthMismatch(len(source), len(target))
        if len(source):
            device.copy_buffer(source, target)

    def scale_vector(self, device: RocmDevice, target: RocmBuffer, factor: float, stream=None) -> None:
        _ffi.check(_ffi.lib().hx_vector_update(device.handle, _ffi.VEC_SCALE, hx_dtype(target.dtype), target.ptr,
                                               len(target), None, 0, float(factor), stream))

    def axpy(self, device: RocmDevice, target: RocmBuffer, source: RocmBuffer, factor: float, stream=None) -> None:
        """target = fmaf(factor, source, target)."""
        _ffi.check(_ffi.lib().hx_vector_update(device.handle, _ffi.VEC_AXPY, hx_dtype(target.dtype), target.ptr,
                                               len(target), source.ptr, len(source), float(factor), stream))

    def xpay(self, device: RocmDevice, target: RocmBuffer, source: RocmBuffer, factor: float, stream=None) -> None:
        """target = fmaf(factor, target, source)."""
        _ffi.check(_ffi.lib().hx_vector_update(device.handle, _ffi.VEC_XPAY, hx_dtype(target.dtype), target.ptr,
                                               len(target), source.ptr, len(source), float(factor), stream))

    def _binary(self, device, op, left, right, output, stream):
        _ffi.check(_ffi.lib().hx_vector_binary(device.handle, op, hx_dtype(left.dtype), left.ptr, len(left),
                                               right.ptr, len(right), output.ptr, len(output), stream))

    def subtract_into(self, device, left, right, output, stream=None) -> None:
        self._binary(device, _ffi.VEC_SUB, left, right, output, stream)

    def add_into(self, device, left, right, output, stream=None) -> None:
        self._binary(device, _ffi.VEC_ADD, left, right, output, stream)

    def multiply_into(self, device, left, right, output, stream=None) -> None:
        self._binary(device, _ffi.VEC_MUL, left, right, output, stream)

    def divide_into(self, device, left, right, output, stream=None) -> None:
        self._binary(device, _ffi.VEC_DIV, left, right, output, stream)

    def prepare_dot(self, device: RocmDevice, left: RocmBuffer, right: RocmBuffer) -> PreparedMapReduction:
        if len(left) != len(right):
            raise errors.LengthMismatch(len(left), len(right))
        return prepare_dot(device, _flat(left), _flat(right))

    def dot_prepared(self, device: RocmDevice, prepared: PreparedMapReduction, left: RocmBuffer,
                     right: RocmBuffer) -> float:
        if not prepared.matches(left, right):
            raise errors.DispatchFailed("prepared dot received different device allocations")
        prepared.dispatch()
        return self._scalar(device, prepared.output)

    def prepare_norm_l2(self, device: RocmDevice, vector: RocmBuffer) -> PreparedMapReduction:
        return prepare_norm_l2(device, _flat(vector))

    def norm_l2_prepared(self, device: RocmDevice, prepared: PreparedMapReduction, vector: RocmBuffer) -> float:
        if not prepared.matches(vector):
            raise errors.DispatchFailed("prepared norm received a different device allocation")
        prepared.dispatch()
        return self._scalar(device, prepared.output)

    def norm_l1(self, device: RocmDevice, vector: RocmBuffer) -> float:
        return self._scalar(device, norm_l1(device, _flat(vector)))

    def norm_max(self, device: RocmDevice, vector: RocmBuffer) -> float:
        return self._scalar(device, norm_max(device, _flat(vector)))
