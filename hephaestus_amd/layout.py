"""Strided layouts and views.

`Layout` mirrors the leto `Layout<N>` the reference pairs with a buffer
(shape, signed element strides, element offset); `StridedView` mirrors
crates/hephaestus-core/src/domain/view.rs:27-41.  Validation of a layout
against its buffer is done by the native planners (hx_layout_* in
include/hx.h), so the rules are the same from every host language.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

from . import _ffi, errors


@dataclass(frozen=True)
class Layout:
    shape: tuple[int, ...]
    strides: tuple[int, ...]
    offset: int = 0

    @staticmethod
    def c_contiguous(shape: Sequence[int]) -> "Layout":
        shape = tuple(int(s) for s in shape)
        strides = []
        acc = 1
        for extent in reversed(shape):
            strides.append(acc)
            acc *= max(extent, 1)
        return Layout(shape, tuple(reversed(strides)), 0)

    @staticmethod
    def try_new(shape: Sequence[int], strides: Sequence[int], offset: int = 0) -> "Layout":
        shape = tuple(int(s) for s in shape)
        strides = tuple(int(s) for s in strides)
        if len(shape) != len(strides):
            raise errors.DispatchFailed(
                f"layout rejected: shape rank {len(shape)} differs from stride rank {len(strides)}"
            )
        if any(s < 0 for s in shape) or offset < 0:
            raise errors.DispatchFailed("layout rejected: negative extent or offset")
        return Layout(shape, strides, int(offset))

    @property
    def rank(self) -> int:
        return len(self.shape)

    def checked_size(self) -> int:
        size = ctypes.c_uint64()
        _ffi.check(_ffi.lib().hx_layout_checked_size(ctypes.byref(_ffi.layout_struct(self)), ctypes.byref(size)))
        return size.value

    def validate_storage_len(self, buf_len: int) -> None:
        _ffi.check(_ffi.lib().hx_layout_validate_storage_len(ctypes.byref(_ffi.layout_struct(self)), buf_len))

    def has_zero_stride_aliasing(self) -> bool:
        return bool(_ffi.lib().hx_layout_has_zero_stride_aliasing(ctypes.byref(_ffi.layout_struct(self))))


@dataclass(frozen=True)
class StridedView:
    """A device buffer read through a layout (core view.rs:27-41)."""

    buffer: object
    layout: Layout
