"""The DeviceApi seam: consumer kernels compiled at run time and launched on
this device (crates/hephaestus-core/src/domain/accelerator/device_api.rs:
10-133; ROCm impl crates/hephaestus-rocm/src/application/device_api.rs:
49-103 and pipeline.rs:175-349) over hx_kernel_compile_cached /
hx_kernel_launch / hx_buffers_alias.

    kernel = device.compile_cached(b"my-key", "my_entry", lambda: SOURCE)
    device.launch(kernel, LaunchGeometry.linear(groups, 256), params, [buf_a, buf_b])

`source` is called only on a cache miss; the kernel's first parameter is
the parameter block (a ctypes.Structure or bytes, passed by value), then
one pointer per operand, in order.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Callable, Sequence

import numpy as np

from . import _ffi, errors


@dataclass(frozen=True)
class LaunchGeometry:
    """A linear grid of `groups` blocks of `width` lanes with `shared_bytes`
    of dynamic LDS (LaunchGeometry, device_api.rs:10-47).  The width is a
    BlockWidth: non-zero (core launch.rs:15-40)."""

    groups: int
    width: int
    shared_bytes: int = 0

    def __post_init__(self):
        if int(self.width) <= 0:
            raise errors.InvalidConfiguration("block width must be non-zero")

    @classmethod
    def linear(cls, groups: int, width: int = 256) -> "LaunchGeometry":
        return cls(int(groups), int(width), 0)

    @classmethod
    def linear_shared(cls, groups: int, width: int, shared_bytes: int) -> "LaunchGeometry":
        return cls(int(groups), int(width), int(shared_bytes))


class RocmCompiledKernel:
    """A kernel compiled and cached for one device (RocmCompiledKernel,
    device_api.rs:25-30).  The device owns it until it is closed."""

    def __init__(self, device, handle: int, key: bytes, entry: str):
        self.device = device
        self.handle = handle
        self.key = key
        self.entry = entry

    def __eq__(self, other) -> bool:
        return isinstance(other, RocmCompiledKernel) and self.handle == other.handle

    def __hash__(self) -> int:
        return hash(self.handle)


def _key_bytes(key) -> bytes:
    if isinstance(key, (bytes, bytearray)):
        return bytes(key)
    return str(key).encode()


def compile_cached(device, key, entry: str, source: Callable[[], str]) -> RocmCompiledKernel:
    """DeviceApi::compile_cached (device_api.rs:83-99): the kernel cached on
    `device` under `key`, else `source()` compiled, loaded and its `entry`
    looked up.  Failed compilations raise DispatchFailed (with the hipRTC
    log) and are not cached; an exception from `source` propagates."""
    keyb = _key_bytes(key)
    keybuf = ctypes.create_string_buffer(keyb, max(1, len(keyb)))
    held: dict = {}

    def provide(_ctx):
        try:
            text = source()
            buf = ctypes.create_string_buffer(str(text).encode())
        except BaseException as exc:  # reported after the C call returns
            held["error"] = exc
            return None
        held["buf"] = buf
        return ctypes.addressof(buf)

    callback = _ffi.SOURCE_FN(provide)
    out = ctypes.c_void_p()
    status = _ffi.lib().hx_kernel_compile_cached(device.handle, keybuf, len(keyb), entry.encode(), callback,
                                                 None, ctypes.byref(out))
    if "error" in held:
        raise held["error"]
    _ffi.check(status)
    return RocmCompiledKernel(device, out.value, keyb, entry)


def device_ptr(buffer) -> int:
    """DeviceApi::device_ptr (device_api.rs:101-102): the buffer's device
    address (an int passes through)."""
    if isinstance(buffer, int):
        return buffer
    return int(buffer.ptr or 0)


def buffers_alias(lhs, rhs) -> bool:
    """DeviceApi::buffers_alias (device_api.rs:105-110): one non-null base,
    or overlapping byte ranges."""
    a, b = device_ptr(lhs), device_ptr(rhs)
    an = 0 if isinstance(lhs, int) else len(lhs) * lhs.itemsize
    bn = 0 if isinstance(rhs, int) else len(rhs) * rhs.itemsize
    return bool(_ffi.lib().hx_buffers_alias(a or None, an, b or None, bn))


def _param_block(params):
    if params is None:
        return None, 0, None
    if isinstance(params, ctypes.Structure) or isinstance(params, ctypes.Array):
        return ctypes.addressof(params), ctypes.sizeof(params), params
    if isinstance(params, np.ndarray):
        params = params.tobytes()
    if isinstance(params, (bytes, bytearray)):
        buf = ctypes.create_string_buffer(bytes(params), max(1, len(params)))
        return ctypes.addressof(buf), len(params), buf
    raise errors.InvalidConfiguration(f"unsupported parameter block {type(params).__name__}")


def launch(device, kernel: RocmCompiledKernel, geometry: LaunchGeometry, params=None,
           operands: Sequence = (), stream=None) -> None:
    """DeviceApi::launch (device_api.rs:116-132): `kernel` over `geometry`
    with `params` (by value) followed by each operand's device address, on
    `stream` (the device stream by default)."""
    addr, nbytes, keep = _param_block(params)
    ptrs = (ctypes.c_void_p * max(1, len(operands)))(*[device_ptr(o) for o in operands])
    _ffi.check(_ffi.lib().hx_kernel_launch(device.handle, kernel.handle, int(geometry.groups), int(geometry.width),
                                           int(geometry.shared_bytes), addr, nbytes, ptrs, len(operands), stream))
    del keep
