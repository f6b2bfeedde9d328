"""`RocmDevice` / `RocmBuffer`: the ComputeDevice and DeviceBuffer<T> seams
(crates/hephaestus-core/src/domain/device.rs:90-224, buffer.rs:7-19) over
the C ABI.  Host data is exchanged as numpy arrays of float32 / uint32 /
int32; device memory is owned by `RocmBuffer` and freed when it is
garbage-collected (the reference frees in Drop: crates/hephaestus-rocm/src/
infrastructure/buffer.rs:16-80).
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass

import numpy as np

from . import _ffi, errors

DTYPES = {
    np.dtype(np.float32): _ffi.DTYPE_F32,
    np.dtype(np.uint32): _ffi.DTYPE_U32,
    np.dtype(np.int32): _ffi.DTYPE_I32,
}


def hx_dtype(dtype) -> int:
    try:
        return DTYPES[np.dtype(dtype)]
    except KeyError:
        raise errors.InvalidConfiguration(f"unsupported element type {np.dtype(dtype)}") from None


@dataclass(frozen=True)
class Topology:
    """Probed hardware topology (query_topology, rocm query.rs:104-177)."""

    name: str
    arch: str
    compute_units: int
    warp_width: int
    max_threads_per_block: int
    max_threads_per_unit: int
    lds_bytes_per_block: int
    l2_bytes: int
    total_memory_bytes: int
    free_memory_bytes: int
    clock_khz: int
    memory_clock_khz: int
    memory_bus_width_bits: int


class DevicePreference(enum.Enum):
    """DevicePreference (core device.rs:10-17)."""

    HighPerformance = 0
    LowPower = 1


class DeviceFeature(enum.IntEnum):
    """DeviceFeature (core device.rs:19-36), hx_device_feature values."""

    TimestampQuery = 0
    ShaderF64 = 1
    ShaderF16 = 2
    MappablePrimaryBuffers = 3
    ImmediateData = 4


@dataclass(frozen=True)
class DeviceLimits:
    """DeviceLimits (core device.rs:38-80); the optional per-stage binding
    limits are None on ROCm (query.rs:85-86)."""

    max_buffer_size: int = 0
    max_compute_workgroup_size_x: int = 0
    max_compute_workgroup_size_y: int = 0
    max_compute_workgroup_size_z: int = 0
    max_compute_invocations_per_workgroup: int = 0
    max_compute_workgroup_storage_size: int = 0
    max_immediate_size: int = 0
    max_storage_buffers_per_shader_stage: int | None = None
    max_buffers_and_acceleration_structures_per_shader_stage: int | None = None

    def _struct(self) -> _ffi.HxDeviceLimits:
        s = _ffi.HxDeviceLimits()
        for name, _ in _ffi.HxDeviceLimits._fields_:
            setattr(s, name, int(getattr(self, name)))
        return s

    @classmethod
    def _from(cls, s: _ffi.HxDeviceLimits) -> "DeviceLimits":
        return cls(**{name: getattr(s, name) for name, _ in _ffi.HxDeviceLimits._fields_})


@dataclass(frozen=True)
class PlacementHint:
    """A placement request (themis PlacementHint, as the reference's devices
    read it: Current, Any, Numa(node), Domain(id) or Tier(tier)).  `tier` is
    the memory tier's name and `host_allocatable` whether it can hold a
    primary buffer; budget-only tiers cannot."""

    kind: str = "Current"
    value: object = None
    host_allocatable: bool = True

    @classmethod
    def current(cls) -> "PlacementHint":
        return cls("Current")

    @classmethod
    def any(cls) -> "PlacementHint":
        return cls("Any")

    @classmethod
    def numa(cls, node: int) -> "PlacementHint":
        return cls("Numa", int(node))

    @classmethod
    def domain(cls, domain) -> "PlacementHint":
        return cls("Domain", domain)

    @classmethod
    def tier(cls, tier: str, host_allocatable: bool = True) -> "PlacementHint":
        return cls("Tier", tier, bool(host_allocatable))

    @staticmethod
    def check_primary(hint: "PlacementHint") -> None:
        """allocation_tier (ROCm device.rs:167-185)."""
        if hint.kind == "Tier" and not hint.host_allocatable:
            raise errors.AllocationFailed(
                f"ROCm primary buffers cannot be allocated from budget-only tier {hint.value}")


class RocmBuffer:
    """A typed, device-resident linear buffer of `len` elements."""

    def __init__(self, device: "RocmDevice", ptr: int | None, length: int, dtype):
        self.device = device
        self.ptr = ptr or None
        self._len = int(length)
        self.dtype = np.dtype(dtype)

    def __len__(self) -> int:
        return self._len

    def len(self) -> int:
        return self._len

    def is_empty(self) -> bool:
        return self._len == 0

    def tier(self) -> str:
        return "device-hbm"

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    def free(self) -> None:
        if self.ptr and self.device is not None and self.device.handle:
            _ffi.check(_ffi.lib().hx_free(self.device.handle, self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class RocmDevice:
    """An acquired AMD GPU (RocmDevice::try_with_ordinal, rocm device.rs:109-165)."""

    def __init__(self, handle: int):
        self.handle = handle
        info = _ffi.HxDeviceInfo()
        _ffi.check(_ffi.lib().hx_device_get_info(self.handle, ctypes.byref(info)))
        self._topology = Topology(
            name=info.name.decode(errors="replace"),
            arch=info.arch.decode(errors="replace"),
            compute_units=info.compute_units,
            warp_width=info.warp_size,
            max_threads_per_block=info.max_threads_per_block,
            max_threads_per_unit=info.max_threads_per_cu,
            lds_bytes_per_block=info.lds_bytes_per_block,
            l2_bytes=info.l2_bytes,
            total_memory_bytes=info.total_memory_bytes,
            free_memory_bytes=info.free_memory_bytes,
            clock_khz=info.clock_khz,
            memory_clock_khz=info.memory_clock_khz,
            memory_bus_width_bits=info.memory_bus_width_bits,
        )
        stream = ctypes.c_void_p()
        _ffi.check(_ffi.lib().hx_device_stream(self.handle, ctypes.byref(stream)))
        self.stream = stream.value

    # -- acquisition ---------------------------------------------------
    @staticmethod
    def device_count() -> int:
        count = ctypes.c_int32()
        _ffi.check(_ffi.lib().hx_device_count(ctypes.byref(count)))
        return count.value

    @classmethod
    def try_with_ordinal(cls, ordinal: int) -> "RocmDevice":
        handle = ctypes.c_void_p()
        _ffi.check(_ffi.lib().hx_device_open(int(ordinal), ctypes.byref(handle)))
        return cls(handle.value)

    @classmethod
    def try_default(cls) -> "RocmDevice":
        return cls.try_with_ordinal(0)

    # -- ComputeDeviceAcquisition (ROCm acquisition.rs:8-35) -------------
    @classmethod
    def try_acquire_device(cls, label: str = "", device_preference=DevicePreference.HighPerformance,
                           optional_features=(), required_limits: DeviceLimits = DeviceLimits()) -> "RocmDevice":
        """The first device, if it meets `required_limits` (label,
        preference and optional features do not select among AMD devices)."""
        device = cls.try_default()
        try:
            cls.require_limits(device.device_limits(), required_limits)
        except BaseException:
            device.close()
            raise
        return device

    @classmethod
    def try_acquire_devices(cls, label_prefix: str = "", max_devices: int = 1,
                            device_preference=DevicePreference.HighPerformance, optional_features=(),
                            required_limits: DeviceLimits = DeviceLimits()) -> list:
        devices = []
        try:
            for ordinal in range(min(cls.device_count(), int(max_devices))):
                device = cls.try_with_ordinal(ordinal)
                devices.append(device)
                cls.require_limits(device.device_limits(), required_limits)
        except BaseException:
            for d in devices:
                d.close()
            raise
        return devices

    @staticmethod
    def require_limits(actual: DeviceLimits, required: DeviceLimits) -> None:
        """DeviceUnavailable for the first limit below the required one
        (ROCm device.rs:187-238)."""
        a, r = actual._struct(), required._struct()
        _ffi.check(_ffi.lib().hx_require_limits(ctypes.byref(a), ctypes.byref(r)))

    # -- ComputeDeviceCapabilities (ROCm capabilities.rs:5-21) -----------
    def device_limits(self) -> DeviceLimits:
        s = _ffi.HxDeviceLimits()
        _ffi.check(_ffi.lib().hx_device_get_limits(self.handle, ctypes.byref(s)))
        return DeviceLimits._from(s)

    def supports_device_feature(self, feature: DeviceFeature) -> bool:
        return bool(_ffi.lib().hx_device_supports_feature(self.handle, int(feature)))

    def close(self) -> None:
        if self.handle:
            _ffi.check(_ffi.lib().hx_device_close(self.handle))
            self.handle = None

    # -- ComputeDevice -------------------------------------------------
    def backend_name(self) -> str:
        return "rocm"

    def topology(self) -> Topology:
        return self._topology

    def synchronize(self) -> None:
        _ffi.check(_ffi.lib().hx_synchronize(self.handle))

    def _alloc(self, dtype, length: int, zeroed: bool) -> RocmBuffer:
        # Any plain-old-data element type can be stored and moved (the
        # reference's Buffer<T: Pod>); compute entry points check theirs.
        if np.dtype(dtype).hasobject:
            raise errors.InvalidConfiguration(f"unsupported element type {np.dtype(dtype)}")
        ptr = ctypes.c_void_p()
        nbytes = int(length) * np.dtype(dtype).itemsize
        _ffi.check(_ffi.lib().hx_alloc(self.handle, nbytes, 1 if zeroed else 0, ctypes.byref(ptr)))
        return RocmBuffer(self, ptr.value, length, dtype)

    def alloc_zeroed(self, dtype, length: int) -> RocmBuffer:
        return self._alloc(dtype, length, True)

    def alloc_uninitialized(self, dtype, length: int) -> RocmBuffer:
        return self._alloc(dtype, length, False)

    def upload(self, host) -> RocmBuffer:
        host = np.ascontiguousarray(host)
        buf = self.alloc_uninitialized(host.dtype, host.size)
        self.write_buffer(buf, host)
        return buf

    # The *_with_hint forms (core device.rs:103-143): every hint places a
    # primary buffer in device memory, except a tier that cannot hold
    # primary buffers (ROCm device.rs:167-185).
    def alloc_zeroed_with_hint(self, dtype, length: int, hint: "PlacementHint") -> RocmBuffer:
        PlacementHint.check_primary(hint)
        return self._alloc(dtype, length, True)

    def alloc_uninitialized_with_hint(self, dtype, length: int, hint: "PlacementHint") -> RocmBuffer:
        PlacementHint.check_primary(hint)
        return self._alloc(dtype, length, False)

    def upload_with_hint(self, host, hint: "PlacementHint") -> RocmBuffer:
        PlacementHint.check_primary(hint)
        return self.upload(host)

    def write_buffer(self, buffer: RocmBuffer, host) -> None:
        host = np.ascontiguousarray(host, dtype=buffer.dtype)
        _ffi.check(
            _ffi.lib().hx_upload(
                self.handle, buffer.ptr, len(buffer), host.ctypes.data, host.size, buffer.itemsize
            )
        )

    def write_sub_buffer(self, buffer: RocmBuffer, offset: int, host) -> None:
        host = np.ascontiguousarray(host, dtype=buffer.dtype)
        _ffi.check(
            _ffi.lib().hx_write_sub(
                self.handle, buffer.ptr, len(buffer), int(offset), host.ctypes.data, host.size,
                buffer.itemsize,
            )
        )

    def download(self, buffer: RocmBuffer, out: np.ndarray) -> None:
        if not (isinstance(out, np.ndarray) and out.flags.c_contiguous and out.dtype == buffer.dtype):
            raise errors.InvalidConfiguration("download target must be a C-contiguous array of the buffer dtype")
        _ffi.check(
            _ffi.lib().hx_download(
                self.handle, buffer.ptr, len(buffer), out.ctypes.data, out.size, buffer.itemsize
            )
        )

    def download_owned(self, buffer: RocmBuffer) -> np.ndarray:
        out = np.empty(len(buffer), dtype=buffer.dtype)
        self.download(buffer, out)
        return out

    def copy_buffer(self, src: RocmBuffer, dst: RocmBuffer) -> None:
        if src.dtype != dst.dtype:
            raise errors.InvalidConfiguration("copy_buffer between different element types")
        _ffi.check(
            _ffi.lib().hx_copy(self.handle, src.ptr, len(src), dst.ptr, len(dst), src.itemsize)
        )

    def copy_buffer_async(self, src: RocmBuffer, dst: RocmBuffer, stream=None) -> None:
        """copy_buffer queued on `stream` without waiting (hx_copy_async)."""
        if src.dtype != dst.dtype:
            raise errors.InvalidConfiguration("copy_buffer between different element types")
        _ffi.check(
            _ffi.lib().hx_copy_async(self.handle, src.ptr, len(src), dst.ptr, len(dst), src.itemsize, stream)
        )

    # -- synthetic inputs (RandomInitOps analog) -----------------------
    def fill_uniform_int(self, buffer: RocmBuffer, seed: int, lo: int, hi: int, stream=None) -> None:
        _ffi.check(
            _ffi.lib().hx_fill_random(
                self.handle, buffer.ptr, len(buffer), hx_dtype(buffer.dtype), _ffi.DIST_UNIFORM_INT,
                int(seed), float(lo), float(hi), stream,
            )
        )

    def fill_uniform_real(self, buffer: RocmBuffer, seed: int, lo: float, hi: float, stream=None) -> None:
        _ffi.check(
            _ffi.lib().hx_fill_random(
                self.handle, buffer.ptr, len(buffer), hx_dtype(buffer.dtype), _ffi.DIST_UNIFORM_REAL,
                int(seed), float(lo), float(hi), stream,
            )
        )

    def fill_normal(self, buffer: RocmBuffer, seed: int, mean: float = 0.0, std: float = 1.0, stream=None) -> None:
        _ffi.check(
            _ffi.lib().hx_fill_random(
                self.handle, buffer.ptr, len(buffer), hx_dtype(buffer.dtype), _ffi.DIST_NORMAL,
                int(seed), float(mean), float(std), stream,
            )
        )

    # -- DeviceApi (core accelerator/device_api.rs:69-133) --------------
    def compile_cached(self, key, entry: str, source):
        """Run-time compiled kernel cached under `key` (device_api.py)."""
        from . import device_api

        return device_api.compile_cached(self, key, entry, source)

    def launch(self, kernel, geometry, params=None, operands=(), stream=None) -> None:
        from . import device_api

        device_api.launch(self, kernel, geometry, params, operands, stream)

    @staticmethod
    def device_ptr(buffer) -> int:
        from . import device_api

        return device_api.device_ptr(buffer)

    @staticmethod
    def buffers_alias(lhs, rhs) -> bool:
        from . import device_api

        return device_api.buffers_alias(lhs, rhs)

    # -- events ---------------------------------------------------------
    def event(self) -> "Event":
        return Event(self)


class Event:
    """A HIP event recorded on a stream (timing of kernels on that stream)."""

    def __init__(self, device: RocmDevice):
        self.device = device
        ev = ctypes.c_void_p()
        _ffi.check(_ffi.lib().hx_event_create(device.handle, ctypes.byref(ev)))
        self.handle = ev.value

    def record(self, stream=None) -> None:
        _ffi.check(_ffi.lib().hx_event_record(self.device.handle, self.handle, stream))

    def synchronize(self) -> None:
        _ffi.check(_ffi.lib().hx_event_synchronize(self.handle))

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        _ffi.check(_ffi.lib().hx_event_elapsed_ms(self.handle, stop.handle, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            if self.handle:
                _ffi.lib().hx_event_destroy(self.handle)
        except Exception:
            pass
