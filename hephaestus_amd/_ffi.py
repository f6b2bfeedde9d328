"""ctypes binding of include/hx.h.

Loading fails loudly when the native library has not been built: there is no
Python or CPU fallback for any operation of this package.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import (
    POINTER,
    Structure,
    c_char,
    c_char_p,
    c_double,
    c_float,
    c_int32,
    c_uint32,
    c_uint64,
    c_void_p,
)
from pathlib import Path

from . import errors

LIB_PATH = Path(
    os.environ.get(
        "HEPHAESTUS_AMD_LIB",
        Path(__file__).resolve().parent / "lib" / "libhephaestus_amd.so",
    )
)

HX_MAX_RANK = 4

# hx_status
OK = 0
ADAPTER_UNAVAILABLE = 1
DEVICE_UNAVAILABLE = 2
ALLOCATION_FAILED = 3
LENGTH_MISMATCH = 4
DISPATCH_FAILED = 5
INVALID_CONFIGURATION = 6
TRANSFER_FAILED = 7

# hx_dtype
DTYPE_F32, DTYPE_U32, DTYPE_I32 = 0, 1, 2
# hx_op
OP_SUM, OP_PROD, OP_MIN, OP_MAX, OP_ARGMAX, OP_MEAN = 0, 1, 2, 3, 4, 5
# hx_scan_kind / hx_scan_direction
SCAN_INCLUSIVE, SCAN_EXCLUSIVE = 0, 1
SCAN_FORWARD, SCAN_REVERSE = 0, 1
# hx_distribution
DIST_UNIFORM_INT, DIST_UNIFORM_REAL, DIST_NORMAL = 0, 1, 2
MAP_SUM, MAP_DOT, MAP_NORM_L1, MAP_NORM_L2, MAP_NORM_MAX = 0, 1, 2, 3, 4
VEC_SCALE, VEC_AXPY, VEC_XPAY, VEC_ADD, VEC_SUB, VEC_MUL, VEC_DIV = 0, 1, 2, 3, 4, 5, 6


class HxLayout(Structure):
    _fields_ = [
        ("rank", c_uint32),
        ("reserved", c_uint32),
        ("shape", c_uint64 * HX_MAX_RANK),
        ("strides", ctypes.c_int64 * HX_MAX_RANK),
        ("offset", c_uint64),
    ]


class HxAffine(Structure):
    _fields_ = [("a", c_float), ("b", c_float), ("enabled", c_uint32), ("reserved", c_uint32)]


class HxDeviceLimits(Structure):
    _fields_ = [
        ("max_buffer_size", c_uint64),
        ("max_compute_workgroup_size_x", c_uint32),
        ("max_compute_workgroup_size_y", c_uint32),
        ("max_compute_workgroup_size_z", c_uint32),
        ("max_compute_invocations_per_workgroup", c_uint32),
        ("max_compute_workgroup_storage_size", c_uint32),
        ("max_immediate_size", c_uint32),
    ]


class HxDeviceInfo(Structure):
    _fields_ = [
        ("name", c_char * 96),
        ("arch", c_char * 64),
        ("ordinal", c_int32),
        ("compute_units", c_uint32),
        ("warp_size", c_uint32),
        ("max_threads_per_block", c_uint32),
        ("max_threads_per_cu", c_uint32),
        ("lds_bytes_per_block", c_uint32),
        ("regs_per_block", c_uint32),
        ("clock_khz", c_uint32),
        ("memory_clock_khz", c_uint32),
        ("memory_bus_width_bits", c_uint32),
        ("l2_bytes", c_uint64),
        ("total_memory_bytes", c_uint64),
        ("free_memory_bytes", c_uint64),
    ]


P = c_void_p
U64 = c_uint64
U32 = c_uint32
I32 = c_int32
LP = POINTER(HxLayout)
AP = POINTER(HxAffine)

# hx_kernel_source_fn: returns the address of NUL-terminated source text.
SOURCE_FN = ctypes.CFUNCTYPE(c_void_p, c_void_p)

# name -> (restype, argtypes); one entry per declaration in include/hx.h.
SIGNATURES = {
    "hx_abi_version": (U32, []),
    "hx_status_name": (c_char_p, [I32]),
    "hx_last_error_message": (c_char_p, []),
    "hx_last_length_mismatch": (None, [POINTER(U64), POINTER(U64)]),
    "hx_device_count": (I32, [POINTER(I32)]),
    "hx_device_open": (I32, [I32, POINTER(P)]),
    "hx_device_close": (I32, [P]),
    "hx_stream_release": (I32, [P, P]),
    "hx_device_get_info": (I32, [P, POINTER(HxDeviceInfo)]),
    "hx_device_stream": (I32, [P, POINTER(P)]),
    "hx_device_get_limits": (I32, [P, POINTER(HxDeviceLimits)]),
    "hx_device_supports_feature": (I32, [P, I32]),
    "hx_require_limits": (I32, [POINTER(HxDeviceLimits), POINTER(HxDeviceLimits)]),
    "hx_synchronize": (I32, [P]),
    "hx_alloc": (I32, [P, U64, U32, POINTER(P)]),
    "hx_free": (I32, [P, P]),
    "hx_upload": (I32, [P, P, U64, P, U64, U32]),
    "hx_write_sub": (I32, [P, P, U64, U64, P, U64, U32]),
    "hx_download": (I32, [P, P, U64, P, U64, U32]),
    "hx_copy": (I32, [P, P, U64, P, U64, U32]),
    "hx_copy_async": (I32, [P, P, U64, P, U64, U32, P]),
    "hx_event_create": (I32, [P, POINTER(P)]),
    "hx_event_destroy": (I32, [P]),
    "hx_event_record": (I32, [P, P, P]),
    "hx_event_synchronize": (I32, [P]),
    "hx_event_elapsed_ms": (I32, [P, P, POINTER(c_float)]),
    "hx_validate_reduction_width": (I32, [U32]),
    "hx_reduction_pass_count": (U64, [U64, U32]),
    "hx_layout_checked_size": (I32, [LP, POINTER(U64)]),
    "hx_layout_validate_storage_len": (I32, [LP, U64]),
    "hx_layout_has_zero_stride_aliasing": (I32, [LP]),
    "hx_plan_axis_reduction": (I32, [LP, U64, LP, U64, U32, U32, I32, POINTER(U64), POINTER(U64)]),
    "hx_plan_axis_scan": (I32, [LP, U64, LP, U64, U32, U32, I32, POINTER(U64), POINTER(U64)]),
    "hx_reduce_full": (I32, [P, I32, I32, P, U64, LP, P, U64, LP, AP, P]),
    "hx_argmax_full": (I32, [P, I32, P, U64, LP, P, P, AP, P]),
    "hx_prepare_reduce_full": (I32, [P, I32, I32, P, U64, LP, P, U64, LP, AP, POINTER(P)]),
    "hx_reduce_axis": (I32, [P, I32, I32, P, U64, LP, U32, P, U64, LP, P]),
    "hx_prepare_reduce_axis": (I32, [P, I32, I32, P, U64, LP, U32, P, U64, LP, POINTER(P)]),
    "hx_reduce_rows": (I32, [P, I32, P, U64, U64, U64, U64, U64, AP, P, P, P, U64, P]),
    "hx_prepare_reduce_rows": (I32, [P, I32, P, U64, U64, U64, U64, U64, AP, P, P, P, U64, POINTER(P)]),
    "hx_scan": (I32, [P, I32, I32, I32, I32, P, U64, LP, U32, P, U64, LP, P]),
    "hx_scan_noalloc": (I32, [P, I32, I32, I32, I32, P, U64, LP, U32, P, U64, LP, P]),
    "hx_noalloc_scratch_bytes": (U64, []),
    "hx_debug_set_wait_limits": (I32, [U32, U32]),
    "hx_debug_set_launch_count": (I32, [P, P, P, U64]),
    "hx_debug_tagged_word_hi": (U32, [U32, U32, U32]),
    "hx_debug_slot16_encode": (None, [U32, U32, U64, P]),
    "hx_debug_slot16_decode": (U32, [U32, P, P]),
    "hx_debug_copy_scan_shape": (I32, [P, P, P, U64, P]),
    "hx_prepare_scan": (I32, [P, I32, I32, I32, I32, P, U64, LP, U32, P, U64, LP, POINTER(P)]),
    "hx_segmented_reduce": (I32, [P, I32, I32, P, U64, P, U64, P, U64, P]),
    "hx_prepare_segmented_reduce": (I32, [P, I32, I32, P, U64, P, U64, P, U64, POINTER(P)]),
    "hx_validate_segment_offsets": (I32, [P, P, U64, U64]),
    "hx_map_reduce": (I32, [P, I32, I32, P, U64, LP, P, U64, LP, P, U64, P]),
    "hx_prepare_map_reduce": (I32, [P, I32, I32, P, U64, LP, P, U64, LP, P, U64, POINTER(P)]),
    "hx_trace": (I32, [P, I32, P, U64, LP, P, U64, P]),
    "hx_vector_update": (I32, [P, I32, I32, P, U64, P, U64, c_float, P]),
    "hx_vector_binary": (I32, [P, I32, I32, P, U64, P, U64, P, U64, P]),
    "hx_plan_dispatch": (I32, [P, P]),
    "hx_plan_dispatch_batch": (I32, [P, U64, P]),
    "hx_plan_destroy": (I32, [P]),
    "hx_plan_workspace_bytes": (I32, [P, POINTER(U64)]),
    "hx_fill_random": (I32, [P, P, U64, I32, I32, U64, c_double, c_double, P]),
    "hx_kernel_compile_cached": (I32, [P, P, U64, c_char_p, SOURCE_FN, P, POINTER(P)]),
    "hx_kernel_launch": (I32, [P, P, U32, U32, U32, P, U64, POINTER(P), U64, P]),
    "hx_buffers_alias": (I32, [P, U64, P, U64]),
}

_lib = None


def lib():
    """Load the native library once; raise if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"hephaestus_amd native library missing at {LIB_PATH}; "
                "build it with `python -m hephaestus_amd.build` (there is no fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_message() -> str:
    msg = lib().hx_last_error_message()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Raise the HephaestusError variant for a non-zero hx_status."""
    if status == OK:
        return
    msg = last_message()
    if status == LENGTH_MISMATCH:
        host = c_uint64()
        dev = c_uint64()
        lib().hx_last_length_mismatch(ctypes.byref(host), ctypes.byref(dev))
        raise errors.LengthMismatch(host.value, dev.value)
    cls = errors.BY_STATUS.get(status, errors.DispatchFailed)
    raise cls(msg)


def layout_struct(layout) -> HxLayout:
    rank = len(layout.shape)
    if rank < 1 or rank > HX_MAX_RANK:
        raise errors.DispatchFailed(f"layout rejected: rank {rank} is outside 1..={HX_MAX_RANK}")
    s = HxLayout()
    s.rank = rank
    for d in range(rank):
        s.shape[d] = int(layout.shape[d])
        s.strides[d] = int(layout.strides[d])
    s.offset = int(layout.offset)
    return s


def affine_struct(prologue) -> HxAffine | None:
    if prologue is None:
        return None
    a, b = prologue
    return HxAffine(float(a), float(b), 1, 0)
