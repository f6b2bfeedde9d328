"""hephaestus_amd — MI355X (gfx950) backend for Hephaestus's reduction / scan
path: full and row-wise reduce (sum, max, argmax, ...), inclusive and
exclusive prefix scans, segmented sum and the fused y = fmaf(a, x, b)
prologue, as hand-written HIP kernels behind the C ABI of include/hx.h.

This package is the Python host side of that ABI.  It has no compute path of
its own: every operation is a call into the native library, which must have
been built (`python -m hephaestus_amd.build`); importing an operation without
it raises ImportError.
"""
from . import _ffi, errors
from .device import (
    DeviceFeature,
    DeviceLimits,
    DevicePreference,
    Event,
    PlacementHint,
    RocmBuffer,
    RocmDevice,
    Topology,
)
from .device_api import LaunchGeometry, RocmCompiledKernel
from .errors import (
    AdapterUnavailable,
    AllocationFailed,
    DeviceUnavailable,
    DispatchFailed,
    HephaestusError,
    InvalidConfiguration,
    LengthMismatch,
    TransferFailed,
)
from .layout import Layout, StridedView
from .vector_ops import (
    PreparedMapReduction,
    RocmDenseVectorOps,
    dot,
    norm_l1,
    norm_l2,
    norm_max,
    prepare_dot,
    prepare_norm_l2,
    trace,
)
from .ops import (
    ArgMaxOp,
    CumProdOp,
    CumSumOp,
    MaxOp,
    MeanOp,
    MinOp,
    PreparedPlan,
    ProdOp,
    RocmAxisReductionOps,
    RocmFullReductionOps,
    RocmScanOps,
    RocmSegmentedReductionOps,
    ScanDirection,
    ScanKind,
    SumOp,
    plan_axis_reduction,
    plan_axis_scan,
    reduction_pass_count,
    submit_prepared_axis_reduction_batch,
    submit_prepared_reduction_batch,
    validate_reduction_width,
)

__all__ = [name for name in dir() if not name.startswith("_")]


def native_library_path():
    """Path of the native library this package calls."""
    return _ffi.LIB_PATH


def load_native():
    """Load (and return) the native library; raises if it is missing."""
    return _ffi.lib()
