"""The DeviceApi seam on the GPU: consumer kernels compiled at run time
(hipRTC), cached per device, launched with a parameter block and operands
(crates/hephaestus-core/src/domain/accelerator/device_api.rs:69-133; ROCm
crates/hephaestus-rocm/src/application/device_api.rs:49-103,
pipeline.rs:175-349).  Integer kernels, so every check is bit-exact."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import hephaestus_amd as hx
from hephaestus_amd import LaunchGeometry

pytestmark = pytest.mark.gpu

AFFINE_SRC = r"""
struct AffineParams { unsigned int n; unsigned int mul; unsigned int add; unsigned int pad; };
extern "C" __global__ void affine_u32(AffineParams p, const unsigned int *x, unsigned int *y) {
    unsigned int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) y[i] = x[i] * p.mul + p.add;
}
"""


class AffineParams(ctypes.Structure):
    _fields_ = [("n", ctypes.c_uint32), ("mul", ctypes.c_uint32), ("add", ctypes.c_uint32),
                ("pad", ctypes.c_uint32)]


def test_compile_launch_and_cache(device):
    calls = []

    def source():
        calls.append(1)
        return AFFINE_SRC

    k1 = device.compile_cached(b"test-affine", "affine_u32", source)
    k2 = device.compile_cached(b"test-affine", "affine_u32", source)
    assert k1 == k2 and len(calls) == 1, "a cache hit must not ask for the source"
    n = 100_003
    x = np.arange(n, dtype=np.uint32) * np.uint32(2654435761)
    xb, yb = device.upload(x), device.alloc_zeroed(np.uint32, n)
    geom = LaunchGeometry.linear((n + 255) // 256, 256)
    device.launch(k1, geom, AffineParams(n, 0x9E3779B9, 12345, 0), [xb, yb])
    device.synchronize()
    want = (x * np.uint32(0x9E3779B9) + np.uint32(12345)).astype(np.uint32)
    assert np.array_equal(device.download_owned(yb), want)
    # A parameter block given as bytes is the same block.
    raw = np.array([n, 3, 7, 0], dtype=np.uint32).tobytes()
    device.launch(k1, geom, raw, [xb, yb])
    device.synchronize()
    assert np.array_equal(device.download_owned(yb), (x * np.uint32(3) + np.uint32(7)).astype(np.uint32))
    # Another key compiles again.
    k3 = device.compile_cached(b"test-affine-2", "affine_u32", source)
    assert k3 != k1 and len(calls) == 2


def test_failed_compilation_reports_the_log_and_is_not_cached(device):
    with pytest.raises(hx.DispatchFailed) as info:
        device.compile_cached(b"test-broken", "broken", lambda: 'extern "C" __global__ void broken( { }')
    assert "hiprtcCompileProgram" in str(info.value)
    k = device.compile_cached(b"test-broken", "affine_u32", lambda: AFFINE_SRC)
    assert k.handle


def test_missing_entry_and_source_errors(device):
    with pytest.raises(hx.DispatchFailed, match="hipModuleGetFunction"):
        device.compile_cached(b"test-missing-entry", "no_such_kernel", lambda: AFFINE_SRC)

    def bad_source():
        raise ValueError("no source today")

    with pytest.raises(ValueError, match="no source today"):
        device.compile_cached(b"test-source-raises", "affine_u32", bad_source)
    # Neither failure was cached.
    assert device.compile_cached(b"test-missing-entry", "affine_u32", lambda: AFFINE_SRC).handle
    assert device.compile_cached(b"test-source-raises", "affine_u32", lambda: AFFINE_SRC).handle
    # A failed runtime call leaves no error behind for the library's next
    # launch (HIP also records it as the thread's last error).
    with pytest.raises(hx.DispatchFailed, match="hipModuleGetFunction"):
        device.compile_cached(b"test-missing-entry-2", "no_such_kernel", lambda: AFFINE_SRC)
    x = np.arange(70_000, dtype=np.uint32)
    xb, yb = device.upload(x), device.alloc_zeroed(np.uint32, x.size)
    lay = hx.Layout.c_contiguous([x.size])
    hx.RocmScanOps().scan_axis_into(device, hx.CumSumOp, hx.StridedView(xb, lay), 0, hx.ScanDirection.Forward,
                                    hx.StridedView(yb, lay))
    assert np.array_equal(device.download_owned(yb), np.cumsum(x, dtype=np.uint32))


MIXED_SRC = r"""
struct Mixed { unsigned long long tag; unsigned int n; float scale; int bias; unsigned int lanes; };
extern "C" __global__ void mixed(Mixed p, const unsigned int *a, const unsigned int *b, unsigned int *out,
                                 unsigned long long *echo) {
    unsigned int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) out[i] = a[i] ^ (b[i] + (unsigned int)p.bias);
    if (i == 0) {
        echo[0] = p.tag;
        echo[1] = (unsigned long long)__float_as_uint(p.scale);
        echo[2] = (unsigned long long)p.lanes;
        echo[3] = (unsigned long long)blockDim.x * gridDim.x;
    }
}
"""


class Mixed(ctypes.Structure):
    _fields_ = [("tag", ctypes.c_uint64), ("n", ctypes.c_uint32), ("scale", ctypes.c_float),
                ("bias", ctypes.c_int32), ("lanes", ctypes.c_uint32)]


def test_parameter_block_by_value_with_several_operands(device):
    k = device.compile_cached(b"test-mixed", "mixed", lambda: MIXED_SRC)
    n = 5000
    rng = np.random.default_rng(3)
    a = rng.integers(0, 2**32, n, dtype=np.uint32)
    b = rng.integers(0, 2**32, n, dtype=np.uint32)
    ab, bb = device.upload(a), device.upload(b)
    out = device.alloc_zeroed(np.uint32, n)
    echo = device.alloc_zeroed(np.uint32, 8)  # four u64 words
    geom = LaunchGeometry.linear(40, 128)
    device.launch(k, geom, Mixed(0x0123456789ABCDEF, n, 1.5, -7, 128), [ab, bb, out, echo])
    device.synchronize()
    assert np.array_equal(device.download_owned(out), a ^ (b + np.uint32(2**32 - 7)))
    words = device.download_owned(echo).view(np.uint64)
    assert words[0] == 0x0123456789ABCDEF
    assert words[1] == np.float32(1.5).view(np.uint32)
    assert words[2] == 128 and words[3] == 40 * 128


REVERSE_SRC = r"""
extern "C" __global__ void reverse_blocks(unsigned int n, const unsigned int *x, unsigned int *y) {
    extern __shared__ unsigned int tile[];
    unsigned int base = blockIdx.x * blockDim.x, t = threadIdx.x;
    tile[t] = base + t < n ? x[base + t] : 0u;
    __syncthreads();
    unsigned int r = blockDim.x - 1 - t;
    if (base + t < n) y[base + t] = tile[r];
}
"""


def test_dynamic_shared_memory_and_caller_stream(device):
    k = device.compile_cached(b"test-reverse", "reverse_blocks", lambda: REVERSE_SRC)
    width, groups = 256, 64
    n = width * groups
    x = np.arange(n, dtype=np.uint32)
    xb, yb = device.upload(x), device.alloc_zeroed(np.uint32, n)
    hip = ctypes.CDLL("libamdhip64.so")
    stream = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    try:
        device.launch(k, LaunchGeometry.linear_shared(groups, width, width * 4), np.uint32(n).tobytes(), [xb, yb],
                      stream=stream.value)
        assert hip.hipStreamSynchronize(stream) == 0
    finally:
        hip.hipStreamDestroy(stream)
    assert np.array_equal(device.download_owned(yb), x.reshape(groups, width)[:, ::-1].ravel())


SCAN_SRC = r"""
// A consumer-authored line scan: one block per line of a row-major
// [lines, len] u32 matrix, walking the line in blockDim-wide windows; each
// window is scanned in LDS by doubling strides (Hillis-Steele) and offset by
// the running total of the windows before it.
struct LineScan { unsigned int lines; unsigned int len; };
extern "C" __global__ void line_scan(LineScan p, const unsigned int *in, unsigned int *out) {
    extern __shared__ unsigned int win[];
    const unsigned int line = blockIdx.x, w = blockDim.x, t = threadIdx.x;
    if (line >= p.lines) return;
    const unsigned int *src = in + (unsigned long long)line * p.len;
    unsigned int *dst = out + (unsigned long long)line * p.len;
    unsigned int carry = 0;
    for (unsigned int base = 0; base < p.len; base += w) {
        unsigned int v = base + t < p.len ? src[base + t] : 0u;
        win[t] = v;
        __syncthreads();
        for (unsigned int d = 1; d < w; d <<= 1) {
            unsigned int add = t >= d ? win[t - d] : 0u;
            __syncthreads();
            win[t] += add;
            __syncthreads();
        }
        if (base + t < p.len) dst[base + t] = carry + win[t];
        carry += win[w - 1];
        __syncthreads();
    }
}
"""


class LineScan(ctypes.Structure):
    _fields_ = [("lines", ctypes.c_uint32), ("len", ctypes.c_uint32)]


@pytest.mark.parametrize("lines,length", [(1, 1), (3, 1000), (37, 4099), (256, 777)])
def test_consumer_line_scan_matches_the_oracle(device, oracle, lines, length):
    k = device.compile_cached(b"test-line-scan", "line_scan", lambda: SCAN_SRC)
    x = oracle.uniform_int(lines * length, seed=lines + length, lo=0, hi=2**32 - 1)
    xb, yb = device.upload(x), device.alloc_zeroed(np.uint32, lines * length)
    width = 128
    device.launch(k, LaunchGeometry.linear_shared(lines, width, width * 4), LineScan(lines, length), [xb, yb])
    device.synchronize()
    got = device.download_owned(yb).reshape(lines, length)
    for r in range(lines):
        assert np.array_equal(got[r], oracle.scan_sum(x[r * length:(r + 1) * length]))
    # The library's own scan agrees with the consumer kernel.
    lay = hx.Layout.c_contiguous([lines, length])
    zb = device.alloc_zeroed(np.uint32, lines * length)
    hx.RocmScanOps().scan_axis_into(device, hx.CumSumOp, hx.StridedView(xb, lay), 1, hx.ScanDirection.Forward,
                                    hx.StridedView(zb, lay))
    assert np.array_equal(device.download_owned(zb).reshape(lines, length), got)


def test_launch_validation(device):
    k = device.compile_cached(b"test-affine", "affine_u32", lambda: AFFINE_SRC)
    with pytest.raises(hx.InvalidConfiguration):
        LaunchGeometry(1, 0)
    lib = hx._ffi.lib()
    status = lib.hx_kernel_launch(device.handle, k.handle, 1, 0, 0, None, 0, None, 0, None)
    assert status == hx._ffi.INVALID_CONFIGURATION
    status = lib.hx_kernel_launch(device.handle, None, 1, 64, 0, None, 0, None, 0, None)
    assert status == hx._ffi.INVALID_CONFIGURATION
    with pytest.raises(hx.InvalidConfiguration, match="argument segment"):
        device.launch(k, LaunchGeometry.linear(1, 64), bytes(8192), [])


def test_buffers_alias(device):
    a = device.alloc_zeroed(np.uint32, 1024)
    b = device.alloc_zeroed(np.uint32, 1024)
    assert hx.RocmDevice.buffers_alias(a, a)
    assert not hx.RocmDevice.buffers_alias(a, b)
    assert hx.RocmDevice.device_ptr(a) == a.ptr


def test_concurrent_compiles_of_one_key_share_one_kernel(device):
    """Threads racing to compile the same key all get the one cached kernel
    (the loser of the race unloads its own module)."""
    import threading

    start = threading.Barrier(4)
    handles, errors_seen = [], []

    def work():
        try:
            start.wait()
            handles.append(device.compile_cached(b"test-race", "affine_u32", lambda: AFFINE_SRC).handle)
        except Exception as exc:
            errors_seen.append(exc)

    threads = [threading.Thread(target=work) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors_seen, errors_seen
    assert len(handles) == 4 and len(set(handles)) == 1
    # and the kernel works
    n = 4096
    x = np.arange(n, dtype=np.uint32)
    xb, yb = device.upload(x), device.alloc_zeroed(np.uint32, n)
    device.launch(hx.RocmCompiledKernel(device, handles[0], b"test-race", "affine_u32"),
                  LaunchGeometry.linear(n // 256, 256), AffineParams(n, 2, 1, 0), [xb, yb])
    device.synchronize()
    assert np.array_equal(device.download_owned(yb), x * np.uint32(2) + np.uint32(1))


def test_capabilities_and_acquisition(device):
    """ComputeDeviceCapabilities and ComputeDeviceAcquisition (ROCm
    capabilities.rs:5-21, acquisition.rs:8-35, query.rs:28-101)."""
    lim = device.device_limits()
    topo = device.topology()
    assert lim.max_compute_invocations_per_workgroup == topo.max_threads_per_block == 1024
    assert lim.max_compute_workgroup_size_x == 1024
    assert lim.max_compute_workgroup_size_y >= 1 and lim.max_compute_workgroup_size_z >= 1
    assert lim.max_compute_workgroup_storage_size >= 65536
    assert 0 < lim.max_buffer_size <= topo.total_memory_bytes
    assert lim.max_immediate_size == 0
    assert lim.max_storage_buffers_per_shader_stage is None
    for f in hx.DeviceFeature:
        assert device.supports_device_feature(f) is False
    d2 = hx.RocmDevice.try_acquire_device("test", hx.DevicePreference.HighPerformance, [],
                                          hx.DeviceLimits(max_compute_invocations_per_workgroup=1024))
    d2.close()
    with pytest.raises(hx.DeviceUnavailable, match="max_compute_invocations_per_workgroup 1024 is below required 2048"):
        hx.RocmDevice.try_acquire_device("test", hx.DevicePreference.LowPower, [hx.DeviceFeature.ShaderF64],
                                         hx.DeviceLimits(max_compute_invocations_per_workgroup=2048))
    devices = hx.RocmDevice.try_acquire_devices("test", 8)
    assert 1 <= len(devices) <= hx.RocmDevice.device_count()
    for d in devices:
        d.close()


def test_allocation_with_placement_hints(device):
    """alloc_*_with_hint / upload_with_hint (core device.rs:103-143): every
    hint gives device memory, a budget-only tier is AllocationFailed (ROCm
    device.rs:167-185)."""
    for hint in (hx.PlacementHint.current(), hx.PlacementHint.any(), hx.PlacementHint.numa(0),
                 hx.PlacementHint.domain("gpu0"), hx.PlacementHint.tier("Device")):
        b = device.alloc_zeroed_with_hint(np.uint32, 17, hint)
        assert np.array_equal(device.download_owned(b), np.zeros(17, np.uint32))
        u = device.upload_with_hint(np.arange(5, dtype=np.float32), hint)
        assert np.array_equal(device.download_owned(u), np.arange(5, dtype=np.float32))
        assert len(device.alloc_uninitialized_with_hint(np.int32, 3, hint)) == 3
    with pytest.raises(hx.AllocationFailed, match="budget-only tier Pooled"):
        device.alloc_zeroed_with_hint(np.uint32, 4, hx.PlacementHint.tier("Pooled", host_allocatable=False))
