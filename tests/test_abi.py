"""The C-ABI boundary without a GPU: the library loads, exports every entry
point include/hx.h declares, and its host-side planners reproduce the
reference planners' results and messages (crates/hephaestus-core/src/
domain/reduction.rs:339-570, scan.rs:87-344).  CPU only."""
from __future__ import annotations

import ctypes
import json
import re
import subprocess
from pathlib import Path

import pytest

import hephaestus_amd as hx
from hephaestus_amd import _ffi

REPO = Path(__file__).resolve().parent.parent
KATS = json.loads((REPO / "tests" / "golden" / "reference_kats.json").read_text())
MSG = KATS["messages"]


def declared_symbols() -> set[str]:
    text = (REPO / "include" / "hx.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _ffi.LIB_PATH
    assert lib.exists(), "native library not built"
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = declared_symbols()
    assert len(declared) >= 40
    assert declared <= exported, sorted(declared - exported)


def test_ctypes_signatures_cover_the_header():
    assert declared_symbols() == set(_ffi.SIGNATURES)
    hx.load_native()  # every signature resolves


def test_library_embeds_gfx950_code_objects_only():
    blob = _ffi.LIB_PATH.read_bytes()  # the library built in this tree
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"--gfx942", b"--gfx90a", b"--gfx1100"):
        assert other not in blob


def test_abi_version_and_status_names():
    lib = hx.load_native()
    assert lib.hx_abi_version() == 1
    names = [lib.hx_status_name(i).decode() for i in range(8)]
    assert names == ["Ok", "AdapterUnavailable", "DeviceUnavailable", "AllocationFailed",
                     "LengthMismatch", "DispatchFailed", "InvalidConfiguration", "TransferFailed"]


def test_device_acquisition_without_gpu_is_adapter_unavailable():
    if hx.RocmDevice.device_count() > 0:
        pytest.skip("a GPU is present")
    with pytest.raises(hx.AdapterUnavailable) as err:
        hx.RocmDevice.try_default()
    assert "ROCm device ordinal 0 unavailable; device count 0" in str(err.value)


# ------------------------------------------------------------------ planners
def test_reduction_pass_count_matches_reference_table():
    for n, want in KATS["planner"]["pass_count_w256"]:
        assert hx.reduction_pass_count(n, 256) == want
    for n, want in KATS["planner"]["pass_count_w128"]:
        assert hx.reduction_pass_count(n, 128) == want


def test_reduction_width_must_be_power_of_two():
    hx.validate_reduction_width(128)
    with pytest.raises(hx.DispatchFailed) as err:
        hx.validate_reduction_width(192)
    assert err.value.message == MSG["width_192"]


L = hx.Layout.c_contiguous


def test_plan_axis_reduction_dense_and_empty():
    # reduction.rs:510-521 and :539-545
    assert hx.plan_axis_reduction(L([3, 4]), 12, L([3, 1]), 3, 1) == (3, 4)
    assert hx.plan_axis_reduction(L([0, 4]), 0, L([0, 1]), 0, 1) == (0, 4)


def test_plan_axis_reduction_rejections():
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([3, 4]), 12, L([3, 4]), 12, 1)
    assert e.value.message.startswith(MSG["axis_shape_prefix"])
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([2, 2]), 4, L([1, 2]), 2, 0, buffers_alias=True)
    assert e.value.message == MSG["axis_alias"]
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([2, 2]), 4, L([1, 2]), 2, 2)
    assert e.value.message == "axis 2 is out of bounds for rank-2 reduction"
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([3, 4]), 12, L([3, 1]), 3, 1, width=192)
    assert e.value.message == MSG["width_192"]
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([2, 2]), 4, hx.Layout.try_new([1, 2], [0, 0]), 2, 0)
    assert "zero-stride aliasing" in e.value.message
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_reduction(L([3, 4]), 11, L([3, 1]), 3, 1)
    assert e.value.message.startswith("layout rejected:")


def test_plan_axis_scan_matches_reference_planner_tests():
    # scan.rs:278-343
    assert hx.plan_axis_scan(L([3, 4]), 12, L([3, 4]), 12, 1) == (3, 4)
    assert hx.plan_axis_scan(L([2, 5]), 10, L([2, 5]), 10, 0) == (5, 2)
    assert hx.plan_axis_scan(L([0, 4]), 0, L([0, 4]), 0, 1)[0] == 0
    assert hx.plan_axis_scan(L([3, 1024]), 3072, L([3, 1024]), 3072, 1) == (3, 1024)
    assert hx.plan_axis_scan(L([100]), 100, L([100]), 100, 0) == (1, 100)
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_scan(L([2, 2]), 4, L([2, 2]), 4, 0, buffers_alias=True)
    assert e.value.message == MSG["scan_alias"]
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_scan(L([2, 2]), 4, L([2, 2]), 4, 0, width=3)
    assert e.value.message == "scan block width 3 must be a power of two"
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_scan(L([2, 4]), 8, L([4, 2]), 8, 1)
    assert e.value.message.startswith(MSG["scan_shape_prefix"])
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_scan(L([3, 4]), 12, L([3, 4]), 12, 2)
    assert e.value.message == "scan axis 2 is out of bounds for rank-2 scan"
    with pytest.raises(hx.DispatchFailed) as e:
        hx.plan_axis_scan(L([2, 2, 2]), 8, L([2, 2, 2]), 8, 0)
    assert "rank 1 and 2 only" in e.value.message


def test_layout_queries():
    assert L([3, 4]).checked_size() == 12
    assert L([0, 4]).checked_size() == 0
    t = hx.Layout.try_new([4, 3], [1, 4], 0)
    t.validate_storage_len(12)
    with pytest.raises(hx.DispatchFailed):
        t.validate_storage_len(11)
    d = hx.Layout.try_new([3], [4], 0)  # the diagonal view of a 3x3
    d.validate_storage_len(9)
    neg = hx.Layout.try_new([3], [-1], 2)
    neg.validate_storage_len(3)
    with pytest.raises(hx.DispatchFailed):
        hx.Layout.try_new([3], [-1], 1).validate_storage_len(3)
    assert hx.Layout.try_new([2, 2], [0, 1]).has_zero_stride_aliasing()
    assert not hx.Layout.try_new([1, 2], [0, 1]).has_zero_stride_aliasing()
    with pytest.raises(hx.DispatchFailed):
        hx.Layout.try_new([2**40, 2**40], [1, 1]).checked_size()


def test_length_mismatch_carries_both_lengths():
    err = hx.LengthMismatch(3, 4)
    assert (err.host_len, err.device_len) == (3, 4)
    assert str(err) == "host length 3 does not match device buffer length 4"
    assert issubclass(hx.DispatchFailed, hx.HephaestusError)


def test_null_device_handles_are_rejected_on_the_host():
    lib = hx.load_native()
    st = lib.hx_synchronize(None)
    assert st == _ffi.INVALID_CONFIGURATION
    assert _ffi.last_message() == "null device handle"
    out = ctypes.c_void_p()
    assert lib.hx_alloc(None, 16, 1, ctypes.byref(out)) == _ffi.INVALID_CONFIGURATION


def test_transfer_byte_counts_that_overflow_are_rejected_on_the_host():
    lib = hx.load_native()
    n = 1 << 62
    for fn in (lib.hx_upload, lib.hx_download, lib.hx_copy):
        assert fn(None, 0x1000, n, 0x2000, n, 8) == _ffi.INVALID_CONFIGURATION
        assert _ffi.last_message() == f"{n} elements of 8 bytes exceed the address range"
    assert lib.hx_write_sub(None, 0x1000, n + 1, 1, 0x2000, n, 8) == _ffi.INVALID_CONFIGURATION


def test_batch_submission_checks_its_arguments_on_the_host():
    """hx_plan_dispatch_batch rejects a null array or a null entry before any
    plan runs; an empty batch is a no-op."""
    lib = hx.load_native()
    assert lib.hx_plan_dispatch_batch(None, 0, None) == _ffi.OK
    assert lib.hx_plan_dispatch_batch(None, 2, None) == _ffi.INVALID_CONFIGURATION
    assert _ffi.last_message() == "null plan array"
    arr = (ctypes.c_void_p * 3)(None, None, None)
    assert lib.hx_plan_dispatch_batch(arr, 3, None) == _ffi.INVALID_CONFIGURATION
    assert _ffi.last_message() == "null plan at batch index 0"


def test_entry_points_validate_before_touching_the_device():
    """Every device entry point rejects a bad operand before it needs the
    device, so these run without a GPU (and leave outputs untouched)."""
    lib = hx.load_native()
    lay = _ffi.layout_struct(L([3, 4]))
    out2 = _ffi.layout_struct(L([2]))
    st = lib.hx_reduce_full(None, _ffi.OP_SUM, _ffi.DTYPE_F32, 0x1000, 12, ctypes.byref(lay),
                            0x2000, 2, ctypes.byref(out2), None, None)
    assert st == _ffi.DISPATCH_FAILED and _ffi.last_message() == MSG["full_multi_output"]
    scan_lay = _ffi.layout_struct(L([3, 4]))
    st = lib.hx_scan(None, _ffi.OP_SUM, _ffi.DTYPE_F32, 0, 0, 0x1000, 12, ctypes.byref(scan_lay), 2,
                     0x2000, 12, ctypes.byref(scan_lay), None)
    assert st == _ffi.DISPATCH_FAILED
    assert _ffi.last_message() == "scan axis 2 is out of bounds for rank-2 scan"
    st = lib.hx_scan(None, _ffi.OP_MAX, _ffi.DTYPE_F32, 0, 0, 0x1000, 12, ctypes.byref(scan_lay), 1,
                     0x2000, 12, ctypes.byref(scan_lay), None)
    assert st == _ffi.DISPATCH_FAILED and "CumSumOp" in _ffi.last_message()
    empty = _ffi.layout_struct(hx.Layout.c_contiguous([3, 0]))
    out31 = _ffi.layout_struct(hx.Layout.c_contiguous([3, 1]))
    st = lib.hx_reduce_axis(None, _ffi.OP_MEAN, _ffi.DTYPE_U32, None, 0, ctypes.byref(empty), 1,
                            0x2000, 3, ctypes.byref(out31), None)
    assert st == _ffi.DISPATCH_FAILED and _ffi.last_message() == MSG["mean_empty_axis1"]
    st = lib.hx_reduce_axis(None, _ffi.OP_SUM, _ffi.DTYPE_U32, 0x1000, 12, ctypes.byref(lay), 1,
                            0x1000, 3, ctypes.byref(out31), None)
    assert st == _ffi.DISPATCH_FAILED and _ffi.last_message() == MSG["axis_alias"]
    st = lib.hx_segmented_reduce(None, _ffi.OP_SUM, _ffi.DTYPE_I32, 0x1000, 10, 0x2000, 4, 0x3000, 2, None)
    assert st == _ffi.LENGTH_MISMATCH
    aff = _ffi.HxAffine(0.5, 0.25, 1, 0)
    st = lib.hx_reduce_full(None, _ffi.OP_SUM, _ffi.DTYPE_U32, 0x1000, 12, ctypes.byref(lay),
                            0x2000, 1, ctypes.byref(_ffi.layout_struct(L([1]))), ctypes.byref(aff), None)
    assert st == _ffi.INVALID_CONFIGURATION and "f32" in _ffi.last_message()


def test_integer_mean_counts_beyond_the_divisor_type_are_rejected():
    """An integer mean divides in the element type (the reference's
    `acc / (T)axis_len`); counts the type cannot hold are rejected on the
    host, before the device is touched, instead of being truncated.  Counts
    that fit reach the device step (here: the null device handle)."""
    lib = hx.load_native()
    one = ctypes.byref(_ffi.layout_struct(L([1])))
    cases = [(_ffi.DTYPE_I32, 2**31, "i32 divisor"), (_ffi.DTYPE_U32, 2**32, "u32 divisor")]
    for dtype, n, text in cases:
        lay = ctypes.byref(_ffi.layout_struct(L([n])))
        st = lib.hx_reduce_full(None, _ffi.OP_MEAN, dtype, 0x1000, n, lay, 0x2000, 1, one, None, None)
        assert st == _ffi.DISPATCH_FAILED and text in _ffi.last_message(), _ffi.last_message()
        fits = ctypes.byref(_ffi.layout_struct(L([n - 1])))
        st = lib.hx_reduce_full(None, _ffi.OP_MEAN, dtype, 0x1000, n - 1, fits, 0x2000, 1, one, None, None)
        assert st == _ffi.INVALID_CONFIGURATION and _ffi.last_message() == "null device handle"
        # axis form: 2 rows of n elements reduced along axis 1
        rows = ctypes.byref(_ffi.layout_struct(L([2, n])))
        out = ctypes.byref(_ffi.layout_struct(L([2, 1])))
        st = lib.hx_reduce_axis(None, _ffi.OP_MEAN, dtype, 0x1000, 2 * n, rows, 1, 0x2000, 2, out, None)
        assert st == _ffi.DISPATCH_FAILED and text in _ffi.last_message(), _ffi.last_message()
    # f32 means divide in f64: no such limit
    lay = ctypes.byref(_ffi.layout_struct(L([2**33])))
    st = lib.hx_reduce_full(None, _ffi.OP_MEAN, _ffi.DTYPE_F32, 0x1000, 2**33, lay, 0x2000, 1, one, None, None)
    assert st == _ffi.INVALID_CONFIGURATION and _ffi.last_message() == "null device handle"


def test_buffers_alias_rule():
    """hx_buffers_alias: one non-null base (the reference's rule, rocm
    buffer.rs:47-49) or overlapping byte ranges; null never aliases."""
    lib = hx.load_native()
    assert lib.hx_buffers_alias(0x1000, 64, 0x1000, 64) == 1
    assert lib.hx_buffers_alias(0x1000, 0, 0x1000, 0) == 1
    assert lib.hx_buffers_alias(0x1000, 64, 0x1040, 64) == 0  # adjacent
    assert lib.hx_buffers_alias(0x1000, 65, 0x1040, 64) == 1  # one byte of overlap
    assert lib.hx_buffers_alias(0x1040, 64, 0x1000, 65) == 1
    assert lib.hx_buffers_alias(None, 64, None, 64) == 0
    assert lib.hx_buffers_alias(None, 64, 0x1000, 64) == 0


def test_device_api_rejects_null_handles_before_the_device():
    """The DeviceApi entry points check their handles before any HIP call,
    so these run without a GPU; the source callback is never reached."""
    lib = hx.load_native()
    calls = []

    def provide(_ctx):
        calls.append(1)
        return None

    cb = _ffi.SOURCE_FN(provide)
    out = ctypes.c_void_p(1)
    st = lib.hx_kernel_compile_cached(None, b"k", 1, b"entry", cb, None, ctypes.byref(out))
    assert st == _ffi.INVALID_CONFIGURATION and _ffi.last_message() == "null device handle"
    assert out.value is None and not calls
    st = lib.hx_kernel_launch(None, None, 1, 64, 0, None, 0, None, 0, None)
    assert st == _ffi.INVALID_CONFIGURATION and _ffi.last_message() == "null kernel handle"
    with pytest.raises(hx.InvalidConfiguration):
        hx.LaunchGeometry.linear(4, 0)
    g = hx.LaunchGeometry.linear_shared(4, 64, 256)
    assert (g.groups, g.width, g.shared_bytes) == (4, 64, 256)


def test_require_limits_messages():
    """require_limits (ROCm device.rs:187-238): the first field short of the
    requirement, in DeviceLimits order, is DeviceUnavailable with the
    reference's message; equal values satisfy."""
    have = hx.DeviceLimits(max_buffer_size=100, max_compute_workgroup_size_x=1024, max_compute_workgroup_size_y=1024,
                           max_compute_workgroup_size_z=1024, max_compute_invocations_per_workgroup=1024,
                           max_compute_workgroup_storage_size=65536, max_immediate_size=0)
    hx.RocmDevice.require_limits(have, have)
    hx.RocmDevice.require_limits(have, hx.DeviceLimits())
    with pytest.raises(hx.DeviceUnavailable) as info:
        hx.RocmDevice.require_limits(have, hx.DeviceLimits(max_buffer_size=200, max_immediate_size=4))
    assert _ffi.last_message() == "ROCm device limit max_buffer_size 100 is below required 200"
    with pytest.raises(hx.DeviceUnavailable):
        hx.RocmDevice.require_limits(have, hx.DeviceLimits(max_compute_invocations_per_workgroup=2048))
    assert _ffi.last_message() == "ROCm device limit max_compute_invocations_per_workgroup 1024 is below required 2048"
    with pytest.raises(hx.DeviceUnavailable):
        hx.RocmDevice.require_limits(have, hx.DeviceLimits(max_immediate_size=1))
    assert _ffi.last_message() == "ROCm device limit max_immediate_size 0 is below required 1"
    assert "below required" in str(info.value)


def test_partial_slots_never_match_lookback_status_words():
    """Look-back statuses (flag 1 aggregate, 2 inclusive prefix) and the
    partial slots of the one-launch reductions share a workspace region and
    one tag counter.  Through the library's own encoders: a slot word of any
    tag never equals a status word of any tag (the slot layout carries flag
    3), and within each kind distinct tags give distinct words.  Checked for
    every tag of the eager range [1, 2^14 - 1) and the reserved captured tag
    (2^14 - 1)."""
    lib = hx.load_native()
    tags = list(range(1, 1 << 14))
    slot = {lib.hx_debug_tagged_word_hi(1, t, 0): t for t in tags}
    agg = {lib.hx_debug_tagged_word_hi(0, t, 1): t for t in tags}
    pre = {lib.hx_debug_tagged_word_hi(0, t, 2): t for t in tags}
    for words in (slot, agg, pre):
        assert len(words) == len(tags)          # injective in the tag
        assert 0 not in words                   # zeroed memory is never current
    assert not (set(slot) & set(agg)), "a slot word equals an aggregate status word"
    assert not (set(slot) & set(pre)), "a slot word equals a prefix status word"
    assert not (set(agg) & set(pre))
    # The collision the old slot layout had: a slot of tag 4t + f read a
    # status word of tag t with flag f.
    for t in (1, 2, 1000, (1 << 12) - 1):
        for f in (1, 2):
            assert lib.hx_debug_tagged_word_hi(1, 4 * t + f, 0) != lib.hx_debug_tagged_word_hi(0, t, f)
    # Every high half of the 64-bit formats stays below 2^16: no dword of them
    # can pass for a check dword of the f32 scan slots (>= 2^18).
    assert max(max(slot), max(agg), max(pre)) < (1 << 16)


def test_captured_and_eager_tags_are_disjoint_in_status_words():
    """The tag reserved for captured dispatches (2^14 - 1) encodes to words
    that no eager tag in [1, 2^14 - 1) produces."""
    lib = hx.load_native()
    cap = 0x3FFF
    captured = {lib.hx_debug_tagged_word_hi(0, cap, f) for f in (1, 2)} | {lib.hx_debug_tagged_word_hi(1, cap, 0)}
    for t in range(1, cap):
        eager = {lib.hx_debug_tagged_word_hi(0, t, f) for f in (1, 2)} | {lib.hx_debug_tagged_word_hi(1, t, 0)}
        assert not (eager & captured)


def _slot16(lib, tag, flag, bits):
    out = (ctypes.c_uint32 * 4)()
    lib.hx_debug_slot16_encode(tag, flag, bits, out)
    return list(out)


def _unslot16(lib, tag, dwords):
    q = (ctypes.c_uint32 * 4)(*dwords)
    b = ctypes.c_uint64()
    f = lib.hx_debug_slot16_decode(tag, q, ctypes.byref(b))
    return f, b.value


def test_f32_scan_slots_round_trip_and_reject_torn_reads():
    """The 16-byte status slot of the f32 scans (f64 carries), through the
    library's own codec.  An aggregate or prefix written with tag t reads
    back bit-exact under tag t and as not ready under any other tag.  A read
    that mixes dwords of the two writes of one launch (aggregate, then
    prefix), of an earlier launch's slot, of zeroed memory or of the 64-bit
    status / partial-slot words that share the area is never accepted: the
    slot needs only 32-bit single-copy atomicity."""
    import itertools
    import struct

    lib = hx.load_native()
    vals = [0.0, -0.0, 1.0, -3.5, 2.0 ** 40 + 0.25, 5e-324, float("inf"), float("-inf"), float("nan"),
            123456.789, -1e300]
    bits = [struct.unpack("<Q", struct.pack("<d", v))[0] for v in vals] + [0x0123456789ABCDEF, 0xFFFFFFFFFFFFFFFF]
    tags = [1, 2, 3, 4, 5, 255, 256, 4096, (1 << 14) - 2, (1 << 14) - 1]
    for t in tags:
        for f in (1, 2):
            for b in bits:
                assert _unslot16(lib, t, _slot16(lib, t, f, b)) == (f, b)
                for other in (t - 1, t + 1, t ^ 1):
                    if 1 <= other < (1 << 14) and other != t:
                        assert _unslot16(lib, other, _slot16(lib, t, f, b))[0] == 0
    # Torn mixes: each dword from one of several sources; accepted only when
    # all four come from one write of this tag.
    t = 77
    a = _slot16(lib, t, 1, bits[4])                     # aggregate
    p = _slot16(lib, t, 2, bits[9])                     # inclusive prefix
    a_same = _slot16(lib, t, 1, bits[4] ^ 0xFFFF0000FFFF)  # differs only in value
    old = _slot16(lib, t - 1, 2, bits[4])               # an earlier launch
    zero = [0, 0, 0, 0]
    packed = [0x12345678, (t << 2) | 1, 0x9ABCDEF0, (t << 2) | 2]   # two u32 status words of tag t
    part = [0x0000BEEF, (t << 2) | 3, 0xFFFFFFFF, (t << 2) | 3]     # a partial slot of tag t
    sources = [a, p, old, zero, packed, part]
    for pick in itertools.product(range(len(sources)), repeat=4):
        q = [sources[pick[i]][i] for i in range(4)]
        f, b = _unslot16(lib, t, q)
        if all(k == 0 for k in pick):
            assert (f, b) == (1, bits[4])
        elif all(k == 1 for k in pick):
            assert (f, b) == (2, bits[9])
        else:
            assert f == 0, (pick, q)
    # Two writes with the same tag and flag never happen (one writer per
    # slot and flag); a mix of such writes would be accepted, which is why
    # waiters never publish into these slots.
    assert _unslot16(lib, t, [a[0], a_same[1], a[2], a[3]])[0] == 1
