"""ctypes wrapper of the CPU oracle (oracle/hx_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Each function
below names the C function it wraps; the semantics and the reference
citations are in hx_oracle.h.
"""
from __future__ import annotations

import ctypes
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

NONE_INDEX = 0xFFFFFFFF


class Affine(ctypes.Structure):
    _fields_ = [("a", c_float), ("b", c_float), ("enabled", c_int32)]


_SIG = {
    "hxo_splitmix64_at": (c_uint64, [c_uint64, c_uint64]),
    "hxo_fill_uniform_int": (None, [c_void_p, c_uint64, c_uint64, c_int64, c_int64]),
    "hxo_fill_uniform_real": (None, [c_void_p, c_uint64, c_uint64, c_float, c_float]),
    "hxo_fill_normal": (None, [c_void_p, c_uint64, c_uint64, c_double, c_double]),
    "hxo_sum_u32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_prod_u32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_sum_f32": (c_double, [c_void_p, c_uint64, POINTER(Affine), POINTER(c_double)]),
    "hxo_max_u32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_max_i32": (c_int32, [c_void_p, c_uint64]),
    "hxo_max_f32": (c_float, [c_void_p, c_uint64, POINTER(Affine)]),
    "hxo_min_u32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_min_i32": (c_int32, [c_void_p, c_uint64]),
    "hxo_min_f32": (c_float, [c_void_p, c_uint64, POINTER(Affine)]),
    "hxo_argmax_u32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_argmax_i32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_argmax_f32": (c_uint32, [c_void_p, c_uint64, POINTER(Affine)]),
    "hxo_rows_f32": (None, [c_void_p, c_uint64, c_uint64, c_uint64, POINTER(Affine), c_void_p, c_void_p, c_void_p, c_void_p]),
    "hxo_rows_u32": (None, [c_void_p, c_uint64, c_uint64, c_uint64, c_void_p, c_void_p, c_void_p]),
    "hxo_rows_i32": (None, [c_void_p, c_uint64, c_uint64, c_uint64, c_void_p, c_void_p, c_void_p]),
    "hxo_scan_sum_u32": (None, [c_void_p, c_uint64, c_int, c_int, c_void_p]),
    "hxo_scan_prod_u32": (None, [c_void_p, c_uint64, c_int, c_int, c_void_p]),
    "hxo_scan_sum_f32": (None, [c_void_p, c_uint64, c_int, c_int, c_void_p, c_void_p]),
    "hxo_check_f32_bound": (c_uint64, [c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, POINTER(c_double)]),
    "hxo_ceil_log2": (c_uint32, [c_uint64]),
    "hxo_check_scan_f32": (c_uint64, [c_void_p, c_void_p, c_uint64, c_int, c_uint64, POINTER(c_double)]),
    "hxo_segmented_sum_u32": (None, [c_void_p, c_uint64, c_void_p, c_uint64, c_void_p]),
    "hxo_geometric_offsets": (c_uint64, [c_uint64, c_double, c_uint64, c_void_p, c_uint64]),
    "hxo_dot_u32": (c_uint32, [c_void_p, c_void_p, c_uint64]),
    "hxo_dot_f32": (c_double, [c_void_p, c_void_p, c_uint64, POINTER(c_double)]),
    "hxo_norm_l1_i32": (c_uint32, [c_void_p, c_uint64]),
    "hxo_norm_l1_f32": (c_double, [c_void_p, c_uint64]),
    "hxo_sum_squares_f32": (c_double, [c_void_p, c_uint64]),
    "hxo_norm_max_i32": (c_int32, [c_void_p, c_uint64]),
    "hxo_norm_max_f32": (c_float, [c_void_p, c_uint64]),
    "hxo_fma_arrays": (None, [c_void_p, c_void_p, c_float, c_uint64, c_void_p]),
    "hxo_sum_f32_threads": (c_double, [c_void_p, c_uint64, c_int]),
    "hxo_scan_excl_u32_threads": (None, [c_void_p, c_uint64, c_void_p, c_int]),
    "hxo_rows_f32_threads": (None, [c_void_p, c_uint64, c_uint64, c_uint64, POINTER(Affine), c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_int]),
    "hxo_segmented_sum_u32_threads": (None, [c_void_p, c_uint64, c_void_p, c_uint64, c_void_p, c_int]),
    "hxo_scan_incl_f32_threads": (None, [c_void_p, c_uint64, c_void_p, c_int]),
}

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "-B", "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def _aff(prologue):
    if prologue is None:
        return None
    return ctypes.byref(Affine(float(prologue[0]), float(prologue[1]), 1))


# ---- generator -----------------------------------------------------------
def splitmix64_at(seed: int, i: int) -> int:
    return int(lib().hxo_splitmix64_at(seed, i))


def uniform_int(n: int, seed: int, lo: int, hi: int, dtype=np.uint32) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    lib().hxo_fill_uniform_int(_ptr(out), n, seed, lo, hi)
    return out.view(dtype)


def uniform_real(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().hxo_fill_uniform_real(_ptr(out), n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().hxo_fill_normal(_ptr(out), n, seed, mean, std)
    return out


# ---- map-reductions (norms.rs:32-490) ----------------------------------------
def dot(a: np.ndarray, b: np.ndarray):
    """u32/i32: wrapped Σ a·b (same dtype).  f32: (f64 Σ a·b of exact products,
    Σ|a·b|)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype
    if a.dtype == np.float32:
        m = c_double()
        return float(lib().hxo_dot_f32(_ptr(a), _ptr(b), a.size, ctypes.byref(m))), float(m.value)
    v = lib().hxo_dot_u32(_ptr(a.view(np.uint32)), _ptr(b.view(np.uint32)), a.size)
    return np.array([v], dtype=np.uint32).view(a.dtype)[0]


def norm_l1(x: np.ndarray):
    """u32: wrapped Σx; i32: wrapped Σ|x| (|INT_MIN| = INT_MIN); f32: f64 Σ|x|."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return float(lib().hxo_norm_l1_f32(_ptr(x), x.size))
    if x.dtype == np.int32:
        return np.array([lib().hxo_norm_l1_i32(_ptr(x), x.size)], np.uint32).view(np.int32)[0]
    return np.uint32(lib().hxo_sum_u32(_ptr(x), x.size))


def norm_l2(x: np.ndarray) -> float:
    """f32: sqrt of the f64 sum of exact squares."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(np.sqrt(lib().hxo_sum_squares_f32(_ptr(x), x.size)))


def norm_max(x: np.ndarray):
    """max |x| with the MaxOp identity (f32::MIN, i32::MIN, 0) when empty."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return np.float32(lib().hxo_norm_max_f32(_ptr(x), x.size))
    if x.dtype == np.int32:
        return np.int32(lib().hxo_norm_max_i32(_ptr(x), x.size))
    return np.uint32(lib().hxo_max_u32(_ptr(x), x.size))


def fma_arrays(x: np.ndarray, y: np.ndarray, f: float) -> np.ndarray:
    """fmaf(f, x[i], y[i]) for every i (axpy: x = source, y = target)."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    out = np.empty_like(x)
    lib().hxo_fma_arrays(_ptr(x), _ptr(y), float(f), x.size, _ptr(out))
    return out


# ---- full reductions -------------------------------------------------------
def full_sum(x: np.ndarray, prologue=None):
    """u32/i32: wrapped sum (same dtype).  f32: (f64 sum, f64 sum|y|)."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        a = c_double()
        s = lib().hxo_sum_f32(_ptr(x), x.size, _aff(prologue), ctypes.byref(a))
        return float(s), float(a.value)
    v = lib().hxo_sum_u32(_ptr(x.view(np.uint32)), x.size)
    return np.array([v], dtype=np.uint32).view(x.dtype)[0]


def full_prod(x: np.ndarray):
    x = np.ascontiguousarray(x)
    v = lib().hxo_prod_u32(_ptr(x.view(np.uint32)), x.size)
    return np.array([v], dtype=np.uint32).view(x.dtype)[0]


def full_max(x: np.ndarray, prologue=None):
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return np.float32(lib().hxo_max_f32(_ptr(x), x.size, _aff(prologue)))
    if x.dtype == np.int32:
        return np.int32(lib().hxo_max_i32(_ptr(x), x.size))
    return np.uint32(lib().hxo_max_u32(_ptr(x), x.size))


def full_min(x: np.ndarray, prologue=None):
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return np.float32(lib().hxo_min_f32(_ptr(x), x.size, _aff(prologue)))
    if x.dtype == np.int32:
        return np.int32(lib().hxo_min_i32(_ptr(x), x.size))
    return np.uint32(lib().hxo_min_u32(_ptr(x), x.size))


def full_argmax(x: np.ndarray, prologue=None) -> int:
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        return int(lib().hxo_argmax_f32(_ptr(x), x.size, _aff(prologue)))
    if x.dtype == np.int32:
        return int(lib().hxo_argmax_i32(_ptr(x), x.size))
    return int(lib().hxo_argmax_u32(_ptr(x), x.size))


# ---- rows ----------------------------------------------------------------
def rows(x: np.ndarray, nrows: int, cols: int, ld: int | None = None, prologue=None):
    """Per row: (sum, abs_sum|None, max, argmax); f32 sums are f64."""
    x = np.ascontiguousarray(x)
    ld = cols if ld is None else ld
    argmax = np.empty(nrows, dtype=np.uint32)
    if x.dtype == np.float32:
        s = np.empty(nrows, dtype=np.float64)
        a = np.empty(nrows, dtype=np.float64)
        m = np.empty(nrows, dtype=np.float32)
        lib().hxo_rows_f32(_ptr(x), nrows, cols, ld, _aff(prologue), _ptr(s), _ptr(a), _ptr(m), _ptr(argmax))
        return s, a, m, argmax
    s = np.empty(nrows, dtype=x.dtype)
    m = np.empty(nrows, dtype=x.dtype)
    fn = lib().hxo_rows_i32 if x.dtype == np.int32 else lib().hxo_rows_u32
    fn(_ptr(x), nrows, cols, ld, _ptr(s), _ptr(m), _ptr(argmax))
    return s, None, m, argmax


# ---- scans ---------------------------------------------------------------
def scan_sum(x: np.ndarray, exclusive=False, reverse=False):
    """u32/i32: wrapped scan (same dtype).  f32: (f64 ref, f64 abs prefix)."""
    x = np.ascontiguousarray(x)
    if x.dtype == np.float32:
        ref = np.empty(x.size, dtype=np.float64)
        ab = np.empty(x.size, dtype=np.float64)
        lib().hxo_scan_sum_f32(_ptr(x), x.size, int(exclusive), int(reverse), _ptr(ref), _ptr(ab))
        return ref, ab
    out = np.empty(x.size, dtype=np.uint32)
    lib().hxo_scan_sum_u32(_ptr(x.view(np.uint32)), x.size, int(exclusive), int(reverse), _ptr(out))
    return out.view(x.dtype)


def scan_prod(x: np.ndarray, exclusive=False, reverse=False):
    x = np.ascontiguousarray(x)
    out = np.empty(x.size, dtype=np.uint32)
    lib().hxo_scan_prod_u32(_ptr(x.view(np.uint32)), x.size, int(exclusive), int(reverse), _ptr(out))
    return out.view(x.dtype)


def ceil_log2(n: int) -> int:
    return int(lib().hxo_ceil_log2(n))


def check_f32_bound(got: np.ndarray, ref: np.ndarray, abs_prefix: np.ndarray, n_for_log: int):
    """(violations, worst |err|/(eps*sum|x|)) for the f32 bound 2*ceil(log2 n)*eps_f32*sum|x|."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float64)
    abs_prefix = np.ascontiguousarray(abs_prefix, dtype=np.float64)
    w = c_double()
    bad = lib().hxo_check_f32_bound(_ptr(got), _ptr(ref), _ptr(abs_prefix), got.size, n_for_log, ctypes.byref(w))
    return int(bad), float(w.value)


def check_scan_f32(x: np.ndarray, got: np.ndarray, exclusive=False, n_for_log=None):
    """Streaming bound check of a forward f32 scan: (violations, worst)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    got = np.ascontiguousarray(got, dtype=np.float32)
    w = c_double()
    bad = lib().hxo_check_scan_f32(_ptr(x), _ptr(got), x.size, int(exclusive),
                                   x.size if n_for_log is None else n_for_log, ctypes.byref(w))
    return int(bad), float(w.value)


# ---- segmented -------------------------------------------------------------
def segmented_sum(x: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint32)
    s = offsets.size - 1
    out = np.empty(max(s, 0), dtype=np.uint32)
    lib().hxo_segmented_sum_u32(_ptr(x.view(np.uint32)), x.size, _ptr(offsets), s, _ptr(out))
    return out.view(x.dtype)


def geometric_offsets(n: int, mean: float, seed: int) -> np.ndarray:
    cap = n + 2
    buf = np.empty(cap, dtype=np.uint32)
    s = lib().hxo_geometric_offsets(n, mean, seed, _ptr(buf), cap)
    return buf[: s + 1].copy()


# ---- CPU baselines ---------------------------------------------------------
def sum_f32_threads(x: np.ndarray, threads: int) -> float:
    return float(lib().hxo_sum_f32_threads(_ptr(x), x.size, threads))


def scan_excl_u32_threads(x: np.ndarray, out: np.ndarray, threads: int) -> None:
    lib().hxo_scan_excl_u32_threads(_ptr(x), x.size, _ptr(out), threads)


def rows_threads(x: np.ndarray, nrows: int, cols: int, threads: int, ld: int | None = None, prologue=None):
    """rows() on `threads` pthreads: (sum f64, abs sum f64, max f32, argmax u32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    ld = cols if ld is None else ld
    s, a = np.empty(nrows, np.float64), np.empty(nrows, np.float64)
    m, i = np.empty(nrows, np.float32), np.empty(nrows, np.uint32)
    lib().hxo_rows_f32_threads(_ptr(x), nrows, cols, ld, _aff(prologue), _ptr(s), _ptr(a), _ptr(m), _ptr(i),
                               threads)
    return s, a, m, i


def segmented_sum_threads(x: np.ndarray, offsets: np.ndarray, threads: int) -> np.ndarray:
    x = np.ascontiguousarray(x)
    offsets = np.ascontiguousarray(offsets, dtype=np.uint32)
    s = offsets.size - 1
    out = np.empty(max(s, 0), dtype=np.uint32)
    lib().hxo_segmented_sum_u32_threads(_ptr(x.view(np.uint32)), x.size, _ptr(offsets), s, _ptr(out), threads)
    return out.view(x.dtype)


def scan_incl_f32_threads(x: np.ndarray, out: np.ndarray, threads: int) -> None:
    lib().hxo_scan_incl_f32_threads(_ptr(x), x.size, _ptr(out), threads)
