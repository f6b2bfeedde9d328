"""Pins the CPU oracle (oracle/hx_oracle.c) before it is trusted as the
parity checker: against the reference's own known-answer vectors
(tests/golden/reference_kats.json), closed forms, library routines (numpy,
math.fsum, fractions) and hand-built special cases.  CPU only."""
from __future__ import annotations

import json
import math
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())
F32_MIN = np.float32(-3.4028235e38)
F32_MAX = np.float32(3.4028235e38)


def bits(x) -> int:
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


# ---------------------------------------------------------------- generator
def test_splitmix64_matches_published_stream(oracle):
    k = KATS["splitmix64"]
    got = [oracle.splitmix64_at(k["seed"], i) for i in range(5)]
    assert got == [int(v) for v in k["outputs"]]


def test_splitmix64_python_restatement_agrees(oracle):
    mask = (1 << 64) - 1

    def sm(seed, i):
        z = (seed + (i + 1) * 0x9E3779B97F4A7C15) & mask
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)

    for seed in (0, 1, 42, 2**63 + 5):
        for i in (0, 1, 2, 1000, 2**40):
            assert oracle.splitmix64_at(seed, i) == sm(seed, i)


def test_uniform_int_range_and_formula(oracle):
    x = oracle.uniform_int(1 << 16, seed=7, lo=0, hi=255)
    assert x.min() == 0 and x.max() == 255
    h = np.array([oracle.splitmix64_at(7, i) for i in range(64)], dtype=np.uint64)
    assert np.array_equal(x[:64], (h >> np.uint64(56)).astype(np.uint32))
    y = oracle.uniform_int(1 << 16, seed=3, lo=-1000, hi=1000, dtype=np.int32)
    assert y.min() == -1000 and y.max() == 1000
    assert abs(float(y.mean())) < 10


def test_uniform_real_is_exact_grid(oracle):
    x = oracle.uniform_real(1 << 16, seed=1, lo=-1.0, hi=1.0)
    assert x.min() >= -1.0 and x.max() < 1.0
    # every value is k * 2^-23 for an integer k (2u - 1 is exact in f32)
    k = x.astype(np.float64) * 2.0**23
    assert np.array_equal(k, np.round(k))
    h = oracle.splitmix64_at(1, 5)
    assert x[5] == np.float32((h >> 40) * 2.0**-24 * 2.0 - 1.0)


def test_normal_moments(oracle):
    z = oracle.normal(1 << 18, seed=11)
    assert abs(float(z.mean())) < 0.01
    assert abs(float(z.std()) - 1.0) < 0.01


# ------------------------------------------------------ reference fixtures
def test_full_reduction_kats(oracle):
    k = KATS["full_reduction"]
    xf = np.array(k["input"], dtype=np.float32)
    xu = np.array(k["input"], dtype=np.uint32)
    s, a = oracle.full_sum(xf)
    assert s == k["sum"] and a == k["sum"]
    assert oracle.full_sum(xu) == k["sum"]
    assert oracle.full_prod(xu) == k["prod"]
    assert oracle.full_min(xf) == k["min"] and oracle.full_max(xf) == k["max"]
    diag = np.array(k["diagonal"]["input"], dtype=np.float32)[::4]
    assert oracle.full_sum(diag)[0] == k["diagonal"]["sum"]
    assert oracle.full_prod(np.full(12, 2, np.uint32)) == k["rebind_all_twos_prod"]["value"]


def test_axis_reduction_kats(oracle):
    k = KATS["axis_reduction"]
    x = np.array(k["input"], dtype=np.float32).reshape(3, 4)
    s1, _, m1, _ = oracle.rows(x.ravel(), 3, 4)
    assert list(s1) == [10, 26, 42] and list(m1) == k["max_axis1"]
    xt = np.ascontiguousarray(x.T)
    s0, _, m0, _ = oracle.rows(xt.ravel(), 4, 3)
    assert list(s0) == k["sum_axis0"] and list(m0) == k["max_axis0"]
    assert list(s0 / 3) == k["mean_axis0"] and list(s1 / 4) == k["mean_axis1"]
    assert [oracle.full_min(r) for r in x] == k["min_axis1"]
    assert [oracle.full_min(c) for c in xt] == k["min_axis0"]
    xu = np.array(k["input"], dtype=np.uint32).reshape(3, 4)
    assert [int(oracle.full_prod(c)) for c in xu.T.copy()] == k["prod_axis0"]
    assert [int(oracle.full_prod(r)) for r in xu] == k["prod_axis1"]


def test_rocm_axis_u32_kats(oracle):
    k = KATS["rocm_axis_u32"]
    x = np.array(k["input"], dtype=np.uint32).reshape(3, 4)
    s, _, m, _ = oracle.rows(x.ravel(), 3, 4)
    assert list(s) == k["sum_rows"] and list(m) == k["max_rows"]
    sc, _, _, _ = oracle.rows(x.T.copy().ravel(), 4, 3)
    assert list(sc) == k["sum_cols"]
    assert [int(oracle.full_min(r)) for r in x] == k["min_rows"]
    assert [int(oracle.full_prod(r)) for r in x] == k["prod_rows"]
    assert [int(oracle.full_prod(c)) for c in x.T.copy()] == k["prod_cols"]
    # The reference asserts 17_600 for column 3; 4 * 40 * 11 is 1760.
    assert 4 * 40 * 11 == k["prod_cols"][3] != k["prod_cols_as_asserted_by_reference"][3]
    assert int(oracle.full_prod(np.zeros(0, np.uint32))) == 1  # empty product = identity


def test_scan_kats(oracle):
    k = KATS["scan"]
    x = np.array(k["input"], dtype=np.uint32).reshape(3, 4)
    fwd = np.concatenate([oracle.scan_sum(r) for r in x])
    rev = np.concatenate([oracle.scan_sum(r, reverse=True) for r in x])
    prod = np.concatenate([oracle.scan_prod(r) for r in x])
    col = np.stack([oracle.scan_sum(c) for c in x.T.copy()], axis=1).ravel()
    assert list(fwd) == k["cumsum_axis1_forward"]
    assert list(rev) == k["cumsum_axis1_reverse"]
    assert list(prod) == k["cumprod_axis1_forward"]
    assert list(col) == k["cumsum_axis0_forward"]
    xf = x.astype(np.float32)
    ref, _ = oracle.scan_sum(xf[0])
    assert list(ref) == k["cumsum_axis1_forward"][:4]


def test_rocm_scan_i32_kats(oracle):
    k = KATS["rocm_scan_i32"]
    x = np.array(k["input"], dtype=np.int32).reshape(2, 4)

    def rows(fn, **kw):
        return list(np.concatenate([fn(r, **kw) for r in x]))

    def cols(fn, **kw):
        return list(np.stack([fn(c, **kw) for c in x.T.copy()], axis=1).ravel())

    assert rows(oracle.scan_sum) == k["cumsum_axis1"]
    assert rows(oracle.scan_sum, reverse=True) == k["reverse_axis1"]
    assert cols(oracle.scan_sum, reverse=True) == k["suffix_axis0"]
    assert cols(oracle.scan_sum) == k["cumsum_axis0"]
    assert rows(oracle.scan_prod) == k["cumprod_axis1"]
    assert cols(oracle.scan_prod) == k["cumprod_axis0"]
    assert rows(oracle.scan_prod, reverse=True) == k["suffix_prod_axis1"]
    assert cols(oracle.scan_prod, reverse=True) == k["suffix_prod_axis0"]
    long = np.array([i % 7 - 3 for i in range(1025)], dtype=np.int32)
    acc, expect = 0, []
    for v in long:
        acc += int(v)
        expect.append(acc)
    assert list(oracle.scan_sum(long)) == expect


def test_rocm_reduce_u32_kats(oracle):
    for n in KATS["rocm_reduce_u32"]["sizes"]:
        x = np.array([i % 17 for i in range(n)], dtype=np.uint32)
        assert int(oracle.full_sum(x)) == sum(i % 17 for i in range(n))
        assert int(oracle.full_min(x)) == 0 and int(oracle.full_max(x)) == 16
    assert int(oracle.full_sum(np.zeros(0, np.uint32))) == 0


# ------------------------------------------------------------- closed forms
def test_u32_sum_wraps_mod_2_32(oracle):
    n = 1 << 20
    x = np.arange(n, dtype=np.uint32)
    assert int(oracle.full_sum(x)) == (n * (n - 1) // 2) % 2**32
    y = np.full(1000, 0xFFFFFFFF, dtype=np.uint32)
    assert int(oracle.full_sum(y)) == (1000 * 0xFFFFFFFF) % 2**32
    z = np.array([2**31 - 1, 1], dtype=np.int32)
    assert int(oracle.full_sum(z)) == -(2**31)  # two's complement wrap


def test_scan_closed_forms(oracle):
    n = 5000
    ones = np.ones(n, dtype=np.uint32)
    assert np.array_equal(oracle.scan_sum(ones), np.arange(1, n + 1, dtype=np.uint32))
    assert np.array_equal(oracle.scan_sum(ones, exclusive=True), np.arange(n, dtype=np.uint32))
    assert np.array_equal(oracle.scan_sum(ones, reverse=True), np.arange(n, 0, -1, dtype=np.uint32))
    x = np.random.default_rng(0).integers(0, 2**32, n, dtype=np.uint32)
    inc = oracle.scan_sum(x)
    exc = oracle.scan_sum(x, exclusive=True)
    assert np.array_equal(inc - x, exc)  # exclusive = inclusive - x (mod 2^32)
    assert np.array_equal(inc, np.cumsum(x, dtype=np.uint32))  # numpy wraps the same way
    rev = oracle.scan_sum(x, reverse=True)
    assert np.array_equal(rev, np.cumsum(x[::-1], dtype=np.uint32)[::-1])
    p = oracle.scan_prod(np.full(40, 3, np.uint32))
    assert int(p[-1]) == pow(3, 40, 2**32)
    pe = oracle.scan_prod(np.full(5, 3, np.uint32), exclusive=True)
    assert list(pe) == [1, 3, 9, 27, 81]


def test_f32_sum_matches_fsum(oracle):
    x = oracle.uniform_real(1 << 16, seed=5, lo=-1.0, hi=1.0)
    s, a = oracle.full_sum(x)
    assert s == pytest.approx(math.fsum(map(float, x)), abs=1e-12)
    assert a == pytest.approx(math.fsum(abs(float(v)) for v in x), rel=1e-15)
    ref, ab = oracle.scan_sum(x[:4096])
    assert ref[-1] == pytest.approx(math.fsum(map(float, x[:4096])), abs=1e-12)
    assert np.all(np.diff(ab) >= 0)
    refx, _ = oracle.scan_sum(x[:10], exclusive=True)
    assert refx[0] == 0.0 and refx[1] == float(x[0])


def test_max_min_argmax_match_numpy_on_plain_data(oracle):
    rng = np.random.default_rng(1)
    for dtype in (np.float32, np.int32, np.uint32):
        if dtype == np.float32:
            x = rng.standard_normal(10007).astype(np.float32)
        else:
            x = rng.integers(np.iinfo(dtype).min, np.iinfo(dtype).max, 10007, dtype=dtype)
        assert oracle.full_max(x) == x.max()
        assert oracle.full_min(x) == x.min()
        assert oracle.full_argmax(x) == int(np.argmax(x))


def test_argmax_ties_go_to_lowest_index(oracle):
    x = np.array([1, 5, 3, 5, 5, 0], dtype=np.float32)
    assert oracle.full_argmax(x) == 1
    assert oracle.full_argmax(np.full(100, 7, np.uint32)) == 0
    assert oracle.full_argmax(np.arange(100, dtype=np.int32)) == 99


def test_special_values(oracle):
    nan = np.float32("nan")
    inf = np.float32("inf")
    x = np.array([nan, 1.0, nan, -2.0], dtype=np.float32)
    assert oracle.full_max(x) == 1.0 and oracle.full_argmax(x) == 1
    assert oracle.full_min(x) == -2.0
    allnan = np.array([nan, nan], dtype=np.float32)
    assert oracle.full_max(allnan) == F32_MIN  # MaxOp identity f32::MIN
    assert oracle.full_argmax(allnan) == 0xFFFFFFFF
    ninf = np.array([-inf, -inf], dtype=np.float32)
    assert oracle.full_max(ninf) == F32_MIN  # identity dominates -inf
    assert oracle.full_argmax(ninf) == 0
    assert oracle.full_min(np.array([inf], np.float32)) == F32_MAX
    z = np.array([-0.0, 0.0, -0.0], dtype=np.float32)
    assert bits(oracle.full_max(z)) == 0x00000000  # +0 above -0
    assert oracle.full_argmax(z) == 1
    assert bits(oracle.full_min(z)) == 0x80000000
    assert oracle.full_argmax(np.zeros(0, np.float32)) == 0xFFFFFFFF
    assert oracle.full_max(np.zeros(0, np.int32)) == np.iinfo(np.int32).min
    assert oracle.full_max(np.zeros(0, np.uint32)) == 0


def test_compensated_sums_of_infinities_and_nans_are_ieee_sums(oracle):
    """Once a term is infinite or NaN the compensated sums return what IEEE
    addition gives in any order: +inf or -inf for infinities of one sign
    among finite terms, NaN for infinities of both signs or any NaN.  (The
    compensation itself turns NaN at the first infinity, inf - inf; a sum
    that added it returned NaN for a row holding +inf.)  f32 extremes that
    overflow f32 stay finite in f64, compensated exactly."""
    nan, inf = np.float32("nan"), np.float32("inf")
    cases = [([inf, 2.0, 1.0], math.inf), ([1.0, -inf, 3.0, -inf], -math.inf), ([2.0, inf, -inf], None),
             ([1.0, nan, inf], None), ([F32_MAX, F32_MAX, 1.0], 2.0 * float(F32_MAX) + 1.0),
             ([F32_MAX, 1.0, F32_MIN], 1.0)]
    for terms, want in cases:
        x = np.array(terms, np.float32)
        got = [oracle.full_sum(x)[0], oracle.rows(x, 1, x.size)[0][0], oracle.scan_sum(x)[0][-1],
               oracle.dot(x, np.ones_like(x))[0]]
        for g in got:
            assert math.isnan(g) if want is None else g == want, (terms, got)
    # Magnitudes: |inf| terms make the absolute sums +inf, with or without NaN.
    x = np.array([1.0, -inf, 2.0], np.float32)
    assert oracle.full_sum(x)[1] == math.inf and oracle.norm_l1(x) == math.inf
    assert oracle.norm_l2(x) == math.inf


def test_prologue_is_correctly_rounded_fma(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(200).astype(np.float32) * np.float32(1e3)
    for a, b in ((0.5, 0.25), (1.0 / 3.0, -7.1), (3.0, 1e-8)):
        a32, b32 = np.float32(a), np.float32(b)
        for i, v in enumerate(x[:50]):
            exact = Fraction(float(a32)) * Fraction(float(v)) + Fraction(float(b32))
            want = np.float32(float(exact))  # one rounding from an exact rational
            # float(Fraction) rounds to f64 first; re-check for the f32 tie cases
            if abs(Fraction(float(want)) - exact) > abs(Fraction(float(np.nextafter(want, np.float32(np.inf)))) - exact):
                want = np.nextafter(want, np.float32(np.inf))
            if abs(Fraction(float(want)) - exact) > abs(Fraction(float(np.nextafter(want, np.float32(-np.inf)))) - exact):
                want = np.nextafter(want, np.float32(-np.inf))
            got = oracle.full_max(np.array([v], np.float32), prologue=(a32, b32))
            assert bits(got) == bits(want), (a, b, v)
        s, _ = oracle.full_sum(x, prologue=(a32, b32))
        expect = math.fsum(float(np.float32(float(Fraction(float(a32)) * Fraction(float(v)) + Fraction(float(b32))))) for v in x)
        assert s == pytest.approx(expect, rel=1e-9)


def test_bound_checker_flags_planted_errors(oracle):
    x = oracle.uniform_real(4096, seed=9, lo=0.0, hi=1.0)
    ref, ab = oracle.scan_sum(x)
    got = ref.astype(np.float32)  # correctly rounded: within bound
    bad, worst = oracle.check_f32_bound(got, ref, ab, 4096)
    assert bad == 0 and worst <= 0.5
    planted = got.copy()
    # dropped term at position 1000: error |x[1000]| far above 24 eps * sum
    planted[1000] = np.float32(ref[1000] - x[1000])
    assert oracle.check_f32_bound(planted, ref, ab, 4096)[0] == 1
    planted = got.copy()
    planted[7] = np.float32("nan")
    assert oracle.check_f32_bound(planted, ref, ab, 4096)[0] == 1
    # the bound itself: 2 * ceil(log2 n) * eps * sum|x|
    n = 4096
    tol = 2 * oracle.ceil_log2(n) * 2.0**-23 * ab[-1]
    edge = got.copy()
    edge[-1] = np.float32(ref[-1] + 1.5 * tol)
    assert oracle.check_f32_bound(edge, ref, ab, n)[0] == 1
    assert oracle.ceil_log2(1) == 0 and oracle.ceil_log2(2) == 1
    assert oracle.ceil_log2(2**28) == 28 and oracle.ceil_log2(2**28 + 1) == 29


def test_segmented_sum_brute_force(oracle):
    rng = np.random.default_rng(3)
    x = rng.integers(-1000, 1001, 5000, dtype=np.int32)
    offsets = np.array([0, 0, 3, 3, 4, 1000, 1000, 4999, 5000, 5000], dtype=np.uint32)
    got = oracle.segmented_sum(x, offsets)
    want = [int(x[offsets[s]:offsets[s + 1]].astype(np.int64).sum()) for s in range(len(offsets) - 1)]
    assert list(got.astype(np.int64)) == want


def test_geometric_offsets(oracle):
    n = 1 << 22
    off = oracle.geometric_offsets(n, 300.0, seed=4)
    lens = np.diff(off.astype(np.int64))
    assert off[0] == 0 and off[-1] == n
    assert lens.min() >= 1
    assert abs(float(lens[:-1].mean()) - 300.0) < 5.0


# ---- map-reductions (dot, norms) -------------------------------------------
def test_map_reduction_kats(oracle):
    k = KATS["map_reduction"]
    m = np.array(k["matrix_i32"], np.int32)
    assert oracle.norm_l1(m) == k["norm_l1"]
    assert oracle.norm_max(m) == k["norm_max"]
    lhs = np.array(k["dot_lhs_i32"], np.int32)[k["dot_lhs_offset"]:]
    assert oracle.dot(lhs, np.array(k["dot_rhs_i32"], np.int32)) == k["dot"]
    tr = np.array(k["trace_i32"], np.int32).reshape(3, 3)
    assert oracle.full_sum(np.ascontiguousarray(np.diagonal(tr))) == k["trace"]
    assert oracle.norm_l2(np.array(k["l2_f32"], np.float32)) == k["norm_l2"]
    dv = KATS["dense_vector"]
    assert oracle.dot(np.array(dv["dot_a"], np.float32), np.array(dv["dot_b"], np.float32))[0] == dv["dot"]
    v = np.array(dv["norm_vector"], np.float32)
    assert oracle.norm_l1(v) == dv["norm_l1"] and oracle.norm_max(v) == dv["norm_max"]
    assert oracle.norm_l2(v) == dv["norm_l2"]
    assert oracle.norm_l2(np.array(dv["norm_vector_rebound"], np.float32)) == dv["norm_l2_rebound"]


def test_map_reductions_against_library_routines(oracle):
    rng = np.random.default_rng(3)
    a = rng.standard_normal(10007).astype(np.float32)
    b = rng.standard_normal(10007).astype(np.float32)
    got, mags = oracle.dot(a, b)
    want = math.fsum(float(x) * float(y) for x, y in zip(a, b))  # exact products, exact sum
    assert got == pytest.approx(want, rel=0, abs=1e-12 * mags)
    assert oracle.norm_l1(a) == pytest.approx(math.fsum(abs(float(x)) for x in a), rel=1e-15)
    assert oracle.norm_l2(a) == pytest.approx(float(np.linalg.norm(a.astype(np.float64))), rel=1e-14)
    assert oracle.norm_max(a) == np.max(np.abs(a))
    # Cauchy-Schwarz and the dot of a vector with itself.
    assert abs(got) <= oracle.norm_l2(a) * oracle.norm_l2(b) * (1 + 1e-12)
    assert oracle.dot(a, a)[0] == pytest.approx(oracle.norm_l2(a) ** 2, rel=1e-12)
    # Integer forms wrap mod 2^32, |INT_MIN| = INT_MIN.
    i = rng.integers(-2**31, 2**31, 5000, dtype=np.int64).astype(np.int32)
    j = rng.integers(-2**31, 2**31, 5000, dtype=np.int64).astype(np.int32)
    wrap = lambda v: np.array([v & 0xFFFFFFFF], np.uint32).view(np.int32)[0]
    assert oracle.dot(i, j) == wrap(sum(int(x) * int(y) for x, y in zip(i, j)))
    assert oracle.norm_l1(i) == wrap(sum(abs(int(x)) for x in i))
    edge = np.array([-2**31, 5, -7], np.int32)
    assert oracle.norm_max(edge) == 7  # |INT_MIN| stays INT_MIN and never wins
    assert oracle.norm_max(np.array([-2**31], np.int32)) == -2**31
    assert oracle.norm_max(np.zeros(0, np.float32)) == np.float32(-3.4028234663852886e38)
    nan = np.array([1.0, np.nan, -3.0], np.float32)
    assert oracle.norm_max(nan) == 3.0


def test_fma_arrays_is_single_rounding(oracle):
    """fmaf(f, x, y) rounds once: checked against exact rational arithmetic
    on values whose separately rounded product would differ."""
    x = np.array([1.0 + 2.0**-23, 3.0, 0.1], np.float32)
    y = np.array([-1.0, 1e-8, -0.3], np.float32)
    f = np.float32(1.0 - 2.0**-24)
    got = oracle.fma_arrays(x, y, float(f))
    for i in range(3):
        exact = Fraction(float(f)) * Fraction(float(x[i])) + Fraction(float(y[i]))
        assert got[i] == np.float32(float(exact)), i
    # the separately rounded form differs on the first element
    assert np.float32(f * x[0]) + y[0] != got[0]


# ---- the streaming f32 scan checker (the only checker of the 2^30 scan) ----
def _tol(x: np.ndarray, i: int, exclusive: bool, n_for_log: int) -> float:
    """The north-star bound at output i from first principles:
    2 * ceil(log2 n) * 2^-23 * (exact sum of |x| over the prefix), with the
    prefix sum taken by math.fsum and ceil(log2 n) by integer bit length."""
    m = i if exclusive else i + 1
    return 2 * (n_for_log - 1).bit_length() * 2.0**-23 * math.fsum(abs(float(v)) for v in x[:m])


@pytest.mark.parametrize("lo", [0.0, -1.0])
@pytest.mark.parametrize("exclusive", [False, True])
def test_streaming_scan_checker_agrees_with_the_array_checker(oracle, lo, exclusive):
    """hxo_check_scan_f32 re-derives the prefix and the bound on the fly; on
    the same outputs it must report what hxo_check_f32_bound reports from
    the stored f64 prefix: same violation count, same worst ratio."""
    n = 1 << 17
    x = oracle.uniform_real(n, seed=21, lo=lo, hi=1.0)
    ref, ab = oracle.scan_sum(x, exclusive=exclusive)
    rng = np.random.default_rng(4)
    tol = 2 * oracle.ceil_log2(n) * 2.0**-23 * ab
    # correctly rounded, jittered inside the bound, and jittered across it
    for scale in (0.0, 0.6, 1.8):
        got = (ref + rng.uniform(-scale, scale, n) * tol).astype(np.float32)
        want = oracle.check_f32_bound(got, ref, ab, n)
        have = oracle.check_scan_f32(x, got, exclusive=exclusive)
        assert have[0] == want[0], scale
        assert have[1] == pytest.approx(want[1], rel=1e-12, abs=1e-12), scale
        if scale == 0.0:
            assert want[0] == 0 and want[1] <= 0.5
        elif scale == 0.6:
            assert want[0] == 0
        else:
            assert want[0] > n // 10


def test_streaming_scan_checker_flags_planted_errors(oracle):
    """Plausible scan bugs must each fail the streaming check, and outputs
    within the bound must pass; the bound's constants are pinned against a
    from-scratch evaluation (math.fsum, bit length)."""
    n = 1 << 17
    x = oracle.uniform_real(n, seed=22, lo=0.0, hi=1.0)
    inc, _ = oracle.scan_sum(x)
    exc, _ = oracle.scan_sum(x, exclusive=True)
    good_inc = inc.astype(np.float32)
    good_exc = exc.astype(np.float32)
    assert oracle.check_scan_f32(x, good_inc)[0] == 0
    assert oracle.check_scan_f32(x, good_exc, exclusive=True)[0] == 0

    # a dropped term at i (and every later output, as a real bug would do)
    i = 1000 + int(np.argmax(x[1000:2000] > 0.5))
    dropped = (inc - np.where(np.arange(n) >= i, float(x[i]), 0.0)).astype(np.float32)
    bad, worst = oracle.check_scan_f32(x, dropped)
    assert bad >= 1 and worst > 2 * oracle.ceil_log2(n)
    # one NaN
    nan = good_inc.copy()
    nan[77] = np.float32("nan")
    assert oracle.check_scan_f32(x, nan)[0] == 1
    # an exclusive result shifted by one position (that is, the inclusive one),
    # and the inclusive form checked as exclusive
    assert oracle.check_scan_f32(x, good_inc, exclusive=True)[0] > n // 2
    assert oracle.check_scan_f32(x, good_exc)[0] > n // 2
    # an exclusive scan one element late: out[i] = sum x[0..i-1)
    late = np.concatenate([[0.0], exc[:-1]]).astype(np.float32)
    assert oracle.check_scan_f32(x, late, exclusive=True)[0] > n // 2
    # the wrong sign of one term
    flip = (inc - 2.0 * np.where(np.arange(n) >= i, float(x[i]), 0.0)).astype(np.float32)
    assert oracle.check_scan_f32(x, flip)[0] >= n - i - 1

    # the bound itself, at three positions, from first principles
    for k in (0, 4097, n - 1):
        for exclusive, base in ((False, inc), (True, exc)):
            if exclusive and k == 0:
                continue  # exclusive out[0] = 0 with zero tolerance
            t = _tol(x, k, exclusive, n)
            for factor, expect in ((0.5, 0), (0.97, 0), (1.03, 1), (1.5, 1)):
                got = (good_exc if exclusive else good_inc).copy()
                got[k] = np.float32(base[k] + factor * t)
                # f32 rounding of the planted value moves it by at most half
                # an ulp, inside the 3% margins around the bound
                assert abs(float(got[k]) - (base[k] + factor * t)) < 0.02 * t
                assert oracle.check_scan_f32(x, got, exclusive=exclusive)[0] == expect, (k, exclusive, factor)
    # exclusive out[0] must be exactly 0 (an empty prefix has no tolerance)
    zero = good_exc.copy()
    zero[0] = np.float32(1e-30)
    assert oracle.check_scan_f32(x, zero, exclusive=True)[0] == 1
    # n_for_log widens the bound by ceil(log2 n_for_log) / ceil(log2 n)
    t = _tol(x, n - 1, False, n)
    wide = good_inc.copy()
    wide[-1] = np.float32(inc[-1] + 1.5 * t)
    assert oracle.check_scan_f32(x, wide)[0] == 1
    assert oracle.check_scan_f32(x, wide, n_for_log=n * n)[0] == 0


def test_streaming_scan_checker_matches_math_fsum_prefixes(oracle):
    """The streaming checker's prefix is exact to f64 rounding: an output set
    to the correctly rounded math.fsum prefix has worst ratio <= 0.5 (one
    f32 rounding), for a signed input with heavy cancellation."""
    rng = np.random.default_rng(6)
    x = (rng.standard_normal(3000) * 1e3).astype(np.float32)
    x[1::2] = -x[::2][: x[1::2].size]  # pairs cancel: partial sums stay small
    prefix = [math.fsum(map(float, x[: i + 1])) for i in range(x.size)]
    got = np.array(prefix, dtype=np.float32)
    bad, worst = oracle.check_scan_f32(x, got)
    assert bad == 0 and worst <= 0.5


def test_rows_with_padded_leading_dimension(oracle):
    """hxo_rows_* with ld > cols read row r at r*ld: each row must match the
    same function on that row alone, and numpy."""
    rng = np.random.default_rng(7)
    rows, cols, ld = 9, 37, 40
    for dtype in (np.float32, np.int32, np.uint32):
        if dtype == np.float32:
            buf = rng.standard_normal(rows * ld).astype(np.float32)
        else:
            info = np.iinfo(dtype)
            buf = rng.integers(info.min, info.max, rows * ld, dtype=dtype)
        pro = (0.5, 0.25) if dtype == np.float32 else None
        s, a, m, i = oracle.rows(buf, rows, cols, ld, prologue=pro)
        for r in range(rows):
            row = np.ascontiguousarray(buf[r * ld: r * ld + cols])
            s1, a1, m1, i1 = oracle.rows(row, 1, cols, prologue=pro)
            assert s[r] == s1[0] and m[r] == m1[0] and i[r] == i1[0], (dtype, r)
            y = oracle.fma_arrays(row, np.full(cols, 0.25, np.float32), 0.5) if pro else row
            assert m[r] == y.max() and i[r] == int(np.argmax(y)), (dtype, r)
            if dtype == np.float32:
                assert a[r] == a1[0]
                assert s[r] == pytest.approx(math.fsum(map(float, y)), abs=1e-12)
            else:
                assert int(s[r]) == int(np.sum(y, dtype=dtype))  # numpy wraps mod 2^32
        # the padding between rows is never read: poisoning it changes nothing
        poisoned = buf.copy()
        for r in range(rows):
            poisoned[r * ld + cols: (r + 1) * ld] = dtype(7) if dtype != np.float32 else np.float32(1e30)
        s2, _, m2, i2 = oracle.rows(poisoned, rows, cols, ld, prologue=pro)
        assert np.array_equal(s2, s) and np.array_equal(m2, m) and np.array_equal(i2, i)


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_multithreaded_scan_baseline_equals_sequential(oracle, threads):
    """The pthread CPU baseline computes the same exclusive scan as the
    sequential oracle (ragged split points, wrap-around)."""
    n = 100_003
    x = oracle.uniform_int(n, seed=8, lo=0, hi=2**32 - 1)
    out = np.empty_like(x)
    oracle.scan_excl_u32_threads(x, out, threads)
    assert np.array_equal(out, oracle.scan_sum(x, exclusive=True))
    assert np.array_equal(out, (np.cumsum(x, dtype=np.uint32) - x))


@pytest.mark.parametrize("threads", [1, 3, 16])
def test_multithreaded_sum_baseline(oracle, threads):
    """The all-core f32 sum baseline (plain f64 partials in thread order):
    exact on integer-valued inputs (every partial and total below 2^53), and
    within the f32 bound of the compensated oracle on random inputs.  A
    dropped or doubled chunk fails the exact case."""
    n = 1_000_003
    xi = (oracle.uniform_int(n, seed=21, lo=0, hi=1000).astype(np.float32) - np.float32(500))
    exact = int(np.sum(xi.astype(np.int64)))
    assert oracle.sum_f32_threads(xi, threads) == float(exact)
    x = oracle.uniform_real(n, seed=22, lo=-1.0, hi=1.0)
    ref, ab = oracle.full_sum(x)
    assert abs(oracle.sum_f32_threads(x, threads) - ref) <= 2 * oracle.ceil_log2(n) * 2.0**-23 * ab


@pytest.mark.parametrize("threads", [1, 5, 16])
def test_multithreaded_rows_baseline_equals_sequential(oracle, threads):
    """The all-core rows baseline is the sequential rows fold per row range:
    bit-identical sums, maxima and argmaxes (ragged row split, padded rows,
    with and without the prologue)."""
    rows, cols, ld = 101, 333, 340
    x = oracle.normal(rows * ld, seed=23)
    for pro in (None, (0.5, 0.25)):
        want = oracle.rows(x, rows, cols, ld, prologue=pro)
        got = oracle.rows_threads(x, rows, cols, threads, ld=ld, prologue=pro)
        for g, w in zip(got, want):
            assert np.array_equal(g, w)


@pytest.mark.parametrize("threads", [1, 7, 16])
def test_multithreaded_segmented_baseline_equals_sequential(oracle, threads):
    """All-core segmented sum == the sequential oracle, bit-exact, including
    empty segments and fewer segments than threads."""
    n = 200_003
    x = oracle.uniform_int(n, seed=24, lo=-1000, hi=1000, dtype=np.int32)
    for mean in (3.0, 300.0, 1e6):
        off = oracle.geometric_offsets(n, mean, seed=25)
        assert np.array_equal(oracle.segmented_sum_threads(x, off, threads), oracle.segmented_sum(x, off))
    off = np.array([0, 0, 5, 5, n], np.uint32)
    assert np.array_equal(oracle.segmented_sum_threads(x, off, threads), oracle.segmented_sum(x, off))


@pytest.mark.parametrize("threads", [1, 4, 16])
def test_multithreaded_f32_scan_baseline(oracle, threads):
    """All-core inclusive f32 scan: exact on integer-valued inputs whose
    prefixes stay below 2^24 (a wrong chunk carry or a shifted index fails
    it), and within 2*ceil(log2 n)*eps*sum|x| of the compensated oracle on
    uniform[0, 1) inputs."""
    n = 500_009
    xi = oracle.uniform_int(n, seed=26, lo=0, hi=31).astype(np.float32)
    out = np.empty_like(xi)
    oracle.scan_incl_f32_threads(xi, out, threads)
    assert np.array_equal(out, np.cumsum(xi.astype(np.int64)).astype(np.float32))
    x = oracle.uniform_real(n, seed=27, lo=0.0, hi=1.0)
    oracle.scan_incl_f32_threads(x, out, threads)
    bad, _ = oracle.check_scan_f32(x, out)
    assert bad == 0
