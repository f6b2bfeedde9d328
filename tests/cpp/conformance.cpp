// C++ conformance program: the reference's conformance clauses and ROCm
// contract cases, written against the C++ host interface
// (hephaestus_amd/host/hephaestus.hpp) the way the reference's Rust clauses
// are written against its traits.  Known-answer values are the ones in
// tests/golden/reference_kats.json (cited per clause); the larger cases
// compare with sequential host folds.
//
// Exit status: 0 when every clause passes, 1 otherwise, 77 when no GPU is
// present (the usual "skipped" code).
#include "../../hephaestus_amd/host/hephaestus.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <numeric>
#include <string>
#include <vector>

using namespace hephaestus;

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond)                                                                                        \
    do {                                                                                                   \
        ++g_checks;                                                                                        \
        if (!(cond)) {                                                                                     \
            ++g_failures;                                                                                  \
            std::printf("  FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);                                  \
        }                                                                                                  \
    } while (0)

template <typename T> bool same(const std::vector<T> &a, const std::vector<T> &b) { return a == b; }

template <typename F> void expect_error(ErrorKind kind, const char *msg_prefix, F &&f) {
    ++g_checks;
    try {
        f();
        ++g_failures;
        std::printf("  FAIL: expected an error starting with \"%s\"\n", msg_prefix);
    } catch (const Error &e) {
        if (e.kind() != kind || std::strncmp(e.what(), msg_prefix, std::strlen(msg_prefix)) != 0) {
            ++g_failures;
            std::printf("  FAIL: got kind %d \"%s\", expected \"%s\"\n", (int)e.kind(), e.what(), msg_prefix);
        }
    }
}

std::vector<float> rows_fixture() { // full_reduction.rs:57-60, scan.rs:45-60
    std::vector<float> v;
    for (int r = 0; r < 3; ++r) v.insert(v.end(), {1.f, 2.f, 3.f, 2.f});
    return v;
}

// ---------------------------------------------------- transfer.rs:27-115
void transfer_contract(RocmDevice &dev) {
    const uint32_t bits[5] = {0x3fc00000u, 0x80000000u, 0x7fc01234u, 0x00800000u, 0xc0500000u};
    std::vector<uint32_t> pattern(bits, bits + 5);
    auto buf = dev.upload(pattern);
    CHECK(buf.len() == 5);
    CHECK(same(dev.download_owned(buf), pattern));

    auto zeros = dev.alloc_zeroed<float>(4);
    CHECK(same(dev.download_owned(zeros), std::vector<float>(4, 0.f)));
    dev.write_buffer(zeros, std::vector<float>{9.f, 8.f, 7.f, 6.f});
    dev.write_sub_buffer(zeros, 1, std::vector<float>{0.5f, 0.25f});
    const std::vector<float> after{9.f, 0.5f, 0.25f, 6.f};
    CHECK(same(dev.download_owned(zeros), after));
    auto copy = dev.alloc_zeroed<float>(4);
    dev.copy_buffer(zeros, copy);
    CHECK(same(dev.download_owned(copy), after));

    std::vector<float> small(3);
    try {
        dev.download(copy, small);
        CHECK(false);
    } catch (const Error &e) {
        CHECK(e.kind() == ErrorKind::LengthMismatch);
        CHECK(e.host_len() == 3 && e.device_len() == 4);
    }
    auto longer = dev.alloc_zeroed<float>(5);
    expect_error(ErrorKind::LengthMismatch, "", [&] { dev.copy_buffer(copy, longer); });
    expect_error(ErrorKind::LengthMismatch, "", [&] { dev.write_buffer(copy, std::vector<float>{1.f, 1.f}); });
    expect_error(ErrorKind::LengthMismatch, "", [&] { dev.write_sub_buffer(copy, 3, std::vector<float>{1.f, 1.f}); });
    CHECK(same(dev.download_owned(copy), after)); // rejections wrote nothing
}

// --------------------------------------------- full_reduction.rs:57-231
void full_reduction_contract(RocmDevice &dev) {
    RocmFullReductionOps ops;
    auto in = dev.upload(rows_fixture());
    const Layout l34 = Layout::c_contiguous({3, 4}), l1 = Layout::c_contiguous({1});
    auto out = dev.alloc_zeroed<float>(1);
    auto value = [&] { return dev.download_owned(out)[0]; };

    ops.reduce_full_into<SumOp, float>(dev, {in, l34}, {out, l1});
    CHECK(value() == 24.f);
    ops.reduce_full_into<ProdOp, float>(dev, {in, l34}, {out, l1});
    CHECK(value() == 1728.f);
    ops.reduce_full_into<MinOp, float>(dev, {in, l34}, {out, l1});
    CHECK(value() == 1.f);
    ops.reduce_full_into<MaxOp, float>(dev, {in, l34}, {out, l1});
    CHECK(value() == 3.f);

    const Layout transposed = Layout::strided({4, 3}, {1, 4}, 0); // :135-145
    ops.reduce_full_into<SumOp, float>(dev, {in, transposed}, {out, l1});
    CHECK(value() == 24.f);
    ops.reduce_full_into<ProdOp, float>(dev, {in, transposed}, {out, l1});
    CHECK(value() == 1728.f);

    auto nine = dev.upload(std::vector<float>{1, 2, 3, 4, 5, 6, 7, 8, 9});
    const Layout diag = Layout::strided({3}, {4}, 0); // :147-171
    ops.reduce_full_into<SumOp, float>(dev, {nine, diag}, {out, l1});
    CHECK(value() == 15.f);

    // Prepared handle observes later writes (:173-208).
    auto plan = ops.prepare_reduce_full<ProdOp, float>(dev, {in, l34}, {out, l1});
    dev.write_buffer(in, std::vector<float>(12, 2.f));
    ops.dispatch_full(dev, plan);
    CHECK(value() == 4096.f);

    // A 2-element output is rejected and left untouched (:213-231).
    auto two = dev.upload(std::vector<float>{-1.f, -2.f});
    const Layout l2 = Layout::c_contiguous({2});
    expect_error(ErrorKind::DispatchFailed, "full reduction output must have exactly 1 element",
                 [&] { ops.reduce_full_into<SumOp, float>(dev, {in, l34}, {two, l2}); });
    CHECK(same(dev.download_owned(two), std::vector<float>{-1.f, -2.f}));
}

// --------------------------------------------- axis_reduction.rs:58-552
void axis_reduction_contract(RocmDevice &dev) {
    RocmAxisReductionOps ops;
    std::vector<float> x(12);
    std::iota(x.begin(), x.end(), 1.f);
    auto in = dev.upload(x);
    const Layout l34 = Layout::c_contiguous({3, 4});
    const Layout o0 = Layout::c_contiguous({1, 4}), o1 = Layout::c_contiguous({3, 1});
    auto r0 = dev.alloc_zeroed<float>(4);
    auto r1 = dev.alloc_zeroed<float>(3);

    ops.prod_axis_into(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    CHECK(same(dev.download_owned(r0), std::vector<float>{45, 120, 231, 384}));
    ops.prod_axis_into(dev, StridedView<float>{in, l34}, 1, StridedView<float>{r1, o1});
    CHECK(same(dev.download_owned(r1), std::vector<float>{24, 1680, 11880}));
    ops.reduce_axis_into<SumOp>(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    CHECK(same(dev.download_owned(r0), std::vector<float>{15, 18, 21, 24}));
    ops.min_axis_into(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    CHECK(same(dev.download_owned(r0), std::vector<float>{1, 2, 3, 4}));
    ops.max_axis_into(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    CHECK(same(dev.download_owned(r0), std::vector<float>{9, 10, 11, 12}));
    ops.min_axis_into(dev, StridedView<float>{in, l34}, 1, StridedView<float>{r1, o1});
    CHECK(same(dev.download_owned(r1), std::vector<float>{1, 5, 9}));
    ops.max_axis_into(dev, StridedView<float>{in, l34}, 1, StridedView<float>{r1, o1});
    CHECK(same(dev.download_owned(r1), std::vector<float>{4, 8, 12}));
    ops.mean_axis_into(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    CHECK(same(dev.download_owned(r0), std::vector<float>{5, 6, 7, 8}));
    ops.mean_axis_into(dev, StridedView<float>{in, l34}, 1, StridedView<float>{r1, o1});
    CHECK(same(dev.download_owned(r1), std::vector<float>{2.5f, 6.5f, 10.5f}));

    const Layout transposed = Layout::strided({4, 3}, {1, 4}, 0);
    auto t1 = dev.alloc_zeroed<float>(4);
    const Layout to1 = Layout::c_contiguous({4, 1});
    ops.prod_axis_into(dev, StridedView<float>{in, transposed}, 1, StridedView<float>{t1, to1});
    CHECK(same(dev.download_owned(t1), std::vector<float>{45, 120, 231, 384}));

    auto plan = ops.prepare_reduce_axis_into<ProdOp>(dev, StridedView<float>{in, l34}, 0, StridedView<float>{r0, o0});
    dev.write_buffer(in, std::vector<float>(12, 2.f));
    plan.dispatch();
    CHECK(same(dev.download_owned(r0), std::vector<float>{8, 8, 8, 8}));

    expect_error(ErrorKind::DispatchFailed, "axis reduction output buffer must not alias input buffer",
                 [&] { ops.reduce_axis_into<SumOp>(dev, StridedView<float>{in, l34}, 0, StridedView<float>{in, o0}); });
}

// ------------------------------------------------------- scan.rs:45-205
void scan_contract(RocmDevice &dev) {
    RocmScanOps ops;
    auto in = dev.upload(rows_fixture());
    const Layout l34 = Layout::c_contiguous({3, 4});
    auto out = dev.alloc_zeroed<float>(12);
    auto rep = [](std::vector<float> row) {
        std::vector<float> v;
        for (int r = 0; r < 3; ++r) v.insert(v.end(), row.begin(), row.end());
        return v;
    };
    ops.scan_axis_into<CumSumOp, float>(dev, {in, l34}, 1, ScanDirection::Forward, {out, l34});
    CHECK(same(dev.download_owned(out), rep({1, 3, 6, 8})));
    ops.scan_axis_into<CumSumOp, float>(dev, {in, l34}, 1, ScanDirection::Reverse, {out, l34});
    CHECK(same(dev.download_owned(out), rep({8, 7, 5, 2})));
    ops.scan_axis_into<CumProdOp, float>(dev, {in, l34}, 1, ScanDirection::Forward, {out, l34});
    CHECK(same(dev.download_owned(out), rep({1, 2, 6, 12})));
    ops.scan_axis_into<CumSumOp, float>(dev, {in, l34}, 0, ScanDirection::Forward, {out, l34});
    CHECK(same(dev.download_owned(out), std::vector<float>{1, 2, 3, 2, 2, 4, 6, 4, 3, 6, 9, 6}));

    const std::vector<float> before = dev.download_owned(out);
    expect_error(ErrorKind::DispatchFailed, "scan axis 2 is out of bounds",
                 [&] { ops.scan_axis_into<CumSumOp, float>(dev, {in, l34}, 2, ScanDirection::Forward, {out, l34}); });
    CHECK(same(dev.download_owned(out), before)); // untouched (:129-149)

    auto plan = ops.prepare_scan_axis<CumSumOp, float>(dev, {in, l34}, 1, ScanDirection::Forward, {out, l34});
    dev.write_buffer(in, std::vector<float>(12, 1.f));
    ops.dispatch_scan(dev, plan);
    CHECK(same(dev.download_owned(out), rep({1, 2, 3, 4})));
}

// ----------------------------------- rocm tests/contract.rs:1533-1717 (i32)
void rocm_scan_contract(RocmDevice &dev) {
    RocmScanOps ops;
    auto in = dev.upload(std::vector<int32_t>{1, 2, 3, 4, 5, 6, 7, 8});
    const Layout l24 = Layout::c_contiguous({2, 4});
    auto out = dev.alloc_zeroed<int32_t>(8);
    auto run = [&](auto op, uint32_t axis, ScanDirection dir) {
        ops.scan_axis_into<decltype(op), int32_t>(dev, {in, l24}, axis, dir, {out, l24});
        return dev.download_owned(out);
    };
    using V = std::vector<int32_t>;
    CHECK(same(run(CumSumOp{}, 1, ScanDirection::Forward), V{1, 3, 6, 10, 5, 11, 18, 26}));
    CHECK(same(run(CumSumOp{}, 1, ScanDirection::Reverse), V{10, 9, 7, 4, 26, 21, 15, 8}));
    CHECK(same(run(CumSumOp{}, 0, ScanDirection::Reverse), V{6, 8, 10, 12, 5, 6, 7, 8}));
    CHECK(same(run(CumSumOp{}, 0, ScanDirection::Forward), V{1, 2, 3, 4, 6, 8, 10, 12}));
    CHECK(same(run(CumProdOp{}, 1, ScanDirection::Forward), V{1, 2, 6, 24, 5, 30, 210, 1680}));
    CHECK(same(run(CumProdOp{}, 0, ScanDirection::Forward), V{1, 2, 3, 4, 5, 12, 21, 32}));
    CHECK(same(run(CumProdOp{}, 1, ScanDirection::Reverse), V{24, 24, 12, 4, 1680, 336, 56, 8}));
    CHECK(same(run(CumProdOp{}, 0, ScanDirection::Reverse), V{5, 12, 21, 32, 5, 6, 7, 8}));

    // 1 x 1025 of (i % 7) - 3 against a sequential scan.
    V x(1025), want(1025);
    for (int i = 0; i < 1025; ++i) x[i] = i % 7 - 3;
    std::partial_sum(x.begin(), x.end(), want.begin());
    auto lin = dev.upload(x);
    auto lout = dev.alloc_zeroed<int32_t>(1025);
    const Layout l = Layout::c_contiguous({1, 1025});
    ops.scan_axis_into<CumSumOp, int32_t>(dev, {lin, l}, 1, ScanDirection::Forward, {lout, l});
    CHECK(same(dev.download_owned(lout), want));
}

// ------------------------------- rocm tests/contract.rs:811-933 (u32 reduce)
void rocm_reduce_contract(RocmDevice &dev) {
    RocmFullReductionOps ops;
    for (uint64_t n : {513ull, 1027ull}) {
        std::vector<uint32_t> x(n);
        for (uint64_t i = 0; i < n; ++i) x[i] = (uint32_t)(i % 17);
        auto in = dev.upload(x);
        auto out = dev.alloc_zeroed<uint32_t>(1);
        const Layout l = Layout::c_contiguous({n}), l1 = Layout::c_contiguous({1});
        ops.reduce_full_into<SumOp, uint32_t>(dev, {in, l}, {out, l1});
        CHECK(dev.download_owned(out)[0] == std::accumulate(x.begin(), x.end(), 0u));
        ops.reduce_full_into<MinOp, uint32_t>(dev, {in, l}, {out, l1});
        CHECK(dev.download_owned(out)[0] == 0u);
        ops.reduce_full_into<MaxOp, uint32_t>(dev, {in, l}, {out, l1});
        CHECK(dev.download_owned(out)[0] == 16u);
        // Prepared min and max submitted as one batch (prepared_reduction.rs:
        // 164-174; cuda tests/contract.rs:717-726 holds the same clause).
        auto out_min = dev.alloc_zeroed<uint32_t>(1), out_max = dev.alloc_zeroed<uint32_t>(1);
        auto pmin = ops.prepare_reduce_full<MinOp, uint32_t>(dev, {in, l}, {out_min, l1});
        auto pmax = ops.prepare_reduce_full<MaxOp, uint32_t>(dev, {in, l}, {out_max, l1});
        submit_prepared_reduction_batch({&pmin, &pmax});
        CHECK(dev.download_owned(out_min)[0] == 0u);
        CHECK(dev.download_owned(out_max)[0] == 16u);
    }
    auto empty = dev.alloc_zeroed<uint32_t>(0);
    auto out = dev.upload(std::vector<uint32_t>{7});
    const Layout l0 = Layout::c_contiguous({0}), l1 = Layout::c_contiguous({1});
    ops.reduce_full_into<SumOp, uint32_t>(dev, {empty, l0}, {out, l1});
    CHECK(dev.download_owned(out)[0] == 0u); // empty sum -> identity (:848-857)
}

// --------------------------------------------- dense_vector.rs:36-184
void dense_vector_contract(RocmDevice &dev) {
    RocmDenseVectorOps ops;
    using V = std::vector<float>;
    auto source = dev.upload(V{1, 2, 3, 4});
    auto target = dev.alloc_zeroed<float>(4);
    ops.copy_vector(dev, source, target);
    CHECK(same(dev.download_owned(target), V{1, 2, 3, 4}));
    auto short_target = dev.alloc_zeroed<float>(3);
    expect_error(ErrorKind::LengthMismatch, "", [&] { ops.copy_vector(dev, source, short_target); });
    ops.scale_vector(dev, target, 2.0f);
    CHECK(same(dev.download_owned(target), V{2, 4, 6, 8}));
    auto y = dev.upload(V{4, 5, 6, 8});
    ops.axpy(dev, y, source, 2.0f);
    CHECK(same(dev.download_owned(y), V{6, 9, 12, 16}));
    auto z = dev.upload(V{4, 5, 6, 8});
    ops.xpay(dev, z, source, 2.0f);
    CHECK(same(dev.download_owned(z), V{9, 12, 15, 20}));
    auto left = dev.upload(V{8, 6, 4, 2}), right = dev.upload(V{2, 4, 8, 0.5f});
    auto out = dev.alloc_zeroed<float>(4);
    ops.subtract_into(dev, left, right, out);
    CHECK(same(dev.download_owned(out), V{6, 2, -4, 1.5f}));
    ops.add_into(dev, left, right, out);
    CHECK(same(dev.download_owned(out), V{10, 10, 12, 2.5f}));
    ops.multiply_into(dev, left, right, out);
    CHECK(same(dev.download_owned(out), V{16, 24, 32, 1}));
    ops.divide_into(dev, left, right, out);
    CHECK(same(dev.download_owned(out), V{4, 1.5f, 0.5f, 4}));
    auto a = dev.upload(V{1, 2, 3, 4}), b = dev.upload(V{8, 4, 2, 1});
    auto pd = ops.prepare_dot(dev, a, b);
    CHECK(ops.dot_prepared(dev, pd, a, b) == 26.0f);
    CHECK(ops.dot_prepared(dev, pd, a, b) == 26.0f);
    dev.write_buffer(a, V{2, 2, 2, 2});
    CHECK(ops.dot_prepared(dev, pd, a, b) == 30.0f);
    auto foreign = dev.upload(V{1, 1, 1, 1});
    expect_error(ErrorKind::DispatchFailed, "prepared dot received different device allocations",
                 [&] { ops.dot_prepared(dev, pd, foreign, b); });
    auto v = dev.upload(V{2, 3, 6, 0});
    CHECK(ops.norm_l1(dev, v) == 11.0f);
    CHECK(ops.norm_max(dev, v) == 6.0f);
    auto pn = ops.prepare_norm_l2(dev, v);
    CHECK(std::fabs(ops.norm_l2_prepared(dev, pn, v) - 7.0f) <= 7.0f * 1.1920929e-7f);
    dev.write_buffer(v, V{9, 12, 20, 0});
    CHECK(std::fabs(ops.norm_l2_prepared(dev, pn, v) - 25.0f) <= 25.0f * 1.1920929e-7f);
}

// ----------------------------------- rocm tests/contract.rs:2615-2737
void map_reduction_contract(RocmDevice &dev) {
    auto m = dev.upload(std::vector<int32_t>{-3, 4, -5, 6, -7, 8});
    const Layout lm = Layout::c_contiguous({2, 3});
    CHECK(dev.download_owned(norm_l1<int32_t>(dev, {m, lm}))[0] == 33);
    CHECK(dev.download_owned(norm_max<int32_t>(dev, {m, lm}))[0] == 8);
    auto lhs = dev.upload(std::vector<int32_t>{99, 1, 2, 3, 4, 5});
    auto rhs = dev.upload(std::vector<int32_t>{6, 7, 8, 9, 10});
    const Layout ll = Layout::strided({5}, {1}, 1), lr = Layout::c_contiguous({5});
    CHECK(dev.download_owned(dot<int32_t>(dev, {lhs, ll}, {rhs, lr}))[0] == 130);
    auto t = dev.upload(std::vector<int32_t>{1, 2, 3, 4, 5, 6, 7, 8, 9});
    const Layout l33 = Layout::c_contiguous({3, 3});
    CHECK(dev.download_owned(trace<int32_t>(dev, {t, l33}))[0] == 15);
    auto l2 = dev.upload(std::vector<float>{3, 4});
    const Layout l2l = Layout::c_contiguous({2});
    CHECK(dev.download_owned(norm_l2<float>(dev, {l2, l2l}))[0] == 5.0f);
    const Layout wrong = Layout::c_contiguous({4});
    expect_error(ErrorKind::DispatchFailed, "dot product shape mismatch",
                 [&] { dot<int32_t>(dev, {lhs, ll}, {rhs, wrong}); });
    expect_error(ErrorKind::DispatchFailed, "trace requires a square matrix", [&] { trace<int32_t>(dev, {m, lm}); });
}

// ------------------------------------------ the path's additions, at size
uint64_t splitmix(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void additions_at_size(RocmDevice &dev) {
    // u32 exclusive scan over several 32768-element tiles and superblocks.
    const uint64_t n = (3u << 21) + 12345;
    std::vector<uint32_t> x(n), want(n);
    for (uint64_t i = 0; i < n; ++i) x[i] = (uint32_t)(splitmix(2, i) >> 32);
    uint32_t acc = 0;
    for (uint64_t i = 0; i < n; ++i) {
        want[i] = acc;
        acc += x[i];
    }
    auto in = dev.upload(x);
    auto out = dev.alloc_zeroed<uint32_t>(n);
    const Layout l = Layout::c_contiguous({n});
    RocmScanOps().scan_axis_into<CumSumOp, uint32_t>(dev, {in, l}, 0, ScanDirection::Forward, {out, l},
                                                      ScanKind::Exclusive);
    CHECK(same(dev.download_owned(out), want));

    // f32 sum within 2*ceil(log2 n)*eps*sum|x| of an f64 accumulation.
    std::vector<float> f(n);
    double ref = 0.0, abs_sum = 0.0;
    for (uint64_t i = 0; i < n; ++i) {
        f[i] = (float)((int64_t)(splitmix(1, i) >> 40) - (1 << 23)) * (1.0f / (1 << 23));
        ref += f[i];
        abs_sum += std::fabs(f[i]);
    }
    auto fin = dev.upload(f);
    auto fout = dev.alloc_zeroed<float>(1);
    const Layout l1 = Layout::c_contiguous({1});
    RocmFullReductionOps().reduce_full_into<SumOp, float>(dev, {fin, l}, {fout, l1});
    const double bound = 2.0 * std::ceil(std::log2((double)n)) * std::ldexp(1.0, -23) * abs_sum;
    CHECK(std::fabs((double)dev.download_owned(fout)[0] - ref) <= bound);

    // Argmax ties resolve to the lowest index.
    std::vector<float> t(100000, 1.0f);
    t[777] = 5.0f;
    t[4242] = 5.0f;
    t[99999] = 5.0f;
    auto tin = dev.upload(t);
    auto idx = dev.alloc_zeroed<uint32_t>(1);
    const Layout lt = Layout::c_contiguous({t.size()});
    RocmFullReductionOps().argmax_full_into<float>(dev, {tin, lt}, idx);
    CHECK(dev.download_owned(idx)[0] == 777u);

    // Fused rows: sum, max, argmax of fmaf(0.5, x, 0.25) per row.
    const uint64_t rows = 64, cols = 1000;
    std::vector<float> m(rows * cols);
    for (uint64_t i = 0; i < m.size(); ++i) m[i] = (float)((int)(splitmix(3, i) % 2001) - 1000) / 7.0f;
    auto min_ = dev.upload(m);
    auto s = dev.alloc_zeroed<float>(rows), mx = dev.alloc_zeroed<float>(rows);
    auto am = dev.alloc_zeroed<uint32_t>(rows);
    const Affine pro{0.5f, 0.25f};
    RocmAxisReductionOps().reduce_rows_fused<float>(dev, min_, rows, cols, cols, &pro, &s, &mx, &am);
    auto gs = dev.download_owned(s), gm = dev.download_owned(mx);
    auto ga = dev.download_owned(am);
    for (uint64_t r = 0; r < rows; ++r) {
        double sum = 0.0, abs_sum_r = 0.0;
        float best = -std::numeric_limits<float>::max();
        uint32_t bi = 0;
        for (uint64_t c = 0; c < cols; ++c) {
            const float y = std::fma(0.5f, m[r * cols + c], 0.25f);
            sum += y;
            abs_sum_r += std::fabs(y);
            if (y > best) {
                best = y;
                bi = (uint32_t)c;
            }
        }
        const double b = 2.0 * std::ceil(std::log2((double)cols)) * std::ldexp(1.0, -23) * abs_sum_r;
        CHECK(std::fabs((double)gs[r] - sum) <= b);
        CHECK(gm[r] == best);
        CHECK(ga[r] == bi);
    }

    // Segmented sum, bit-exact, with empty segments.
    const uint64_t sn = 200000;
    std::vector<int32_t> v(sn);
    for (uint64_t i = 0; i < sn; ++i) v[i] = (int32_t)(splitmix(4, i) % 2001) - 1000;
    std::vector<uint32_t> off{0};
    for (uint64_t i = 0; off.back() < sn; ++i) {
        const uint64_t len = splitmix(5, i) % 600; // 0 gives an empty segment
        off.push_back((uint32_t)std::min<uint64_t>(sn, off.back() + len));
    }
    std::vector<int32_t> swant(off.size() - 1);
    for (size_t k = 0; k + 1 < off.size(); ++k) {
        uint32_t a = 0;
        for (uint32_t i = off[k]; i < off[k + 1]; ++i) a += (uint32_t)v[i];
        swant[k] = (int32_t)a;
    }
    auto vin = dev.upload(v);
    auto oin = dev.upload(off);
    auto sout = dev.alloc_zeroed<int32_t>(swant.size());
    RocmSegmentedReductionOps().segmented_sum_into<int32_t>(dev, vin, oin, sout);
    CHECK(same(dev.download_owned(sout), swant));
}

// ------------------------------------------- accelerator/device_api.rs
// A consumer kernel through the DeviceApi seam: compiled once per key (the
// source callback runs only on a miss), launched with a parameter block
// followed by operand addresses; a broken source is DispatchFailed.
void device_api_contract(RocmDevice &dev) {
    static const char *kSrc = R"(
struct Params { unsigned int n; unsigned int k; };
extern "C" __global__ void add_k(Params p, const unsigned int *x, unsigned int *y) {
    unsigned int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) y[i] = x[i] + p.k;
}
)";
    int calls = 0;
    auto source = [&]() {
        ++calls;
        return std::string(kSrc);
    };
    RocmDevice::Kernel k1 = dev.compile_cached("cpp-add-k", "add_k", source);
    RocmDevice::Kernel k2 = dev.compile_cached("cpp-add-k", "add_k", source);
    CHECK(k1 == k2 && calls == 1);
    struct Params {
        uint32_t n, k;
    };
    const uint32_t n = 1000;
    std::vector<uint32_t> x(n);
    for (uint32_t i = 0; i < n; ++i) x[i] = i * 7u;
    RocmBuffer<uint32_t> xb = dev.upload(x);
    RocmBuffer<uint32_t> yb = dev.alloc_zeroed<uint32_t>(n);
    dev.launch(k1, LaunchGeometry::linear((n + 127) / 128, 128), Params{n, 42u},
               {RocmDevice::device_ptr(xb), RocmDevice::device_ptr(yb)});
    dev.synchronize();
    std::vector<uint32_t> want(n);
    for (uint32_t i = 0; i < n; ++i) want[i] = i * 7u + 42u;
    CHECK(same(dev.download_owned(yb), want));
    CHECK(RocmDevice::buffers_alias(xb, xb) && !RocmDevice::buffers_alias(xb, yb));
    expect_error(ErrorKind::DispatchFailed, "hiprtcCompileProgram",
                 [&] { dev.compile_cached("cpp-broken", "broken", [] { return std::string("not c++ {"); }); });
    // ComputeDeviceCapabilities / require_limits
    const hx_device_limits lim = dev.device_limits();
    CHECK(lim.max_compute_invocations_per_workgroup == 1024 && lim.max_immediate_size == 0);
    CHECK(!dev.supports_device_feature(HX_FEATURE_SHADER_F64));
    hx_device_limits need = lim;
    need.max_compute_workgroup_storage_size = lim.max_compute_workgroup_storage_size + 1;
    expect_error(ErrorKind::DeviceUnavailable, "ROCm device limit max_compute_workgroup_storage_size",
                 [&] { RocmDevice::require_limits(lim, need); });
}

} // namespace

int main() {
    int32_t count = 0;
    if (hx_device_count(&count) != HX_OK || count == 0) {
        std::printf("no ROCm device: skipped\n");
        return 77;
    }
    RocmDevice dev = RocmDevice::try_default();
    const Topology topo = dev.topology();
    std::printf("device %s (%s), %u CUs, backend %s\n", topo.name.c_str(), topo.arch.c_str(), topo.compute_units,
                dev.backend_name());
    const std::pair<const char *, std::function<void(RocmDevice &)>> clauses[] = {
        {"transfer", transfer_contract},
        {"full_reduction", full_reduction_contract},
        {"axis_reduction", axis_reduction_contract},
        {"scan", scan_contract},
        {"rocm_scan_i32", rocm_scan_contract},
        {"rocm_reduce_u32", rocm_reduce_contract},
        {"dense_vector", dense_vector_contract},
        {"rocm_map_reduction", map_reduction_contract},
        {"additions_at_size", additions_at_size},
        {"device_api", device_api_contract},
    };
    for (const auto &c : clauses) {
        const int before = g_failures;
        try {
            c.second(dev);
        } catch (const Error &e) {
            ++g_failures;
            std::printf("  FAIL: unexpected error kind %d: %s\n", (int)e.kind(), e.what());
        }
        std::printf("%-20s %s\n", c.first, g_failures == before ? "ok" : "FAILED");
        std::fflush(stdout);
    }
    std::printf("%d checks, %d failures\n", g_checks, g_failures);
    return g_failures == 0 ? 0 : 1;
}
