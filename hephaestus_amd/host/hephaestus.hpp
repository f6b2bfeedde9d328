// hephaestus.hpp — C++17 host interface over the C ABI (include/hx.h).
//
// Mirrors the reference's Rust seams so C++ callers read like the
// reference's own code:
//   ComputeDevice / ComputeDeviceAcquisition  crates/hephaestus-core/src/domain/device.rs:90-281
//   DeviceBuffer<T>                           crates/hephaestus-core/src/domain/buffer.rs:7-19
//   StridedView / Layout                      crates/hephaestus-core/src/domain/view.rs:27-41
//   FullReductionOps                          crates/hephaestus-core/src/domain/reduction.rs:243-309
//   AxisReductionOps                          crates/hephaestus-core/src/domain/reduction.rs:74-223
//   ScanOps / ScanDirection                   crates/hephaestus-core/src/domain/scan.rs:36-264
//   DenseVectorOps                            crates/hephaestus-core/src/domain/vector.rs:57-200
//   dot / trace / norms                       crates/hephaestus-rocm/src/application/linalg/norms.rs:394-490
//   DeviceApi / LaunchGeometry                crates/hephaestus-core/src/domain/accelerator/device_api.rs:10-133
//   ComputeDeviceCapabilities / limits        crates/hephaestus-core/src/domain/device.rs:38-80,225-238
//   HephaestusError                           crates/hephaestus-core/src/domain/error.rs:8-58
// Errors are thrown as hephaestus::Error carrying the variant and the
// native message; every entry point validates before it writes, so a
// thrown call leaves its outputs untouched.  Header-only; link
// libhephaestus_amd.so.
#pragma once

#include "../../include/hx.h"

#include <array>
#include <cstdint>
#include <exception>
#include <functional>
#include <initializer_list>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

namespace hephaestus {

// ------------------------------------------------------------------ errors
enum class ErrorKind {
    AdapterUnavailable = HX_ERR_ADAPTER_UNAVAILABLE,
    DeviceUnavailable = HX_ERR_DEVICE_UNAVAILABLE,
    AllocationFailed = HX_ERR_ALLOCATION_FAILED,
    LengthMismatch = HX_ERR_LENGTH_MISMATCH,
    DispatchFailed = HX_ERR_DISPATCH_FAILED,
    InvalidConfiguration = HX_ERR_INVALID_CONFIGURATION,
    TransferFailed = HX_ERR_TRANSFER_FAILED,
};

class Error : public std::runtime_error {
  public:
    Error(ErrorKind kind, const std::string &msg, uint64_t host_len = 0, uint64_t device_len = 0)
        : std::runtime_error(msg), kind_(kind), host_len_(host_len), device_len_(device_len) {}
    ErrorKind kind() const { return kind_; }
    // LengthMismatch { host_len, device_len } (error.rs:30-36).
    uint64_t host_len() const { return host_len_; }
    uint64_t device_len() const { return device_len_; }

  private:
    ErrorKind kind_;
    uint64_t host_len_, device_len_;
};

inline void check(hx_status s) {
    if (s == HX_OK) return;
    uint64_t h = 0, d = 0;
    if (s == HX_ERR_LENGTH_MISMATCH) hx_last_length_mismatch(&h, &d);
    throw Error(static_cast<ErrorKind>(s), hx_last_error_message(), h, d);
}

// ------------------------------------------------------------ element types
template <typename T> struct Scalar;
template <> struct Scalar<float> { static constexpr hx_dtype dtype = HX_DTYPE_F32; };
template <> struct Scalar<uint32_t> { static constexpr hx_dtype dtype = HX_DTYPE_U32; };
template <> struct Scalar<int32_t> { static constexpr hx_dtype dtype = HX_DTYPE_I32; };

// ------------------------------------------------------- operator markers
// core ops.rs:735-803 (SumOp ... CumProdOp); MeanOp and ArgMaxOp select the
// mean / argmax kernels.
struct SumOp { static constexpr hx_op code = HX_OP_SUM; };
struct ProdOp { static constexpr hx_op code = HX_OP_PROD; };
struct MinOp { static constexpr hx_op code = HX_OP_MIN; };
struct MaxOp { static constexpr hx_op code = HX_OP_MAX; };
struct MeanOp { static constexpr hx_op code = HX_OP_MEAN; };
struct ArgMaxOp { static constexpr hx_op code = HX_OP_ARGMAX; };
struct CumSumOp { static constexpr hx_op code = HX_OP_SUM; };
struct CumProdOp { static constexpr hx_op code = HX_OP_PROD; };

enum class ScanDirection { Forward = HX_SCAN_FORWARD, Reverse = HX_SCAN_REVERSE };
enum class ScanKind { Inclusive = HX_SCAN_INCLUSIVE, Exclusive = HX_SCAN_EXCLUSIVE };

// Fused prologue y = fmaf(a, x, b) (f32 only).
struct Affine {
    float a = 1.0f, b = 0.0f;
};

// ------------------------------------------------------------------ layout
// Shape, strides (elements, may be negative) and offset of a view over a
// linear buffer; rank <= 4.
class Layout {
  public:
    static Layout c_contiguous(std::vector<uint64_t> shape) {
        Layout l;
        l.raw_.rank = static_cast<uint32_t>(shape.size());
        int64_t stride = 1;
        for (size_t d = shape.size(); d-- > 0;) {
            l.raw_.shape[d] = shape[d];
            l.raw_.strides[d] = stride;
            stride *= static_cast<int64_t>(shape[d]);
        }
        return l;
    }
    static Layout strided(std::vector<uint64_t> shape, std::vector<int64_t> strides, uint64_t offset) {
        if (shape.size() != strides.size() || shape.size() > HX_MAX_RANK)
            throw Error(ErrorKind::InvalidConfiguration, "layout rejected: rank mismatch");
        Layout l;
        l.raw_.rank = static_cast<uint32_t>(shape.size());
        for (size_t d = 0; d < shape.size(); ++d) {
            l.raw_.shape[d] = shape[d];
            l.raw_.strides[d] = strides[d];
        }
        l.raw_.offset = offset;
        return l;
    }
    uint32_t rank() const { return raw_.rank; }
    uint64_t size() const {
        uint64_t n = 1;
        for (uint32_t d = 0; d < raw_.rank; ++d) n *= raw_.shape[d];
        return n;
    }
    const hx_layout *raw() const { return &raw_; }

  private:
    hx_layout raw_{};
};

class RocmDevice;

// ------------------------------------------------------------------ buffer
// RocmBuffer<T> (rocm infrastructure/buffer.rs:16-80): owns one device
// allocation of len() elements; a zero-length buffer holds no allocation.
template <typename T> class RocmBuffer {
  public:
    RocmBuffer() = default;
    RocmBuffer(const RocmBuffer &) = delete;
    RocmBuffer &operator=(const RocmBuffer &) = delete;
    RocmBuffer(RocmBuffer &&o) noexcept { *this = std::move(o); }
    RocmBuffer &operator=(RocmBuffer &&o) noexcept {
        release();
        dev_ = o.dev_;
        ptr_ = o.ptr_;
        len_ = o.len_;
        o.ptr_ = nullptr;
        o.len_ = 0;
        return *this;
    }
    ~RocmBuffer() { release(); }

    uint64_t len() const { return len_; }
    bool is_empty() const { return len_ == 0; }
    T *device_ptr() const { return ptr_; }

  private:
    friend class RocmDevice;
    RocmBuffer(hx_device *dev, T *ptr, uint64_t len) : dev_(dev), ptr_(ptr), len_(len) {}
    void release() {
        if (ptr_ && dev_) hx_free(dev_, ptr_);
        ptr_ = nullptr;
    }
    hx_device *dev_ = nullptr;
    T *ptr_ = nullptr;
    uint64_t len_ = 0;
};

template <typename T> struct StridedView {
    const RocmBuffer<T> &buffer;
    const Layout &layout;
};

struct Topology {
    std::string name, arch;
    uint32_t compute_units = 0, warp_size = 0;
    uint64_t total_memory_bytes = 0;
};

// ------------------------------------------------------------------ device
// LaunchGeometry (device_api.rs:10-47): `groups` blocks of `width` lanes
// with `shared_bytes` of dynamic LDS.
struct LaunchGeometry {
    uint32_t groups, width, shared_bytes;
    static LaunchGeometry linear(uint32_t groups, uint32_t width) { return {groups, width, 0}; }
    static LaunchGeometry linear_shared(uint32_t groups, uint32_t width, uint32_t shared_bytes) {
        return {groups, width, shared_bytes};
    }
};

class RocmDevice {
  public:
    // ComputeDeviceAcquisition: the first device / a given ordinal.
    static RocmDevice try_default() { return try_with_ordinal(0); }
    static RocmDevice try_with_ordinal(int32_t ordinal) {
        hx_device *d = nullptr;
        check(hx_device_open(ordinal, &d));
        return RocmDevice(d);
    }
    static int32_t device_count() {
        int32_t n = 0;
        check(hx_device_count(&n));
        return n;
    }
    // ComputeDeviceAcquisition::try_acquire_device (ROCm acquisition.rs:9-18).
    static RocmDevice try_acquire_device(const hx_device_limits &required) {
        RocmDevice d = try_default();
        require_limits(d.device_limits(), required);
        return d;
    }
    static void require_limits(const hx_device_limits &actual, const hx_device_limits &required) {
        check(hx_require_limits(&actual, &required));
    }

    RocmDevice(RocmDevice &&o) noexcept : dev_(o.dev_) { o.dev_ = nullptr; }
    RocmDevice(const RocmDevice &) = delete;
    ~RocmDevice() {
        if (dev_) hx_device_close(dev_);
    }

    const char *backend_name() const { return "rocm"; }
    hx_device *raw() const { return dev_; }

    Topology topology() const {
        hx_device_info i{};
        check(hx_device_get_info(dev_, &i));
        return Topology{i.name, i.arch, i.compute_units, i.warp_size, i.total_memory_bytes};
    }
    void synchronize() { check(hx_synchronize(dev_)); }
    // ComputeDeviceCapabilities (ROCm capabilities.rs:5-21).
    hx_device_limits device_limits() const {
        hx_device_limits l{};
        check(hx_device_get_limits(dev_, &l));
        return l;
    }
    bool supports_device_feature(hx_device_feature f) const { return hx_device_supports_feature(dev_, f) != 0; }

    template <typename T> RocmBuffer<T> alloc_zeroed(uint64_t len) { return alloc<T>(len, true); }
    template <typename T> RocmBuffer<T> alloc_uninitialized(uint64_t len) { return alloc<T>(len, false); }

    template <typename T> RocmBuffer<T> upload(const std::vector<T> &host) {
        RocmBuffer<T> b = alloc_uninitialized<T>(host.size());
        write_buffer(b, host);
        return b;
    }
    template <typename T> void write_buffer(RocmBuffer<T> &b, const std::vector<T> &host) {
        check(hx_upload(dev_, b.device_ptr(), b.len(), host.data(), host.size(), sizeof(T)));
    }
    template <typename T> void write_sub_buffer(RocmBuffer<T> &b, uint64_t offset, const std::vector<T> &host) {
        check(hx_write_sub(dev_, b.device_ptr(), b.len(), offset, host.data(), host.size(), sizeof(T)));
    }
    template <typename T> void download(const RocmBuffer<T> &b, std::vector<T> &host) {
        check(hx_download(dev_, b.device_ptr(), b.len(), host.data(), host.size(), sizeof(T)));
    }
    template <typename T> std::vector<T> download_owned(const RocmBuffer<T> &b) {
        std::vector<T> host(b.len());
        download(b, host);
        return host;
    }
    template <typename T> void copy_buffer(const RocmBuffer<T> &src, RocmBuffer<T> &dst) {
        check(hx_copy(dev_, src.device_ptr(), src.len(), dst.device_ptr(), dst.len(), sizeof(T)));
    }

    // -- DeviceApi (device_api.rs:69-133) -------------------------------
    using Kernel = const hx_kernel *;
    using DevicePtr = void *;
    // compile_cached: `source` runs only on a cache miss.  An exception it
    // throws is caught before the C ABI and rethrown here.
    Kernel compile_cached(const std::string &key, const std::string &entry,
                          const std::function<std::string()> &source) {
        struct Ctx {
            const std::function<std::string()> *source;
            std::string text;
            std::exception_ptr error;
        } ctx{&source, {}, nullptr};
        hx_kernel *k = nullptr;
        const hx_status s = hx_kernel_compile_cached(
            dev_, key.data(), key.size(), entry.c_str(),
            [](void *c) -> const char * {
                Ctx *x = static_cast<Ctx *>(c);
                try {
                    x->text = (*x->source)();
                } catch (...) {
                    x->error = std::current_exception();
                    return nullptr;
                }
                return x->text.c_str();
            },
            &ctx, &k);
        if (ctx.error) std::rethrow_exception(ctx.error);
        check(s);
        return k;
    }
    template <typename T> static DevicePtr device_ptr(const RocmBuffer<T> &b) { return b.device_ptr(); }
    template <typename T> static bool buffers_alias(const RocmBuffer<T> &a, const RocmBuffer<T> &b) {
        return hx_buffers_alias(a.device_ptr(), a.len() * sizeof(T), b.device_ptr(), b.len() * sizeof(T)) != 0;
    }
    // launch: `params` by value as the kernel's first argument, then each
    // operand's address.
    template <typename P>
    void launch(Kernel kernel, const LaunchGeometry &g, const P &params, std::initializer_list<DevicePtr> operands) {
        static_assert(std::is_trivially_copyable<P>::value, "the parameter block is copied bytewise");
        std::vector<void *> ops(operands);
        check(hx_kernel_launch(dev_, kernel, g.groups, g.width, g.shared_bytes, &params, sizeof(P), ops.data(),
                               ops.size(), nullptr));
    }

  private:
    explicit RocmDevice(hx_device *d) : dev_(d) {}
    template <typename T> RocmBuffer<T> alloc(uint64_t len, bool zeroed) {
        void *p = nullptr;
        check(hx_alloc(dev_, len * sizeof(T), zeroed ? 1u : 0u, &p));
        return RocmBuffer<T>(dev_, static_cast<T *>(p), len);
    }
    hx_device *dev_ = nullptr;
};

// ------------------------------------------------------------------- plans
// The Prepared associated types: a dispatch bound to its operands, owning
// its workspace; dispatch() re-reads the bound buffers every time.
class PreparedPlan {
  public:
    explicit PreparedPlan(hx_plan *p) : plan_(p) {}
    PreparedPlan(PreparedPlan &&o) noexcept : plan_(o.plan_) { o.plan_ = nullptr; }
    PreparedPlan(const PreparedPlan &) = delete;
    ~PreparedPlan() {
        if (plan_) hx_plan_destroy(plan_);
    }
    void dispatch(hx_stream stream = nullptr) const { check(hx_plan_dispatch(plan_, stream)); }
    uint64_t workspace_bytes() const {
        uint64_t b = 0;
        check(hx_plan_workspace_bytes(plan_, &b));
        return b;
    }
    hx_plan *handle() const { return plan_; }

  private:
    hx_plan *plan_ = nullptr;
};

// submit_prepared_reduction_batch (rocm application/prepared_reduction.rs:
// 164-174): the plans run in order on one stream, no host sync in between.
inline void submit_prepared_reduction_batch(std::initializer_list<const PreparedPlan *> plans,
                                            hx_stream stream = nullptr) {
    std::vector<hx_plan *> handles;
    handles.reserve(plans.size());
    for (const PreparedPlan *p : plans) handles.push_back(p->handle());
    check(hx_plan_dispatch_batch(handles.data(), handles.size(), stream));
}
// submit_prepared_axis_reduction_batch (rocm application/
// prepared_axis_reduction.rs:84-92): the same for prepared axis reductions.
inline void submit_prepared_axis_reduction_batch(RocmDevice &, std::initializer_list<const PreparedPlan *> plans,
                                                 hx_stream stream = nullptr) {
    submit_prepared_reduction_batch(plans, stream);
}

namespace detail {
inline const hx_affine *affine(const Affine *p, hx_affine &storage) {
    if (!p) return nullptr;
    storage = hx_affine{p->a, p->b, 1u, 0u};
    return &storage;
}
} // namespace detail

// ---------------------------------------------------------- FullReductionOps
class RocmFullReductionOps {
  public:
    template <typename Op, typename T>
    void reduce_full_into(RocmDevice &dev, StridedView<T> input, StridedView<T> output,
                          const Affine *prologue = nullptr, hx_stream stream = nullptr) const {
        hx_affine a;
        check(hx_reduce_full(dev.raw(), Op::code, Scalar<T>::dtype, input.buffer.device_ptr(), input.buffer.len(),
                             input.layout.raw(), output.buffer.device_ptr(), output.buffer.len(),
                             output.layout.raw(), detail::affine(prologue, a), stream));
    }
    template <typename Op, typename T>
    PreparedPlan prepare_reduce_full(RocmDevice &dev, StridedView<T> input, StridedView<T> output,
                                     const Affine *prologue = nullptr) const {
        hx_affine a;
        hx_plan *p = nullptr;
        check(hx_prepare_reduce_full(dev.raw(), Op::code, Scalar<T>::dtype, input.buffer.device_ptr(),
                                     input.buffer.len(), input.layout.raw(), output.buffer.device_ptr(),
                                     output.buffer.len(), output.layout.raw(), detail::affine(prologue, a), &p));
        return PreparedPlan(p);
    }
    void dispatch_full(RocmDevice &, const PreparedPlan &plan, hx_stream stream = nullptr) const {
        plan.dispatch(stream);
    }
    // Index of the maximum (ties to the lowest index, NaN ignored).
    template <typename T>
    void argmax_full_into(RocmDevice &dev, StridedView<T> input, RocmBuffer<uint32_t> &index,
                          RocmBuffer<T> *value = nullptr, const Affine *prologue = nullptr,
                          hx_stream stream = nullptr) const {
        if (index.len() != 1) throw Error(ErrorKind::DispatchFailed, "argmax index output must hold 1 element");
        if (value && value->len() != 1) throw Error(ErrorKind::DispatchFailed, "argmax value output must hold 1 element");
        hx_affine a;
        check(hx_argmax_full(dev.raw(), Scalar<T>::dtype, input.buffer.device_ptr(), input.buffer.len(),
                             input.layout.raw(), value ? value->device_ptr() : nullptr, index.device_ptr(),
                             detail::affine(prologue, a), stream));
    }
};

// ---------------------------------------------------------- AxisReductionOps
class RocmAxisReductionOps {
  public:
    template <typename Op, typename T, typename U>
    void reduce_axis_into(RocmDevice &dev, StridedView<T> input, uint32_t axis, StridedView<U> output,
                          hx_stream stream = nullptr) const {
        static_assert(std::is_same<T, U>::value || std::is_same<Op, ArgMaxOp>::value,
                      "output element type must match the input (u32 for argmax)");
        check(hx_reduce_axis(dev.raw(), Op::code, Scalar<T>::dtype, input.buffer.device_ptr(), input.buffer.len(),
                             input.layout.raw(), axis, output.buffer.device_ptr(), output.buffer.len(),
                             output.layout.raw(), stream));
    }
    template <typename T> void prod_axis_into(RocmDevice &d, StridedView<T> in, uint32_t axis, StridedView<T> out) const {
        reduce_axis_into<ProdOp>(d, in, axis, out);
    }
    template <typename T> void min_axis_into(RocmDevice &d, StridedView<T> in, uint32_t axis, StridedView<T> out) const {
        reduce_axis_into<MinOp>(d, in, axis, out);
    }
    template <typename T> void max_axis_into(RocmDevice &d, StridedView<T> in, uint32_t axis, StridedView<T> out) const {
        reduce_axis_into<MaxOp>(d, in, axis, out);
    }
    template <typename T> void mean_axis_into(RocmDevice &d, StridedView<T> in, uint32_t axis, StridedView<T> out) const {
        reduce_axis_into<MeanOp>(d, in, axis, out);
    }
    template <typename Op, typename T, typename U>
    PreparedPlan prepare_reduce_axis_into(RocmDevice &dev, StridedView<T> input, uint32_t axis,
                                          StridedView<U> output) const {
        hx_plan *p = nullptr;
        check(hx_prepare_reduce_axis(dev.raw(), Op::code, Scalar<T>::dtype, input.buffer.device_ptr(),
                                     input.buffer.len(), input.layout.raw(), axis, output.buffer.device_ptr(),
                                     output.buffer.len(), output.layout.raw(), &p));
        return PreparedPlan(p);
    }
    // Sum, max and argmax of y = fmaf(a, x, b) per row from ONE read; any
    // output may be null.
    template <typename T>
    void reduce_rows_fused(RocmDevice &dev, const RocmBuffer<T> &input, uint64_t rows, uint64_t cols,
                           uint64_t row_stride, const Affine *prologue, RocmBuffer<T> *out_sum,
                           RocmBuffer<T> *out_max, RocmBuffer<uint32_t> *out_argmax,
                           hx_stream stream = nullptr) const {
        uint64_t out_len = rows;
        if (out_sum) out_len = out_sum->len();
        else if (out_max) out_len = out_max->len();
        else if (out_argmax) out_len = out_argmax->len();
        hx_affine a;
        check(hx_reduce_rows(dev.raw(), Scalar<T>::dtype, input.device_ptr(), input.len(), rows, cols, row_stride, 0,
                             detail::affine(prologue, a), out_sum ? out_sum->device_ptr() : nullptr,
                             out_max ? out_max->device_ptr() : nullptr,
                             out_argmax ? out_argmax->device_ptr() : nullptr, out_len, stream));
    }
    // The prepared form (prepared_axis_reduction.rs:20-222): dispatch
    // re-reads the bound input and allocates nothing.
    template <typename T>
    PreparedPlan prepare_reduce_rows_fused(RocmDevice &dev, const RocmBuffer<T> &input, uint64_t rows,
                                           uint64_t cols, uint64_t row_stride, const Affine *prologue,
                                           RocmBuffer<T> *out_sum, RocmBuffer<T> *out_max,
                                           RocmBuffer<uint32_t> *out_argmax) const {
        uint64_t out_len = rows;
        if (out_sum) out_len = out_sum->len();
        else if (out_max) out_len = out_max->len();
        else if (out_argmax) out_len = out_argmax->len();
        hx_affine a;
        hx_plan *p = nullptr;
        check(hx_prepare_reduce_rows(dev.raw(), Scalar<T>::dtype, input.device_ptr(), input.len(), rows, cols,
                                     row_stride, 0, detail::affine(prologue, a),
                                     out_sum ? out_sum->device_ptr() : nullptr,
                                     out_max ? out_max->device_ptr() : nullptr,
                                     out_argmax ? out_argmax->device_ptr() : nullptr, out_len, &p));
        return PreparedPlan(p);
    }
};

// ------------------------------------------------------------------ ScanOps
class RocmScanOps {
  public:
    template <typename Op, typename T>
    void scan_axis_into(RocmDevice &dev, StridedView<T> input, uint32_t axis, ScanDirection direction,
                        StridedView<T> output, ScanKind kind = ScanKind::Inclusive,
                        hx_stream stream = nullptr) const {
        check(hx_scan(dev.raw(), Op::code, Scalar<T>::dtype, static_cast<hx_scan_kind>(kind),
                      static_cast<hx_scan_direction>(direction), input.buffer.device_ptr(), input.buffer.len(),
                      input.layout.raw(), axis, output.buffer.device_ptr(), output.buffer.len(),
                      output.layout.raw(), stream));
    }
    template <typename Op, typename T>
    PreparedPlan prepare_scan_axis(RocmDevice &dev, StridedView<T> input, uint32_t axis, ScanDirection direction,
                                   StridedView<T> output, ScanKind kind = ScanKind::Inclusive) const {
        hx_plan *p = nullptr;
        check(hx_prepare_scan(dev.raw(), Op::code, Scalar<T>::dtype, static_cast<hx_scan_kind>(kind),
                              static_cast<hx_scan_direction>(direction), input.buffer.device_ptr(),
                              input.buffer.len(), input.layout.raw(), axis, output.buffer.device_ptr(),
                              output.buffer.len(), output.layout.raw(), &p));
        return PreparedPlan(p);
    }
    void dispatch_scan(RocmDevice &, const PreparedPlan &plan, hx_stream stream = nullptr) const {
        plan.dispatch(stream);
    }
};

// ------------------------------------------------------ segmented reduction
// out[s] = sum of values[offsets[s] .. offsets[s+1]) (CSR row_ptr offsets,
// core sparse.rs:179-220), integer sums wrapping mod 2^32.
class RocmSegmentedReductionOps {
  public:
    template <typename T>
    void segmented_sum_into(RocmDevice &dev, const RocmBuffer<T> &values, const RocmBuffer<uint32_t> &offsets,
                            RocmBuffer<T> &out, hx_stream stream = nullptr) const {
        check(hx_segmented_reduce(dev.raw(), HX_OP_SUM, Scalar<T>::dtype, values.device_ptr(), values.len(),
                                  offsets.device_ptr(), offsets.len(), out.device_ptr(), out.len(), stream));
    }
    void validate_offsets(RocmDevice &dev, const RocmBuffer<uint32_t> &offsets, uint64_t n) const {
        check(hx_validate_segment_offsets(dev.raw(), offsets.device_ptr(), offsets.len(), n));
    }
};

// --------------------------------------------------------- map-reductions
// dot / trace / norm_l1 / norm_l2 / norm_max (rocm linalg/norms.rs:394-490):
// strided views in, a new one-element device buffer out.
template <typename T> RocmBuffer<T> dot(RocmDevice &dev, StridedView<T> a, StridedView<T> b, hx_stream stream = nullptr) {
    RocmBuffer<T> out = dev.alloc_uninitialized<T>(1);
    check(hx_map_reduce(dev.raw(), HX_MAP_DOT, Scalar<T>::dtype, a.buffer.device_ptr(), a.buffer.len(), a.layout.raw(),
                        b.buffer.device_ptr(), b.buffer.len(), b.layout.raw(), out.device_ptr(), 1, stream));
    return out;
}
template <typename T> RocmBuffer<T> trace(RocmDevice &dev, StridedView<T> m, hx_stream stream = nullptr) {
    RocmBuffer<T> out = dev.alloc_uninitialized<T>(1);
    check(hx_trace(dev.raw(), Scalar<T>::dtype, m.buffer.device_ptr(), m.buffer.len(), m.layout.raw(),
                   out.device_ptr(), 1, stream));
    return out;
}
namespace detail {
template <typename T> RocmBuffer<T> norm(RocmDevice &dev, hx_map_reduction kind, StridedView<T> v, hx_stream stream) {
    RocmBuffer<T> out = dev.alloc_uninitialized<T>(1);
    check(hx_map_reduce(dev.raw(), kind, Scalar<T>::dtype, v.buffer.device_ptr(), v.buffer.len(), v.layout.raw(),
                        nullptr, 0, nullptr, out.device_ptr(), 1, stream));
    return out;
}
} // namespace detail
template <typename T> RocmBuffer<T> norm_l1(RocmDevice &d, StridedView<T> v, hx_stream s = nullptr) {
    return detail::norm(d, HX_MAP_NORM_L1, v, s);
}
template <typename T> RocmBuffer<T> norm_l2(RocmDevice &d, StridedView<T> v, hx_stream s = nullptr) {
    return detail::norm(d, HX_MAP_NORM_L2, v, s);
}
template <typename T> RocmBuffer<T> norm_max(RocmDevice &d, StridedView<T> v, hx_stream s = nullptr) {
    return detail::norm(d, HX_MAP_NORM_MAX, v, s);
}

// ------------------------------------------------------- DenseVectorOps
// DenseVectorOps<RocmDevice, f32> (core vector.rs:57-200): whole buffers as
// vectors, scalar results returned to the host.
class RocmDenseVectorOps {
  public:
    // A prepared dot / L2 norm: the plan, its output and the allocations it
    // was prepared against.
    struct Prepared {
        PreparedPlan plan;
        RocmBuffer<float> output;
        const float *a, *b;
    };

    void copy_vector(RocmDevice &dev, const RocmBuffer<float> &source, RocmBuffer<float> &target) const {
        if (source.len() != target.len())
            throw Error(ErrorKind::LengthMismatch, "copy_vector length mismatch", source.len(), target.len());
        if (source.len()) dev.copy_buffer(source, target);
    }
    void scale_vector(RocmDevice &dev, RocmBuffer<float> &target, float factor) const {
        check(hx_vector_update(dev.raw(), HX_VEC_SCALE, HX_DTYPE_F32, target.device_ptr(), target.len(), nullptr, 0,
                               factor, nullptr));
    }
    void axpy(RocmDevice &dev, RocmBuffer<float> &target, const RocmBuffer<float> &source, float factor) const {
        check(hx_vector_update(dev.raw(), HX_VEC_AXPY, HX_DTYPE_F32, target.device_ptr(), target.len(),
                               source.device_ptr(), source.len(), factor, nullptr));
    }
    void xpay(RocmDevice &dev, RocmBuffer<float> &target, const RocmBuffer<float> &source, float factor) const {
        check(hx_vector_update(dev.raw(), HX_VEC_XPAY, HX_DTYPE_F32, target.device_ptr(), target.len(),
                               source.device_ptr(), source.len(), factor, nullptr));
    }
    void subtract_into(RocmDevice &d, const RocmBuffer<float> &l, const RocmBuffer<float> &r, RocmBuffer<float> &o) const {
        binary(d, HX_VEC_SUB, l, r, o);
    }
    void add_into(RocmDevice &d, const RocmBuffer<float> &l, const RocmBuffer<float> &r, RocmBuffer<float> &o) const {
        binary(d, HX_VEC_ADD, l, r, o);
    }
    void multiply_into(RocmDevice &d, const RocmBuffer<float> &l, const RocmBuffer<float> &r, RocmBuffer<float> &o) const {
        binary(d, HX_VEC_MUL, l, r, o);
    }
    void divide_into(RocmDevice &d, const RocmBuffer<float> &l, const RocmBuffer<float> &r, RocmBuffer<float> &o) const {
        binary(d, HX_VEC_DIV, l, r, o);
    }
    Prepared prepare_dot(RocmDevice &dev, const RocmBuffer<float> &left, const RocmBuffer<float> &right) const {
        if (left.len() != right.len())
            throw Error(ErrorKind::LengthMismatch, "dot length mismatch", left.len(), right.len());
        return prepare(dev, HX_MAP_DOT, left, &right);
    }
    float dot_prepared(RocmDevice &dev, const Prepared &p, const RocmBuffer<float> &left,
                       const RocmBuffer<float> &right) const {
        if (p.a != left.device_ptr() || p.b != right.device_ptr())
            throw Error(ErrorKind::DispatchFailed, "prepared dot received different device allocations");
        p.plan.dispatch();
        return dev.download_owned(p.output)[0];
    }
    Prepared prepare_norm_l2(RocmDevice &dev, const RocmBuffer<float> &v) const {
        return prepare(dev, HX_MAP_NORM_L2, v, nullptr);
    }
    float norm_l2_prepared(RocmDevice &dev, const Prepared &p, const RocmBuffer<float> &v) const {
        if (p.a != v.device_ptr())
            throw Error(ErrorKind::DispatchFailed, "prepared norm received a different device allocation");
        p.plan.dispatch();
        return dev.download_owned(p.output)[0];
    }
    float norm_l1(RocmDevice &dev, const RocmBuffer<float> &v) const {
        const Layout l = Layout::c_contiguous({v.len()});
        return dev.download_owned(hephaestus::norm_l1<float>(dev, {v, l}))[0];
    }
    float norm_max(RocmDevice &dev, const RocmBuffer<float> &v) const {
        const Layout l = Layout::c_contiguous({v.len()});
        return dev.download_owned(hephaestus::norm_max<float>(dev, {v, l}))[0];
    }

  private:
    void binary(RocmDevice &d, hx_vector_op op, const RocmBuffer<float> &l, const RocmBuffer<float> &r,
                RocmBuffer<float> &o) const {
        check(hx_vector_binary(d.raw(), op, HX_DTYPE_F32, l.device_ptr(), l.len(), r.device_ptr(), r.len(),
                               o.device_ptr(), o.len(), nullptr));
    }
    Prepared prepare(RocmDevice &dev, hx_map_reduction kind, const RocmBuffer<float> &a,
                     const RocmBuffer<float> *b) const {
        const Layout la = Layout::c_contiguous({a.len()});
        RocmBuffer<float> out = dev.alloc_uninitialized<float>(1);
        hx_plan *plan = nullptr;
        check(hx_prepare_map_reduce(dev.raw(), kind, HX_DTYPE_F32, a.device_ptr(), a.len(), la.raw(),
                                    b ? b->device_ptr() : nullptr, b ? b->len() : 0, b ? la.raw() : nullptr,
                                    out.device_ptr(), 1, &plan));
        return Prepared{PreparedPlan(plan), std::move(out), a.device_ptr(), b ? b->device_ptr() : nullptr};
    }
};

} // namespace hephaestus
