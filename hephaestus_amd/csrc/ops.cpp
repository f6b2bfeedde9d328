// Device entry points of the C ABI: validate (always before any write, so a
// rejected call leaves its outputs untouched), then launch on the chosen
// stream.  Immediate forms use the workspace of the stream they launch on
// (Immediate); hx_prepare_* returns a plan that owns its workspace, so
// hx_plan_dispatch allocates nothing.
#include "hx_internal.hpp"

#include <new>

using namespace hx;

namespace {

constexpr uint32_t kDefaultWidth = 256; // BlockWidth::DEFAULT, core launch.rs:26-29

const char *op_name(hx_op op) {
    switch (op) {
    case HX_OP_SUM: return "sum";
    case HX_OP_PROD: return "prod";
    case HX_OP_MIN: return "min";
    case HX_OP_MAX: return "max";
    case HX_OP_ARGMAX: return "argmax";
    case HX_OP_MEAN: return "mean";
    }
    return "unknown";
}

hx_status check_dtype(hx_dtype d) {
    if (d != HX_DTYPE_F32 && d != HX_DTYPE_U32 && d != HX_DTYPE_I32)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)d);
    return HX_OK;
}

hx_status check_op(hx_op op) {
    if ((int)op < HX_OP_SUM || (int)op > HX_OP_MEAN)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown reduction operator %d", (int)op);
    return HX_OK;
}

hx_status read_prologue(const hx_affine *pro, hx_dtype dtype, bool *affine, float *a, float *b) {
    *affine = false;
    *a = 1.0f;
    *b = 0.0f;
    if (!pro || !pro->enabled) return HX_OK;
    if (dtype != HX_DTYPE_F32)
        return fail(HX_ERR_INVALID_CONFIGURATION, "the affine prologue fmaf(a, x, b) needs f32 operands");
    *affine = true;
    *a = pro->a;
    *b = pro->b;
    return HX_OK;
}

bool aliases(const void *a, const void *b) { return a != nullptr && a == b; }

// Integer means divide the wrapped sum by the element count in the element
// type, as the reference's `acc / (T)axis_len` does (rocm axis_reduction.rs:
// 78-108); a count that the type cannot hold has no such divisor, so it is
// rejected rather than truncated.
hx_status check_mean_divisor(hx_dtype dtype, uint64_t n) {
    if (dtype == HX_DTYPE_I32 && n > 0x7FFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "mean of %llu i32 elements: the count exceeds the i32 divisor range",
                    (unsigned long long)n);
    if (dtype == HX_DTYPE_U32 && n > 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "mean of %llu u32 elements: the count exceeds the u32 divisor range",
                    (unsigned long long)n);
    return HX_OK;
}

// ---------------------------------------------------------------- full

// rocm full_reduction_seam.rs:65-78: output storage, output size == 1,
// input size, input storage.
hx_status plan_full(hx_op op, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                    const hx_layout *in_layout, void *out, uint64_t out_buf_len,
                    const hx_layout *out_layout, const hx_affine *pro, FullReduceArgs *a) {
    HX_TRY(check_dtype(dtype));
    HX_TRY(check_op(op));
    if (op == HX_OP_ARGMAX)
        return fail(HX_ERR_DISPATCH_FAILED, "full argmax returns an index: use hx_argmax_full");
    HX_TRY(layout_basic_check(out_layout, "output"));
    HX_TRY(hx_layout_validate_storage_len(out_layout, out_buf_len));
    uint64_t out_size = 0;
    HX_TRY(hx_layout_checked_size(out_layout, &out_size));
    if (out_size != 1)
        return fail(HX_ERR_DISPATCH_FAILED, "full reduction output must have exactly 1 element");
    HX_TRY(layout_basic_check(in_layout, "input"));
    uint64_t n = 0;
    HX_TRY(hx_layout_checked_size(in_layout, &n));
    HX_TRY(hx_layout_validate_storage_len(in_layout, in_buf_len));
    if (!out) return fail(HX_ERR_DISPATCH_FAILED, "full reduction output buffer is null");
    if (n > 0 && !in) return fail(HX_ERR_DISPATCH_FAILED, "full reduction input buffer is null");
    bool affine;
    float pa, pb;
    HX_TRY(read_prologue(pro, dtype, &affine, &pa, &pb));
    *a = FullReduceArgs{};
    a->op = op;
    a->dtype = dtype;
    a->base = in;
    a->layout = *in_layout;
    a->n = n;
    // Sum, product, min, max and mean are order-independent here (exact
    // integer / key arithmetic, f64 accumulation), so any view that covers a
    // dense block of memory, transposed or reversed, is streamed as that
    // block from its lowest element.
    uint64_t first = in_layout->offset;
    a->flat = layout_covers_dense_range(*in_layout, &first);
    a->flat_offset = first;
    a->affine = affine;
    a->a = pa;
    a->b = pb;
    a->out_value = (char *)out + out_layout->offset * 4;
    a->out_index = nullptr;
    if (op == HX_OP_MEAN && n == 0)
        return fail(HX_ERR_DISPATCH_FAILED, "mean is undefined for an empty operand");
    if (op == HX_OP_MEAN) HX_TRY(check_mean_divisor(dtype, n));
    return HX_OK;
}

struct FullPlan final : hx_plan {
    FullReduceArgs args;
    bool tagged() const override { return true; }
    hx_status dispatch(hipStream_t stream) override {
        return launch_full_reduce(args, ws, ws_bytes, lookback, stream);
    }
};

hx_status run_full(hx_device *dev, const FullReduceArgs &a, hipStream_t stream) {
    Immediate im;
    HX_TRY(im.open(dev, stream));
    void *ws = nullptr;
    HX_TRY(im.workspace(full_reduce_workspace_bytes(a.n), &ws));
    return launch_full_reduce(a, ws, im.workspace_bytes(), im.lookback(), stream);
}

// ---------------------------------------------------------------- axis

hx_status plan_axis(hx_op op, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                    const hx_layout *in_layout, uint32_t axis, void *out, uint64_t out_buf_len,
                    const hx_layout *out_layout, AxisArgs *a) {
    HX_TRY(check_dtype(dtype));
    HX_TRY(check_op(op));
    HX_TRY(layout_basic_check(in_layout, "input"));
    if (op == HX_OP_MIN || op == HX_OP_MAX || op == HX_OP_MEAN || op == HX_OP_ARGMAX) {
        // rocm axis_reduction.rs:114-136 (axis_len, reject_empty_axis)
        if (axis >= 2 || axis >= in_layout->rank)
            return fail(HX_ERR_DISPATCH_FAILED, "axis %u is out of bounds for rank-2 reduction", axis);
        if (in_layout->shape[axis] == 0)
            return fail(HX_ERR_DISPATCH_FAILED, "%s_axis is undefined for empty axis %u", op_name(op),
                        axis);
    }
    uint64_t out_len = 0, axis_len = 0;
    HX_TRY(hx_plan_axis_reduction(in_layout, in_buf_len, out_layout, out_buf_len, axis, kDefaultWidth,
                                  aliases(in, out) ? 1 : 0, &out_len, &axis_len));
    if (op == HX_OP_ARGMAX && axis_len > 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "argmax axis length %llu exceeds the u32 index range",
                    (unsigned long long)axis_len);
    if (op == HX_OP_MEAN) HX_TRY(check_mean_divisor(dtype, axis_len));
    *a = AxisArgs{};
    a->op = op;
    a->dtype = dtype;
    a->in = in;
    a->out = out;
    a->outer = out_len;
    a->axis_len = axis_len;
    a->in_axis_stride = in_layout->strides[axis];
    a->in_outer_stride = in_layout->strides[1 - axis];
    a->in_offset = in_layout->offset;
    a->out_stride = out_layout->strides[1 - axis];
    a->out_offset = out_layout->offset;
    // Reversed dimensions are read from their other end, so lines and
    // neighbouring outputs ascend in memory (unit strides take the vector
    // paths).  The reduced axis only where the order of its elements cannot
    // show: argmax reports the first index of the maximum.  The outer axis
    // always, together with the outputs, which keep pairing with their lines.
    if (op != HX_OP_ARGMAX && axis_len > 1 && a->in_axis_stride < 0) {
        a->in_offset += (axis_len - 1) * a->in_axis_stride;
        a->in_axis_stride = -a->in_axis_stride;
    }
    if (out_len > 1 && a->in_outer_stride < 0) {
        a->in_offset += (out_len - 1) * a->in_outer_stride;
        a->out_offset += (out_len - 1) * a->out_stride;
        a->in_outer_stride = -a->in_outer_stride;
        a->out_stride = -a->out_stride;
    }
    return HX_OK;
}

struct AxisPlan final : hx_plan {
    AxisArgs args;
    hx_status dispatch(hipStream_t stream) override { return launch_axis_reduce(args, ws, ws_bytes, stream); }
};

// Fused rows: validation shared by the immediate and prepared forms.
hx_status plan_rows(hx_dtype dtype, const void *in, uint64_t in_buf_len, uint64_t rows, uint64_t cols,
                    uint64_t row_stride, uint64_t offset, const hx_affine *prologue, void *out_sum, void *out_max,
                    uint32_t *out_argmax, uint64_t out_len, RowsArgs *args) {
    HX_TRY(check_dtype(dtype));
    bool affine;
    float pa, pb;
    HX_TRY(read_prologue(prologue, dtype, &affine, &pa, &pb));
    if (!out_sum && !out_max && !out_argmax)
        return fail(HX_ERR_DISPATCH_FAILED, "row reduction needs at least one output");
    if (out_len != rows) return length_mismatch(out_len, rows);
    if ((out_max || out_argmax) && cols == 0 && rows > 0)
        return fail(HX_ERR_DISPATCH_FAILED, "%s_axis is undefined for empty axis 1",
                    out_argmax ? "argmax" : "max");
    if (out_argmax && cols > 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "argmax row length %llu exceeds the u32 index range",
                    (unsigned long long)cols);
    if (rows > 1 && row_stride < cols)
        return fail(HX_ERR_DISPATCH_FAILED, "row stride %llu is shorter than the row length %llu",
                    (unsigned long long)row_stride, (unsigned long long)cols);
    if (rows > 0 && cols > 0) {
        const unsigned __int128 last =
            (unsigned __int128)offset + (unsigned __int128)(rows - 1) * row_stride + (cols - 1);
        if (last >= in_buf_len)
            return fail(HX_ERR_DISPATCH_FAILED,
                        "layout rejected: rows need %llu elements but the buffer holds %llu",
                        (unsigned long long)(last + 1), (unsigned long long)in_buf_len);
        if (!in) return fail(HX_ERR_DISPATCH_FAILED, "row reduction input is null");
    }
    if (aliases(in, out_sum) || aliases(in, out_max) || aliases(in, out_argmax))
        return fail(HX_ERR_DISPATCH_FAILED, "axis reduction output buffer must not alias input buffer");
    RowsArgs &a = *args;
    a = RowsArgs{};
    a.dtype = dtype;
    a.base = in;
    a.rows = rows;
    a.cols = cols;
    a.row_stride = row_stride;
    a.offset = offset;
    a.affine = affine;
    a.a = pa;
    a.b = pb;
    a.out_sum = out_sum;
    a.out_max = out_max;
    a.out_argmax = out_argmax;
    return HX_OK;
}

struct RowsPlan final : hx_plan {
    RowsArgs args;
    hx_status dispatch(hipStream_t stream) override { return launch_rows(args, ws, ws_bytes, stream); }
};

// ---------------------------------------------------------------- scan

hx_status plan_scan(hx_op op, hx_dtype dtype, hx_scan_kind kind, hx_scan_direction direction,
                    const void *in, uint64_t in_buf_len, const hx_layout *in_layout, uint32_t axis,
                    void *out, uint64_t out_buf_len, const hx_layout *out_layout, ScanArgs *a) {
    HX_TRY(check_dtype(dtype));
    if (op != HX_OP_SUM && op != HX_OP_PROD)
        return fail(HX_ERR_DISPATCH_FAILED, "scan supports sum (CumSumOp) and prod (CumProdOp), got %s",
                    op_name(op));
    if (kind != HX_SCAN_INCLUSIVE && kind != HX_SCAN_EXCLUSIVE)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown scan kind %d", (int)kind);
    if (direction != HX_SCAN_FORWARD && direction != HX_SCAN_REVERSE)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown scan direction %d", (int)direction);
    uint64_t lines = 0, len = 0;
    HX_TRY(hx_plan_axis_scan(in_layout, in_buf_len, out_layout, out_buf_len, axis, kDefaultWidth,
                             aliases(in, out) ? 1 : 0, &lines, &len));
    *a = ScanArgs{};
    a->op = op;
    a->dtype = dtype;
    a->exclusive = kind == HX_SCAN_EXCLUSIVE;
    a->reverse = direction == HX_SCAN_REVERSE;
    a->in = in;
    a->out = out;
    a->lines = lines;
    a->len = len;
    a->in_elem_stride = in_layout->strides[axis];
    a->out_elem_stride = out_layout->strides[axis];
    a->in_line_stride = in_layout->rank == 2 ? in_layout->strides[1 - axis] : 0;
    a->out_line_stride = out_layout->rank == 2 ? out_layout->strides[1 - axis] : 0;
    a->in_offset = in_layout->offset;
    a->out_offset = out_layout->offset;
    if (len > 1 && a->in_elem_stride < 0 && a->out_elem_stride < 0) {
        // Lines that run backwards in both operands: the same elements in
        // the same order are the mirrored lines scanned the other way, and
        // those read and write with ascending addresses.
        a->in_offset += (len - 1) * a->in_elem_stride;
        a->out_offset += (len - 1) * a->out_elem_stride;
        a->in_elem_stride = -a->in_elem_stride;
        a->out_elem_stride = -a->out_elem_stride;
        a->reverse = !a->reverse;
    }
    return HX_OK;
}

struct ScanPlan final : hx_plan {
    ScanArgs args;
    bool tagged() const override { return scan_uses_lookback(args); }
    hx_status dispatch(hipStream_t stream) override {
        return launch_scan(args, ws, ws_bytes, lookback, stream);
    }
};

// ----------------------------------------------------------- segmented

hx_status plan_segmented(hx_op op, hx_dtype dtype, const void *values, uint64_t n,
                         const uint32_t *offsets, uint64_t num_offsets, void *out, uint64_t out_len,
                         SegmentedArgs *a) {
    HX_TRY(check_dtype(dtype));
    if (op != HX_OP_SUM)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce supports sum only, got %s", op_name(op));
    if (dtype == HX_DTYPE_F32)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented sum supports u32 and i32 values");
    if (num_offsets == 0)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "segment offsets need at least one entry (offsets[0] = 0)");
    if (n > 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce of %llu values exceeds the u32 offset range",
                    (unsigned long long)n);
    const uint64_t segments = num_offsets - 1;
    if (out_len != segments) return length_mismatch(out_len, segments);
    if (n > 0 && !values) return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce values are null");
    if (!offsets) return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce offsets are null");
    if (segments > 0 && !out) return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce output is null");
    if (aliases(out, values) || aliases(out, offsets))
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce output must not alias its inputs");
    if (((uintptr_t)values) % 4 != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce values must be 4-byte aligned");
    *a = SegmentedArgs{};
    a->op = op;
    a->dtype = dtype;
    a->values = values;
    a->n = n;
    a->offsets = offsets;
    a->num_segments = segments;
    a->out = out;
    return HX_OK;
}

struct SegmentedPlan final : hx_plan {
    SegmentedArgs args;
    bool tagged() const override { return true; }
    hx_status dispatch(hipStream_t stream) override {
        return launch_segmented(args, ws, ws_bytes, nullptr, 0, lookback, stream);
    }
};

template <typename Plan>
hx_status finish_plan(hx_device *dev, Plan *plan, uint64_t ws_bytes, hx_plan **out) {
    plan->dev = dev;
    hx_status s = alloc_workspace(dev, ws_bytes, &plan->ws);
    if (s != HX_OK) {
        delete plan;
        return s;
    }
    plan->ws_bytes = ws_bytes;
    *out = plan;
    return ok();
}

} // namespace

extern "C" {

hx_status hx_reduce_full(hx_device *dev, hx_op op, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                         const hx_layout *in_layout, void *out, uint64_t out_buf_len,
                         const hx_layout *out_layout, const hx_affine *prologue, hx_stream stream) {
    FullReduceArgs a;
    HX_TRY(plan_full(op, dtype, in, in_buf_len, in_layout, out, out_buf_len, out_layout, prologue, &a));
    HX_TRY(bind_device(dev));
    HX_TRY(run_full(dev, a, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_prepare_reduce_full(hx_device *dev, hx_op op, hx_dtype dtype, const void *in,
                                 uint64_t in_buf_len, const hx_layout *in_layout, void *out,
                                 uint64_t out_buf_len, const hx_layout *out_layout,
                                 const hx_affine *prologue, hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    FullReduceArgs a;
    HX_TRY(plan_full(op, dtype, in, in_buf_len, in_layout, out, out_buf_len, out_layout, prologue, &a));
    HX_TRY(bind_device(dev));
    FullPlan *p = new (std::nothrow) FullPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = a;
    return finish_plan(dev, p, full_reduce_workspace_bytes(a.n), plan);
}

hx_status hx_argmax_full(hx_device *dev, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                         const hx_layout *in_layout, void *out_value, uint32_t *out_index,
                         const hx_affine *prologue, hx_stream stream) {
    HX_TRY(check_dtype(dtype));
    HX_TRY(layout_basic_check(in_layout, "input"));
    uint64_t n = 0;
    HX_TRY(hx_layout_checked_size(in_layout, &n));
    HX_TRY(hx_layout_validate_storage_len(in_layout, in_buf_len));
    if (!out_index) return fail(HX_ERR_DISPATCH_FAILED, "argmax index output is null");
    if (n > 0xFFFFFFFFull - 1)
        return fail(HX_ERR_DISPATCH_FAILED, "argmax supports at most 4294967294 elements, got %llu",
                    (unsigned long long)n);
    if (n > 0 && !in) return fail(HX_ERR_DISPATCH_FAILED, "argmax input buffer is null");
    FullReduceArgs a{};
    bool affine;
    float pa, pb;
    HX_TRY(read_prologue(prologue, dtype, &affine, &pa, &pb));
    a.op = HX_OP_ARGMAX;
    a.dtype = dtype;
    a.base = in;
    a.layout = *in_layout;
    a.n = n;
    // Indices follow logical order: only a row-major view is the flat range;
    // a permuted dense one (a transpose) is read in memory order with each
    // element's logical index carried along.
    a.flat = layout_is_c_contiguous(*in_layout);
    a.flat_offset = in_layout->offset;
    // A view read entirely backwards is the flat range from its far end:
    // view index n - 1 - e, so the first index of the maximum is still found
    // by the smallest index on ties.
    uint64_t first = 0;
    if (!a.flat && layout_is_reversed_c_contiguous(*in_layout, &first)) {
        a.flat = true;
        a.reversed = true;
        a.flat_offset = first;
    }
    a.memory_order = !a.flat && layout_is_permuted_dense(*in_layout);
    a.affine = affine;
    a.a = pa;
    a.b = pb;
    a.out_value = out_value;
    a.out_index = out_index;
    HX_TRY(bind_device(dev));
    HX_TRY(run_full(dev, a, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_reduce_axis(hx_device *dev, hx_op op, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                         const hx_layout *in_layout, uint32_t axis, void *out, uint64_t out_buf_len,
                         const hx_layout *out_layout, hx_stream stream) {
    AxisArgs a;
    HX_TRY(plan_axis(op, dtype, in, in_buf_len, in_layout, axis, out, out_buf_len, out_layout, &a));
    HX_TRY(bind_device(dev));
    const hipStream_t s = pick_stream(dev, stream);
    Immediate im;
    HX_TRY(im.open(dev, s));
    const uint64_t bytes = axis_reduce_workspace_bytes(a);
    void *scratch = nullptr;
    HX_TRY(im.scratch(bytes, &scratch));
    HX_TRY(launch_axis_reduce(a, scratch, bytes, s));
    return ok();
}

hx_status hx_prepare_reduce_axis(hx_device *dev, hx_op op, hx_dtype dtype, const void *in,
                                 uint64_t in_buf_len, const hx_layout *in_layout, uint32_t axis,
                                 void *out, uint64_t out_buf_len, const hx_layout *out_layout,
                                 hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    AxisArgs a;
    HX_TRY(plan_axis(op, dtype, in, in_buf_len, in_layout, axis, out, out_buf_len, out_layout, &a));
    HX_TRY(bind_device(dev));
    AxisPlan *p = new (std::nothrow) AxisPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = a;
    return finish_plan(dev, p, axis_reduce_workspace_bytes(a), plan);
}

hx_status hx_reduce_rows(hx_device *dev, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                         uint64_t rows, uint64_t cols, uint64_t row_stride, uint64_t offset,
                         const hx_affine *prologue, void *out_sum, void *out_max,
                         uint32_t *out_argmax, uint64_t out_len, hx_stream stream) {
    RowsArgs a;
    HX_TRY(plan_rows(dtype, in, in_buf_len, rows, cols, row_stride, offset, prologue, out_sum, out_max, out_argmax,
                     out_len, &a));
    HX_TRY(bind_device(dev));
    const hipStream_t s = pick_stream(dev, stream);
    Immediate im;
    HX_TRY(im.open(dev, s));
    const uint64_t bytes = rows_workspace_bytes(a);
    void *scratch = nullptr;
    HX_TRY(im.scratch(bytes, &scratch));
    HX_TRY(launch_rows(a, scratch, bytes, s));
    return ok();
}

hx_status hx_prepare_reduce_rows(hx_device *dev, hx_dtype dtype, const void *in, uint64_t in_buf_len,
                                 uint64_t rows, uint64_t cols, uint64_t row_stride, uint64_t offset,
                                 const hx_affine *prologue, void *out_sum, void *out_max,
                                 uint32_t *out_argmax, uint64_t out_len, hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    RowsArgs a;
    HX_TRY(plan_rows(dtype, in, in_buf_len, rows, cols, row_stride, offset, prologue, out_sum, out_max, out_argmax,
                     out_len, &a));
    HX_TRY(bind_device(dev));
    RowsPlan *p = new (std::nothrow) RowsPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = a;
    return finish_plan(dev, p, rows_workspace_bytes(a), plan);
}

hx_status hx_scan(hx_device *dev, hx_op op, hx_dtype dtype, hx_scan_kind kind,
                  hx_scan_direction direction, const void *in, uint64_t in_buf_len,
                  const hx_layout *in_layout, uint32_t axis, void *out, uint64_t out_buf_len,
                  const hx_layout *out_layout, hx_stream stream) {
    ScanArgs a;
    HX_TRY(plan_scan(op, dtype, kind, direction, in, in_buf_len, in_layout, axis, out, out_buf_len,
                     out_layout, &a));
    HX_TRY(bind_device(dev));
    hipStream_t s = pick_stream(dev, stream);
    Immediate im;
    HX_TRY(im.open(dev, s));
    void *ws = nullptr;
    const uint64_t bytes = scan_workspace_bytes(a);
    if (!scan_uses_lookback(a)) {
        HX_TRY(im.scratch(bytes, &ws));
        HX_TRY(launch_scan(a, ws, bytes, im.lookback(), s));
        return ok();
    }
    HX_TRY(im.workspace(bytes, &ws));
    HX_TRY(launch_scan(a, ws, im.workspace_bytes(), im.lookback(), s));
    return ok();
}

uint64_t hx_noalloc_scratch_bytes(void) { return noalloc_scratch_bytes(); }

hx_status hx_scan_noalloc(hx_device *dev, hx_op op, hx_dtype dtype, hx_scan_kind kind,
                          hx_scan_direction direction, const void *in, uint64_t in_buf_len,
                          const hx_layout *in_layout, uint32_t axis, void *out, uint64_t out_buf_len,
                          const hx_layout *out_layout, hx_stream stream) {
    ScanArgs a;
    HX_TRY(plan_scan(op, dtype, kind, direction, in, in_buf_len, in_layout, axis, out, out_buf_len,
                     out_layout, &a));
    HX_TRY(bind_device(dev));
    std::lock_guard<std::mutex> guard(dev->noalloc_mu);
    HX_TRY(launch_scan_noalloc(a, dev->noalloc_scratch, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_prepare_scan(hx_device *dev, hx_op op, hx_dtype dtype, hx_scan_kind kind,
                          hx_scan_direction direction, const void *in, uint64_t in_buf_len,
                          const hx_layout *in_layout, uint32_t axis, void *out, uint64_t out_buf_len,
                          const hx_layout *out_layout, hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    ScanArgs a;
    HX_TRY(plan_scan(op, dtype, kind, direction, in, in_buf_len, in_layout, axis, out, out_buf_len,
                     out_layout, &a));
    HX_TRY(bind_device(dev));
    ScanPlan *p = new (std::nothrow) ScanPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = a;
    return finish_plan(dev, p, scan_workspace_bytes(a), plan);
}

hx_status hx_segmented_reduce(hx_device *dev, hx_op op, hx_dtype dtype, const void *values, uint64_t n,
                              const uint32_t *offsets, uint64_t num_offsets, void *out,
                              uint64_t out_len, hx_stream stream) {
    SegmentedArgs a;
    HX_TRY(plan_segmented(op, dtype, values, n, offsets, num_offsets, out, out_len, &a));
    HX_TRY(bind_device(dev));
    hipStream_t s = pick_stream(dev, stream);
    Immediate im;
    HX_TRY(im.open(dev, s));
    void *ws = nullptr, *aux = nullptr;
    const uint64_t lookback = segmented_lookback_bytes(a), aux_bytes = segmented_aux_bytes(a);
    HX_TRY(im.scratch(aux_bytes, &aux));
    if (lookback) HX_TRY(im.workspace(lookback, &ws));
    HX_TRY(launch_segmented(a, ws, lookback ? im.workspace_bytes() : 0, aux, aux_bytes, im.lookback(), s));
    return ok();
}

hx_status hx_prepare_segmented_reduce(hx_device *dev, hx_op op, hx_dtype dtype, const void *values,
                                      uint64_t n, const uint32_t *offsets, uint64_t num_offsets,
                                      void *out, uint64_t out_len, hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    SegmentedArgs a;
    HX_TRY(plan_segmented(op, dtype, values, n, offsets, num_offsets, out, out_len, &a));
    HX_TRY(bind_device(dev));
    SegmentedPlan *p = new (std::nothrow) SegmentedPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = a;
    return finish_plan(dev, p, segmented_workspace_bytes(a), plan);
}

hx_status hx_validate_segment_offsets(hx_device *dev, const uint32_t *offsets, uint64_t num_offsets,
                                      uint64_t n) {
    if (num_offsets == 0)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "segment offsets need at least one entry (offsets[0] = 0)");
    if (!offsets) return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce offsets are null");
    HX_TRY(bind_device(dev));
    HX_TRY(validate_offsets_on_device(dev, offsets, num_offsets, n));
    return ok();
}

hx_status hx_fill_random(hx_device *dev, void *dst, uint64_t n, hx_dtype dtype, hx_distribution dist,
                         uint64_t seed, double p0, double p1, hx_stream stream) {
    HX_TRY(check_dtype(dtype));
    if (n > 0 && !dst) return fail(HX_ERR_DISPATCH_FAILED, "fill destination is null");
    HX_TRY(bind_device(dev));
    HX_TRY(launch_fill_random(dst, n, dtype, dist, seed, p0, p1, pick_stream(dev, stream)));
    return ok();
}

} // extern "C"
