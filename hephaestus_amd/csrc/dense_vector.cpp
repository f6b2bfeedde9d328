// Entry points of the map-reductions (dot, norms, trace) and the dense f32
// vector forms.  Validation runs first and in the reference's order, so a
// rejected call writes nothing.
#include "hx_internal.hpp"

#include <new>

using namespace hx;

namespace {

hx_status check_dtype(hx_dtype d) {
    if (d != HX_DTYPE_F32 && d != HX_DTYPE_U32 && d != HX_DTYPE_I32)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)d);
    return HX_OK;
}

bool same_shape(const hx_layout &a, const hx_layout &b) {
    if (a.rank != b.rank) return false;
    for (uint32_t d = 0; d < a.rank; ++d)
        if (a.shape[d] != b.shape[d]) return false;
    return true;
}

// Same strides over every extent above one (the shapes already match).
bool same_strides(const hx_layout &a, const hx_layout &b) {
    for (uint32_t d = 0; d < a.rank; ++d)
        if (a.shape[d] > 1 && a.strides[d] != b.strides[d]) return false;
    return true;
}

// One operand of a map-reduction: layout checks of the reference's
// StridedOperand (leto Layout validation) against its buffer.
hx_status check_operand(const void *buf, uint64_t buf_len, const hx_layout *l, const char *what, uint64_t *n) {
    HX_TRY(layout_basic_check(l, what));
    HX_TRY(hx_layout_checked_size(l, n));
    HX_TRY(hx_layout_validate_storage_len(l, buf_len));
    if (*n > 0 && !buf) return fail(HX_ERR_DISPATCH_FAILED, "map-reduction %s buffer is null", what);
    return HX_OK;
}

hx_status plan_map(hx_map_reduction map, hx_dtype dtype, const void *a, uint64_t a_buf_len, const hx_layout *a_layout,
                   const void *b, uint64_t b_buf_len, const hx_layout *b_layout, void *out, uint64_t out_buf_len,
                   MapReduceArgs *args) {
    HX_TRY(check_dtype(dtype));
    if ((int)map < HX_MAP_SUM || (int)map > HX_MAP_NORM_MAX)
        return fail(HX_ERR_INVALID_CONFIGURATION, "unknown map-reduction %d", (int)map);
    if (map == HX_MAP_NORM_L2 && dtype != HX_DTYPE_F32)
        return fail(HX_ERR_INVALID_CONFIGURATION, "the L2 norm is defined for f32 operands only");
    uint64_t n = 0, nb = 0;
    HX_TRY(check_operand(a, a_buf_len, a_layout, "lhs", &n));
    if (map == HX_MAP_DOT) {
        HX_TRY(check_operand(b, b_buf_len, b_layout, "rhs", &nb));
        if (!same_shape(*a_layout, *b_layout))
            return fail(HX_ERR_DISPATCH_FAILED, "dot product shape mismatch: lhs %s, rhs %s",
                        shape_string(*a_layout).c_str(), shape_string(*b_layout).c_str());
    }
    if (!out || out_buf_len < 1) return fail(HX_ERR_DISPATCH_FAILED, "map-reduction output must hold 1 element");
    *args = MapReduceArgs{};
    args->map = map;
    args->dtype = dtype;
    args->a = a;
    args->a_layout = *a_layout;
    args->b = map == HX_MAP_DOT ? b : a;
    args->b_layout = map == HX_MAP_DOT ? *b_layout : *a_layout;
    args->n = n;
    // The order of a sum does not change its value here (exact integer
    // arithmetic; f64 accumulation of exact f32 products), so views that
    // cover a dense range (transposed or reversed) are streamed as that range
    // with vector loads, from its lowest element.  A dot pairs a[k] with b[k]
    // along both ranges, which pairs the right elements when both views have
    // the same strides; their vector loads need only 4-byte alignment, so
    // the two may start at any element offsets.
    uint64_t a0 = 0, b0 = 0;
    bool flat = layout_covers_dense_range(*a_layout, &a0);
    if (map == HX_MAP_DOT)
        flat = flat && same_strides(*a_layout, *b_layout) && layout_covers_dense_range(*b_layout, &b0);
    else
        b0 = a0;
    args->flat = flat;
    if (flat) {
        args->a_layout.offset = a0;
        args->b_layout.offset = b0;
    }
    args->out = out;
    return HX_OK;
}

struct MapPlan final : hx_plan {
    MapReduceArgs args;
    bool tagged() const override { return true; }
    hx_status dispatch(hipStream_t stream) override {
        return launch_map_reduce(args, ws, ws_bytes, lookback, stream);
    }
};

hx_status run_map(hx_device *dev, const MapReduceArgs &a, hipStream_t stream) {
    Immediate im;
    HX_TRY(im.open(dev, stream));
    void *ws = nullptr;
    HX_TRY(im.workspace(map_reduce_workspace_bytes(a.n), &ws));
    return launch_map_reduce(a, ws, im.workspace_bytes(), im.lookback(), stream);
}

hx_status check_f32_vector(hx_dtype dtype) {
    if (dtype != HX_DTYPE_F32)
        return fail(HX_ERR_INVALID_CONFIGURATION, "dense vector operations are defined for f32 only");
    return HX_OK;
}

} // namespace

extern "C" {

hx_status hx_map_reduce(hx_device *dev, hx_map_reduction map, hx_dtype dtype, const void *a, uint64_t a_buf_len,
                        const hx_layout *a_layout, const void *b, uint64_t b_buf_len, const hx_layout *b_layout,
                        void *out, uint64_t out_buf_len, hx_stream stream) {
    MapReduceArgs args;
    HX_TRY(plan_map(map, dtype, a, a_buf_len, a_layout, b, b_buf_len, b_layout, out, out_buf_len, &args));
    HX_TRY(bind_device(dev));
    HX_TRY(run_map(dev, args, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_prepare_map_reduce(hx_device *dev, hx_map_reduction map, hx_dtype dtype, const void *a,
                                uint64_t a_buf_len, const hx_layout *a_layout, const void *b, uint64_t b_buf_len,
                                const hx_layout *b_layout, void *out, uint64_t out_buf_len, hx_plan **plan) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan out-pointer");
    *plan = nullptr;
    MapReduceArgs args;
    HX_TRY(plan_map(map, dtype, a, a_buf_len, a_layout, b, b_buf_len, b_layout, out, out_buf_len, &args));
    HX_TRY(bind_device(dev));
    MapPlan *p = new (std::nothrow) MapPlan();
    if (!p) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of plan failed");
    p->args = args;
    p->dev = dev;
    const uint64_t bytes = map_reduce_workspace_bytes(args.n);
    hx_status s = alloc_workspace(dev, bytes, &p->ws);
    if (s != HX_OK) {
        delete p;
        return s;
    }
    p->ws_bytes = bytes;
    *plan = p;
    return ok();
}

hx_status hx_trace(hx_device *dev, hx_dtype dtype, const void *in, uint64_t in_buf_len, const hx_layout *in_layout,
                   void *out, uint64_t out_buf_len, hx_stream stream) {
    HX_TRY(check_dtype(dtype));
    HX_TRY(layout_basic_check(in_layout, "trace input"));
    if (in_layout->rank != 2 || in_layout->shape[0] != in_layout->shape[1])
        return fail(HX_ERR_DISPATCH_FAILED, "trace requires a square matrix, got shape %s",
                    shape_string(*in_layout).c_str());
    HX_TRY(hx_layout_validate_storage_len(in_layout, in_buf_len));
    // The diagonal as a rank-1 view (norms.rs:430-439).
    hx_layout diag{};
    diag.rank = 1;
    diag.shape[0] = in_layout->shape[0];
    diag.strides[0] = in_layout->strides[0] + in_layout->strides[1];
    diag.offset = in_layout->offset;
    return hx_map_reduce(dev, HX_MAP_SUM, dtype, in, in_buf_len, &diag, nullptr, 0, nullptr, out, out_buf_len,
                         stream);
}

hx_status hx_vector_update(hx_device *dev, hx_vector_op op, hx_dtype dtype, void *target, uint64_t target_len,
                           const void *source, uint64_t source_len, float factor, hx_stream stream) {
    HX_TRY(check_f32_vector(dtype));
    if (op != HX_VEC_SCALE && op != HX_VEC_AXPY && op != HX_VEC_XPAY)
        return fail(HX_ERR_INVALID_CONFIGURATION, "vector update takes SCALE, AXPY or XPAY, got %d", (int)op);
    if (op != HX_VEC_SCALE && target_len != source_len) return length_mismatch(target_len, source_len);
    if (target_len == 0) return ok();
    if (!target || (op != HX_VEC_SCALE && !source))
        return fail(HX_ERR_DISPATCH_FAILED, "dense vector operand is null");
    HX_TRY(bind_device(dev));
    return launch_vector_op(op, (const float *)target, (const float *)source, (float *)target, target_len, factor,
                            pick_stream(dev, stream));
}

hx_status hx_vector_binary(hx_device *dev, hx_vector_op op, hx_dtype dtype, const void *left, uint64_t left_len,
                           const void *right, uint64_t right_len, void *out, uint64_t out_len, hx_stream stream) {
    HX_TRY(check_f32_vector(dtype));
    if (op != HX_VEC_ADD && op != HX_VEC_SUB && op != HX_VEC_MUL && op != HX_VEC_DIV)
        return fail(HX_ERR_INVALID_CONFIGURATION, "vector binary takes ADD, SUB, MUL or DIV, got %d", (int)op);
    // rocm vector.rs:237-241: left vs right, then left vs output.
    if (left_len != right_len) return length_mismatch(left_len, right_len);
    if (left_len != out_len) return length_mismatch(left_len, out_len);
    if (left_len == 0) return ok();
    if (!left || !right || !out) return fail(HX_ERR_DISPATCH_FAILED, "dense vector operand is null");
    HX_TRY(bind_device(dev));
    return launch_vector_op(op, (const float *)left, (const float *)right, (float *)out, left_len, 0.0f,
                            pick_stream(dev, stream));
}

} // extern "C"
