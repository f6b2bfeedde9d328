// Host-side planning: layout checks and the dispatch planners that every
// device entry point runs before it touches memory.  They restate the
// reference's backend-neutral planners (crates/hephaestus-core/src/domain/
// reduction.rs:339-500, scan.rs:87-178) and the leto Layout queries those
// planners call (checked_size, validate_storage_len,
// has_zero_stride_aliasing).  The reference narrows extents to u32 and
// strides to i32 because its kernels index with 32-bit integers
// (core planning.rs:16-29); these kernels index with 64-bit offsets, so
// those range checks are deliberately absent.
#include "hx_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <string>

namespace hx {

std::string shape_string(const hx_layout &l) {
    std::string s = "[";
    for (uint32_t d = 0; d < l.rank; ++d) {
        if (d) s += ", ";
        s += std::to_string((unsigned long long)l.shape[d]);
    }
    return s + "]";
}

hx_status layout_basic_check(const hx_layout *l, const char *what) {
    if (!l) return fail(HX_ERR_INVALID_CONFIGURATION, "null %s layout", what);
    if (l->rank < 1 || l->rank > HX_MAX_RANK)
        return fail(HX_ERR_DISPATCH_FAILED, "layout rejected: %s rank %u is outside 1..=%u", what,
                    l->rank, HX_MAX_RANK);
    return HX_OK;
}

static bool checked_size(const hx_layout &l, uint64_t *size) {
    unsigned __int128 s = 1;
    for (uint32_t d = 0; d < l.rank; ++d) {
        s *= l.shape[d];
        if (s > (unsigned __int128)UINT64_MAX) return false;
    }
    *size = (uint64_t)s;
    return true;
}

bool layout_is_c_contiguous(const hx_layout &l) {
    int64_t expect = 1;
    for (int d = (int)l.rank - 1; d >= 0; --d) {
        if (l.shape[d] > 1 && l.strides[d] != expect) return false;
        expect *= (int64_t)(l.shape[d] ? l.shape[d] : 1);
    }
    return true;
}

namespace {
// Rows from dimensions listed outermost first (extent, stride, second
// stride), merging neighbours adjacent under both strides.
RowsView rows_from_dims(const uint64_t *shape, const int64_t *stride, const int64_t *lstride, int n) {
    uint64_t ext[HX_MAX_RANK];
    int64_t str[HX_MAX_RANK], lst[HX_MAX_RANK];
    int m = 0;
    for (int d = 0; d < n; ++d) {
        if (shape[d] == 1) continue;
        if (m > 0 && str[m - 1] == stride[d] * (int64_t)shape[d] && lst[m - 1] == lstride[d] * (int64_t)shape[d]) {
            ext[m - 1] *= shape[d];
            str[m - 1] = stride[d];
            lst[m - 1] = lstride[d];
            continue;
        }
        ext[m] = shape[d];
        str[m] = stride[d];
        lst[m] = lstride[d];
        ++m;
    }
    RowsView v;
    if (m == 0) return v; // one element
    v.cols = ext[m - 1];
    v.cstride = str[m - 1];
    v.cstride2 = lst[m - 1];
    v.orank = (uint32_t)(m - 1);
    for (int k = 0; k < m - 1; ++k) {
        v.oshape[k] = ext[m - 2 - k];
        v.ostride[k] = str[m - 2 - k];
        v.ostride2[k] = lst[m - 2 - k];
        v.rows *= ext[m - 2 - k];
    }
    return v;
}

void logical_strides(const hx_layout &l, int64_t *lstride) {
    int64_t s = 1;
    for (int d = (int)l.rank - 1; d >= 0; --d) {
        lstride[d] = s;
        s *= (int64_t)(l.shape[d] ? l.shape[d] : 1);
    }
}
} // namespace

RowsView layout_rows(const hx_layout &l) {
    int64_t lstride[HX_MAX_RANK];
    logical_strides(l, lstride);
    return rows_from_dims(l.shape, l.strides, lstride, (int)l.rank);
}

RowsView layout_rows_pair(const hx_layout &a, const hx_layout &b) {
    return rows_from_dims(a.shape, a.strides, b.strides, (int)a.rank);
}

bool layout_pair_transposed(const hx_layout &a, const hx_layout &b, PairTranspose *t) {
    if (a.rank != b.rank) return false;
    int dims[3], m = 0;
    for (uint32_t d = 0; d < a.rank; ++d) {
        if (a.shape[d] != b.shape[d]) return false;
        if (a.shape[d] <= 1) continue;
        if (m == 3) return false;
        dims[m++] = (int)d;
    }
    if (m < 2) return false;
    for (int pass = 0; pass < 2; ++pass) {
        const bool a_col = pass == 0;
        const hx_layout &c = a_col ? a : b, &r = a_col ? b : a;
        int di = -1, dj = -1;
        for (int k = 0; k < m; ++k) {
            if (di < 0 && c.strides[dims[k]] == 1) di = dims[k];
            if (dj < 0 && r.strides[dims[k]] == 1) dj = dims[k];
        }
        if (di < 0 || dj < 0 || di == dj) continue;
        if (c.strides[dj] <= 0 || r.strides[di] <= 0) continue;
        int db = -1;
        for (int k = 0; k < m; ++k)
            if (dims[k] != di && dims[k] != dj) db = dims[k];
        t->a_is_col = a_col;
        t->rows = a.shape[di];
        t->cols = a.shape[dj];
        t->col_ld = c.strides[dj];
        t->row_ld = r.strides[di];
        t->batch = db < 0 ? 1 : a.shape[db];
        t->col_bs = db < 0 ? 0 : c.strides[db];
        t->row_bs = db < 0 ? 0 : r.strides[db];
        return true;
    }
    return false;
}

RowsView layout_rows_memory_order(const hx_layout &l) {
    int64_t lstride[HX_MAX_RANK];
    logical_strides(l, lstride);
    uint64_t shape[HX_MAX_RANK];
    int64_t stride[HX_MAX_RANK], lst[HX_MAX_RANK];
    const int n = (int)l.rank;
    for (int d = 0; d < n; ++d) {
        shape[d] = l.shape[d];
        stride[d] = l.strides[d];
        lst[d] = lstride[d];
    }
    // Decreasing stride: memory order, outermost first (ties keep logical order).
    for (int i = 1; i < n; ++i)
        for (int j = i; j > 0 && stride[j - 1] < stride[j]; --j) {
            std::swap(shape[j - 1], shape[j]);
            std::swap(stride[j - 1], stride[j]);
            std::swap(lst[j - 1], lst[j]);
        }
    return rows_from_dims(shape, stride, lst, n);
}

bool layout_is_permuted_dense(const hx_layout &l) {
    uint64_t ext[HX_MAX_RANK];
    int64_t str[HX_MAX_RANK];
    int m = 0;
    for (uint32_t d = 0; d < l.rank; ++d) {
        if (l.shape[d] <= 1) continue;
        if (l.strides[d] <= 0) return false;
        ext[m] = l.shape[d];
        str[m] = l.strides[d];
        ++m;
    }
    // Sort dimensions by stride; dense means stride_k = prod(extent_{<k}).
    for (int i = 1; i < m; ++i)
        for (int j = i; j > 0 && str[j - 1] > str[j]; --j) {
            std::swap(str[j - 1], str[j]);
            std::swap(ext[j - 1], ext[j]);
        }
    int64_t expect = 1;
    for (int i = 0; i < m; ++i) {
        if (str[i] != expect) return false;
        expect *= (int64_t)ext[i];
    }
    return true;
}

bool layout_covers_dense_range(const hx_layout &l, uint64_t *first) {
    hx_layout m = l;
    int64_t lo = (int64_t)l.offset;
    for (uint32_t d = 0; d < l.rank; ++d)
        if (l.strides[d] < 0 && l.shape[d] > 1) {
            lo += (int64_t)(l.shape[d] - 1) * l.strides[d];
            m.strides[d] = -l.strides[d];
        }
    if (lo < 0) return false;
    m.offset = (uint64_t)lo;
    if (!layout_is_c_contiguous(m) && !layout_is_permuted_dense(m)) return false;
    *first = m.offset;
    return true;
}

bool layout_is_reversed_c_contiguous(const hx_layout &l, uint64_t *first) {
    hx_layout m = l;
    int64_t lo = (int64_t)l.offset;
    bool any = false;
    for (uint32_t d = 0; d < l.rank; ++d) {
        if (l.shape[d] <= 1) continue;
        if (l.strides[d] >= 0) return false;
        lo += (int64_t)(l.shape[d] - 1) * l.strides[d];
        m.strides[d] = -l.strides[d];
        any = true;
    }
    if (!any || lo < 0) return false;
    m.offset = (uint64_t)lo;
    if (!layout_is_c_contiguous(m)) return false;
    *first = m.offset;
    return true;
}

} // namespace hx

using namespace hx;

extern "C" {

hx_status hx_validate_reduction_width(uint32_t width) {
    // core reduction.rs:339-349
    if (width == 0 || (width & (width - 1)) != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "reduction block width %u must be a power of two", width);
    return ok();
}

uint64_t hx_reduction_pass_count(uint64_t len, uint32_t width) {
    // core reduction.rs:356-366
    if (width <= 1) return len > 1 ? UINT64_MAX : 0;
    uint64_t passes = 0;
    while (len > 1) {
        len = (len + width - 1) / width;
        ++passes;
    }
    return passes;
}

hx_status hx_layout_checked_size(const hx_layout *layout, uint64_t *size) {
    HX_TRY(layout_basic_check(layout, "operand"));
    if (!size) return fail(HX_ERR_INVALID_CONFIGURATION, "null size out-pointer");
    if (!checked_size(*layout, size))
        return fail(HX_ERR_DISPATCH_FAILED, "layout rejected: shape %s overflows the element count",
                    shape_string(*layout).c_str());
    return ok();
}

hx_status hx_layout_validate_storage_len(const hx_layout *layout, uint64_t buf_len) {
    uint64_t size = 0;
    HX_TRY(hx_layout_checked_size(layout, &size));
    if (size == 0) return ok();
    __int128 lo = (__int128)layout->offset, hi = (__int128)layout->offset;
    for (uint32_t d = 0; d < layout->rank; ++d) {
        const __int128 span = (__int128)(layout->shape[d] - 1) * layout->strides[d];
        if (span < 0) lo += span;
        else hi += span;
    }
    if (lo < 0)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "layout rejected: layout %s reaches negative element index", shape_string(*layout).c_str());
    if (hi >= (__int128)buf_len)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "layout rejected: layout %s needs %llu elements but the buffer holds %llu",
                    shape_string(*layout).c_str(), (unsigned long long)(hi + 1),
                    (unsigned long long)buf_len);
    return ok();
}

int32_t hx_layout_has_zero_stride_aliasing(const hx_layout *layout) {
    if (!layout) return 0;
    for (uint32_t d = 0; d < layout->rank && d < HX_MAX_RANK; ++d)
        if (layout->strides[d] == 0 && layout->shape[d] > 1) return 1;
    return 0;
}

hx_status hx_plan_axis_reduction(const hx_layout *in, uint64_t in_buf_len, const hx_layout *out,
                                 uint64_t out_buf_len, uint32_t axis, uint32_t width,
                                 int32_t buffers_alias, uint64_t *out_len, uint64_t *axis_len) {
    // core reduction.rs:410-500, same order of checks and messages.
    if (width == 0 || (width & (width - 1)) != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "reduction block width %u must be a power of two", width);
    HX_TRY(layout_basic_check(in, "input"));
    HX_TRY(layout_basic_check(out, "output"));
    if (in->rank != 2 || out->rank != 2)
        return fail(HX_ERR_DISPATCH_FAILED, "axis reduction supports rank 2 only, got rank %u",
                    in->rank != 2 ? in->rank : out->rank);
    if (axis >= 2)
        return fail(HX_ERR_DISPATCH_FAILED, "axis %u is out of bounds for rank-2 reduction", axis);
    hx_layout expected = *in;
    expected.shape[axis] = 1;
    if (expected.shape[0] != out->shape[0] || expected.shape[1] != out->shape[1])
        return fail(HX_ERR_DISPATCH_FAILED,
                    "axis reduction output shape mismatch: input %s, axis %u, out %s",
                    shape_string(*in).c_str(), axis, shape_string(*out).c_str());
    if (buffers_alias)
        return fail(HX_ERR_DISPATCH_FAILED, "axis reduction output buffer must not alias input buffer");
    if (hx_layout_has_zero_stride_aliasing(out))
        return fail(HX_ERR_DISPATCH_FAILED,
                    "axis reduction output layout must not contain zero-stride aliasing");
    HX_TRY(hx_layout_validate_storage_len(in, in_buf_len));
    HX_TRY(hx_layout_validate_storage_len(out, out_buf_len));
    uint64_t n_out = 0;
    HX_TRY(hx_layout_checked_size(out, &n_out));
    if (out_len) *out_len = n_out;
    if (axis_len) *axis_len = in->shape[axis];
    return ok();
}

hx_status hx_plan_axis_scan(const hx_layout *in, uint64_t in_buf_len, const hx_layout *out,
                            uint64_t out_buf_len, uint32_t axis, uint32_t width,
                            int32_t buffers_alias, uint64_t *lines, uint64_t *line_len) {
    // core scan.rs:87-178 (rank 2) and its rank-1 extension.
    if (width == 0 || (width & (width - 1)) != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "scan block width %u must be a power of two", width);
    HX_TRY(layout_basic_check(in, "input"));
    HX_TRY(layout_basic_check(out, "output"));
    if (in->rank > 2)
        // core accelerator/scan.rs:519-526 (rank 2 only there; rank 1 here too)
        return fail(HX_ERR_DISPATCH_FAILED, "rocm scan supports rank 1 and 2 only, got rank %u",
                    in->rank);
    if (axis >= in->rank)
        return fail(HX_ERR_DISPATCH_FAILED, "scan axis %u is out of bounds for rank-%u scan", axis,
                    in->rank);
    bool same = in->rank == out->rank;
    for (uint32_t d = 0; same && d < in->rank; ++d) same = in->shape[d] == out->shape[d];
    if (!same)
        return fail(HX_ERR_DISPATCH_FAILED, "scan output shape mismatch: input %s, out %s",
                    shape_string(*in).c_str(), shape_string(*out).c_str());
    if (buffers_alias)
        return fail(HX_ERR_DISPATCH_FAILED, "scan output buffer must not alias input buffer");
    if (hx_layout_has_zero_stride_aliasing(out))
        return fail(HX_ERR_DISPATCH_FAILED, "scan output layout must not contain zero-stride aliasing");
    HX_TRY(hx_layout_validate_storage_len(in, in_buf_len));
    HX_TRY(hx_layout_validate_storage_len(out, out_buf_len));
    uint64_t size = 0;
    HX_TRY(hx_layout_checked_size(out, &size));
    const uint64_t len = in->shape[axis];
    const uint64_t nlines = size == 0 ? 0 : (in->rank == 2 ? in->shape[1 - axis] : 1);
    if (lines) *lines = nlines;
    if (line_len) *line_len = len;
    return ok();
}

} // extern "C"
