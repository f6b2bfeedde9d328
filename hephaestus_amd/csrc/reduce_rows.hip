// Row-wise and axis reductions for gfx950: AxisReductionOps
// (crates/hephaestus-core/src/domain/reduction.rs:74-223) plus the fused
// row reduce: sum, max and argmax of y = fmaf(a, x, b) out of ONE read of
// each row.
//
// The reference runs one thread per output with a serial loop along the
// axis (crates/hephaestus-rocm/src/application/axis_reduction.rs:16-65): for
// a row-major matrix reduced along axis 1, neighbouring lanes are a whole
// row apart, so no load is coalesced, and sum and max are two full passes.
// Here:
//   rows_kernel  one wave64 per row: lane l reads 16-byte vectors l, l+64,
//                ... of the row (every load instruction covers 1 KiB of
//                contiguous memory), keeps every requested statistic in
//                registers, then combines them with xor-butterflies.  Used
//                whenever the reduced axis has unit stride (or no stride is
//                unit).
//   cols_kernel  one thread per output when the OTHER axis has unit stride
//                (axis-0 reduction of a row-major matrix): each load
//                instruction of a wave covers 64 adjacent outputs.
#include "hx_device.hpp"
#include "hx_internal.hpp"

#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;

enum Flag : int {
    F_SUM = 1,
    F_MAX = 2,
    F_ARG = 4,
    F_MIN = 8,
    F_PROD = 16,
    F_MEAN = 32,
};

struct RowParams {
    const void *base;
    uint64_t rows, cols;
    int64_t row_stride, col_stride;
    uint64_t offset;
    float a, b;
    void *out_sum;  // SUM or MEAN
    void *out_max;
    uint32_t *out_arg;
    void *out_min;
    void *out_prod;
    int64_t out_stride;
    uint64_t out_offset;
};

template <typename T, bool AFFINE> __device__ __forceinline__ T prologue(T x, float, float) { return x; }
template <> __device__ __forceinline__ float prologue<float, true>(float x, float a, float b) {
    return __builtin_fmaf(a, x, b);
}

template <typename T> struct Acc;
template <> struct Acc<float> { using sum = double; using prod = double; };
template <> struct Acc<uint32_t> { using sum = uint32_t; using prod = uint32_t; };
template <> struct Acc<int32_t> { using sum = uint32_t; using prod = uint32_t; };

// Running statistics of one lane (or thread).
template <typename T, int FLAGS> struct Stats {
    using S = typename Acc<T>::sum;
    using Pr = typename Acc<T>::prod;
    S sum = S(0);
    Pr prod = Pr(1);
    uint32_t maxk = Key<T>::max_identity();
    uint32_t mink = Key<T>::min_identity();
    uint64_t arg = 0ull;

    __device__ __forceinline__ void visit(T y, uint32_t j) {
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum += (S)(typename Wrap<T>::type)y;
        if constexpr ((FLAGS & F_PROD) != 0) prod *= (Pr)(typename Wrap<T>::type)y;
        if constexpr ((FLAGS & F_ARG) != 0) {
            arg = umax64(arg, pack_arg(Key<T>::max_key(y), j));
        } else if constexpr ((FLAGS & F_MAX) != 0) {
            uint32_t k = Key<T>::max_key(y);
            maxk = maxk > k ? maxk : k;
        }
        if constexpr ((FLAGS & F_MIN) != 0) {
            uint32_t k = Key<T>::min_key(y);
            mink = mink < k ? mink : k;
        }
    }
    __device__ __forceinline__ void wave_combine() {
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum = wave_sum(sum);
        if constexpr ((FLAGS & F_PROD) != 0) prod = wave_prod(prod);
        if constexpr ((FLAGS & F_ARG) != 0) arg = wave_umax64(arg);
        else if constexpr ((FLAGS & F_MAX) != 0) maxk = wave_umax(maxk);
        if constexpr ((FLAGS & F_MIN) != 0) mink = wave_umin(mink);
    }
    __device__ __forceinline__ void write(const RowParams &p, uint64_t r) const {
        const int64_t o = (int64_t)p.out_offset + (int64_t)r * p.out_stride;
        if constexpr ((FLAGS & F_SUM) != 0) ((T *)p.out_sum)[o] = (T)sum;
        if constexpr ((FLAGS & F_MEAN) != 0) {
            if constexpr (std::is_same<T, float>::value)
                ((float *)p.out_sum)[o] = (float)(sum / (double)p.cols);
            else if constexpr (std::is_same<T, int32_t>::value)
                ((int32_t *)p.out_sum)[o] = (int32_t)sum / (int32_t)p.cols;
            else
                ((uint32_t *)p.out_sum)[o] = (uint32_t)sum / (uint32_t)p.cols;
        }
        if constexpr ((FLAGS & F_PROD) != 0) ((T *)p.out_prod)[o] = (T)prod;
        if constexpr ((FLAGS & F_ARG) != 0) {
            const uint32_t key = (uint32_t)(arg >> 32);
            const bool none = std::is_same<T, float>::value ? (key == 0u) : (arg == 0ull);
            if (p.out_arg) p.out_arg[o] = none ? 0xFFFFFFFFu : arg_index(arg);
            if ((FLAGS & F_MAX) != 0 && p.out_max) {
                uint32_t mk = Key<T>::max_identity();
                if (!none && key > mk) mk = key;
                ((T *)p.out_max)[o] = Key<T>::decode(mk);
            }
        } else if constexpr ((FLAGS & F_MAX) != 0) {
            ((T *)p.out_max)[o] = Key<T>::decode(maxk);
        }
        if constexpr ((FLAGS & F_MIN) != 0) ((T *)p.out_min)[o] = Key<T>::decode(mink);
    }
};

// One wave per row.  VEC: unit column stride and every row start 16-byte
// aligned, so lanes issue global_load_dwordx4.
template <typename T, bool AFFINE, int FLAGS, bool VEC>
__global__ __launch_bounds__(kBlock) void rows_kernel(RowParams p) {
    const int lane = lane_id();
    const uint64_t wave = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    const uint64_t nwaves = (uint64_t)gridDim.x * (kBlock / kWave);
    for (uint64_t r = wave; r < p.rows; r += nwaves) {
        const T *row = (const T *)p.base + ((int64_t)p.offset + (int64_t)r * p.row_stride);
        Stats<T, FLAGS> st;
        if constexpr (VEC) {
            using V = typename Vec4<T>::type;
            const V *vrow = (const V *)row;
            const uint64_t nvec = p.cols >> 2;
            uint64_t v = lane;
            for (; v + 3 * kWave < nvec; v += 4 * kWave) {
                V x[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) x[u] = __builtin_nontemporal_load(&vrow[v + u * kWave]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t j = (uint32_t)(4 * (v + u * kWave));
                    st.visit(prologue<T, AFFINE>((T)x[u].x, p.a, p.b), j);
                    st.visit(prologue<T, AFFINE>((T)x[u].y, p.a, p.b), j + 1);
                    st.visit(prologue<T, AFFINE>((T)x[u].z, p.a, p.b), j + 2);
                    st.visit(prologue<T, AFFINE>((T)x[u].w, p.a, p.b), j + 3);
                }
            }
            for (; v < nvec; v += kWave) {
                V x = __builtin_nontemporal_load(&vrow[v]);
                const uint32_t j = (uint32_t)(4 * v);
                st.visit(prologue<T, AFFINE>((T)x.x, p.a, p.b), j);
                st.visit(prologue<T, AFFINE>((T)x.y, p.a, p.b), j + 1);
                st.visit(prologue<T, AFFINE>((T)x.z, p.a, p.b), j + 2);
                st.visit(prologue<T, AFFINE>((T)x.w, p.a, p.b), j + 3);
            }
            const uint64_t j = 4 * nvec + lane;
            if (j < p.cols) st.visit(prologue<T, AFFINE>(row[j], p.a, p.b), (uint32_t)j);
        } else {
            for (uint64_t j = lane; j < p.cols; j += kWave)
                st.visit(prologue<T, AFFINE>(row[(int64_t)j * p.col_stride], p.a, p.b), (uint32_t)j);
        }
        st.wave_combine();
        if (lane == 0) st.write(p, r);
    }
}

// One thread per output; the reduced axis is walked serially, which is
// coalesced across the wave when the outputs are adjacent in memory.
template <typename T, bool AFFINE, int FLAGS>
__global__ __launch_bounds__(kBlock) void cols_kernel(RowParams p) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t r = (uint64_t)blockIdx.x * kBlock + threadIdx.x; r < p.rows; r += nthreads) {
        const T *line = (const T *)p.base + ((int64_t)p.offset + (int64_t)r * p.row_stride);
        Stats<T, FLAGS> st;
        for (uint64_t j = 0; j < p.cols; ++j)
            st.visit(prologue<T, AFFINE>(line[(int64_t)j * p.col_stride], p.a, p.b), (uint32_t)j);
        st.write(p, r);
    }
}

template <typename T, bool AFFINE, int FLAGS>
hx_status launch_rows_typed(const RowParams &p, bool cols_layout, hipStream_t stream) {
    if (p.rows == 0) return HX_OK;
    if (cols_layout) {
        uint64_t blocks = ceil_div(p.rows, kBlock);
        if (blocks > (1u << 20)) blocks = 1u << 20;
        hipLaunchKernelGGL((cols_kernel<T, AFFINE, FLAGS>), dim3((uint32_t)blocks), dim3(kBlock),
                           0, stream, p);
        return check_launch("cols_kernel");
    }
    const uintptr_t base = (uintptr_t)((const T *)p.base + p.offset);
    const bool vec = p.col_stride == 1 && (base % 16) == 0 && (p.row_stride % 4) == 0;
    uint64_t blocks = ceil_div(p.rows, kBlock / kWave);
    if (blocks > (1u << 20)) blocks = 1u << 20;
    if (vec)
        hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true>), dim3((uint32_t)blocks),
                           dim3(kBlock), 0, stream, p);
    else
        hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, false>), dim3((uint32_t)blocks),
                           dim3(kBlock), 0, stream, p);
    return check_launch("rows_kernel");
}

template <typename T, bool AFFINE>
hx_status launch_rows_flags(const RowParams &p, int flags, bool cols_layout, hipStream_t stream) {
    switch (flags) {
    case F_SUM: return launch_rows_typed<T, AFFINE, F_SUM>(p, cols_layout, stream);
    case F_MAX: return launch_rows_typed<T, AFFINE, F_MAX>(p, cols_layout, stream);
    case F_ARG: return launch_rows_typed<T, AFFINE, F_ARG>(p, cols_layout, stream);
    case F_MIN: return launch_rows_typed<T, AFFINE, F_MIN>(p, cols_layout, stream);
    case F_PROD: return launch_rows_typed<T, AFFINE, F_PROD>(p, cols_layout, stream);
    case F_MEAN: return launch_rows_typed<T, AFFINE, F_MEAN>(p, cols_layout, stream);
    case F_SUM | F_MAX: return launch_rows_typed<T, AFFINE, F_SUM | F_MAX>(p, cols_layout, stream);
    case F_SUM | F_ARG: return launch_rows_typed<T, AFFINE, F_SUM | F_ARG>(p, cols_layout, stream);
    case F_MAX | F_ARG: return launch_rows_typed<T, AFFINE, F_MAX | F_ARG>(p, cols_layout, stream);
    case F_SUM | F_MAX | F_ARG:
        return launch_rows_typed<T, AFFINE, F_SUM | F_MAX | F_ARG>(p, cols_layout, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unsupported row statistic set %d", flags);
}

hx_status launch_rows_any(const RowParams &p, hx_dtype dtype, bool affine, int flags,
                          bool cols_layout, hipStream_t stream) {
    switch (dtype) {
    case HX_DTYPE_F32:
        return affine ? launch_rows_flags<float, true>(p, flags, cols_layout, stream)
                      : launch_rows_flags<float, false>(p, flags, cols_layout, stream);
    case HX_DTYPE_U32: return launch_rows_flags<uint32_t, false>(p, flags, cols_layout, stream);
    case HX_DTYPE_I32: return launch_rows_flags<int32_t, false>(p, flags, cols_layout, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)dtype);
}

} // namespace

hx_status launch_rows(const RowsArgs &a, hipStream_t stream) {
    RowParams p{};
    p.base = a.base;
    p.rows = a.rows;
    p.cols = a.cols;
    p.row_stride = (int64_t)a.row_stride;
    p.col_stride = 1;
    p.offset = a.offset;
    p.a = a.a;
    p.b = a.b;
    p.out_sum = a.out_sum;
    p.out_max = a.out_max;
    p.out_arg = a.out_argmax;
    p.out_stride = 1;
    p.out_offset = 0;
    int flags = (a.out_sum ? F_SUM : 0) | (a.out_argmax ? F_ARG : 0) | (a.out_max ? F_MAX : 0);
    if (flags == 0) return HX_OK;
    return launch_rows_any(p, a.dtype, a.affine, flags, false, stream);
}

hx_status launch_axis_reduce(const AxisArgs &a, hipStream_t stream) {
    RowParams p{};
    p.base = a.in;
    p.rows = a.outer;
    p.cols = a.axis_len;
    p.row_stride = a.in_outer_stride;
    p.col_stride = a.in_axis_stride;
    p.offset = a.in_offset;
    p.out_stride = a.out_stride;
    p.out_offset = a.out_offset;
    int flags = 0;
    switch (a.op) {
    case HX_OP_SUM: flags = F_SUM; p.out_sum = a.out; break;
    case HX_OP_MEAN: flags = F_MEAN; p.out_sum = a.out; break;
    case HX_OP_PROD: flags = F_PROD; p.out_prod = a.out; break;
    case HX_OP_MIN: flags = F_MIN; p.out_min = a.out; break;
    case HX_OP_MAX: flags = F_MAX; p.out_max = a.out; break;
    case HX_OP_ARGMAX: flags = F_ARG; p.out_arg = (uint32_t *)a.out; break;
    }
    // Unit stride along the reduced axis -> lanes along the axis; unit
    // stride across outputs -> threads across outputs.
    const bool axis_unit = a.in_axis_stride == 1 || a.in_axis_stride == -1;
    const bool outer_unit = a.in_outer_stride == 1 || a.in_outer_stride == -1;
    const bool cols_layout = !axis_unit && outer_unit && a.outer >= 64;
    return launch_rows_any(p, a.dtype, false, flags, cols_layout, stream);
}

} // namespace hx
