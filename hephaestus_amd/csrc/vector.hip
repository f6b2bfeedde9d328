// Dense f32 vector recurrences and elementwise arithmetic for gfx950: the
// non-reducing half of DenseVectorOps (crates/hephaestus-core/src/domain/
// vector.rs:57-200), with the expressions of the reference kernels
// (crates/hephaestus-rocm/src/application/vector.rs:36-72):
//   scale  t = t * f          axpy  t = fmaf(f, s, t)     xpay  t = fmaf(f, t, s)
//   add / sub / mul / div     o = l op r
// One streaming kernel per form: 16-byte vectors, two in flight per lane,
// grid-stride, when every operand is 16-byte aligned; a scalar grid-stride
// loop otherwise.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {
namespace {

constexpr int kBlock = 256;
constexpr uint64_t kMaxBlocks = 2048;

template <int OP> __device__ __forceinline__ float apply(float t, float s, float f) {
    if constexpr (OP == HX_VEC_SCALE) return t * f;
    else if constexpr (OP == HX_VEC_AXPY) return __builtin_fmaf(f, s, t);
    else if constexpr (OP == HX_VEC_XPAY) return __builtin_fmaf(f, t, s);
    else if constexpr (OP == HX_VEC_ADD) return t + s;
    else if constexpr (OP == HX_VEC_SUB) return t - s;
    else if constexpr (OP == HX_VEC_MUL) return t * s;
    else return t / s;
}

// out[i] = apply(t[i], s[i], f); for scale s is unused, for the binary
// forms t is the left operand and s the right.
template <int OP, bool VEC>
__global__ __launch_bounds__(kBlock) void vector_kernel(const float *t, const float *s, float *out, uint64_t n, float f) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    constexpr bool kUsesS = OP != HX_VEC_SCALE;
    if constexpr (VEC) {
        const uint64_t nvec = n / 4;
        const f32x4 *vt = (const f32x4 *)t;
        const f32x4 *vs = (const f32x4 *)s;
        f32x4 *vo = (f32x4 *)out;
        for (; i < nvec; i += nthreads) {
            const f32x4 a = load_vec<true>(&vt[i]);
            f32x4 b = a;
            if constexpr (kUsesS) b = load_vec<true>(&vs[i]);
            f32x4 r;
            r.x = apply<OP>(a.x, b.x, f);
            r.y = apply<OP>(a.y, b.y, f);
            r.z = apply<OP>(a.z, b.z, f);
            r.w = apply<OP>(a.w, b.w, f);
            store_vec<true>(r, &vo[i]);
        }
        const uint64_t tail = nvec * 4 + (uint64_t)blockIdx.x * kBlock + threadIdx.x;
        if (blockIdx.x * (uint64_t)kBlock + threadIdx.x < n - nvec * 4)
            out[tail] = apply<OP>(t[tail], kUsesS ? s[tail] : 0.0f, f);
    } else {
        for (; i < n; i += nthreads) out[i] = apply<OP>(t[i], kUsesS ? s[i] : 0.0f, f);
    }
}

template <int OP> hx_status launch_op(const float *t, const float *s, float *out, uint64_t n, float f, hipStream_t stream) {
    const bool vec = ((((uintptr_t)t | (uintptr_t)out | (OP == HX_VEC_SCALE ? 0 : (uintptr_t)s)) & 15u) == 0);
    uint64_t blocks = ceil_div(vec ? ceil_div(n, 4) : n, kBlock);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    if (blocks < 1) blocks = 1;
    if (vec)
        hipLaunchKernelGGL((vector_kernel<OP, true>), dim3((uint32_t)blocks), dim3(kBlock), 0, stream, t, s, out, n, f);
    else
        hipLaunchKernelGGL((vector_kernel<OP, false>), dim3((uint32_t)blocks), dim3(kBlock), 0, stream, t, s, out, n, f);
    return check_launch("vector_kernel");
}

} // namespace

hx_status launch_vector_op(hx_vector_op op, const float *t, const float *s, float *out, uint64_t n, float f,
                           hipStream_t stream) {
    if (n == 0) return ok();
    switch (op) {
    case HX_VEC_SCALE: return launch_op<HX_VEC_SCALE>(t, s, out, n, f, stream);
    case HX_VEC_AXPY: return launch_op<HX_VEC_AXPY>(t, s, out, n, f, stream);
    case HX_VEC_XPAY: return launch_op<HX_VEC_XPAY>(t, s, out, n, f, stream);
    case HX_VEC_ADD: return launch_op<HX_VEC_ADD>(t, s, out, n, f, stream);
    case HX_VEC_SUB: return launch_op<HX_VEC_SUB>(t, s, out, n, f, stream);
    case HX_VEC_MUL: return launch_op<HX_VEC_MUL>(t, s, out, n, f, stream);
    case HX_VEC_DIV: return launch_op<HX_VEC_DIV>(t, s, out, n, f, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown vector operation %d", (int)op);
}

} // namespace hx
