// Dense f32 vector recurrences and elementwise arithmetic for gfx950: the
// non-reducing half of DenseVectorOps (crates/hephaestus-core/src/domain/
// vector.rs:57-200), with the expressions of the reference kernels
// (crates/hephaestus-rocm/src/application/vector.rs:36-72):
//   scale  t = t * f          axpy  t = fmaf(f, s, t)     xpay  t = fmaf(f, t, s)
//   add / sub / mul / div     o = l op r
// Whole 4096-element tiles go to a tile-per-block kernel (all loads of a
// lane before its stores) and the remainder to a 16-byte grid-stride loop.
// The 16-byte vectors need only 4-byte alignment, so operands at any element
// offset take this path; only operands off a 4-byte boundary fall back to a
// scalar grid-stride loop.
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
        const f32x4_a4 *vt = (const f32x4_a4 *)t;
        const f32x4_a4 *vs = (const f32x4_a4 *)s;
        f32x4_a4 *vo = (f32x4_a4 *)out;
        for (; i < nvec; i += nthreads) {
            const f32x4_a4 a = load_a4<true>(&vt[i]);
            f32x4_a4 b = a;
            if constexpr (kUsesS) b = load_a4<true>(&vs[i]);
            f32x4_a4 r;
            r.x = apply<OP>(a.x, b.x, f);
            r.y = apply<OP>(a.y, b.y, f);
            r.z = apply<OP>(a.z, b.z, f);
            r.w = apply<OP>(a.w, b.w, f);
            store_a4<true>(r, &vo[i]);
        }
        const uint64_t tail = nvec * 4 + (uint64_t)blockIdx.x * kBlock + threadIdx.x;
        if (blockIdx.x * (uint64_t)kBlock + threadIdx.x < n - nvec * 4)
            out[tail] = apply<OP>(t[tail], kUsesS ? s[tail] : 0.0f, f);
    } else {
        for (; i < n; i += nthreads) out[i] = apply<OP>(t[i], kUsesS ? s[i] : 0.0f, f);
    }
}

// Whole tiles in the copy kernel's pattern: a block of kTileWaves waves takes
// kTileWaves x 64 x kTileSteps vectors per operand, every lane issuing all
// its loads before its first store, through a block-uniform base and one
// 32-bit lane offset. Measured on 2^28-element axpy (12 bytes/element):
// 2 waves x 8 steps (16 KiB per operand) 6.25-6.3 TB/s; 1x4 and 4x2 6.2;
// 8x8 5.2; 8x16 6.1; 2x16 5.65; the grid-stride form above 4.6-5.0.
constexpr int kTileWaves = 2;
constexpr int kTileSteps = 8;
constexpr uint64_t kTileElems = (uint64_t)kTileWaves * kWave * 4 * kTileSteps;

template <int OP>
__global__ __launch_bounds__(kTileWaves * kWave) void vector_tiles_kernel(const float *t, const float *s, float *out,
                                                                          float f) {
    constexpr bool kUsesS = OP != HX_VEC_SCALE;
    const uint64_t base = (uint64_t)blockIdx.x * kTileElems * 4; // bytes
    const uint32_t lane_off =
        ((uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * kWave * kTileSteps + lane_id()) * 16u;
    f32x4_a4 a[kTileSteps], b[kTileSteps];
#pragma unroll
    for (int j = 0; j < kTileSteps; ++j) {
        a[j] = load_a4<true>((const f32x4_a4 *)((const char *)t + base + lane_off + (uint32_t)j * (kWave * 16)));
        if constexpr (kUsesS)
            b[j] = load_a4<true>((const f32x4_a4 *)((const char *)s + base + lane_off + (uint32_t)j * (kWave * 16)));
    }
    const auto orsrc = stream_rsrc((char *)out + base, (uint32_t)(kTileElems * 4));
#pragma unroll
    for (int j = 0; j < kTileSteps; ++j) {
        f32x4_a4 r;
        const f32x4_a4 y = kUsesS ? b[j] : a[j];
        r.x = apply<OP>(a[j].x, y.x, f);
        r.y = apply<OP>(a[j].y, y.y, f);
        r.z = apply<OP>(a[j].z, y.z, f);
        r.w = apply<OP>(a[j].w, y.w, f);
        stream_store(r, orsrc, lane_off + (uint32_t)j * (kWave * 16));
    }
}

template <int OP> hx_status launch_op(const float *t, const float *s, float *out, uint64_t n, float f, hipStream_t stream) {
    // 16-byte vectors at 4-byte alignment (f32x4_a4): every f32 operand
    // qualifies wherever it starts.
    const bool vec = ((((uintptr_t)t | (uintptr_t)out | (OP == HX_VEC_SCALE ? 0 : (uintptr_t)s)) & 3u) == 0);
    if (vec && n >= kTileElems) {
        const uint64_t tiles = n / kTileElems;
        if (tiles >= 0x80000000ull)
            return fail(HX_ERR_DISPATCH_FAILED, "vector of %llu elements exceeds the grid range", (unsigned long long)n);
        hipLaunchKernelGGL((vector_tiles_kernel<OP>), dim3((uint32_t)tiles), dim3(kTileWaves * kWave), 0, stream, t, s,
                           out, f);
        HX_TRY(check_launch("vector_tiles_kernel"));
        const uint64_t done = tiles * kTileElems;
        t += done;
        if (OP != HX_VEC_SCALE) s += done;
        out += done;
        n -= done;
        if (n == 0) return ok();
    }
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
