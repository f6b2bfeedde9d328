// Seeded synthetic inputs, generated where they are consumed (in HBM) so a
// 4 GiB operand needs no host round trip.  Every element is a pure function
// of (seed, index) (the generator is defined in hx_device.hpp), so any host
// can regenerate the same bits; the RandomInitOps seam of the reference
// (crates/hephaestus-core/src/domain/random.rs) delegates to leto-ops on the
// host instead.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ uint32_t uniform_int(uint64_t h, int64_t lo, uint64_t range) {
    // Multiply-shift of the high 32 bits: lo + floor(h_hi * range / 2^32).
    return (uint32_t)(lo + (int64_t)(((h >> 32) * range) >> 32));
}

__global__ __launch_bounds__(kBlock) void fill_uniform_int_kernel(uint32_t *dst, uint64_t n,
                                                                   uint64_t seed, int64_t lo,
                                                                   uint64_t range) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += nthreads)
        dst[i] = uniform_int(splitmix64_at(seed, i), lo, range);
}

__global__ __launch_bounds__(kBlock) void fill_uniform_real_kernel(float *dst, uint64_t n,
                                                                    uint64_t seed, float lo,
                                                                    float width) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += nthreads) {
        const float u = (float)(splitmix64_at(seed, i) >> 40) * 0x1.0p-24f; // exact
        dst[i] = __builtin_fmaf(width, u, lo);
    }
}

__global__ __launch_bounds__(kBlock) void fill_normal_kernel(float *dst, uint64_t n, uint64_t seed,
                                                              double mean, double stddev) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += nthreads) {
        const uint64_t h1 = splitmix64_at(seed, 2 * i);
        const uint64_t h2 = splitmix64_at(seed, 2 * i + 1);
        const double u1 = (double)((h1 >> 11) + 1) * 0x1.0p-53; // (0, 1]
        const double u2 = (double)(h2 >> 11) * 0x1.0p-53;       // [0, 1)
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = (float)(mean + stddev * z);
    }
}

} // namespace

hx_status launch_fill_random(void *dst, uint64_t n, hx_dtype dtype, hx_distribution dist,
                             uint64_t seed, double p0, double p1, hipStream_t stream) {
    if (n == 0) return HX_OK;
    uint64_t blocks = ceil_div(n, kBlock * 8);
    if (blocks > 16384) blocks = 16384;
    switch (dist) {
    case HX_DIST_UNIFORM_INT: {
        if (dtype == HX_DTYPE_F32)
            return fail(HX_ERR_INVALID_CONFIGURATION, "uniform integers need a u32 or i32 buffer");
        const int64_t lo = (int64_t)p0, hi = (int64_t)p1;
        if (hi < lo) return fail(HX_ERR_INVALID_CONFIGURATION, "empty integer range [%lld, %lld]",
                                 (long long)lo, (long long)hi);
        const uint64_t range = (uint64_t)(hi - lo) + 1;
        if (range > (1ull << 32))
            return fail(HX_ERR_INVALID_CONFIGURATION, "integer range wider than 2^32");
        hipLaunchKernelGGL(fill_uniform_int_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (uint32_t *)dst, n, seed, lo, range);
        return check_launch("fill_uniform_int_kernel");
    }
    case HX_DIST_UNIFORM_REAL:
        if (dtype != HX_DTYPE_F32)
            return fail(HX_ERR_INVALID_CONFIGURATION, "uniform reals need an f32 buffer");
        hipLaunchKernelGGL(fill_uniform_real_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (float *)dst, n, seed, (float)p0, (float)(p1 - p0));
        return check_launch("fill_uniform_real_kernel");
    case HX_DIST_NORMAL:
        if (dtype != HX_DTYPE_F32)
            return fail(HX_ERR_INVALID_CONFIGURATION, "normal samples need an f32 buffer");
        hipLaunchKernelGGL(fill_normal_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (float *)dst, n, seed, p0, p1);
        return check_launch("fill_normal_kernel");
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown distribution %d", (int)dist);
}

} // namespace hx
