// Device-local copy behind hx_copy (copy_buffer, crates/hephaestus-core/src/
// domain/device.rs:197-211).  A plain streaming kernel rather than a DMA
// engine copy: it runs on the compute queue in stream order like every other
// kernel here, and its known traffic (read B, write B) is the yardstick that
// the HBM byte counters of the other kernels are calibrated against.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {
namespace {

constexpr int kBlock = 256;
constexpr uint32_t kMaxBlocks = 2048;

// 16-byte body (both pointers 16-byte aligned), two vectors in flight per
// lane, grid-stride; the tail (< 16 bytes) is copied bytewise.
__global__ __launch_bounds__(kBlock) void copy_vec_kernel(const u32x4 *src, u32x4 *dst, uint64_t nvec,
                                                          const uint8_t *src_tail, uint8_t *dst_tail,
                                                          uint32_t tail) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    for (; i + nthreads < nvec; i += 2 * nthreads) {
        const u32x4 a = load_vec<true>(&src[i]);
        const u32x4 b = load_vec<true>(&src[i + nthreads]);
        store_vec<true>(a, &dst[i]);
        store_vec<true>(b, &dst[i + nthreads]);
    }
    if (i < nvec) store_vec<true>(load_vec<true>(&src[i]), &dst[i]);
    if (blockIdx.x == 0 && threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

// Unaligned pointers: bytewise, grid-stride.
__global__ __launch_bounds__(kBlock) void copy_bytes_kernel(const uint8_t *src, uint8_t *dst, uint64_t bytes) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < bytes; i += nthreads) dst[i] = src[i];
}

} // namespace

hx_status launch_copy(const void *src, void *dst, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0) return ok();
    const bool aligned = (((uintptr_t)src | (uintptr_t)dst) & 15u) == 0;
    if (aligned) {
        const uint64_t nvec = bytes / 16;
        const uint32_t tail = (uint32_t)(bytes - nvec * 16);
        uint64_t blocks = ceil_div(nvec, 2 * kBlock);
        if (blocks > kMaxBlocks) blocks = kMaxBlocks;
        if (blocks < 1) blocks = 1;
        hipLaunchKernelGGL(copy_vec_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, (const u32x4 *)src,
                           (u32x4 *)dst, nvec, (const uint8_t *)src + nvec * 16, (uint8_t *)dst + nvec * 16, tail);
        return check_launch("copy_vec_kernel");
    }
    uint64_t blocks = ceil_div(bytes, kBlock);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, (const uint8_t *)src,
                       (uint8_t *)dst, bytes);
    return check_launch("copy_bytes_kernel");
}

} // namespace hx
