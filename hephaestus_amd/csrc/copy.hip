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

// Streaming copy in the load pattern of the scan tiles: a block of 8 waves
// moves one 256 KiB tile, every lane issuing all 32 of its 16-byte loads
// before its first store (a block-uniform base plus one 32-bit lane offset
// per access).  Whole tiles only; the remainder goes to copy_vec_kernel.
// Measured at 2^28 u32 on MI355X: 32 loads in flight per lane 344 us
// (6.2 TB/s), 16 loads 351 us, 8 loads 373 us; plain (temporal) loads or
// stores cost 4-6%.  Stores go through stream_store (nt | sc1): 349.5 ->
// 340 us against nt stores.  Tiles go to blocks in XCD-contiguous order
// (xcd_contiguous): 337.5 -> 332 us.
constexpr int kTileWaves = 8;
constexpr int kTileSteps = 32;
constexpr uint64_t kTileBytes = (uint64_t)kTileWaves * kWave * 16 * kTileSteps;

__global__ __launch_bounds__(kTileWaves * kWave) void copy_tiles_kernel(const char *src, char *dst) {
    const uint64_t base = (uint64_t)xcd_contiguous(blockIdx.x, gridDim.x) * kTileBytes;
    const uint32_t lane_off =
        ((uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * kWave * kTileSteps + lane_id()) * 16u;
    u32x4_a4 v[kTileSteps];
#pragma unroll
    for (int j = 0; j < kTileSteps; ++j)
        v[j] = load_a4<true>((const u32x4_a4 *)(src + base + lane_off + (uint32_t)j * (kWave * 16)));
    const auto orsrc = stream_rsrc(dst + base, (uint32_t)kTileBytes);
#pragma unroll
    for (int j = 0; j < kTileSteps; ++j) stream_store(v[j], orsrc, lane_off + (uint32_t)j * (kWave * 16));
}

// 16-byte body (both pointers 4-byte aligned: the vectors need no more),
// two vectors in flight per lane, grid-stride; the tail (< 16 bytes) is
// copied bytewise.
__global__ __launch_bounds__(kBlock) void copy_vec_kernel(const u32x4_a4 *src, u32x4_a4 *dst, uint64_t nvec,
                                                          const uint8_t *src_tail, uint8_t *dst_tail,
                                                          uint32_t tail) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x;
    for (; i + nthreads < nvec; i += 2 * nthreads) {
        const u32x4_a4 a = load_a4<true>(&src[i]);
        const u32x4_a4 b = load_a4<true>(&src[i + nthreads]);
        store_a4<true>(a, &dst[i]);
        store_a4<true>(b, &dst[i + nthreads]);
    }
    if (i < nvec) store_a4<true>(load_a4<true>(&src[i]), &dst[i]);
    if (blockIdx.x == 0 && threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

// Pointers off a 4-byte boundary: bytewise, grid-stride.
__global__ __launch_bounds__(kBlock) void copy_bytes_kernel(const uint8_t *src, uint8_t *dst, uint64_t bytes) {
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < bytes; i += nthreads) dst[i] = src[i];
}

// Copy in the access pattern of the integer scan's look-back tiles: block b
// moves tile b (no XCD reordering, since a look-back needs every tile's
// predecessors dispatched first), 8 waves x 16 steps = 128 KiB, each wave
// its own contiguous 16 KiB run, every load issued before the first store.
// The best a single-pass scan in that order and shape could stream; the
// bench reports it beside the library copy (copy_tiles_kernel).
constexpr int kScanShapeWaves = 8;
constexpr int kScanShapeSteps = 16;
constexpr uint64_t kScanShapeBytes = (uint64_t)kScanShapeWaves * kWave * 16 * kScanShapeSteps;

__global__ __launch_bounds__(kScanShapeWaves * kWave) void copy_scan_shape_kernel(const char *src, char *dst) {
    const uint64_t base = (uint64_t)blockIdx.x * kScanShapeBytes;
    const uint32_t lane_off =
        ((uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave) * kWave * kScanShapeSteps + lane_id()) * 16u;
    u32x4_a4 v[kScanShapeSteps];
#pragma unroll
    for (int j = 0; j < kScanShapeSteps; ++j)
        v[j] = load_a4<true>((const u32x4_a4 *)(src + base + lane_off + (uint32_t)j * (kWave * 16)));
    __builtin_amdgcn_sched_barrier(0);
    const auto orsrc = stream_rsrc(dst + base, (uint32_t)kScanShapeBytes);
#pragma unroll
    for (int j = 0; j < kScanShapeSteps; ++j) stream_store(v[j], orsrc, lane_off + (uint32_t)j * (kWave * 16));
}

// Zero `count` 64-bit words.  Used where status words must be cleared on a
// stream that a caller may capture into a HIP graph (a kernel node replays
// correctly where a captured memset node may not).
__global__ __launch_bounds__(kBlock) void clear_words_kernel(uint64_t *words, uint64_t count) {
    const uint64_t stride = (uint64_t)gridDim.x * kBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kBlock + threadIdx.x; i < count; i += stride) words[i] = 0;
}

} // namespace

hx_status launch_clear_words(void *words, uint64_t count, hipStream_t stream) {
    if (count == 0) return HX_OK;
    uint64_t blocks = ceil_div(count, kBlock);
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(clear_words_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, (uint64_t *)words,
                       count);
    return check_launch("clear_words_kernel");
}

hx_status launch_copy_scan_shape(const void *src, void *dst, uint64_t bytes, hipStream_t stream) {
    if (bytes % kScanShapeBytes != 0 || (((uintptr_t)src | (uintptr_t)dst) & 3u) != 0)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "the scan-shaped copy moves whole %llu-byte tiles between 4-byte aligned buffers",
                    (unsigned long long)kScanShapeBytes);
    const uint64_t tiles = bytes / kScanShapeBytes;
    if (tiles >= 0x80000000ull)
        return fail(HX_ERR_DISPATCH_FAILED, "copy of %llu bytes exceeds the grid range", (unsigned long long)bytes);
    if (tiles == 0) return HX_OK;
    hipLaunchKernelGGL(copy_scan_shape_kernel, dim3((uint32_t)tiles), dim3(kScanShapeWaves * kWave), 0, stream,
                       (const char *)src, (char *)dst);
    return check_launch("copy_scan_shape_kernel");
}

hx_status launch_copy(const void *src, void *dst, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0) return ok();
    const bool aligned = (((uintptr_t)src | (uintptr_t)dst) & 3u) == 0; // 16-byte vectors at 4-byte alignment
    if (aligned) {
        const uint64_t tiles = bytes / kTileBytes;
        if (tiles >= 0x80000000ull)
            return fail(HX_ERR_DISPATCH_FAILED, "copy of %llu bytes exceeds the grid range",
                        (unsigned long long)bytes);
        if (tiles > 0) {
            hipLaunchKernelGGL(copy_tiles_kernel, dim3((uint32_t)tiles), dim3(kTileWaves * kWave), 0, stream,
                               (const char *)src, (char *)dst);
            HX_TRY(check_launch("copy_tiles_kernel"));
        }
        const uint64_t done = tiles * kTileBytes;
        const uint64_t rest = bytes - done;
        if (rest == 0) return ok();
        const uint64_t nvec = rest / 16;
        const uint32_t tail = (uint32_t)(rest - nvec * 16);
        uint64_t blocks = ceil_div(nvec, 2 * kBlock);
        if (blocks > kMaxBlocks) blocks = kMaxBlocks;
        if (blocks < 1) blocks = 1;
        const char *s0 = (const char *)src + done;
        char *d0 = (char *)dst + done;
        hipLaunchKernelGGL(copy_vec_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, (const u32x4_a4 *)s0,
                           (u32x4_a4 *)d0, nvec, (const uint8_t *)s0 + nvec * 16, (uint8_t *)d0 + nvec * 16, tail);
        return check_launch("copy_vec_kernel");
    }
    uint64_t blocks = ceil_div(bytes, kBlock);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    hipLaunchKernelGGL(copy_bytes_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream, (const uint8_t *)src,
                       (uint8_t *)dst, bytes);
    return check_launch("copy_bytes_kernel");
}

} // namespace hx
