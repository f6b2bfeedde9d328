// Device acquisition, memory, transfers, events, workspace and plan
// plumbing behind the C ABI.  Mirrors the reference's ROCm infrastructure
// layer (crates/hephaestus-rocm/src/infrastructure/{device,memory,query}.rs)
// with pinned, double-buffered staging instead of synchronous pageable
// hipMemcpy calls.
#include "hx_internal.hpp"

#include <cstdarg>
#include <cstdio>
#include <atomic>
#include <cstring>
#include <new>

namespace {

thread_local std::string t_message;
thread_local uint64_t t_host_len = 0;
thread_local uint64_t t_device_len = 0;

// Transfers at or below this size go through one synchronous hipMemcpy.
constexpr uint64_t kSmallTransfer = 1ull << 20;
// Each of the two pinned staging buffers.
constexpr uint64_t kStagingChunk = 32ull << 20;

} // namespace

namespace hx {

hx_status ok() {
    t_message.clear();
    return HX_OK;
}

hx_status fail(hx_status status, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_message = buf;
    return status;
}

// error.rs:30-36: "host length {host_len} does not match device buffer
// length {device_len}".
hx_status length_mismatch(uint64_t host_len, uint64_t device_len) {
    t_host_len = host_len;
    t_device_len = device_len;
    return fail(HX_ERR_LENGTH_MISMATCH,
                "host length %llu does not match device buffer length %llu",
                (unsigned long long)host_len, (unsigned long long)device_len);
}

hx_status hip_fail(hx_status status, hipError_t err, const char *what) {
    // The runtime also keeps this error as the thread's last error; clear it,
    // or the next launch's check_launch would report it again.
    (void)hipGetLastError();
    return fail(status, "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
}

hx_status bind_device(const hx_device *dev) {
    if (dev == nullptr)
        return fail(HX_ERR_INVALID_CONFIGURATION, "null device handle");
    HX_HIP(hipSetDevice(dev->ordinal), HX_ERR_DEVICE_UNAVAILABLE, "hipSetDevice");
    return HX_OK;
}

hipStream_t pick_stream(const hx_device *dev, hx_stream stream) {
    return stream ? (hipStream_t)stream : dev->stream;
}

hx_status stream_capturing(hipStream_t stream, bool *capturing) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    HX_HIP(hipStreamIsCapturing(stream, &status), HX_ERR_DISPATCH_FAILED, "hipStreamIsCapturing");
    *capturing = status != hipStreamCaptureStatusNone;
    return HX_OK;
}

hx_status check_launch(const char *kernel) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return hip_fail(HX_ERR_DISPATCH_FAILED, err, kernel);
    return HX_OK;
}

hx_status alloc_workspace(hx_device *dev, uint64_t bytes, void **ws) {
    *ws = nullptr;
    if (bytes == 0) return HX_OK;
    void *p = nullptr;
    HX_HIP(hipMalloc(&p, bytes), HX_ERR_ALLOCATION_FAILED, "workspace hipMalloc");
    hipError_t err = hipMemsetAsync(p, 0, bytes, dev->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(dev->stream);
    if (err != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(HX_ERR_ALLOCATION_FAILED, err, "workspace zero-fill");
    }
    *ws = p;
    return HX_OK;
}

namespace {

// Replace `buf` by a zeroed buffer of at least `need` bytes.  The old buffer
// may still be read by launches queued on `stream` (its only user), so the
// stream is drained before it is freed; the zero-fill is queued on `stream`
// ahead of the launches that will use the new buffer.
hx_status grow_stream_buffer(hipStream_t stream, void *&buf, uint64_t &have, uint64_t need, const char *what) {
    if (need <= have) return HX_OK;
    if (buf) {
        HX_HIP(hipStreamSynchronize(stream), HX_ERR_DISPATCH_FAILED, "stream synchronize before buffer growth");
        HX_HIP(hipFree(buf), HX_ERR_ALLOCATION_FAILED, what);
        buf = nullptr;
        have = 0;
    }
    const uint64_t grow = need < (1ull << 20) ? (1ull << 20) : need;
    void *p = nullptr;
    HX_HIP(hipMalloc(&p, grow), HX_ERR_ALLOCATION_FAILED, what);
    hipError_t err = hipMemsetAsync(p, 0, grow, stream);
    if (err != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(HX_ERR_ALLOCATION_FAILED, err, what);
    }
    buf = p;
    have = grow;
    return HX_OK;
}

} // namespace

hx_status Immediate::open(hx_device *dev, hipStream_t stream) {
    dev_ = dev;
    stream_ = stream;
    // An immediate call draws a fresh look-back tag per call and may grow
    // (allocate, zero-fill, synchronize) its stream's buffers: none of that
    // can be recorded into a graph and replayed.
    bool capturing = false;
    HX_TRY(stream_capturing(stream, &capturing));
    if (capturing)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "immediate calls cannot be recorded into a HIP graph (the stream is capturing): capture "
                    "hx_plan_dispatch of a prepared plan, or hx_scan_noalloc, instead");
    {
        std::lock_guard<std::mutex> guard(dev->streams_mu);
        std::unique_ptr<StreamWorkspace> &slot = dev->immediate[stream];
        if (!slot) {
            slot.reset(new (std::nothrow) StreamWorkspace());
            if (!slot) {
                dev->immediate.erase(stream);
                return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of a stream workspace failed");
            }
        }
        // Entries are erased only by hx_stream_release, whose caller
        // guarantees that no other call uses that stream meanwhile.
        sw_ = slot.get();
    }
    lock_ = std::unique_lock<std::mutex>(sw_->mu);
    return HX_OK;
}

hx_status Immediate::workspace(uint64_t bytes, void **ws) {
    const bool grows = bytes > sw_->ws_bytes;
    HX_TRY(grow_stream_buffer(stream_, sw_->ws, sw_->ws_bytes, bytes, "immediate workspace"));
    if (grows) sw_->lookback = LookbackState{};
    *ws = sw_->ws;
    return HX_OK;
}

hx_status Immediate::scratch(uint64_t bytes, void **scratch) {
    *scratch = nullptr;
    if (bytes == 0) return HX_OK;
    HX_TRY(grow_stream_buffer(stream_, sw_->scratch, sw_->scratch_bytes, bytes, "immediate scratch"));
    *scratch = sw_->scratch;
    return HX_OK;
}

hx_status next_lookback_launch(LookbackState &st, void *ws, uint64_t ws_bytes,
                               hipStream_t stream, uint32_t *tag) {
    if (st.captured) {
        *tag = kCapturedTag;
        return HX_OK;
    }
    // Eager tags cycle through [1, kCapturedTag).
    const uint32_t t = (uint32_t)(st.launches % (kCapturedTag - 1u)) + 1u;
    if (t == 1u && st.launches != 0u && ws_bytes > kLookbackOffset) {
        // The tag range wrapped: words from kCapturedTag - 1 launches ago
        // would read as current, so clear them once (a fill kernel, which a
        // graph replays correctly).
        HX_TRY(launch_clear_words((char *)ws + kLookbackOffset, (ws_bytes - kLookbackOffset) / 8, stream));
    }
    *tag = t;
    return HX_OK;
}

void commit_lookback_launch(LookbackState &st) {
    if (!st.captured) st.launches += 1u;
}

namespace {
std::atomic<uint32_t> g_lookback_polls{64};
std::atomic<uint32_t> g_gather_polls{1u << 14};
} // namespace

uint32_t lookback_poll_limit() { return g_lookback_polls.load(std::memory_order_relaxed); }
uint32_t gather_poll_limit() { return g_gather_polls.load(std::memory_order_relaxed); }

} // namespace hx

hx_plan::~hx_plan() {
    if (ws) {
        (void)hipSetDevice(dev->ordinal);
        (void)hipFree(ws);
    }
}

using namespace hx;

extern "C" {

uint32_t hx_abi_version(void) { return HX_ABI_VERSION; }

hx_status hx_debug_set_wait_limits(uint32_t lookback_polls, uint32_t gather_polls) {
    g_lookback_polls.store(lookback_polls, std::memory_order_relaxed);
    g_gather_polls.store(gather_polls, std::memory_order_relaxed);
    return ok();
}

hx_status hx_debug_set_launch_count(hx_device *dev, hx_plan *plan, hx_stream stream, uint64_t launches) {
    if (plan) {
        std::lock_guard<std::mutex> guard(plan->mu);
        plan->lookback.launches = launches;
        return ok();
    }
    if (!dev) return fail(HX_ERR_INVALID_CONFIGURATION, "null device handle");
    const hipStream_t s = pick_stream(dev, stream);
    StreamWorkspace *sw = nullptr;
    {
        std::lock_guard<std::mutex> guard(dev->streams_mu);
        auto it = dev->immediate.find(s);
        if (it == dev->immediate.end())
            return fail(HX_ERR_INVALID_CONFIGURATION, "no immediate workspace has been used on this stream");
        sw = it->second.get();
    }
    std::lock_guard<std::mutex> guard(sw->mu);
    sw->lookback.launches = launches;
    return ok();
}


const char *hx_status_name(hx_status status) {
    switch (status) {
    case HX_OK: return "Ok";
    case HX_ERR_ADAPTER_UNAVAILABLE: return "AdapterUnavailable";
    case HX_ERR_DEVICE_UNAVAILABLE: return "DeviceUnavailable";
    case HX_ERR_ALLOCATION_FAILED: return "AllocationFailed";
    case HX_ERR_LENGTH_MISMATCH: return "LengthMismatch";
    case HX_ERR_DISPATCH_FAILED: return "DispatchFailed";
    case HX_ERR_INVALID_CONFIGURATION: return "InvalidConfiguration";
    case HX_ERR_TRANSFER_FAILED: return "TransferFailed";
    }
    return "Unknown";
}

const char *hx_last_error_message(void) { return t_message.c_str(); }

void hx_last_length_mismatch(uint64_t *host_len, uint64_t *device_len) {
    if (host_len) *host_len = t_host_len;
    if (device_len) *device_len = t_device_len;
}

hx_status hx_device_count(int32_t *count) {
    if (!count) return fail(HX_ERR_INVALID_CONFIGURATION, "null count pointer");
    *count = 0;
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    if (err == hipErrorNoDevice) return ok();
    if (err != hipSuccess)
        return hip_fail(HX_ERR_ADAPTER_UNAVAILABLE, err, "hipGetDeviceCount");
    *count = n;
    return ok();
}

hx_status hx_device_open(int32_t ordinal, hx_device **out) {
    if (!out) return fail(HX_ERR_INVALID_CONFIGURATION, "null device out-pointer");
    *out = nullptr;
    int count = 0;
    hipError_t err = hipGetDeviceCount(&count);
    if (err == hipErrorNoDevice) count = 0;
    else if (err != hipSuccess)
        return hip_fail(HX_ERR_ADAPTER_UNAVAILABLE, err, "hipGetDeviceCount");
    // device.rs:121-126
    if (ordinal < 0 || ordinal >= count)
        return fail(HX_ERR_ADAPTER_UNAVAILABLE,
                    "ROCm device ordinal %d unavailable; device count %d", ordinal, count);

    hx_device *dev = new (std::nothrow) hx_device();
    if (!dev) return fail(HX_ERR_ALLOCATION_FAILED, "host allocation of device handle failed");
    dev->ordinal = ordinal;
    auto bail = [&](hx_status s) {
        if (dev->stream) (void)hipStreamDestroy(dev->stream);
        delete dev;
        return s;
    };
    err = hipSetDevice(ordinal);
    if (err != hipSuccess) return bail(hip_fail(HX_ERR_DEVICE_UNAVAILABLE, err, "hipSetDevice"));
    hipDeviceProp_t prop;
    err = hipGetDeviceProperties(&prop, ordinal);
    if (err != hipSuccess)
        return bail(hip_fail(HX_ERR_DEVICE_UNAVAILABLE, err, "hipGetDeviceProperties"));
    hx_device_info &info = dev->info;
    snprintf(info.name, sizeof info.name, "%s", prop.name);
    snprintf(info.arch, sizeof info.arch, "%s", prop.gcnArchName);
    info.ordinal = ordinal;
    info.compute_units = (uint32_t)prop.multiProcessorCount;
    info.warp_size = (uint32_t)prop.warpSize;
    info.max_threads_per_block = (uint32_t)prop.maxThreadsPerBlock;
    info.max_threads_per_cu = (uint32_t)prop.maxThreadsPerMultiProcessor;
    info.lds_bytes_per_block = (uint32_t)prop.sharedMemPerBlock;
    info.regs_per_block = (uint32_t)prop.regsPerBlock;
    info.clock_khz = (uint32_t)prop.clockRate;
    info.memory_clock_khz = (uint32_t)prop.memoryClockRate;
    info.memory_bus_width_bits = (uint32_t)prop.memoryBusWidth;
    info.l2_bytes = (uint64_t)prop.l2CacheSize;
    info.total_memory_bytes = (uint64_t)prop.totalGlobalMem;
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess) info.free_memory_bytes = free_b;
    // Device limits (ROCm query.rs:28-90).
    {
        hx_device_limits &lim = dev->limits;
        lim.max_buffer_size = info.free_memory_bytes;
        struct {
            hipDeviceAttribute_t attr;
            uint32_t *dst;
            const char *name;
        } q[] = {
            {hipDeviceAttributeMaxBlockDimX, &lim.max_compute_workgroup_size_x, "max_block_dim_x"},
            {hipDeviceAttributeMaxBlockDimY, &lim.max_compute_workgroup_size_y, "max_block_dim_y"},
            {hipDeviceAttributeMaxBlockDimZ, &lim.max_compute_workgroup_size_z, "max_block_dim_z"},
            {hipDeviceAttributeMaxThreadsPerBlock, &lim.max_compute_invocations_per_workgroup,
             "max_threads_per_block"},
            {hipDeviceAttributeMaxSharedMemoryPerBlock, &lim.max_compute_workgroup_storage_size,
             "max_shared_memory_per_block"},
        };
        for (auto &e : q) {
            int v = 0;
            err = hipDeviceGetAttribute(&v, e.attr, ordinal);
            if (err != hipSuccess) return bail(hip_fail(HX_ERR_DEVICE_UNAVAILABLE, err, e.name));
            if (v < 0)
                return bail(fail(HX_ERR_DEVICE_UNAVAILABLE, "ROCm attribute %s returned negative value %d", e.name, v));
            *e.dst = (uint32_t)v;
        }
        lim.max_immediate_size = 0;
    }

    // This device's no-allocation scratch, looked up with the device current.
    {
        hx_status s = lookup_noalloc_scratch(&dev->noalloc_scratch);
        if (s != HX_OK) return bail(s);
    }

    // Default-priority stream (never a priority stream).
    err = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking);
    if (err != hipSuccess)
        return bail(hip_fail(HX_ERR_DEVICE_UNAVAILABLE, err, "hipStreamCreate"));

    // Sanity round trip (device.rs:141-163).
    void *probe = nullptr;
    err = hipMalloc(&probe, sizeof(uint32_t));
    if (err != hipSuccess)
        return bail(fail(HX_ERR_ADAPTER_UNAVAILABLE, "ROCm sanity allocation failed: %s",
                         hipGetErrorString(err)));
    uint32_t host = 42, back = 0;
    err = hipMemcpy(probe, &host, sizeof host, hipMemcpyHostToDevice);
    if (err == hipSuccess) err = hipMemcpy(&back, probe, sizeof back, hipMemcpyDeviceToHost);
    (void)hipFree(probe);
    if (err != hipSuccess)
        return bail(fail(HX_ERR_ADAPTER_UNAVAILABLE, "ROCm sanity transfer failed: %s",
                         hipGetErrorString(err)));
    if (back != host)
        return bail(fail(HX_ERR_ADAPTER_UNAVAILABLE, "ROCm sanity transfer mismatch: [%u] != [%u]",
                         back, host));
    *out = dev;
    return ok();
}

hx_status hx_stream_release(hx_device *dev, hx_stream stream) {
    if (!stream) return ok(); // the device's own stream keeps its buffers until hx_device_close
    HX_TRY(bind_device(dev));
    std::unique_ptr<StreamWorkspace> sw;
    {
        std::lock_guard<std::mutex> guard(dev->streams_mu);
        auto it = dev->immediate.find((hipStream_t)stream);
        if (it == dev->immediate.end()) return ok();
        sw = std::move(it->second);
        dev->immediate.erase(it);
    }
    std::lock_guard<std::mutex> guard(sw->mu);
    // Launches queued on the stream may still read the buffers.
    const hipError_t err = hipStreamSynchronize((hipStream_t)stream);
    if (sw->ws) (void)hipFree(sw->ws);
    if (sw->scratch) (void)hipFree(sw->scratch);
    if (err != hipSuccess) return hip_fail(HX_ERR_DISPATCH_FAILED, err, "stream synchronize before release");
    return ok();
}

hx_status hx_device_close(hx_device *dev) {
    if (!dev) return ok();
    (void)hipSetDevice(dev->ordinal);
    (void)hipDeviceSynchronize();
    for (int i = 0; i < 2; ++i) {
        if (dev->pinned[i]) (void)hipHostFree(dev->pinned[i]);
        if (dev->pinned_ev[i]) (void)hipEventDestroy(dev->pinned_ev[i]);
    }
    for (auto &entry : dev->immediate) {
        if (entry.second->ws) (void)hipFree(entry.second->ws);
        if (entry.second->scratch) (void)hipFree(entry.second->scratch);
    }
    release_kernels(dev);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
    return ok();
}

hx_status hx_device_get_info(const hx_device *dev, hx_device_info *out) {
    if (!dev || !out) return fail(HX_ERR_INVALID_CONFIGURATION, "null argument");
    *out = dev->info;
    return ok();
}

hx_status hx_device_get_limits(const hx_device *dev, hx_device_limits *out) {
    if (!dev || !out) return fail(HX_ERR_INVALID_CONFIGURATION, "null argument");
    *out = dev->limits;
    return ok();
}

int32_t hx_device_supports_feature(const hx_device *dev, hx_device_feature feature) {
    (void)dev;
    (void)feature;
    return 0;
}

hx_status hx_require_limits(const hx_device_limits *actual, const hx_device_limits *required) {
    if (!actual || !required) return fail(HX_ERR_INVALID_CONFIGURATION, "null argument");
    const struct {
        const char *name;
        uint64_t available, needed;
    } rows[] = {
        {"max_buffer_size", actual->max_buffer_size, required->max_buffer_size},
        {"max_compute_workgroup_size_x", actual->max_compute_workgroup_size_x, required->max_compute_workgroup_size_x},
        {"max_compute_workgroup_size_y", actual->max_compute_workgroup_size_y, required->max_compute_workgroup_size_y},
        {"max_compute_workgroup_size_z", actual->max_compute_workgroup_size_z, required->max_compute_workgroup_size_z},
        {"max_compute_invocations_per_workgroup", actual->max_compute_invocations_per_workgroup,
         required->max_compute_invocations_per_workgroup},
        {"max_compute_workgroup_storage_size", actual->max_compute_workgroup_storage_size,
         required->max_compute_workgroup_storage_size},
        {"max_immediate_size", actual->max_immediate_size, required->max_immediate_size},
    };
    for (const auto &r : rows)
        if (r.available < r.needed)
            return fail(HX_ERR_DEVICE_UNAVAILABLE, "ROCm device limit %s %llu is below required %llu", r.name,
                        (unsigned long long)r.available, (unsigned long long)r.needed);
    return ok();
}

hx_status hx_device_stream(const hx_device *dev, hx_stream *out) {
    if (!dev || !out) return fail(HX_ERR_INVALID_CONFIGURATION, "null argument");
    *out = (hx_stream)dev->stream;
    return ok();
}

hx_status hx_synchronize(hx_device *dev) {
    HX_TRY(bind_device(dev));
    HX_HIP(hipDeviceSynchronize(), HX_ERR_DISPATCH_FAILED, "hipDeviceSynchronize");
    return ok();
}

hx_status hx_alloc(hx_device *dev, uint64_t bytes, uint32_t zeroed, void **out) {
    if (!out) return fail(HX_ERR_INVALID_CONFIGURATION, "null allocation out-pointer");
    *out = nullptr;
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok(); // memory.rs:75-88: no HIP call
    void *p = nullptr;
    hipError_t err = hipMalloc(&p, bytes);
    if (err != hipSuccess)
        return fail(HX_ERR_ALLOCATION_FAILED, "hipMalloc of %llu bytes failed: %s",
                    (unsigned long long)bytes, hipGetErrorString(err));
    if (zeroed) {
        err = hipMemsetAsync(p, 0, bytes, dev->stream);
        if (err == hipSuccess) err = hipStreamSynchronize(dev->stream);
        if (err != hipSuccess) {
            (void)hipFree(p);
            return hip_fail(HX_ERR_ALLOCATION_FAILED, err, "zero-fill");
        }
    }
    *out = p;
    return ok();
}

hx_status hx_free(hx_device *dev, void *ptr) {
    if (!ptr) return ok();
    HX_TRY(bind_device(dev));
    HX_HIP(hipFree(ptr), HX_ERR_ALLOCATION_FAILED, "hipFree");
    return ok();
}

} // extern "C"

namespace {

// Both staging buffers and their events, or none: a failed set-up releases
// what it made, and `pinned_bytes` (the chunk size the copy loops step by)
// is set only once everything exists.
hx_status ensure_staging(hx_device *dev) {
    if (dev->pinned_bytes != 0) return HX_OK;
    hipError_t err = hipSuccess;
    const char *what = nullptr;
    for (int i = 0; i < 2 && err == hipSuccess; ++i) {
        if (!dev->pinned[i]) {
            err = hipHostMalloc(&dev->pinned[i], kStagingChunk, hipHostMallocDefault);
            what = "pinned staging hipHostMalloc";
            if (err != hipSuccess) dev->pinned[i] = nullptr;
        }
        if (err == hipSuccess && !dev->pinned_ev[i]) {
            err = hipEventCreateWithFlags(&dev->pinned_ev[i], hipEventDisableTiming);
            what = "staging event";
            if (err != hipSuccess) dev->pinned_ev[i] = nullptr;
        }
    }
    if (err != hipSuccess) {
        for (int i = 0; i < 2; ++i) {
            if (dev->pinned[i]) (void)hipHostFree(dev->pinned[i]);
            if (dev->pinned_ev[i]) (void)hipEventDestroy(dev->pinned_ev[i]);
            dev->pinned[i] = nullptr;
            dev->pinned_ev[i] = nullptr;
        }
        return hip_fail(HX_ERR_TRANSFER_FAILED, err, what);
    }
    dev->pinned_bytes = kStagingChunk;
    return HX_OK;
}

// Host -> device through two pinned buffers: the memcpy into one buffer
// overlaps the DMA out of the other.
hx_status staged_h2d(hx_device *dev, void *dst, const void *src, uint64_t bytes) {
    if (bytes <= kSmallTransfer) {
        HX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, dev->stream),
               HX_ERR_TRANSFER_FAILED, "hipMemcpyAsync H2D");
        HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "H2D synchronize");
        return HX_OK;
    }
    std::lock_guard<std::mutex> lock(dev->staging_mu);
    HX_TRY(ensure_staging(dev));
    // Order after earlier work on the device stream.
    HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "H2D synchronize");
    uint64_t done = 0;
    int slot = 0;
    bool used[2] = {false, false};
    while (done < bytes) {
        uint64_t chunk = bytes - done < dev->pinned_bytes ? bytes - done : dev->pinned_bytes;
        if (used[slot])
            HX_HIP(hipEventSynchronize(dev->pinned_ev[slot]), HX_ERR_TRANSFER_FAILED,
                   "staging wait");
        std::memcpy(dev->pinned[slot], (const char *)src + done, chunk);
        HX_HIP(hipMemcpyAsync((char *)dst + done, dev->pinned[slot], chunk,
                              hipMemcpyHostToDevice, dev->stream),
               HX_ERR_TRANSFER_FAILED, "hipMemcpyAsync H2D");
        HX_HIP(hipEventRecord(dev->pinned_ev[slot], dev->stream), HX_ERR_TRANSFER_FAILED,
               "staging record");
        used[slot] = true;
        done += chunk;
        slot ^= 1;
    }
    HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "H2D synchronize");
    return HX_OK;
}

hx_status staged_d2h(hx_device *dev, void *dst, const void *src, uint64_t bytes) {
    if (bytes <= kSmallTransfer) {
        HX_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, dev->stream),
               HX_ERR_TRANSFER_FAILED, "hipMemcpyAsync D2H");
        HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "D2H synchronize");
        return HX_OK;
    }
    std::lock_guard<std::mutex> lock(dev->staging_mu);
    HX_TRY(ensure_staging(dev));
    uint64_t nchunks = (bytes + dev->pinned_bytes - 1) / dev->pinned_bytes;
    auto chunk_len = [&](uint64_t c) {
        uint64_t off = c * dev->pinned_bytes;
        return bytes - off < dev->pinned_bytes ? bytes - off : dev->pinned_bytes;
    };
    // Keep one DMA in flight while the previous chunk is copied out.
    HX_HIP(hipMemcpyAsync(dev->pinned[0], src, chunk_len(0), hipMemcpyDeviceToHost,
                          dev->stream),
           HX_ERR_TRANSFER_FAILED, "hipMemcpyAsync D2H");
    HX_HIP(hipEventRecord(dev->pinned_ev[0], dev->stream), HX_ERR_TRANSFER_FAILED,
           "staging record");
    for (uint64_t c = 0; c < nchunks; ++c) {
        int slot = (int)(c & 1);
        if (c + 1 < nchunks) {
            int next = slot ^ 1;
            HX_HIP(hipMemcpyAsync(dev->pinned[next],
                                  (const char *)src + (c + 1) * dev->pinned_bytes,
                                  chunk_len(c + 1), hipMemcpyDeviceToHost, dev->stream),
                   HX_ERR_TRANSFER_FAILED, "hipMemcpyAsync D2H");
            HX_HIP(hipEventRecord(dev->pinned_ev[next], dev->stream), HX_ERR_TRANSFER_FAILED,
                   "staging record");
        }
        HX_HIP(hipEventSynchronize(dev->pinned_ev[slot]), HX_ERR_TRANSFER_FAILED,
               "staging wait");
        std::memcpy((char *)dst + c * dev->pinned_bytes, dev->pinned[slot], chunk_len(c));
    }
    HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "D2H synchronize");
    return HX_OK;
}

hx_status check_elem(uint32_t elem_size) {
    if (elem_size == 0)
        return fail(HX_ERR_INVALID_CONFIGURATION, "element size must be non-zero");
    return HX_OK;
}

// Byte count of `len` elements, rejecting lengths whose byte count does not
// fit 64 bits (the transfer would otherwise wrap to a short copy).
hx_status byte_count(uint64_t len, uint32_t elem_size, uint64_t *bytes) {
    if (len > UINT64_MAX / elem_size)
        return fail(HX_ERR_INVALID_CONFIGURATION, "%llu elements of %u bytes exceed the address range",
                    (unsigned long long)len, elem_size);
    *bytes = len * elem_size;
    return HX_OK;
}

} // namespace

extern "C" {

hx_status hx_upload(hx_device *dev, void *dst, uint64_t dst_len, const void *src,
                    uint64_t src_len, uint32_t elem_size) {
    HX_TRY(check_elem(elem_size));
    if (dst_len != src_len) return length_mismatch(src_len, dst_len);
    uint64_t bytes = 0;
    HX_TRY(byte_count(src_len, elem_size, &bytes));
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(HX_ERR_TRANSFER_FAILED, "null transfer pointer");
    HX_TRY(staged_h2d(dev, dst, src, bytes));
    return ok();
}

hx_status hx_write_sub(hx_device *dev, void *dst, uint64_t dst_len, uint64_t offset,
                       const void *src, uint64_t src_len, uint32_t elem_size) {
    HX_TRY(check_elem(elem_size));
    // host lib.rs:157-169: overflow or end beyond the buffer -> LengthMismatch
    uint64_t end = offset + src_len;
    if (end < offset || end > dst_len) return length_mismatch(src_len, dst_len);
    uint64_t bytes = 0, skip = 0;
    HX_TRY(byte_count(end, elem_size, &skip)); // also bounds offset * elem_size
    HX_TRY(byte_count(src_len, elem_size, &bytes));
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(HX_ERR_TRANSFER_FAILED, "null transfer pointer");
    HX_TRY(staged_h2d(dev, (char *)dst + offset * elem_size, src, bytes));
    return ok();
}

hx_status hx_download(hx_device *dev, const void *src, uint64_t src_len, void *dst,
                      uint64_t dst_len, uint32_t elem_size) {
    HX_TRY(check_elem(elem_size));
    if (dst_len != src_len) return length_mismatch(dst_len, src_len);
    uint64_t bytes = 0;
    HX_TRY(byte_count(src_len, elem_size, &bytes));
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok();
    if (!dst || !src) return fail(HX_ERR_TRANSFER_FAILED, "null transfer pointer");
    HX_TRY(staged_d2h(dev, dst, src, bytes));
    return ok();
}

hx_status hx_copy(hx_device *dev, const void *src, uint64_t src_len, void *dst,
                  uint64_t dst_len, uint32_t elem_size) {
    HX_TRY(check_elem(elem_size));
    if (src == dst && src_len == dst_len) return ok(); // host lib.rs:175-177
    if (dst_len != src_len) return length_mismatch(dst_len, src_len);
    uint64_t bytes = 0;
    HX_TRY(byte_count(src_len, elem_size, &bytes));
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok();
    HX_TRY(launch_copy(src, dst, bytes, dev->stream));
    HX_HIP(hipStreamSynchronize(dev->stream), HX_ERR_TRANSFER_FAILED, "D2D synchronize");
    return ok();
}

hx_status hx_debug_copy_scan_shape(hx_device *dev, const void *src, void *dst, uint64_t bytes, hx_stream stream) {
    HX_TRY(bind_device(dev));
    if (bytes > 0 && (!src || !dst)) return fail(HX_ERR_DISPATCH_FAILED, "null copy pointer");
    HX_TRY(launch_copy_scan_shape(src, dst, bytes, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_copy_async(hx_device *dev, const void *src, uint64_t src_len, void *dst, uint64_t dst_len,
                        uint32_t elem_size, hx_stream stream) {
    HX_TRY(check_elem(elem_size));
    if (src == dst && src_len == dst_len) return ok();
    if (dst_len != src_len) return length_mismatch(dst_len, src_len);
    uint64_t bytes = 0;
    HX_TRY(byte_count(src_len, elem_size, &bytes));
    HX_TRY(bind_device(dev));
    if (bytes == 0) return ok();
    HX_TRY(launch_copy(src, dst, bytes, pick_stream(dev, stream)));
    return ok();
}

hx_status hx_event_create(hx_device *dev, hx_event *out) {
    if (!out) return fail(HX_ERR_INVALID_CONFIGURATION, "null event out-pointer");
    HX_TRY(bind_device(dev));
    hipEvent_t ev = nullptr;
    HX_HIP(hipEventCreate(&ev), HX_ERR_DISPATCH_FAILED, "hipEventCreate");
    *out = (hx_event)ev;
    return ok();
}

hx_status hx_event_destroy(hx_event ev) {
    if (ev) HX_HIP(hipEventDestroy((hipEvent_t)ev), HX_ERR_DISPATCH_FAILED, "hipEventDestroy");
    return ok();
}

hx_status hx_event_record(hx_device *dev, hx_event ev, hx_stream stream) {
    HX_TRY(bind_device(dev));
    HX_HIP(hipEventRecord((hipEvent_t)ev, pick_stream(dev, stream)), HX_ERR_DISPATCH_FAILED,
           "hipEventRecord");
    return ok();
}

hx_status hx_event_synchronize(hx_event ev) {
    HX_HIP(hipEventSynchronize((hipEvent_t)ev), HX_ERR_DISPATCH_FAILED, "hipEventSynchronize");
    return ok();
}

hx_status hx_event_elapsed_ms(hx_event start, hx_event stop, float *ms) {
    if (!ms) return fail(HX_ERR_INVALID_CONFIGURATION, "null out-pointer");
    HX_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop), HX_ERR_DISPATCH_FAILED,
           "hipEventElapsedTime");
    return ok();
}

} // extern "C"

namespace {

// One dispatch of `plan` on `s` (plan->mu held).  Under stream capture a
// tagged plan records a clear of its status words and runs with the reserved
// captured tag, so every replay of the graph starts from zeroed words.
hx_status dispatch_locked(hx_plan *plan, hipStream_t s) {
    bool capturing = false;
    HX_TRY(stream_capturing(s, &capturing));
    if (!capturing || !plan->tagged()) return plan->dispatch(s);
    if (plan->ws_bytes > kLookbackOffset)
        HX_TRY(launch_clear_words((char *)plan->ws + kLookbackOffset, (plan->ws_bytes - kLookbackOffset) / 8, s));
    plan->lookback.captured = true;
    const hx_status st = plan->dispatch(s);
    plan->lookback.captured = false;
    return st;
}

} // namespace

extern "C" {

hx_status hx_plan_dispatch(hx_plan *plan, hx_stream stream) {
    if (!plan) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan");
    HX_TRY(bind_device(plan->dev));
    std::lock_guard<std::mutex> guard(plan->mu);
    HX_TRY(dispatch_locked(plan, pick_stream(plan->dev, stream)));
    return ok();
}

hx_status hx_plan_dispatch_batch(hx_plan *const *plans, uint64_t count, hx_stream stream) {
    if (count && !plans) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan array");
    for (uint64_t i = 0; i < count; ++i)
        if (!plans[i]) return fail(HX_ERR_INVALID_CONFIGURATION, "null plan at batch index %llu", (unsigned long long)i);
    for (uint64_t i = 0; i < count; ++i) {
        HX_TRY(bind_device(plans[i]->dev));
        std::lock_guard<std::mutex> guard(plans[i]->mu);
        HX_TRY(dispatch_locked(plans[i], pick_stream(plans[i]->dev, stream)));
    }
    return ok();
}

hx_status hx_plan_destroy(hx_plan *plan) {
    delete plan;
    return ok();
}

hx_status hx_plan_workspace_bytes(const hx_plan *plan, uint64_t *bytes) {
    if (!plan || !bytes) return fail(HX_ERR_INVALID_CONFIGURATION, "null argument");
    *bytes = plan->ws_bytes;
    return ok();
}

} // extern "C"
