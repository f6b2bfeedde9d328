// hx_scan_noalloc: the scans of hx_scan with every byte of their workspace in
// a fixed device array, for callers that cannot allocate (code under HIP
// graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope __device__ array, so each GPU holds its own copy
// for the life of the process.  Host code never passes the array's name to
// a kernel: the name is a host-side stand-in, not a device address.  Each
// device's address is looked up once, with that device current, when the
// device is opened (hx_device_open calls lookup_noalloc_scratch) and kept in
// the device handle; kernels and the clear kernel receive that pointer.
//
// The layout is that of a scan workspace: 256-byte header, then look-back
// status words (or, for chunked column scans, chunk totals).
// The array keeps the last call's contents, so every look-back call first
// clears the status words it will use with a fill kernel (no
// hipMemsetAsync, which a captured graph may replay wrongly) and then runs
// with a fresh tag.  Calls that overlap on one GPU share the array and race;
// calls queued on one stream run in order.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

constexpr uint64_t kNoAllocBytes = 8ull << 20;

static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

uint64_t noalloc_scratch_bytes() { return kNoAllocBytes; }

hx_status lookup_noalloc_scratch(void **ptr) {
    *ptr = nullptr;
    void *p = nullptr;
    HX_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), HX_ERR_DEVICE_UNAVAILABLE,
           "hipGetSymbolAddress of the no-allocation scratch");
    if (p == nullptr)
        return fail(HX_ERR_DEVICE_UNAVAILABLE, "the no-allocation scratch has no device address");
    *ptr = p;
    return HX_OK;
}

hx_status launch_scan_noalloc(const ScanArgs &a, void *scratch_ptr, hipStream_t stream) {
    if (a.lines == 0 || a.len == 0) return HX_OK;
    const uint64_t bytes = scan_workspace_bytes(a);
    if (bytes > kNoAllocBytes)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "scan needs %llu bytes of workspace; the no-allocation scratch holds %llu "
                    "(use hx_scan or hx_prepare_scan)",
                    (unsigned long long)bytes, (unsigned long long)kNoAllocBytes);
    if (scratch_ptr == nullptr)
        return fail(HX_ERR_DEVICE_UNAVAILABLE, "the no-allocation scratch was not set up for this device");
    if (scan_uses_lookback(a) && bytes > kLookbackOffset)
        HX_TRY(launch_clear_words((char *)scratch_ptr + kLookbackOffset, (bytes - kLookbackOffset) / 8, stream));
    // The status words were just cleared, so the first tag is fresh.
    LookbackState fresh;
    return launch_scan(a, scratch_ptr, bytes, fresh, stream);
}

} // namespace hx
