// The reference's vendor seam beneath its generic accelerator layer
// (DeviceApi, crates/hephaestus-core/src/domain/accelerator/
// device_api.rs:69-133; ROCm impl crates/hephaestus-rocm/src/application/
// device_api.rs:49-103 over pipeline.rs:175-349): kernel source compiled at
// run time, cached per device under the caller's key, and launched with a
// parameter block followed by an ordered operand list.  It is what lets a
// consumer run its own kernels on this backend next to the library's.
//
//   hx_kernel_compile_cached  hipRTC for this device's architecture, with
//                             the flags the library's own kernels are built
//                             with; the code object is loaded as a module
//                             and `entry` looked up.  A cache hit never asks
//                             for the source; failed compilations are not
//                             cached.
//   hx_kernel_launch          hipModuleLaunchKernel: argument 0 is the
//                             parameter block (by value), then one device
//                             address per operand, on the caller's stream.
//   hx_buffers_alias          whether two device ranges are one base or
//                             overlap.
//
// Modules live until hx_device_close (release_kernels).
#include "hx_internal.hpp"

#include <hip/hiprtc.h>

#include <cstring>
#include <string>
#include <vector>

namespace hx {
namespace {

// The library's device compile flags (build.py FLAGS) that apply to run-time
// compiled code: optimisation, and no packed FP32 instructions.
const char *const kRtcOptions[] = {"-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};

constexpr uint64_t kMaxKernargBytes = 4096;

hx_status rtc_fail(hiprtcResult r, const char *what, const std::string &log = std::string()) {
    if (log.empty()) return fail(HX_ERR_DISPATCH_FAILED, "%s: %s", what, hiprtcGetErrorString(r));
    return fail(HX_ERR_DISPATCH_FAILED, "%s: %s\n%s", what, hiprtcGetErrorString(r), log.c_str());
}

struct Program {
    hiprtcProgram p = nullptr;
    ~Program() {
        if (p) (void)hiprtcDestroyProgram(&p);
    }
};

// Source text -> code object for the current device (pipeline.rs:175-257).
hx_status compile_to_code(const hx_device *dev, const std::string &source, std::vector<char> &code) {
    Program prog;
    hiprtcResult r = hiprtcCreateProgram(&prog.p, source.c_str(), "hx_kernel_source", 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return rtc_fail(r, "hiprtcCreateProgram");
    std::vector<const char *> opts(std::begin(kRtcOptions), std::end(kRtcOptions));
    const std::string arch = std::string("--offload-arch=") + dev->info.arch;
    opts.push_back(arch.c_str());
    r = hiprtcCompileProgram(prog.p, (int)opts.size(), opts.data());
    if (r != HIPRTC_SUCCESS) {
        std::string log;
        size_t n = 0;
        if (hiprtcGetProgramLogSize(prog.p, &n) == HIPRTC_SUCCESS && n > 1) {
            log.resize(n);
            if (hiprtcGetProgramLog(prog.p, &log[0]) != HIPRTC_SUCCESS) log.clear();
            while (!log.empty() && log.back() == '\0') log.pop_back();
        }
        return rtc_fail(r, "hiprtcCompileProgram", log);
    }
    size_t size = 0;
    r = hiprtcGetCodeSize(prog.p, &size);
    if (r != HIPRTC_SUCCESS) return rtc_fail(r, "hiprtcGetCodeSize");
    code.resize(size);
    r = hiprtcGetCode(prog.p, code.data());
    if (r != HIPRTC_SUCCESS) return rtc_fail(r, "hiprtcGetCode");
    return HX_OK;
}

} // namespace

void release_kernels(hx_device *dev) {
    std::lock_guard<std::mutex> lock(dev->kernels_mu);
    for (auto &entry : dev->kernels)
        if (entry.second && entry.second->module) (void)hipModuleUnload(entry.second->module);
    dev->kernels.clear();
}

} // namespace hx

using namespace hx;

extern "C" {

hx_status hx_kernel_compile_cached(hx_device *dev, const void *key, uint64_t key_len, const char *entry,
                                   hx_kernel_source_fn source, void *ctx, hx_kernel **kernel) {
    if (kernel == nullptr) return fail(HX_ERR_INVALID_CONFIGURATION, "null kernel out-pointer");
    *kernel = nullptr;
    if (dev == nullptr) return fail(HX_ERR_INVALID_CONFIGURATION, "null device handle");
    if (key == nullptr && key_len != 0) return fail(HX_ERR_INVALID_CONFIGURATION, "null cache key");
    if (entry == nullptr) return fail(HX_ERR_DISPATCH_FAILED, "null kernel entry name");
    if (source == nullptr) return fail(HX_ERR_INVALID_CONFIGURATION, "null kernel source callback");
    const std::string k((const char *)key, (size_t)key_len);
    {
        std::lock_guard<std::mutex> lock(dev->kernels_mu);
        auto it = dev->kernels.find(k);
        if (it != dev->kernels.end()) {
            *kernel = it->second.get();
            return ok();
        }
    }
    HX_TRY(bind_device(dev));
    const char *text = source(ctx);
    if (text == nullptr) return fail(HX_ERR_DISPATCH_FAILED, "the kernel source callback returned no source");
    const std::string src(text);
    std::vector<char> code;
    HX_TRY(compile_to_code(dev, src, code));
    auto compiled = std::make_unique<hx_kernel>();
    compiled->owner = dev;
    HX_HIP(hipModuleLoadData(&compiled->module, code.data()), HX_ERR_DISPATCH_FAILED, "hipModuleLoadData");
    hipError_t err = hipModuleGetFunction(&compiled->function, compiled->module, entry);
    if (err != hipSuccess) {
        (void)hipModuleUnload(compiled->module);
        return hip_fail(HX_ERR_DISPATCH_FAILED, err, "hipModuleGetFunction");
    }
    std::lock_guard<std::mutex> lock(dev->kernels_mu);
    auto it = dev->kernels.find(k);
    if (it != dev->kernels.end()) {
        // Another thread compiled the same key meanwhile: keep the first.
        (void)hipModuleUnload(compiled->module);
        *kernel = it->second.get();
        return ok();
    }
    *kernel = compiled.get();
    dev->kernels.emplace(k, std::move(compiled));
    return ok();
}

hx_status hx_kernel_launch(hx_device *dev, const hx_kernel *kernel, uint32_t groups, uint32_t width,
                           uint32_t shared_bytes, const void *params, uint64_t params_bytes,
                           void *const *operands, uint64_t operand_count, hx_stream stream) {
    if (kernel == nullptr || kernel->function == nullptr)
        return fail(HX_ERR_INVALID_CONFIGURATION, "null kernel handle");
    if (width == 0) return fail(HX_ERR_INVALID_CONFIGURATION, "block width must be non-zero");
    if (kernel->owner != dev)
        return fail(HX_ERR_INVALID_CONFIGURATION, "kernel was compiled for another device");
    if (params == nullptr && params_bytes != 0) return fail(HX_ERR_INVALID_CONFIGURATION, "null parameter block");
    if (params_bytes > kMaxKernargBytes)
        return fail(HX_ERR_INVALID_CONFIGURATION, "parameter block of %llu bytes exceeds the %llu-byte argument segment",
                    (unsigned long long)params_bytes, (unsigned long long)kMaxKernargBytes);
    if (operands == nullptr && operand_count != 0) return fail(HX_ERR_INVALID_CONFIGURATION, "null operand list");
    HX_TRY(bind_device(dev));
    // HIP reads each argument through a pointer to the slot holding it: the
    // parameter block first (copied, so the caller's block may go away), then
    // each operand address (device_api.rs ROCm:75-102).
    // The block is padded with zeros to the largest kernel argument segment,
    // so a kernel whose first parameter is larger than params_bytes reads
    // zeros, never past the copy.
    std::vector<unsigned char> block(params_bytes + kMaxKernargBytes, 0);
    if (params_bytes != 0) std::memcpy(block.data(), params, params_bytes);
    std::vector<void *> slots(operands, operands + operand_count);
    std::vector<void *> args;
    args.reserve(slots.size() + 1);
    if (params_bytes != 0) args.push_back(block.data());
    for (auto &s : slots) args.push_back(&s);
    HX_HIP(hipModuleLaunchKernel(kernel->function, groups, 1, 1, width, 1, 1, shared_bytes, pick_stream(dev, stream),
                                 args.empty() ? nullptr : args.data(), nullptr),
           HX_ERR_DISPATCH_FAILED, "hipModuleLaunchKernel");
    return ok();
}

int32_t hx_buffers_alias(const void *a, uint64_t a_bytes, const void *b, uint64_t b_bytes) {
    if (a == nullptr || b == nullptr) return 0;
    if (a == b) return 1; // the reference's rule: one non-null base (buffer.rs:47-49)
    const uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    return (a0 < b0 + b_bytes && b0 < a0 + a_bytes) ? 1 : 0;
}

} // extern "C"
