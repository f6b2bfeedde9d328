// Host-side internals shared by the runtime, the planners and the kernel
// launchers.  Nothing here crosses the C ABI.
#pragma once

#include "../../include/hx.h"

#include <hip/hip_runtime.h>

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>

namespace hx {
// Host-side bookkeeping of one look-back workspace: every launch tags its
// status words with a fresh 14-bit tag, so words left by earlier launches
// (of any look-back kernel) read as "not yet published".  No device-side
// end-of-launch bookkeeping is needed, and therefore no device-scope
// release/acquire (which on multi-XCD CDNA writes back and invalidates the
// L2) on the hot path.
//
// A dispatch recorded into a HIP graph (stream capture) is replayed with the
// tag it was recorded with, so captured dispatches use the one reserved tag
// kCapturedTag, which eager launches never draw, and record a clear of the
// status words in front of the kernel: every replay starts from zeroed words,
// and eager launches never read a replay's words as current.
// Tags stay below 2^14 because the f32 scan slots carry (tag << 2) | flag
// in 16 bits of each dword; eager tags cycle through [1, kCapturedTag) and
// the wrapping launch clears the status words (one fill kernel per 16382
// launches).
constexpr uint32_t kCapturedTag = 0x3FFFu;
struct LookbackState {
    uint64_t launches = 0;  // eager launches so far on this workspace
    bool captured = false;  // the launch being queued is under stream capture
};

// The buffers the immediate (un-prepared) entry points use on ONE stream:
//   ws       header + tagged status words (look-back statuses and the
//            partial slots of the one-launch grid folds);
//   scratch  partials staged outside any look-back protocol (split axis
//            reductions, chunked column scans, segmented tile maps and
//            worklists), kept apart from `ws` so those writes never land on
//            status words.
// Each stream has its own, so launches queued on different streams never
// share a buffer; `mu` is held from the workspace lookup until the call's
// launches are queued (see Immediate).
struct StreamWorkspace {
    std::mutex mu;
    void *ws = nullptr;
    uint64_t ws_bytes = 0;
    LookbackState lookback;
    void *scratch = nullptr;
    uint64_t scratch_bytes = 0;
};
} // namespace hx

// The device handle behind hx_device* (RocmDevice analog:
// crates/hephaestus-rocm/src/infrastructure/device.rs:109-165).
// A run-time compiled kernel (hx_kernel_compile_cached): its module and
// entry point.
struct hx_kernel {
    hipModule_t module = nullptr;
    hipFunction_t function = nullptr;
    const hx_device *owner = nullptr; // the device whose cache holds it
};

struct hx_device {
    int32_t ordinal = -1;
    hipStream_t stream = nullptr;
    hx_device_info info{};
    hx_device_limits limits{};

    // Pinned double-buffered staging for host<->device transfers.
    std::mutex staging_mu;
    void *pinned[2] = {nullptr, nullptr};
    uint64_t pinned_bytes = 0;
    hipEvent_t pinned_ev[2] = {nullptr, nullptr};

    // Immediate-mode buffers, one set per stream handle the caller has used
    // (created on first use, freed by hx_stream_release or at
    // hx_device_close).  A stream handle is only reused by the runtime after
    // the destroyed stream's work has drained, so an entry never serves two
    // live streams at once.
    std::mutex streams_mu;
    std::unordered_map<hipStream_t, std::unique_ptr<hx::StreamWorkspace>> immediate;

    // This device's copy of the no-allocation scratch array (its device
    // address, looked up at hx_device_open with the device current), and the
    // lock held by hx_scan_noalloc from its clear kernel to its scan launch,
    // so calls from several host threads on one stream queue as whole
    // clear + scan pairs.
    void *noalloc_scratch = nullptr;
    std::mutex noalloc_mu;

    // Run-time compiled kernels (hx_kernel_compile_cached), by cache key;
    // their modules are unloaded at hx_device_close.
    std::mutex kernels_mu;
    std::unordered_map<std::string, std::unique_ptr<hx_kernel>> kernels;
};

namespace hx {

// ------------------------------------------------------------- errors

hx_status ok();
hx_status fail(hx_status status, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));
hx_status length_mismatch(uint64_t host_len, uint64_t device_len);
// Map a HIP error to `status` with "<what>: <hip error string>".
hx_status hip_fail(hx_status status, hipError_t err, const char *what);

#define HX_TRY(expr)                                                         \
    do {                                                                     \
        hx_status hx_try_status_ = (expr);                                   \
        if (hx_try_status_ != HX_OK) return hx_try_status_;                  \
    } while (0)

#define HX_HIP(call, status, what)                                           \
    do {                                                                     \
        hipError_t hx_hip_err_ = (call);                                     \
        if (hx_hip_err_ != hipSuccess)                                       \
            return ::hx::hip_fail((status), hx_hip_err_, (what));            \
    } while (0)

hx_status bind_device(const hx_device *dev);
hipStream_t pick_stream(const hx_device *dev, hx_stream stream);
// Whether `stream` is being captured into a HIP graph (any capture status
// other than none, an invalidated capture included).
hx_status stream_capturing(hipStream_t stream, bool *capturing);
// Map the status of a kernel launch (hipGetLastError) to DispatchFailed.
hx_status check_launch(const char *kernel);
// Unload every run-time compiled kernel of the device (hx_device_close).
void release_kernels(hx_device *dev);

// ------------------------------------------------------------- layouts

std::string shape_string(const hx_layout &l);
// Row-major (C-contiguous) over every extent > 1: the view is the flat
// element range [offset, offset + size).
bool layout_is_c_contiguous(const hx_layout &l);
// Strides are a permutation of a dense row-major stride set (all positive):
// the view covers exactly [offset, offset + size) in some order.
bool layout_is_permuted_dense(const hx_layout &l);
// The view covers exactly [*first, *first + size) in some order: with the
// signs of its strides dropped (each reversed dimension read from its other
// end) it is a permuted dense view.  *first is the lowest element it reaches.
bool layout_covers_dense_range(const hx_layout &l, uint64_t *first);
// Every dimension runs backwards and, read from its other end, the view is
// row-major: element k of the view (row-major order) is element n - 1 - k of
// the dense range [*first, *first + size).
bool layout_is_reversed_c_contiguous(const hx_layout &l, uint64_t *first);
// A view as rows: `rows` rows of `cols` elements, element c of a row at
// c * cstride, the row index split over up to three outer dimensions
// (innermost first) from the view's offset.  Each dimension also carries a
// second stride (cstride2, ostride2): the logical (row-major) stride for
// one operand, or a second operand's stride, so a second linear form over
// the same digits follows the walk.  Built by dropping unit dimensions and
// merging dimension pairs adjacent under both strides (stride[d] ==
// stride[d+1] * shape[d+1]).
struct RowsView {
    uint64_t rows = 1, cols = 1;
    int64_t cstride = 1, cstride2 = 1;
    uint32_t orank = 0;
    uint64_t oshape[HX_MAX_RANK - 1] = {1, 1, 1};
    int64_t ostride[HX_MAX_RANK - 1] = {0, 0, 0};
    int64_t ostride2[HX_MAX_RANK - 1] = {0, 0, 0};
};
// Rows in logical (row-major) order; the second form is the logical index.
RowsView layout_rows(const hx_layout &l);
// Rows in memory order (dimensions by decreasing stride) of a view whose
// strides are all positive (layout_is_permuted_dense), the second form the
// logical index: for order-free folds that still need logical indices
// (argmax of a transposed view).
RowsView layout_rows_memory_order(const hx_layout &l);
// Rows of two same-shape views in logical order: the first form walks `a`,
// the second `b`'s strides.
RowsView layout_rows_pair(const hx_layout &a, const hx_layout &b);
// Two same-shape views with two or three extents above one: one view
// contiguous along one of them (the rows), the other along another (the
// columns), both other strides of those two positive, and any third
// extent a batch of such matrices (a transposed matrix paired with a
// row-major one).  Element (b, i, j) of the first at its offset + b *
// col_bs + i + j * col_ld, of the second at its offset + b * row_bs + i *
// row_ld + j.  a_is_col says which operand is contiguous along the rows.
struct PairTranspose {
    bool a_is_col = false;
    uint64_t rows = 0, cols = 0, batch = 1;
    int64_t col_ld = 0, row_ld = 0, col_bs = 0, row_bs = 0;
};
bool layout_pair_transposed(const hx_layout &a, const hx_layout &b, PairTranspose *t);
hx_status layout_basic_check(const hx_layout *l, const char *what);

// ----------------------------------------------------------- workspace
// Every workspace: a reserved 256-byte header, then the tagged status words
// (look-back statuses of the scans and the segmented sum, partial slots of
// the single-launch grid folds), all tagged from the workspace's one
// LookbackState.
constexpr uint64_t kWorkspaceHeader = 256;
constexpr uint64_t kLookbackOffset = kWorkspaceHeader;

hx_status alloc_workspace(hx_device *dev, uint64_t bytes, void **ws);

// Exclusive use of one stream's immediate-mode buffers for the rest of an
// entry point.  The lock is held across buffer growth, the draw of the
// look-back tag and the launches, so calls from several host threads on one
// stream draw distinct tags in launch order, and a buffer is never freed
// while a launch queued on its stream may still use it (growth first waits
// for that stream).  Calls on different streams use different buffers.
class Immediate {
public:
    hx_status open(hx_device *dev, hipStream_t stream);
    // Look-back workspace of at least `bytes` (zeroed when allocated; a new
    // buffer restarts the tag count).
    hx_status workspace(uint64_t bytes, void **ws);
    // Scratch of at least `bytes`; nullptr for 0 bytes.
    hx_status scratch(uint64_t bytes, void **scratch);
    uint64_t workspace_bytes() const { return sw_->ws_bytes; }
    LookbackState &lookback() { return sw_->lookback; }

private:
    hx_device *dev_ = nullptr;
    hipStream_t stream_ = nullptr;
    StreamWorkspace *sw_ = nullptr;
    std::unique_lock<std::mutex> lock_;
};

// Poll limits of the bounded waits (hx_debug_set_wait_limits): look-back
// polls before a waiter computes a missing predecessor, and gather polls per
// partial before the gathering block recomputes it (0: recompute all).
uint32_t lookback_poll_limit();
uint32_t gather_poll_limit();

// Tag for the next look-back launch on a workspace of `ws_bytes`: a fresh
// eager tag in [1, kCapturedTag), with the status area cleared (by a fill
// kernel) when that range wraps; kCapturedTag under capture (the caller has
// cleared the words in front of the launch).
hx_status next_lookback_launch(LookbackState &st, void *ws, uint64_t ws_bytes,
                               hipStream_t stream, uint32_t *tag);
void commit_lookback_launch(LookbackState &st);

// ------------------------------------------------------------- kernels

struct FullReduceArgs {
    hx_op op;
    hx_dtype dtype;
    const void *base;    // buffer base pointer
    hx_layout layout;    // logical view
    uint64_t n;          // logical size
    bool flat;           // view is the flat range [flat_offset, +n)
    bool memory_order;   // not flat: walk rows in memory order (argmax of a permuted dense view)
    bool reversed;       // flat: the view reads the range from its far end (view index n - 1 - e)
    uint64_t flat_offset;
    bool affine;
    float a, b;
    void *out_value;     // T[1] (may be null for argmax)
    uint32_t *out_index; // u32[1] (argmax only)
};
uint64_t full_reduce_workspace_bytes(uint64_t n);
// One launch; its partials are tagged status words of `ws` (tag drawn
// from `lb`).
hx_status launch_full_reduce(const FullReduceArgs &args, void *ws, uint64_t ws_bytes,
                             LookbackState &lb, hipStream_t stream);

struct RowsArgs {
    hx_dtype dtype;
    const void *base;
    uint64_t rows, cols, row_stride, offset;
    bool affine;
    float a, b;
    void *out_sum, *out_max;
    uint32_t *out_argmax;
};
// Split forms (few long rows, or column tiles over a tall matrix) fold
// per-chunk partials through `ws`; 0 bytes when no split is needed.
uint64_t rows_workspace_bytes(const RowsArgs &args);
hx_status launch_rows(const RowsArgs &args, void *ws, uint64_t ws_bytes, hipStream_t stream);

struct AxisArgs {
    hx_op op;
    hx_dtype dtype;
    const void *in;
    void *out;
    uint64_t outer;      // number of outputs
    uint64_t axis_len;   // reduced extent
    int64_t in_outer_stride, in_axis_stride;
    uint64_t in_offset;
    int64_t out_stride;
    uint64_t out_offset;
};
uint64_t axis_reduce_workspace_bytes(const AxisArgs &args);
hx_status launch_axis_reduce(const AxisArgs &args, void *ws, uint64_t ws_bytes, hipStream_t stream);

struct ScanArgs {
    hx_op op;
    hx_dtype dtype;
    bool exclusive, reverse;
    const void *in;
    void *out;
    uint64_t lines, len;
    int64_t in_line_stride, in_elem_stride;
    uint64_t in_offset;
    int64_t out_line_stride, out_elem_stride;
    uint64_t out_offset;
};
uint64_t scan_workspace_bytes(const ScanArgs &args);
// False for chunked column scans, whose workspace holds chunk totals
// instead of look-back status words (immediate calls take it from device
// scratch); true for every other scan.
bool scan_uses_lookback(const ScanArgs &args);
hx_status launch_scan(const ScanArgs &args, void *ws, uint64_t ws_bytes,
                      LookbackState &st, hipStream_t stream);

// The no-allocation scan (noalloc.hip): the device address of the current
// device's scratch array, its size, and a scan whose whole workspace is that
// array (rejected when the scan needs more).
hx_status lookup_noalloc_scratch(void **ptr);
uint64_t noalloc_scratch_bytes();
hx_status launch_scan_noalloc(const ScanArgs &args, void *scratch, hipStream_t stream);

struct SegmentedArgs {
    hx_op op;
    hx_dtype dtype;
    const void *values;
    uint64_t n;
    const uint32_t *offsets;
    uint64_t num_segments; // S (num_offsets - 1)
    void *out;
};
// Immediate calls take the look-back status words from the shared look-back
// workspace and everything else (tile maps, worklists) from the separate
// scratch buffer, so no other data ever lands where a later launch reads
// status words.  A prepared plan holds both in one workspace of
// segmented_workspace_bytes and passes aux = nullptr.
uint64_t segmented_lookback_bytes(const SegmentedArgs &args);
uint64_t segmented_aux_bytes(const SegmentedArgs &args);
uint64_t segmented_workspace_bytes(const SegmentedArgs &args);
hx_status launch_segmented(const SegmentedArgs &args, void *ws, uint64_t ws_bytes, void *aux,
                           uint64_t aux_bytes, LookbackState &st, hipStream_t stream);
hx_status validate_offsets_on_device(hx_device *dev, const uint32_t *offsets,
                                     uint64_t num_offsets, uint64_t n);

struct MapReduceArgs {
    hx_map_reduction map;
    hx_dtype dtype;
    const void *a, *b;
    hx_layout a_layout, b_layout;
    uint64_t n;
    bool flat; // both operands dense row-major with agreeing 16-byte phase
    void *out;
};
uint64_t map_reduce_workspace_bytes(uint64_t n);
// One launch; its partials are tagged status words of `ws` (tag drawn
// from `lb`).
hx_status launch_map_reduce(const MapReduceArgs &args, void *ws, uint64_t ws_bytes, LookbackState &lb,
                            hipStream_t stream);

// Elementwise f32 vector forms: out[i] = op(t[i], s[i], factor).
hx_status launch_vector_op(hx_vector_op op, const float *t, const float *s, float *out, uint64_t n,
                           float factor, hipStream_t stream);

// Stream-ordered device-to-device copy of `bytes` bytes (a streaming kernel).
hx_status launch_copy(const void *src, void *dst, uint64_t bytes, hipStream_t stream);
// The copy in the integer scan's tile shape and order (a bench yardstick):
// whole 128 KiB tiles, block b -> tile b.
hx_status launch_copy_scan_shape(const void *src, void *dst, uint64_t bytes, hipStream_t stream);
// Zero `count` 64-bit words with a fill kernel (safe under graph capture).
hx_status launch_clear_words(void *words, uint64_t count, hipStream_t stream);

hx_status launch_fill_random(void *dst, uint64_t n, hx_dtype dtype,
                             hx_distribution dist, uint64_t seed, double p0,
                             double p1, hipStream_t stream);

// Grid sizing shared by the launchers.
inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

} // namespace hx

// A prepared dispatch (the reference's Prepared associated types, e.g.
// crates/hephaestus-rocm/src/application/full_reduction_seam.rs:33-43).
// `mu` serialises dispatches of one plan from several host threads, so each
// draws its own look-back tag; launches on different streams are ordered by
// the caller.
//
// Under stream capture (hx_plan_dispatch checks), a plan whose launches are
// tagged (tagged()) records a fill kernel over its status words and then its
// launch with kCapturedTag, so the graph can be replayed any number of
// times; plans without tagged words are captured as they are.
struct hx_plan {
    hx_device *dev = nullptr;
    void *ws = nullptr;
    uint64_t ws_bytes = 0;
    hx::LookbackState lookback;
    std::mutex mu;
    virtual ~hx_plan();
    virtual hx_status dispatch(hipStream_t stream) = 0;
    // Whether dispatch() draws a look-back tag for words in ws.
    virtual bool tagged() const { return false; }
};
