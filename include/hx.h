/*
 * hx.h — C ABI of hephaestus-amd, the MI355X (gfx950) reduction / scan backend.
 *
 * Every entry point takes plain pointers, sizes and small POD structs; no C++
 * or framework types cross this boundary.  Device pointers are the values
 * returned by hx_alloc (a hipMalloc allocation); a zero-byte allocation is the
 * null pointer and every operation accepts it for an empty operand.
 *
 * Status codes map one-to-one onto the reference error vocabulary
 * (crates/hephaestus-core/src/domain/error.rs:8-58).  On failure the entry
 * point stores a message in thread-local storage (hx_last_error_message) and
 * leaves every output untouched: validation always runs before the first
 * write (conformance clauses crates/hephaestus-conformance/src/
 * full_reduction.rs:213-231 and scan.rs:129-149).
 *
 * Element counts are uint64_t throughout; the kernels index with 64-bit
 * offsets, so operands of 2^30 elements (4 GiB) and beyond are addressable.
 *
 * Streams: every operation takes an hx_stream (a hipStream_t).  NULL selects
 * the device's own stream, created at hx_device_open with default priority.
 * Operations are stream-ordered and asynchronous; hx_download, hx_upload,
 * hx_write_sub, hx_copy and hx_synchronize are synchronous, like the
 * reference's transfers (crates/hephaestus-rocm/src/infrastructure/
 * memory.rs:102-131,207-258).
 *
 * Threads: a device handle may be shared by host threads, like the
 * reference's Send + Sync device (crates/hephaestus-rocm/src/application/
 * pipeline.rs:101-108).  The immediate (un-prepared) entry points keep their
 * partials and look-back state per stream, and calls on one stream from
 * several threads are serialised from workspace lookup to launch, so
 * immediate calls on any mix of threads and streams never share scratch
 * memory.  A plan (hx_prepare_*) owns one workspace: dispatches of the same
 * plan are serialised across threads, and the caller orders dispatches of
 * one plan that go to different streams (an event, or a synchronize), as
 * for any other work on those streams.
 *
 * Graph capture: hx_plan_dispatch and hx_plan_dispatch_batch may be called
 * on a stream that is being captured into a HIP graph.  A captured dispatch
 * of a plan with look-back statuses or partial slots (scan, full reduce,
 * map-reduction, segmented plans) records a fill kernel that zeroes the
 * plan's status words, then its launches with one tag reserved for captured
 * work, so the graph may be replayed any number of times and reads the
 * plan's bound buffers afresh on each replay.  A replay uses the plan's
 * workspace: replays and eager dispatches of the same plan must be ordered
 * like any two dispatches of it.  The immediate entry points (hx_scan,
 * hx_reduce_full, hx_argmax_full, hx_reduce_axis, hx_reduce_rows,
 * hx_segmented_reduce, hx_map_reduce, hx_trace) draw a fresh tag per call
 * and may grow their stream's buffers, so on a capturing stream they fail
 * with HX_ERR_DISPATCH_FAILED before anything is queued; hx_scan_noalloc,
 * the vector forms, hx_copy_async and hx_fill_random queue plain kernels and
 * may be captured.
 */
#ifndef HX_H
#define HX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HX_ABI_VERSION 1u
#define HX_MAX_RANK 4u

/* ---------------------------------------------------------------- status */

/* crates/hephaestus-core/src/domain/error.rs:8-58 (HephaestusError). */
typedef enum hx_status {
    HX_OK = 0,
    HX_ERR_ADAPTER_UNAVAILABLE = 1,   /* AdapterUnavailable   error.rs:11-15 */
    HX_ERR_DEVICE_UNAVAILABLE = 2,    /* DeviceUnavailable    error.rs:17-21 */
    HX_ERR_ALLOCATION_FAILED = 3,     /* AllocationFailed     error.rs:24-28 */
    HX_ERR_LENGTH_MISMATCH = 4,       /* LengthMismatch       error.rs:30-36 */
    HX_ERR_DISPATCH_FAILED = 5,       /* DispatchFailed       error.rs:38-42 */
    HX_ERR_INVALID_CONFIGURATION = 6, /* InvalidConfiguration error.rs:45-49 */
    HX_ERR_TRANSFER_FAILED = 7        /* TransferFailed       error.rs:51-55 */
} hx_status;

typedef enum hx_dtype {
    HX_DTYPE_F32 = 0, /* DialectScalar<HipC> "float"        core dialect.rs:116-126 */
    HX_DTYPE_U32 = 1, /* "unsigned int"; sums wrap mod 2^32 */
    HX_DTYPE_I32 = 2  /* "int"; two's complement wrap       */
} hx_dtype;

/* Combining operators: crates/hephaestus-core/src/domain/ops.rs:735-803
 * (SumOp, ProdOp, MinOp, MaxOp) with identities ops.rs:926-983.  ARGMAX is
 * an addition to the reference's operators (index of the maximum, ties to
 * the lowest index); MEAN mirrors mean_axis_kernel (crates/hephaestus-rocm/src/application/
 * axis_reduction.rs:67-112). */
typedef enum hx_op {
    HX_OP_SUM = 0,
    HX_OP_PROD = 1,
    HX_OP_MIN = 2,
    HX_OP_MAX = 3,
    HX_OP_ARGMAX = 4,
    HX_OP_MEAN = 5
} hx_op;

typedef enum hx_scan_kind {
    HX_SCAN_INCLUSIVE = 0, /* reference form: core accelerator/scan.rs:56-155 */
    HX_SCAN_EXCLUSIVE = 1  /* addition to the reference: out[i] = fold(x[0..i)) */
} hx_scan_kind;

/* crates/hephaestus-core/src/domain/scan.rs:36-43 (ScanDirection). */
typedef enum hx_scan_direction {
    HX_SCAN_FORWARD = 0,
    HX_SCAN_REVERSE = 1
} hx_scan_direction;

/* Strided view of a linear buffer: the leto Layout<N> that
 * crates/hephaestus-core/src/domain/view.rs:27-41 pairs with a buffer.
 * Element (i0..i{r-1}) lives at offset + sum(i_k * strides[k]). */
typedef struct hx_layout {
    uint32_t rank;
    uint32_t reserved;
    uint64_t shape[HX_MAX_RANK];
    int64_t strides[HX_MAX_RANK];
    uint64_t offset;
} hx_layout;

/* Fused elementwise prologue y = fmaf(a, x, b), applied to every f32 element
 * before it is combined.  The reference spells this as a separate
 * ParameterizedUnaryExpr launch "x * first + second" (core parameterized.rs:
 * 16-45) writing a temporary; here it is fused into the reduction's load. */
typedef struct hx_affine {
    float a;
    float b;
    uint32_t enabled;
    uint32_t reserved;
} hx_affine;

/* Limits and topology: crates/hephaestus-rocm/src/infrastructure/
 * query.rs:29-177 (query_device_limits, query_topology). */
typedef struct hx_device_info {
    char name[96];
    char arch[64];
    int32_t ordinal;
    uint32_t compute_units;
    uint32_t warp_size;
    uint32_t max_threads_per_block;
    uint32_t max_threads_per_cu;
    uint32_t lds_bytes_per_block;
    uint32_t regs_per_block;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_width_bits;
    uint64_t l2_bytes;
    uint64_t total_memory_bytes;
    uint64_t free_memory_bytes;
} hx_device_info;

typedef struct hx_device hx_device; /* opaque: RocmDevice */
typedef struct hx_plan hx_plan;     /* opaque: a prepared dispatch */
typedef void *hx_stream;            /* hipStream_t; NULL = device stream */
typedef void *hx_event;             /* hipEvent_t */

/* ---------------------------------------------------------- diagnostics */

uint32_t hx_abi_version(void);
const char *hx_status_name(hx_status status);
/* Message of the last failed call on this thread ("" after a success). */
const char *hx_last_error_message(void);
/* Lengths carried by the last HX_ERR_LENGTH_MISMATCH on this thread
 * (error.rs:30-36: host_len, device_len). */
void hx_last_length_mismatch(uint64_t *host_len, uint64_t *device_len);

/* ------------------------------------------------- device (ComputeDevice) */

/* hipGetDeviceCount; 0 devices is HX_OK with *count = 0. */
hx_status hx_device_count(int32_t *count);
/* RocmDevice::try_with_ordinal (crates/hephaestus-rocm/src/infrastructure/
 * device.rs:109-165), including the 42 sanity round trip (:141-163).
 * No device / bad ordinal -> HX_ERR_ADAPTER_UNAVAILABLE. */
hx_status hx_device_open(int32_t ordinal, hx_device **out);
hx_status hx_device_close(hx_device *dev);
/* No counterpart in the reference (its launches all go to the null stream).
 * Frees the buffers that immediate calls keep for `stream` (created on its
 * first use, at least 1 MiB of workspace and 1 MiB of scratch) after waiting
 * for the work queued on it.  Call it before destroying a stream that
 * immediate calls have used; otherwise those buffers stay allocated until
 * hx_device_close.  The caller guarantees that no other call uses `stream`
 * meanwhile, as for destroying it.  NULL (the device's own stream) and
 * streams without buffers are no-ops. */
hx_status hx_stream_release(hx_device *dev, hx_stream stream);
hx_status hx_device_get_info(const hx_device *dev, hx_device_info *out);
/* The device's own stream (what a NULL hx_stream selects). */
hx_status hx_device_stream(const hx_device *dev, hx_stream *out);

/* ComputeDeviceCapabilities (core device.rs:225-238; ROCm
 * infrastructure/capabilities.rs:5-21 over query.rs:28-101).  The limits
 * are queried at hx_device_open: max_buffer_size is the free device memory
 * then (query.rs:39), the workgroup limits are the HIP device attributes,
 * max_immediate_size is 0. */
typedef struct hx_device_limits {
    uint64_t max_buffer_size;
    uint32_t max_compute_workgroup_size_x;
    uint32_t max_compute_workgroup_size_y;
    uint32_t max_compute_workgroup_size_z;
    uint32_t max_compute_invocations_per_workgroup;
    uint32_t max_compute_workgroup_storage_size;
    uint32_t max_immediate_size;
} hx_device_limits;
/* DeviceFeature (core device.rs:19-36). */
typedef enum hx_device_feature {
    HX_FEATURE_TIMESTAMP_QUERY = 0,
    HX_FEATURE_SHADER_F64 = 1,
    HX_FEATURE_SHADER_F16 = 2,
    HX_FEATURE_MAPPABLE_PRIMARY_BUFFERS = 3,
    HX_FEATURE_IMMEDIATE_DATA = 4
} hx_device_feature;
hx_status hx_device_get_limits(const hx_device *dev, hx_device_limits *out);
/* supports_device_feature: 0 for every feature, as the reference's ROCm
 * device reports (capabilities.rs:12-20: hipMalloc memory is not
 * host-mappable). */
int32_t hx_device_supports_feature(const hx_device *dev,
                                   hx_device_feature feature);
/* require_limits (ROCm device.rs:187-238), used by try_acquire_device(s)
 * (ROCm acquisition.rs:8-35): HX_ERR_DEVICE_UNAVAILABLE "ROCm device limit
 * <name> <available> is below required <needed>" for the first field of
 * `actual` below `required`, in the order of the struct. */
hx_status hx_require_limits(const hx_device_limits *actual,
                            const hx_device_limits *required);
/* ComputeDevice::synchronize (core device.rs:218-223). */
hx_status hx_synchronize(hx_device *dev);

/* alloc_zeroed / alloc_uninitialized (core device.rs:96-121).  A zero-byte
 * request returns NULL and makes no HIP call (rocm memory.rs:75-88). */
hx_status hx_alloc(hx_device *dev, uint64_t bytes, uint32_t zeroed, void **out);
hx_status hx_free(hx_device *dev, void *ptr);

/* write_buffer (core device.rs:178-184): dst_len must equal src_len
 * (elements of elem_size bytes) or HX_ERR_LENGTH_MISMATCH. Staged through
 * pinned host memory. */
hx_status hx_upload(hx_device *dev, void *dst, uint64_t dst_len,
                    const void *src, uint64_t src_len, uint32_t elem_size);
/* write_sub_buffer (core device.rs:186-195; host semantics
 * crates/hephaestus-host/src/lib.rs:151-172). */
hx_status hx_write_sub(hx_device *dev, void *dst, uint64_t dst_len,
                       uint64_t offset, const void *src, uint64_t src_len,
                       uint32_t elem_size);
/* download (core device.rs:137-144): rejects a length mismatch before any
 * transfer. */
hx_status hx_download(hx_device *dev, const void *src, uint64_t src_len,
                      void *dst, uint64_t dst_len, uint32_t elem_size);
/* copy_buffer (core device.rs:197-211): device-local, complete on return;
 * src == dst is a no-op (host lib.rs:174-183); otherwise the two ranges must
 * not overlap (distinct buffers, as the reference's &src / &mut dst). */
hx_status hx_copy(hx_device *dev, const void *src, uint64_t src_len,
                  void *dst, uint64_t dst_len, uint32_t elem_size);

/* Stream-ordered form of hx_copy (no reference counterpart; copy_buffer is
 * synchronous): the same streaming copy kernel queued on `stream`, returning
 * without waiting.  It is also the read+write bandwidth yardstick that the
 * bench times back to back. */
hx_status hx_copy_async(hx_device *dev, const void *src, uint64_t src_len,
                        void *dst, uint64_t dst_len, uint32_t elem_size,
                        hx_stream stream);

/* ------------------------------------------------------------- timing */

hx_status hx_event_create(hx_device *dev, hx_event *out);
hx_status hx_event_destroy(hx_event ev);
hx_status hx_event_record(hx_device *dev, hx_event ev, hx_stream stream);
hx_status hx_event_synchronize(hx_event ev);
hx_status hx_event_elapsed_ms(hx_event start, hx_event stop, float *ms);

/* ------------------------------------------------- host-side planners */
/* Pure host functions: no device needed; they are what every device entry
 * point runs first. */

/* validate_reduction_width (core reduction.rs:339-349). */
hx_status hx_validate_reduction_width(uint32_t width);
/* reduction_pass_count (core reduction.rs:356-366). */
uint64_t hx_reduction_pass_count(uint64_t len, uint32_t width);
/* Layout::checked_size / validate_storage_len / has_zero_stride_aliasing,
 * as the planners use them (core reduction.rs:449-462). */
hx_status hx_layout_checked_size(const hx_layout *layout, uint64_t *size);
hx_status hx_layout_validate_storage_len(const hx_layout *layout,
                                         uint64_t buf_len);
int32_t hx_layout_has_zero_stride_aliasing(const hx_layout *layout);

/* plan_axis_reduction (core reduction.rs:410-500).  On success *groups is
 * the number of outputs (0 = empty no-op) and *axis_len the reduced
 * extent. */
hx_status hx_plan_axis_reduction(const hx_layout *in, uint64_t in_buf_len,
                                 const hx_layout *out, uint64_t out_buf_len,
                                 uint32_t axis, uint32_t width,
                                 int32_t buffers_alias, uint64_t *out_len,
                                 uint64_t *axis_len);
/* plan_axis_scan (core scan.rs:87-178) generalised to rank 1 and 2:
 * *lines = number of scan lines (0 = empty no-op), *line_len their
 * length. */
hx_status hx_plan_axis_scan(const hx_layout *in, uint64_t in_buf_len,
                            const hx_layout *out, uint64_t out_buf_len,
                            uint32_t axis, uint32_t width,
                            int32_t buffers_alias, uint64_t *lines,
                            uint64_t *line_len);

/* ------------------------------------------------------ FullReductionOps */

/* FullReductionOps::reduce_full_into (core reduction.rs:267-279;
 * ROCm impl crates/hephaestus-rocm/src/application/
 * full_reduction_seam.rs:55-120).  `out` must be a 1-element view
 * (full_reduction_seam.rs:65-73).  op is SUM, PROD, MIN or MAX (MEAN divides
 * the sum by the element count).  `prologue` (may be NULL) applies
 * y = fmaf(a,x,b) to f32 inputs first.  Immediate form: partials live in
 * the workspace of the stream it launches on (see Threads above). */
hx_status hx_reduce_full(hx_device *dev, hx_op op, hx_dtype dtype,
                         const void *in, uint64_t in_buf_len,
                         const hx_layout *in_layout, void *out,
                         uint64_t out_buf_len, const hx_layout *out_layout,
                         const hx_affine *prologue, hx_stream stream);

/* Full argmax (no reference counterpart): index
 * of the maximum of the (prologue-mapped) view in logical row-major order,
 * ties to the lowest index, NaN elements ignored.  out_index (u32[1]) gets
 * the index (UINT32_MAX when there is no non-NaN element); out_value (T[1],
 * may be NULL) gets the MaxOp result (ops.rs:956-958: identity f32::MIN).
 * The logical length must be < 2^32. */
hx_status hx_argmax_full(hx_device *dev, hx_dtype dtype, const void *in,
                         uint64_t in_buf_len, const hx_layout *in_layout,
                         void *out_value, uint32_t *out_index,
                         const hx_affine *prologue, hx_stream stream);

/* FullReductionOps::prepare_reduce_full (core reduction.rs:289-297): binds
 * the operands and owns the workspace, so hx_plan_dispatch allocates
 * nothing and re-reads the bound input each time (rebind contract,
 * conformance full_reduction.rs:173-208). */
hx_status hx_prepare_reduce_full(hx_device *dev, hx_op op, hx_dtype dtype,
                                 const void *in, uint64_t in_buf_len,
                                 const hx_layout *in_layout, void *out,
                                 uint64_t out_buf_len,
                                 const hx_layout *out_layout,
                                 const hx_affine *prologue, hx_plan **plan);

/* ----------------------------------------- AxisReductionOps + fused rows */

/* AxisReductionOps::reduce_axis_into / prod / min / max / mean_axis_into
 * (core reduction.rs:97-197): rank-2 input, `axis` collapsed to length 1 in
 * `out`.  MIN/MAX/MEAN reject an empty axis with "{min,max,mean}_axis is
 * undefined for empty axis {axis}" (rocm axis_reduction.rs:125-136). */
hx_status hx_reduce_axis(hx_device *dev, hx_op op, hx_dtype dtype,
                         const void *in, uint64_t in_buf_len,
                         const hx_layout *in_layout, uint32_t axis, void *out,
                         uint64_t out_buf_len, const hx_layout *out_layout,
                         hx_stream stream);
/* AxisReductionOps::prepare_reduce_axis_into (core reduction.rs:206-215). */
hx_status hx_prepare_reduce_axis(hx_device *dev, hx_op op, hx_dtype dtype,
                                 const void *in, uint64_t in_buf_len,
                                 const hx_layout *in_layout, uint32_t axis,
                                 void *out, uint64_t out_buf_len,
                                 const hx_layout *out_layout, hx_plan **plan);

/* Fused row-wise reduce (no single reference counterpart): for each of
 * `rows` rows of `cols` elements (row r starts at in + offset +
 * r*row_stride, unit column stride), ONE read computes any of
 *   out_sum[r]    = sum of y          (T; f32 accumulates in f64)
 *   out_max[r]    = MaxOp fold of y   (T)
 *   out_argmax[r] = lowest index of the max of y (u32; UINT32_MAX if none)
 * with y = fmaf(a, x, b) when `prologue` is enabled (f32 only).  Any output
 * may be NULL.  Replaces separate sum_axis/max_axis launches
 * (rocm axis_reduction.rs:16-65, one serial thread per row). */
hx_status hx_reduce_rows(hx_device *dev, hx_dtype dtype, const void *in,
                         uint64_t in_buf_len, uint64_t rows, uint64_t cols,
                         uint64_t row_stride, uint64_t offset,
                         const hx_affine *prologue, void *out_sum,
                         void *out_max, uint32_t *out_argmax,
                         uint64_t out_len, hx_stream stream);

/* Prepared form of hx_reduce_rows, as prepare_reduce_axis_into is of
 * reduce_axis_into (crates/hephaestus-rocm/src/application/
 * prepared_axis_reduction.rs:20-222): binds the operands, validates once and
 * owns the workspace of the split forms, so hx_plan_dispatch allocates
 * nothing, re-reads the bound input on every dispatch, and the plan can go
 * to hx_plan_dispatch_batch (submit_prepared_axis_reduction_batch,
 * prepared_axis_reduction.rs:84-92). */
hx_status hx_prepare_reduce_rows(hx_device *dev, hx_dtype dtype, const void *in,
                                 uint64_t in_buf_len, uint64_t rows,
                                 uint64_t cols, uint64_t row_stride,
                                 uint64_t offset, const hx_affine *prologue,
                                 void *out_sum, void *out_max,
                                 uint32_t *out_argmax, uint64_t out_len,
                                 hx_plan **plan);

/* ---------------------------------------------------------------- ScanOps */

/* ScanOps::scan_axis_into (core scan.rs:219-233) over rank-1 or rank-2
 * views; op is SUM (CumSumOp) or PROD (CumProdOp); kind adds the exclusive
 * form; direction REVERSE is the suffix scan (accelerator/scan.rs:430-435).
 * A contiguous line runs the single-pass decoupled look-back scan; f32 sums
 * carry the inter-tile prefix in f64. */
hx_status hx_scan(hx_device *dev, hx_op op, hx_dtype dtype, hx_scan_kind kind,
                  hx_scan_direction direction, const void *in,
                  uint64_t in_buf_len, const hx_layout *in_layout,
                  uint32_t axis, void *out, uint64_t out_buf_len,
                  const hx_layout *out_layout, hx_stream stream);
/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): hx_scan with the same arguments and
 * results, whose whole workspace is a fixed 8 MiB device array per GPU
 * (hx_noalloc_scratch_bytes), so it calls no hipMalloc, hipFree or
 * allocating library routine.  A scan that needs more workspace (1-D scans
 * beyond about 2^31 elements, large single-pass column scans) is rejected
 * with HX_ERR_DISPATCH_FAILED before anything is launched.  Every call on a GPU shares that GPU's array: calls
 * queued on one stream run in order, calls that overlap on one GPU (other
 * streams, other threads) race. */
hx_status hx_scan_noalloc(hx_device *dev, hx_op op, hx_dtype dtype,
                          hx_scan_kind kind, hx_scan_direction direction,
                          const void *in, uint64_t in_buf_len,
                          const hx_layout *in_layout, uint32_t axis, void *out,
                          uint64_t out_buf_len, const hx_layout *out_layout,
                          hx_stream stream);
/* Size in bytes of each GPU's no-allocation scratch array. */
uint64_t hx_noalloc_scratch_bytes(void);
/* ScanOps::prepare_scan_axis (core scan.rs:242-252). */
hx_status hx_prepare_scan(hx_device *dev, hx_op op, hx_dtype dtype,
                          hx_scan_kind kind, hx_scan_direction direction,
                          const void *in, uint64_t in_buf_len,
                          const hx_layout *in_layout, uint32_t axis, void *out,
                          uint64_t out_buf_len, const hx_layout *out_layout,
                          hx_plan **plan);

/* ------------------------------------------------------- segmented reduce */

/* Segmented sum (no reference counterpart; offsets follow the CSR row_ptr
 * convention of core sparse.rs:179-220: num_offsets = S+1 entries,
 * offsets[0] = 0, offsets[S] = n, non-decreasing):
 *   out[s] = sum of values[offsets[s] .. offsets[s+1])   (mod 2^32 for ints)
 * Offsets live in device memory and are not re-validated on the hot path;
 * the kernel clamps every offset into [0, n] so malformed offsets cannot
 * read out of bounds.  hx_validate_segment_offsets checks them. */
hx_status hx_segmented_reduce(hx_device *dev, hx_op op, hx_dtype dtype,
                              const void *values, uint64_t n,
                              const uint32_t *offsets, uint64_t num_offsets,
                              void *out, uint64_t out_len, hx_stream stream);
hx_status hx_prepare_segmented_reduce(hx_device *dev, hx_op op, hx_dtype dtype,
                                      const void *values, uint64_t n,
                                      const uint32_t *offsets,
                                      uint64_t num_offsets, void *out,
                                      uint64_t out_len, hx_plan **plan);
/* Synchronous device check of the row_ptr rules (validate_csr,
 * core sparse.rs:179-220); HX_ERR_DISPATCH_FAILED names the first rule
 * broken. */
hx_status hx_validate_segment_offsets(hx_device *dev, const uint32_t *offsets,
                                      uint64_t num_offsets, uint64_t n);

/* ------------------------------------- map-reductions (dot, norms, trace) */

/* rocm linalg/norms.rs:32-490: a map fused into a full reduction.  `out`
 * receives one element of `dtype`.  DOT needs b with the same logical shape
 * as a ("dot product shape mismatch: lhs [..], rhs [..]", norms.rs:402-411);
 * the other maps read a only (b may be NULL).  NORM_L2 is f32 only
 * (norms.rs:452-456: L2NormScalar is implemented for f32).  f32 sums
 * accumulate in f64 (products and squares of f32 values are exact there);
 * integer sums and products wrap mod 2^32.  Empty operands give the
 * identity: 0, or for NORM_MAX the MaxOp identity (ops.rs:956-958). */
typedef enum hx_map_reduction {
    HX_MAP_SUM = 0,      /* IdentityMap + SumOp (trace)                  */
    HX_MAP_DOT = 1,      /* DotMap: sum of a[i] * b[i]                   */
    HX_MAP_NORM_L1 = 2,  /* AbsMap: sum of |a[i]|                        */
    HX_MAP_NORM_L2 = 3,  /* SquareMap + sqrt: sqrt(sum of a[i]^2)        */
    HX_MAP_NORM_MAX = 4  /* MaxAbsMap + MaxOp: max of |a[i]|             */
} hx_map_reduction;
hx_status hx_map_reduce(hx_device *dev, hx_map_reduction map, hx_dtype dtype,
                        const void *a, uint64_t a_buf_len,
                        const hx_layout *a_layout, const void *b,
                        uint64_t b_buf_len, const hx_layout *b_layout,
                        void *out, uint64_t out_buf_len, hx_stream stream);
/* prepare_map_reduction (rocm prepared_map_reduction.rs:63-213): binds the
 * operands; dispatch re-reads them. */
hx_status hx_prepare_map_reduce(hx_device *dev, hx_map_reduction map,
                                hx_dtype dtype, const void *a,
                                uint64_t a_buf_len, const hx_layout *a_layout,
                                const void *b, uint64_t b_buf_len,
                                const hx_layout *b_layout, void *out,
                                uint64_t out_buf_len, hx_plan **plan);
/* trace (norms.rs:416-444): rank-2 square view ("trace requires a square
 * matrix, got shape [r, c]"), summed along the diagonal view with stride
 * strides[0] + strides[1]; an empty matrix gives 0. */
hx_status hx_trace(hx_device *dev, hx_dtype dtype, const void *in,
                   uint64_t in_buf_len, const hx_layout *in_layout, void *out,
                   uint64_t out_buf_len, hx_stream stream);

/* ------------------------------------------- dense f32 vector recurrences */

/* DenseVectorOps (core vector.rs:57-200; rocm vector.rs:36-72, 141-271), f32
 * only like the reference's ROCm implementation.  Lengths must agree
 * (HX_ERR_LENGTH_MISMATCH with (left, right) lengths, vector.rs:119-128);
 * empty vectors are a no-op.
 *   SCALE  target = target * factor              (source unused)
 *   AXPY   target = fmaf(factor, source, target)
 *   XPAY   target = fmaf(factor, target, source)
 * hx_vector_binary: out = left op right, op one of ADD SUB MUL DIV. */
typedef enum hx_vector_op {
    HX_VEC_SCALE = 0,
    HX_VEC_AXPY = 1,
    HX_VEC_XPAY = 2,
    HX_VEC_ADD = 3,
    HX_VEC_SUB = 4,
    HX_VEC_MUL = 5,
    HX_VEC_DIV = 6
} hx_vector_op;
hx_status hx_vector_update(hx_device *dev, hx_vector_op op, hx_dtype dtype,
                           void *target, uint64_t target_len,
                           const void *source, uint64_t source_len,
                           float factor, hx_stream stream);
hx_status hx_vector_binary(hx_device *dev, hx_vector_op op, hx_dtype dtype,
                           const void *left, uint64_t left_len,
                           const void *right, uint64_t right_len, void *out,
                           uint64_t out_len, hx_stream stream);

/* ---------------------------------------------------------------- plans */

/* dispatch_full / dispatch_prepared / dispatch_scan (core reduction.rs:
 * 222,304-308; scan.rs:259-263): re-run a prepared plan on `stream`.
 * Allocates nothing.  Concurrent calls on one plan are serialised; a plan
 * dispatched on two streams must be ordered by the caller between them.
 * May be captured into a HIP graph (see Graph capture above). */
hx_status hx_plan_dispatch(hx_plan *plan, hx_stream stream);
/* submit_prepared_reduction_batch (rocm application/prepared_reduction.rs:
 * 164-174): dispatch `count` plans in order on `stream` with no host
 * synchronisation between them; returns the first error.  A null entry is
 * rejected before any plan runs. */
hx_status hx_plan_dispatch_batch(hx_plan *const *plans, uint64_t count,
                                 hx_stream stream);
hx_status hx_plan_destroy(hx_plan *plan);
/* Bytes of device workspace the plan owns. */
hx_status hx_plan_workspace_bytes(const hx_plan *plan, uint64_t *bytes);

/* ------------------------------------------------------------ DeviceApi */
/* The vendor seam beneath the reference's generic accelerator layer
 * (DeviceApi, core accelerator/device_api.rs:69-133; ROCm impl
 * crates/hephaestus-rocm/src/application/device_api.rs:49-103 over
 * pipeline.rs:175-349): kernel source compiled at run time with hipRTC for
 * this device's architecture, cached per device under a caller key, and
 * launched with a parameter block and an ordered operand list.  Consumers
 * run their own kernels through it next to the library's. */

typedef struct hx_kernel hx_kernel; /* owned by the device; valid until
                                       hx_device_close */

/* Returns the NUL-terminated source to compile, or NULL to fail the call.
 * Called only on a cache miss (compile_cached's `source: impl FnOnce`);
 * the text is copied before hx_kernel_compile_cached returns.  It must not
 * unwind (throw or longjmp) through the library. */
typedef const char *(*hx_kernel_source_fn)(void *ctx);

/* compile_cached (device_api.rs:83-99, pipeline.rs:259-322): the kernel
 * cached under `key` (key_len bytes, compared bytewise), else source(ctx)
 * compiled (-O3, no packed FP32 instructions, the device's
 * --offload-arch), loaded as a module, and `entry` looked up.  Compile,
 * load and lookup failures are HX_ERR_DISPATCH_FAILED (a compile failure
 * carries the hipRTC log) and are not cached. */
hx_status hx_kernel_compile_cached(hx_device *dev, const void *key,
                                   uint64_t key_len, const char *entry,
                                   hx_kernel_source_fn source, void *ctx,
                                   hx_kernel **kernel);

/* launch (device_api.rs:116-132; ROCm device_api.rs:75-102): `groups`
 * blocks of `width` lanes (LaunchGeometry, device_api.rs:16-24) with
 * `shared_bytes` of dynamic LDS.  The argument list is the parameter block
 * (params_bytes at `params`, passed by value as the kernel's first
 * argument; omitted when params_bytes is 0) followed by each operand's
 * device address.  width 0, a parameter block over 4 KiB, or a kernel
 * compiled for another device is HX_ERR_INVALID_CONFIGURATION; the
 * runtime's launch errors are HX_ERR_DISPATCH_FAILED.  Stream-ordered on
 * `stream`. */
hx_status hx_kernel_launch(hx_device *dev, const hx_kernel *kernel,
                           uint32_t groups, uint32_t width,
                           uint32_t shared_bytes, const void *params,
                           uint64_t params_bytes, void *const *operands,
                           uint64_t operand_count, hx_stream stream);

/* buffers_alias (device_api.rs:105-110; ROCm buffer.rs:47-49): 1 when both
 * addresses are non-null and equal (the reference's rule) or the byte
 * ranges [a, a + a_bytes) and [b, b + b_bytes) overlap, else 0. */
int32_t hx_buffers_alias(const void *a, uint64_t a_bytes, const void *b,
                         uint64_t b_bytes);

/* --------------------------------------------------- synthetic inputs */

/* RandomInitOps analog (core random.rs), counter-based so every element is
 * a pure function of (seed, index): h_i = SplitMix64 output i for `seed`
 * (state seed + (i+1)*0x9E3779B97F4A7C15, Steele-Lea-Flood 2014 mixer).
 *   HX_DIST_UNIFORM_INT  : lo + ((h_i >> 32) * (hi-lo+1) >> 32), ints in
 *                          [p0, p1]
 *   HX_DIST_UNIFORM_REAL : fmaf(p1-p0, u, p0), u = (h_i >> 40) * 2^-24
 *   HX_DIST_NORMAL       : Box-Muller in f64 from h_{2i}, h_{2i+1}, mean p0,
 *                          std p1, rounded to f32. */
typedef enum hx_distribution {
    HX_DIST_UNIFORM_INT = 0,
    HX_DIST_UNIFORM_REAL = 1,
    HX_DIST_NORMAL = 2
} hx_distribution;
hx_status hx_fill_random(hx_device *dev, void *dst, uint64_t n, hx_dtype dtype,
                         hx_distribution dist, uint64_t seed, double p0,
                         double p1, hx_stream stream);

/* ------------------------------------------------------------ diagnostics */

/* No counterpart in the reference.  For tests of the forward-progress
 * fallbacks: sets, for launches queued afterwards by this process, how many
 * polls a look-back (scans, segmented sums) makes before it computes a
 * missing predecessor itself (default 64), and how many polls the gathering
 * block of a one-launch reduction (full reduce, map-reductions) makes per
 * partial before it recomputes that partial from the operand (default
 * 16384).  0 takes every fallback at once; for the gather, 0 skips the
 * partials entirely, so the gathering block recomputes every one.  Results
 * are the same at every setting (integer results bit-identical, f32
 * reductions bit-identical, f32 scans within their bound); only time
 * changes.  Not for production use: a small limit makes large inputs slow. */
hx_status hx_debug_set_wait_limits(uint32_t lookback_polls, uint32_t gather_polls);
/* No counterpart in the reference.  For tests of the look-back tag range:
 * sets how many launches the library counts as already made on a
 * workspace -- `plan`'s when it is not NULL, else the immediate workspace of
 * `stream` on `dev` (HX_ERR_INVALID_CONFIGURATION if that stream has none
 * yet).  Eager tags cycle through [1, 2^14 - 1); the launch that wraps the
 * range back to tag 1 first clears the workspace's status words, so
 * presetting the count to 2^14 - 2 makes the next launch the wrap. */
hx_status hx_debug_set_launch_count(hx_device *dev, hx_plan *plan,
                                    hx_stream stream, uint64_t launches);
/* No counterpart in the reference.  The high 32 bits of a tagged word as the
 * kernels build it: kind 0 a look-back status word with `flag` (1 aggregate,
 * 2 inclusive prefix), kind 1 a partial slot of a one-launch reduction
 * (`flag` ignored).  Both kinds share a workspace region and one tag
 * counter; a test checks that no slot word equals any status word. */
uint32_t hx_debug_tagged_word_hi(uint32_t kind, uint32_t tag, uint32_t flag);
/* No counterpart in the reference.  The 16-byte status slot of the f32 scans
 * (f64 carries), as the kernels encode and decode it: four dwords, each
 * ((tag << 2 | flag) << 16) | 16 bits of `bits` (tags below 2^14).  decode
 * returns the flag (1 aggregate, 2 inclusive prefix) and the value when all
 * four dwords carry `tag` and one flag, else 0 ("not ready"), so a read that
 * mixes dwords of two writes is never accepted.  Host-only, for tests. */
void hx_debug_slot16_encode(uint32_t tag, uint32_t flag, uint64_t bits, uint32_t *dwords);
uint32_t hx_debug_slot16_decode(uint32_t tag, const uint32_t *dwords, uint64_t *bits);
/* No counterpart in the reference.  A bench yardstick: copies `bytes` (a
 * multiple of 131072) from src to dst in the access pattern of the integer
 * scan's look-back tiles -- block b moves 128 KiB tile b, each of 8 waves a
 * contiguous 16 KiB run, every load issued before the first store -- the
 * order and shape a single-pass scan is held to, unlike hx_copy_async's
 * 256 KiB tiles in XCD-contiguous order. */
hx_status hx_debug_copy_scan_shape(hx_device *dev, const void *src, void *dst,
                                   uint64_t bytes, hx_stream stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* HX_H */
