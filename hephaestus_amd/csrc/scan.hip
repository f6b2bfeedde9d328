// Prefix scans for gfx950: ScanOps (crates/hephaestus-core/src/domain/
// scan.rs:197-264), extended with the exclusive form and rank-1 operands.
//
// The reference launches ONE 256-lane block per scan line; each lane walks a
// contiguous chunk serially, lane 0 folds the chunk totals, and a second sweep
// re-reads and re-writes the output (core accelerator/scan.rs:56-155).  A 1-D
// scan of 2^28 elements therefore runs on one CU.  Here every line is cut
// into tiles of 4096 elements that all CUs process in a single pass:
//
//   * a block takes a virtual tile ticket from an agent-scope counter, so
//     every tile it may wait on was taken by a block that is already running
//     (forward progress without any dispatch-order assumption);
//   * the tile is loaded with 16-byte vectors, wave-striped: step j of wave w
//     holds 256 contiguous elements, lane l four of them; each step is a
//     4-element register scan plus a 6-step wave64 scan of lane totals;
//   * the tile aggregate is published, then wave 0 looks back over up to 64
//     predecessors per poll (one status word per lane) until it meets an
//     inclusive prefix; the tile publishes its own inclusive prefix;
//   * every element is written exactly once, 16-byte vectors again.
//
// Status words carry a 30-bit launch tag, so a new launch never needs the
// status array cleared: the last block to finish bumps the tag and resets
// the ticket counter.  Integer scans publish (tag, flag, value) in ONE 64-bit
// word.  f32 scans carry the inter-tile prefix in f64 (two value arrays and a
// flag word released after the value), which keeps the error of every output
// within a few ulp of the f32-rounded exact prefix at 2^30 elements.
#include "hx_device.hpp"
#include "hx_internal.hpp"

#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;
constexpr int kSteps = 4;                            // vectors per lane
constexpr int kWaveElems = kWave * 4 * kSteps;       // 1024
constexpr int kTile = kWaves * kWaveElems;           // 4096
constexpr uint64_t kLookbackOffset = 256 + 64 * 1024; // after header + reduce area

constexpr uint32_t kInvalid = 0, kAggregate = 1, kPrefix = 2;

__device__ __forceinline__ uint32_t epoch_tag(uint32_t epoch) { return (epoch % 0x3FFFFFFFu) + 1u; }

// (tag, flag, value) in one 64-bit word: [63:34] tag, [33:32] flag, [31:0] value.
struct PackedStatus {
    using C = uint32_t;
    uint64_t *words;
    __device__ __forceinline__ void publish(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        st_relaxed(&words[t], ((uint64_t)((tag << 2) | flag) << 32) | (uint64_t)v);
    }
    __device__ __forceinline__ void read(uint64_t t, uint32_t tag, uint32_t &flag, C &v) const {
        const uint64_t w = ld_relaxed(&words[t]);
        const uint32_t hi = (uint32_t)(w >> 32);
        flag = ((hi >> 2) == tag) ? (hi & 3u) : kInvalid;
        v = (uint32_t)w;
    }
};

// f64 carries: the value is stored first, then the flag word with release
// semantics; a reader acquires the flag before reading the value.  The
// aggregate and the inclusive prefix live in different arrays so a reader
// that saw "aggregate" can never read a later prefix by mistake.
struct F64Status {
    using C = double;
    uint32_t *flags;
    double *agg;
    double *incl;
    __device__ __forceinline__ void publish(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        if (flag == kAggregate) st_relaxed_f64(&agg[t], v);
        else st_relaxed_f64(&incl[t], v);
        st_release32(&flags[t], (tag << 2) | flag);
    }
    __device__ __forceinline__ void read(uint64_t t, uint32_t tag, uint32_t &flag, C &v) const {
        const uint32_t f = ld_acquire(&flags[t]);
        flag = ((f >> 2) == tag) ? (f & 3u) : kInvalid;
        if (flag == kAggregate) v = ld_relaxed_f64(&agg[t]);
        else if (flag == kPrefix) v = ld_relaxed_f64(&incl[t]);
    }
};

struct ScanParams {
    const void *in;
    void *out;
    uint64_t lines, len, tiles_per_line, total_tiles;
    int64_t in_line_stride, in_elem_stride;
    int64_t out_line_stride, out_elem_stride;
    uint64_t in_offset, out_offset;
    WorkspaceHeader *hdr;
};

// Wave 0 of tile `ticket` folds the values of its predecessors in the same
// line, nearest first, up to and including the first inclusive prefix.
template <typename Op, typename Status>
__device__ typename Status::C lookback(const Status &st, uint64_t ticket, uint64_t line_first,
                                       uint32_t tag) {
    using C = typename Status::C;
    const int lane = lane_id();
    C excl = Op::template identity<C>();
    int64_t pred = (int64_t)ticket - 1;
    for (;;) {
        const int64_t idx = pred - lane;
        const bool in_line = idx >= (int64_t)line_first;
        uint32_t flag = kPrefix;
        C val = Op::template identity<C>();
        for (;;) {
            if (in_line) st.read((uint64_t)idx, tag, flag, val);
            const uint64_t pm = ballot(flag == kPrefix);
            const uint64_t im = ballot(flag == kInvalid);
            // Lanes 0..first-prefix must all be valid.
            const uint64_t need = pm ? (((pm & (~pm + 1ull)) << 1) - 1ull) : ~0ull;
            if ((im & need) == 0ull) break;
            __builtin_amdgcn_s_sleep(1);
        }
        const uint64_t pm = ballot(flag == kPrefix);
        const int first = pm ? (__ffsll((long long)pm) - 1) : kWave;
        const C contrib = (lane <= first) ? val : Op::template identity<C>();
        excl = Op::combine(wave_reduce<Op, C>(contrib), excl);
        if (pm) break;
        pred -= kWave;
    }
    return excl;
}

template <typename T, typename C, typename Op>
__device__ __forceinline__ T finalize(C tile_excl, T within) {
    if constexpr (std::is_same<T, float>::value) {
        return (float)Op::combine(tile_excl, (double)within);
    } else {
        return Op::combine((T)tile_excl, within);
    }
}

template <typename T, typename Op, typename Status, bool EXCL, bool VEC, bool REV>
__global__ __launch_bounds__(kBlock) void scan_tiles_kernel(ScanParams p, Status st) {
    using C = typename Status::C;
    __shared__ uint32_t s_ticket;
    __shared__ uint32_t s_tag;
    __shared__ T s_wave_tot[kWaves];
    __shared__ C s_excl;

    if (threadIdx.x == 0) {
        s_ticket = fetch_add32(&p.hdr->tile_counter, 1u);
        s_tag = epoch_tag(ld_relaxed32(&p.hdr->epoch));
    }
    __syncthreads();
    const uint64_t ticket = s_ticket;
    const uint32_t tag = s_tag;
    const uint64_t line = ticket / p.tiles_per_line;
    const uint64_t tin = ticket - line * p.tiles_per_line;
    const int w = threadIdx.x / kWave;
    const int lane = lane_id();
    const int64_t ib = (int64_t)p.in_offset + (int64_t)line * p.in_line_stride;
    const int64_t ob = (int64_t)p.out_offset + (int64_t)line * p.out_line_stride;
    const uint64_t e0 = tin * kTile + (uint64_t)w * kWaveElems + (uint64_t)lane * 4;
    const T *in = (const T *)p.in;
    T *out = (T *)p.out;
    const T ident = Op::template identity<T>();

    T x[kSteps][4];
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
        if constexpr (VEC) {
            if (e + 3 < p.len) {
                using V = typename Vec4<T>::type;
                const V v = __builtin_nontemporal_load((const V *)(in + ib + (int64_t)e));
                x[j][0] = (T)v.x;
                x[j][1] = (T)v.y;
                x[j][2] = (T)v.z;
                x[j][3] = (T)v.w;
                continue;
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint64_t i = e + c;
            const uint64_t li = REV ? (p.len - 1 - i) : i;
            x[j][c] = (i < p.len) ? in[ib + (int64_t)li * p.in_elem_stride] : ident;
        }
    }

    // Per step: register scan of 4, wave scan of lane totals, running carry.
    T carry = ident;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const T p0 = x[j][0];
        const T p1 = Op::combine(p0, x[j][1]);
        const T p2 = Op::combine(p1, x[j][2]);
        const T p3 = Op::combine(p2, x[j][3]);
        const T incl = wave_inclusive_scan<Op, T>(p3);
        T lex = __shfl_up(incl, 1, kWave);
        if (lane == 0) lex = ident;
        const T step_tot = __shfl(incl, kWave - 1, kWave);
        const T base = Op::combine(carry, lex);
        if constexpr (EXCL) {
            x[j][0] = base;
            x[j][1] = Op::combine(base, p0);
            x[j][2] = Op::combine(base, p1);
            x[j][3] = Op::combine(base, p2);
        } else {
            x[j][0] = Op::combine(base, p0);
            x[j][1] = Op::combine(base, p1);
            x[j][2] = Op::combine(base, p2);
            x[j][3] = Op::combine(base, p3);
        }
        carry = Op::combine(carry, step_tot);
    }
    if (lane == 0) s_wave_tot[w] = carry;
    __syncthreads();
    T wave_excl = ident;
    T tile_agg = ident;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
        if (k < w) wave_excl = Op::combine(wave_excl, s_wave_tot[k]);
        tile_agg = Op::combine(tile_agg, s_wave_tot[k]);
    }

    if (w == 0) {
        const C agg = (C)tile_agg;
        C excl = Op::template identity<C>();
        if (tin == 0) {
            if (lane == 0) st.publish(ticket, tag, kPrefix, agg);
        } else {
            if (lane == 0) st.publish(ticket, tag, kAggregate, agg);
            excl = lookback<Op>(st, ticket, ticket - tin, tag);
            if (lane == 0) st.publish(ticket, tag, kPrefix, Op::combine(excl, agg));
        }
        if (lane == 0) s_excl = excl;
    }
    __syncthreads();
    const C tile_excl = s_excl;

#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
        T r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) r[c] = finalize<T, C, Op>(tile_excl, Op::combine(wave_excl, x[j][c]));
        if constexpr (VEC) {
            if (e + 3 < p.len) {
                using V = typename Vec4<T>::type;
                V v;
                v.x = r[0];
                v.y = r[1];
                v.z = r[2];
                v.w = r[3];
                __builtin_nontemporal_store(v, (V *)(out + ob + (int64_t)e));
                continue;
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint64_t i = e + c;
            const uint64_t li = REV ? (p.len - 1 - i) : i;
            if (i < p.len) out[ob + (int64_t)li * p.out_elem_stride] = r[c];
        }
    }

    if (threadIdx.x == 0) {
        const uint32_t d = fetch_add32_acqrel(&p.hdr->tile_done, 1u);
        if (d == (uint32_t)(p.total_tiles - 1)) {
            st_relaxed32(&p.hdr->tile_counter, 0u);
            st_relaxed32(&p.hdr->tile_done, 0u);
            st_relaxed32(&p.hdr->epoch, ld_relaxed32(&p.hdr->epoch) + 1u);
        }
    }
}

// Many short strided lines whose starts are adjacent in memory (axis-0 scan
// of a row-major matrix): one thread per line walks it serially, so each load
// instruction of a wave covers 64 adjacent lines.  f32 sums accumulate in f64.
template <typename T, typename Op, bool EXCL, bool REV>
__global__ __launch_bounds__(kBlock) void scan_lines_serial_kernel(ScanParams p) {
    using A = typename std::conditional<std::is_same<T, float>::value, double, T>::type;
    const uint64_t nthreads = (uint64_t)gridDim.x * kBlock;
    const T *in = (const T *)p.in;
    T *out = (T *)p.out;
    for (uint64_t line = (uint64_t)blockIdx.x * kBlock + threadIdx.x; line < p.lines; line += nthreads) {
        const int64_t ib = (int64_t)p.in_offset + (int64_t)line * p.in_line_stride;
        const int64_t ob = (int64_t)p.out_offset + (int64_t)line * p.out_line_stride;
        A acc = Op::template identity<A>();
        for (uint64_t i = 0; i < p.len; ++i) {
            const uint64_t li = REV ? (p.len - 1 - i) : i;
            const A v = (A)in[ib + (int64_t)li * p.in_elem_stride];
            if constexpr (EXCL) {
                out[ob + (int64_t)li * p.out_elem_stride] = (T)acc;
                acc = Op::combine(acc, v);
            } else {
                acc = Op::combine(acc, v);
                out[ob + (int64_t)li * p.out_elem_stride] = (T)acc;
            }
        }
    }
}

uint64_t status_bytes(uint64_t tiles, bool f64) {
    if (!f64) return tiles * 8;
    const uint64_t flag_bytes = (tiles * 4 + 7) & ~7ull;
    return flag_bytes + 2 * tiles * 8;
}

template <typename T, typename Op, typename Status, bool EXCL>
hx_status launch_tiles(const ScanParams &p, const Status &st, bool vec, bool rev, hipStream_t stream) {
    const dim3 grid((uint32_t)p.total_tiles), block(kBlock);
    if (vec)
        hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, true, false>), grid, block, 0,
                           stream, p, st);
    else if (rev)
        hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, false, true>), grid, block, 0,
                           stream, p, st);
    else
        hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, false, false>), grid, block, 0,
                           stream, p, st);
    return check_launch("scan_tiles_kernel");
}

template <typename T, typename Op, bool EXCL>
hx_status launch_serial(const ScanParams &p, bool rev, hipStream_t stream) {
    uint64_t blocks = ceil_div(p.lines, kBlock);
    if (blocks > (1u << 20)) blocks = 1u << 20;
    if (rev)
        hipLaunchKernelGGL((scan_lines_serial_kernel<T, Op, EXCL, true>), dim3((uint32_t)blocks),
                           dim3(kBlock), 0, stream, p);
    else
        hipLaunchKernelGGL((scan_lines_serial_kernel<T, Op, EXCL, false>), dim3((uint32_t)blocks),
                           dim3(kBlock), 0, stream, p);
    return check_launch("scan_lines_serial_kernel");
}

bool serial_mode(const ScanArgs &a) {
    const bool contiguous = a.in_elem_stride == 1 && a.out_elem_stride == 1;
    const bool adjacent = (a.in_line_stride == 1 || a.in_line_stride == -1) &&
                          (a.out_line_stride == 1 || a.out_line_stride == -1);
    return !contiguous && adjacent && a.lines >= 256;
}

template <typename T, typename Op>
hx_status launch_op(const ScanArgs &a, void *ws, hipStream_t stream) {
    ScanParams p{};
    p.in = a.in;
    p.out = a.out;
    p.lines = a.lines;
    p.len = a.len;
    p.tiles_per_line = ceil_div(a.len, kTile);
    p.total_tiles = p.tiles_per_line * a.lines;
    p.in_line_stride = a.in_line_stride;
    p.in_elem_stride = a.in_elem_stride;
    p.out_line_stride = a.out_line_stride;
    p.out_elem_stride = a.out_elem_stride;
    p.in_offset = a.in_offset;
    p.out_offset = a.out_offset;
    p.hdr = (WorkspaceHeader *)ws;
    if (a.lines == 0 || a.len == 0) return HX_OK;

    if (serial_mode(a)) {
        return a.exclusive ? launch_serial<T, Op, true>(p, a.reverse, stream)
                           : launch_serial<T, Op, false>(p, a.reverse, stream);
    }
    if (p.total_tiles >= 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "scan of %llu tiles exceeds the u32 ticket range",
                    (unsigned long long)p.total_tiles);
    const bool contiguous = a.in_elem_stride == 1 && a.out_elem_stride == 1;
    const uintptr_t ibase = (uintptr_t)((const T *)a.in + a.in_offset);
    const uintptr_t obase = (uintptr_t)((T *)a.out + a.out_offset);
    const bool vec = contiguous && !a.reverse && ibase % 16 == 0 && obase % 16 == 0 &&
                     a.in_line_stride % 4 == 0 && a.out_line_stride % 4 == 0;
    char *area = (char *)ws + kLookbackOffset;
    if constexpr (std::is_same<T, float>::value) {
        F64Status st;
        st.flags = (uint32_t *)area;
        st.agg = (double *)(area + ((p.total_tiles * 4 + 7) & ~7ull));
        st.incl = st.agg + p.total_tiles;
        return a.exclusive ? launch_tiles<T, Op, F64Status, true>(p, st, vec, a.reverse, stream)
                           : launch_tiles<T, Op, F64Status, false>(p, st, vec, a.reverse, stream);
    } else {
        PackedStatus st;
        st.words = (uint64_t *)area;
        return a.exclusive ? launch_tiles<T, Op, PackedStatus, true>(p, st, vec, a.reverse, stream)
                           : launch_tiles<T, Op, PackedStatus, false>(p, st, vec, a.reverse, stream);
    }
}

} // namespace

uint64_t scan_workspace_bytes(const ScanArgs &a, int *format) {
    const bool f64 = a.dtype == HX_DTYPE_F32;
    *format = f64 ? kWsLookbackF64 : kWsLookbackPacked;
    if (serial_mode(a)) return kWorkspaceHeader;
    const uint64_t tiles = ceil_div(a.len, kTile) * a.lines;
    return kLookbackOffset + status_bytes(tiles, f64);
}

hx_status launch_scan(const ScanArgs &a, void *ws, hipStream_t stream) {
    const bool prod = a.op == HX_OP_PROD;
    switch (a.dtype) {
    case HX_DTYPE_F32:
        return prod ? launch_op<float, OpProd>(a, ws, stream) : launch_op<float, OpSum>(a, ws, stream);
    case HX_DTYPE_U32:
    case HX_DTYPE_I32:
        // Two's complement: i32 sums and products have the bits of u32 ones.
        return prod ? launch_op<uint32_t, OpProd>(a, ws, stream)
                    : launch_op<uint32_t, OpSum>(a, ws, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)a.dtype);
}

} // namespace hx
