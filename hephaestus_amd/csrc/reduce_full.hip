// Full (whole-operand) reductions for gfx950: FullReductionOps
// (crates/hephaestus-core/src/domain/reduction.rs:243-309).
//
// The reference runs a 256-lane LDS halving tree with one element per thread
// and one launch per tree pass (crates/hephaestus-rocm/src/application/
// reduction.rs:16-52, prepared_reduction.rs:39-132), after a strided staging
// copy (full_reduction_seam.rs:102-120).  Here ONE launch does the whole job
// and reads the operand exactly once:
//   * every block grid-strides over the operand with 16-byte loads, folds
//     into registers (f32 sums in f64), reduces its 4 waves with
//     xor-butterflies and publishes one partial;
//   * the last block (dispatched last) gathers the partials, folds them in
//     index order and writes the result.
// A partial is published as self-tagged 64-bit words -- high half the launch
// tag in the look-back layout with the slot flag (slot_word_hi), low half 32
// bits of the value -- with relaxed agent-scope stores, and the gathering
// block accepts a partial only when every half carries this launch's tag.
// No release/acquire pair is needed: a "last block done" counter would need
// a device-scope acq_rel per block, which on multi-XCD CDNA writes back and
// invalidates the L2 each time (measured 2.5x slower at 8192 blocks).  A
// partial still missing after a long bounded wait is recomputed by the
// gathering block from the operand, bit-identically, so the launch finishes
// whatever the dispatch order.
// The grid size is a function of n only, so the combination order and the
// result bits do not depend on the GPU's CU count.
#include "hx_device.hpp"
#include "hx_internal.hpp"
#include "rows_walk.hpp"

#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxBlocks = 768; // 16-byte partial slots: 12 KiB of status words

// The grid: a function of n and the element type only (so is the
// combination tree), one block per 4096 integer or 8192 f32 elements up to
// 768 blocks, three per CU on 256 CUs.  At 2^28 f32 a sweep over 512..4096
// blocks and 1/2/4 loads in flight per lane put 768 blocks with two 16-byte
// non-temporal loads per lane at 7.08 TB/s (151.6 us), ahead of 1024 blocks
// (6.9) and 8192 (3.9).  Small, launch-bound operands gain from fewer blocks
// (fewer partials to gather): 2^20 elements, per-launch median, 512 / 256 /
// 128 / 64 blocks: f32 4.96 / 4.12 / 3.88 / 4.31 us, u32 4.51 / 3.72 / 4.06
// / 4.36; the bench's 2^20 f32 sum, three interleaved runs of 2000 launches:
// 256 blocks 4.26-4.40 us, 128 blocks 3.97-4.29, 64 blocks 4.36-4.47.
constexpr uint64_t kElemsPerBlock = 4096, kElemsPerBlockF32 = 8192;
inline uint32_t full_reduce_blocks(uint64_t n, bool f32) {
    uint64_t blocks = ceil_div(n, f32 ? kElemsPerBlockF32 : kElemsPerBlock);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    return blocks < 1 ? 1u : (uint32_t)blocks;
}

enum Kind { kSum = 0, kProd = 1, kMin = 2, kMax = 3, kArgmax = 4, kMean = 5 };

// Per-kind accumulation policy.
template <typename T, int K> struct Policy;

template <typename T> struct Policy<T, kSum> {
    using Acc = typename SumAcc<typename Wrap<T>::type>::type;
    __device__ static Acc identity() { return Acc(0); }
    template <typename Y> __device__ static Acc lift(Y y, uint64_t) { return (Acc)(typename Wrap<T>::type)y; }
    __device__ static Acc combine(Acc a, Acc b) { return a + b; }
    __device__ static Acc wave(Acc a) { return wave_sum(a); }
};
template <> struct Policy<float, kSum> {
    using Acc = double;
    __device__ static Acc identity() { return 0.0; }
    __device__ static Acc lift(float y, uint64_t) { return (double)y; }
    __device__ static Acc combine(Acc a, Acc b) { return a + b; }
    __device__ static Acc wave(Acc a) { return wave_sum(a); }
};
template <typename T> struct Policy<T, kMean> : Policy<T, kSum> {};

template <typename T> struct Policy<T, kProd> {
    using W = typename Wrap<T>::type;
    using Acc = W;
    __device__ static Acc identity() { return Acc(1); }
    __device__ static Acc lift(T y, uint64_t) { return (W)y; }
    __device__ static Acc combine(Acc a, Acc b) { return a * b; }
    __device__ static Acc wave(Acc a) { return wave_prod(a); }
};
template <> struct Policy<float, kProd> {
    using Acc = double;
    __device__ static Acc identity() { return 1.0; }
    __device__ static Acc lift(float y, uint64_t) { return (double)y; }
    __device__ static Acc combine(Acc a, Acc b) { return a * b; }
    __device__ static Acc wave(Acc a) { return wave_prod(a); }
};

template <typename T> struct Policy<T, kMax> {
    using Acc = uint32_t;
    __device__ static Acc identity() { return Key<T>::max_identity(); }
    __device__ static Acc lift(T y, uint64_t) { return Key<T>::max_key(y); }
    __device__ static Acc combine(Acc a, Acc b) { return a > b ? a : b; }
    __device__ static Acc wave(Acc a) { return wave_umax(a); }
};
template <typename T> struct Policy<T, kMin> {
    using Acc = uint32_t;
    __device__ static Acc identity() { return Key<T>::min_identity(); }
    __device__ static Acc lift(T y, uint64_t) { return Key<T>::min_key(y); }
    __device__ static Acc combine(Acc a, Acc b) { return a < b ? a : b; }
    __device__ static Acc wave(Acc a) { return wave_umin(a); }
};
template <typename T> struct Policy<T, kArgmax> {
    using Acc = uint64_t;
    __device__ static Acc identity() { return 0ull; }
    __device__ static Acc lift(T y, uint64_t i) { return pack_arg(Key<T>::max_key(y), (uint32_t)i); }
    __device__ static Acc combine(Acc a, Acc b) { return umax64(a, b); }
    __device__ static Acc wave(Acc a) { return wave_umax64(a); }
};

struct FullParams {
    const void *base;
    uint64_t n;
    uint64_t offset; // element offset of the view (flat) / layout offset
    RowsGeom g;      // non-flat views
    float a, b;
    void *out_value;
    uint32_t *out_index;
    uint64_t *slots;     // partial slots (PartialSlot), 16 bytes per block
    uint32_t tag;        // this launch's tag
    uint32_t poll_limit; // gather polls per partial before recomputing it
    // Flat views: element e of the range has view index e, or n - 1 - e
    // when the view reads the range from its far end (rev; argmax reports
    // view indices).
    uint64_t idx_last;
    uint32_t rev;
};

template <typename T, bool AFFINE> __device__ __forceinline__ T prologue(T x, float, float) { return x; }
template <> __device__ __forceinline__ float prologue<float, true>(float x, float a, float b) {
    return __builtin_fmaf(a, x, b);
}

template <typename P>
__device__ __forceinline__ typename P::Acc block_reduce(typename P::Acc v,
                                                        typename P::Acc *lds) {
    v = P::wave(v);
    const int w = threadIdx.x / kWave;
    if (lane_id() == 0) lds[w] = v;
    __syncthreads();
    typename P::Acc r = lds[0];
#pragma unroll
    for (int k = 1; k < kBlock / kWave; ++k) r = P::combine(r, lds[k]);
    __syncthreads();
    return r;
}

template <typename T, int K>
__device__ __forceinline__ void write_result_impl(const FullParams &p, typename Policy<T, K>::Acc r) {
    if constexpr (K == kSum || K == kProd) {
        *(T *)p.out_value = (T)r;
    } else if constexpr (K == kMean) {
        if constexpr (std::is_same<T, float>::value) {
            *(float *)p.out_value = (float)(r / (double)p.n);
        } else if constexpr (std::is_same<T, int32_t>::value) {
            // n <= INT32_MAX here (the host rejects larger integer means)
            *(int32_t *)p.out_value = (int32_t)r / (int32_t)p.n;
        } else {
            // n <= UINT32_MAX here
            *(uint32_t *)p.out_value = (uint32_t)r / (uint32_t)p.n;
        }
    } else if constexpr (K == kMax || K == kMin) {
        *(T *)p.out_value = Key<T>::decode(r);
    } else { // argmax
        uint32_t key = (uint32_t)(r >> 32);
        bool none = std::is_same<T, float>::value ? (key == 0u) : (r == 0ull);
        if (p.out_index) *p.out_index = none ? 0xFFFFFFFFu : arg_index(r);
        if (p.out_value) {
            uint32_t mk = Key<T>::max_identity();
            if (!none && key > mk) mk = key;
            *(T *)p.out_value = Key<T>::decode(mk);
        }
    }
}


// Four elements with view indices e .. e + 3, or e .. e - 3 when rev.
template <typename P, typename T, bool AFFINE, typename V>
__device__ __forceinline__ typename P::Acc fold4(const V &v, uint64_t e, bool rev, float a, float b) {
    using Acc = typename P::Acc;
    const Acc a0 = P::lift(prologue<T, AFFINE>((T)v.x, a, b), e);
    const Acc a1 = P::lift(prologue<T, AFFINE>((T)v.y, a, b), rev ? e - 1 : e + 1);
    const Acc a2 = P::lift(prologue<T, AFFINE>((T)v.z, a, b), rev ? e - 2 : e + 2);
    const Acc a3 = P::lift(prologue<T, AFFINE>((T)v.w, a, b), rev ? e - 3 : e + 3);
    return P::combine(P::combine(a0, a1), P::combine(a2, a3));
}

// How a view is walked: the flat element range, or rows (RowsGeom) of
// 16-byte vector units (contiguous rows) or of single elements.
enum Mode { kFlat = 0, kRowsVec = 1, kRowsScalar = 2 };
// Walkers (units in flight per thread) of the row modes.  A 65536 x 4000
// slice of 4096-wide f32 rows: 2 walkers 262 us, 4 walkers 170 us (dense:
// 153 us), with the row tail loaded by unrolled predicated loads (a
// runtime-indexed tail loop cost 35%).
template <int MODE> struct Walkers { static constexpr int value = 4; };

// Unit of walker `w`: its elements in x[0..count), returned count.
template <typename T, int MODE, bool NT>
__device__ __forceinline__ uint32_t load_unit(const RowsGeom &g, const T *src, const RowWalker &w, T (&x)[4]) {
    if constexpr (MODE == kRowsVec) {
        const uint64_t c0 = 4 * w.unit;
        if (c0 + 4 <= g.cols) {
            using V = typename Vec4A4<T>::type;
            const V q = load_a4<NT>((const V *)(src + w.off));
            x[0] = (T)q.x;
            x[1] = (T)q.y;
            x[2] = (T)q.z;
            x[3] = (T)q.w;
            return 4;
        }
        const uint32_t cnt = (uint32_t)(g.cols - c0);
#pragma unroll
        for (uint32_t c = 0; c < 3; ++c)
            if (c < cnt) x[c] = src[w.off + c];
        return cnt;
    } else {
        x[0] = src[w.off];
        return 1;
    }
}

// Fold of `cnt` elements whose logical indices are e0, e0 + es, ...
template <typename P, typename T, bool AFFINE>
__device__ __forceinline__ typename P::Acc fold_n(const T (&x)[4], uint32_t cnt, uint64_t e0, uint64_t es, float a,
                                                  float b) {
    using Acc = typename P::Acc;
    if (cnt == 4) {
        const Acc a0 = P::lift(prologue<T, AFFINE>(x[0], a, b), e0);
        const Acc a1 = P::lift(prologue<T, AFFINE>(x[1], a, b), e0 + es);
        const Acc a2 = P::lift(prologue<T, AFFINE>(x[2], a, b), e0 + 2 * es);
        const Acc a3 = P::lift(prologue<T, AFFINE>(x[3], a, b), e0 + 3 * es);
        return P::combine(P::combine(a0, a1), P::combine(a2, a3));
    }
    Acc r = P::identity();
#pragma unroll
    for (uint32_t c = 0; c < 3; ++c)
        if (c < cnt) r = P::combine(r, P::lift(prologue<T, AFFINE>(x[c], a, b), e0 + c * es));
    return r;
}

// The fold of "block" vb of a G-block grid, per thread (the thread's
// grid-stride share), before the block reduction.  The gathering block
// calls it with another block's index to recompute a missing partial.
// kFlat: the view is the contiguous element range [offset, offset + n);
// UNROLL independent 16-byte loads are in flight per thread per trip.
// Row modes: Walkers<MODE> units in flight, unit j of the thread's share
// at item tid + j * nthreads, each walker stepping by Walkers * nthreads
// items (the host's RowsGeom step).  NT marks loads non-temporal
// (streamed, not kept in the caches).
template <typename P, typename T, bool AFFINE, int MODE, int UNROLL, bool NT>
__device__ __forceinline__ typename P::Acc thread_fold(const FullParams &p, uint32_t vb, uint32_t G) {
    using Acc = typename P::Acc;
    const uint64_t n = p.n;
    const uint64_t tid = (uint64_t)vb * kBlock + threadIdx.x;
    const uint64_t nthreads = (uint64_t)G * kBlock;
    Acc acc = P::identity();

    if constexpr (MODE == kFlat) {
        const T *src = (const T *)p.base + p.offset;
        // Peel up to 3 leading elements so the body is 16-byte aligned.
        uint64_t mis = ((uintptr_t)src >> 2) & 3u;
        uint64_t head = mis ? (4 - mis) : 0;
        if (head > n) head = n;
        const bool rev = p.rev != 0;
        auto vidx = [&](uint64_t e) { return rev ? p.idx_last - e : e; };
        if (tid < head) acc = P::combine(acc, P::lift(prologue<T, AFFINE>(src[tid], p.a, p.b), vidx(tid)));
        const uint64_t nvec = (n - head) >> 2;
        using V = typename Vec4<T>::type;
        const V *vsrc = (const V *)(src + head);
        uint64_t vi = tid;
        for (; vi + (UNROLL - 1) * nthreads < nvec; vi += UNROLL * nthreads) {
            V v[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) v[u] = load_vec<NT>(&vsrc[vi + u * nthreads]);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u)
                acc = P::combine(acc, fold4<P, T, AFFINE>(v[u], vidx(head + 4 * (vi + u * nthreads)), rev, p.a, p.b));
        }
        for (; vi < nvec; vi += nthreads)
            acc = P::combine(acc, fold4<P, T, AFFINE>(load_vec<NT>(&vsrc[vi]), vidx(head + 4 * vi), rev, p.a, p.b));
        const uint64_t tail0 = head + 4 * nvec;
        if (tail0 + tid < n) {
            const uint64_t e = tail0 + tid;
            acc = P::combine(acc, P::lift(prologue<T, AFFINE>(src[e], p.a, p.b), vidx(e)));
        }
    } else {
        constexpr int W = Walkers<MODE>::value;
        const RowsGeom &g = p.g;
        const T *src = (const T *)p.base;
        const uint64_t items = g.rows * g.units;
        RowWalker w[W];
#pragma unroll
        for (int k = 0; k < W; ++k) w[k].init(g, (int64_t)p.offset, 0, tid + (uint64_t)k * nthreads);
        for (uint64_t j = tid; j < items; j += (uint64_t)W * nthreads) {
            T x[W][4];
            uint32_t cnt[W];
#pragma unroll
            for (int k = 0; k < W; ++k)
                cnt[k] = (j + (uint64_t)k * nthreads < items) ? load_unit<T, MODE, NT>(g, src, w[k], x[k]) : 0u;
#pragma unroll
            for (int k = 0; k < W; ++k) {
                if (cnt[k] != 0u)
                    acc = P::combine(acc, fold_n<P, T, AFFINE>(x[k], cnt[k], (uint64_t)w[k].off2, (uint64_t)g.cstride2,
                                                               p.a, p.b));
                w[k].advance(g);
            }
        }
    }
    return acc;
}

template <typename T, int K, bool AFFINE, int MODE, int UNROLL = 2, bool NT = true>
__global__ __launch_bounds__(kBlock) void full_reduce_kernel(FullParams p) {
    using P = Policy<T, K>;
    using Acc = typename P::Acc;
    using Slot = PartialSlot<Acc>;
    __shared__ Acc lds[kBlock / kWave];
    __shared__ Acc vals[kMaxBlocks];
    __shared__ uint32_t missing[kMaxBlocks / 32];

    const uint32_t G = gridDim.x;
    const uint32_t last = G - 1;
    const Acc part = block_reduce<P>(thread_fold<P, T, AFFINE, MODE, UNROLL, NT>(p, blockIdx.x, G), lds);
    if (blockIdx.x != last) {
        if (threadIdx.x == 0) Slot::publish(p.slots + (uint64_t)blockIdx.x * Slot::kWords, p.tag, part);
        return;
    }

    // The last block gathers every partial into LDS ...
    gather_partials<kBlock, kMaxBlocks>(p.slots, p.tag, p.poll_limit, G, part, vals, missing, [&](uint32_t k) {
        return block_reduce<P>(thread_fold<P, T, AFFINE, MODE, UNROLL, NT>(p, k, G), lds);
    });
    // ... and folds them in index order: thread t takes t, t + 256, ...
    Acc r = P::identity();
    for (uint32_t k = threadIdx.x; k < G; k += kBlock) r = P::combine(r, vals[k]);
    r = block_reduce<P>(r, lds);
    if (threadIdx.x == 0) write_result_impl<T, K>(p, r);
}

// n == 0: the result is the operator identity (ops.rs:926-983); empty
// argmax has no index.
template <typename T, int K> __global__ void full_reduce_empty_kernel(FullParams p) {
    using P = Policy<T, K>;
    if (threadIdx.x == 0 && blockIdx.x == 0) write_result_impl<T, K>(p, P::identity());
}

template <typename T, int K, bool AFFINE>
hx_status launch_typed(const FullReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    FullParams p{};
    p.base = a.base;
    p.n = a.n;
    p.offset = a.flat ? a.flat_offset : a.layout.offset;
    p.a = a.a;
    p.b = a.b;
    p.out_value = a.out_value;
    p.out_index = a.out_index;
    p.slots = (uint64_t *)((char *)ws + kLookbackOffset);
    p.poll_limit = gather_poll_limit();
    p.idx_last = a.n - 1;
    p.rev = a.reversed ? 1u : 0u;
    if (a.n == 0) {
        if constexpr (K == kMean) {
            return fail(HX_ERR_DISPATCH_FAILED, "mean is undefined for an empty operand");
        } else {
            hipLaunchKernelGGL((full_reduce_empty_kernel<T, K>), dim3(1), dim3(64), 0, stream, p);
            return check_launch("full_reduce_empty_kernel");
        }
    }
    const uint32_t blocks = full_reduce_blocks(a.n, std::is_same<T, float>::value);
    if (ws_bytes < full_reduce_workspace_bytes(a.n))
        return fail(HX_ERR_DISPATCH_FAILED, "full-reduction workspace of %llu bytes is below %llu",
                    (unsigned long long)ws_bytes, (unsigned long long)full_reduce_workspace_bytes(a.n));
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    if (a.flat) {
        hipLaunchKernelGGL((full_reduce_kernel<T, K, AFFINE, kFlat>), dim3(blocks), dim3(kBlock), 0, stream, p);
    } else {
        const RowsView rv = a.memory_order ? layout_rows_memory_order(a.layout) : layout_rows(a.layout);
        const bool vec = rv.cstride == 1 && rv.cols >= 4;
        p.g = rows_geom(rv, vec, (uint64_t)(vec ? Walkers<kRowsVec>::value : Walkers<kRowsScalar>::value) *
                                     blocks * kBlock);
        if (vec)
            hipLaunchKernelGGL((full_reduce_kernel<T, K, AFFINE, kRowsVec>), dim3(blocks), dim3(kBlock), 0, stream,
                               p);
        else
            hipLaunchKernelGGL((full_reduce_kernel<T, K, AFFINE, kRowsScalar>), dim3(blocks), dim3(kBlock), 0,
                               stream, p);
    }
    HX_TRY(check_launch("full_reduce_kernel"));
    commit_lookback_launch(lb);
    return HX_OK;
}

template <typename T, bool AFFINE>
hx_status launch_kind(const FullReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    switch (a.op) {
    case HX_OP_SUM: return launch_typed<T, kSum, AFFINE>(a, ws, ws_bytes, lb, stream);
    case HX_OP_PROD: return launch_typed<T, kProd, AFFINE>(a, ws, ws_bytes, lb, stream);
    case HX_OP_MIN: return launch_typed<T, kMin, AFFINE>(a, ws, ws_bytes, lb, stream);
    case HX_OP_MAX: return launch_typed<T, kMax, AFFINE>(a, ws, ws_bytes, lb, stream);
    case HX_OP_ARGMAX: return launch_typed<T, kArgmax, AFFINE>(a, ws, ws_bytes, lb, stream);
    case HX_OP_MEAN: return launch_typed<T, kMean, AFFINE>(a, ws, ws_bytes, lb, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown reduction operator %d", (int)a.op);
}

} // namespace

// Two 64-bit slot words per block (the widest partial) after the header,
// where every tagged status word of a workspace lives; sized for the larger
// (integer) grid, whatever the element type.
uint64_t full_reduce_workspace_bytes(uint64_t n) {
    return kLookbackOffset + (uint64_t)full_reduce_blocks(n, false) * 16;
}

// High half of a tagged word as the kernels build it (the host-side copy of
// the same inline functions): kind 0 a look-back status with `flag`, kind 1
// a partial slot.
uint32_t tagged_word_hi(uint32_t kind, uint32_t tag, uint32_t flag) {
    return kind == 0 ? status_word_hi(tag, flag) : slot_word_hi(tag);
}

hx_status launch_full_reduce(const FullReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb,
                             hipStream_t stream) {
    switch (a.dtype) {
    case HX_DTYPE_F32:
        return a.affine ? launch_kind<float, true>(a, ws, ws_bytes, lb, stream)
                        : launch_kind<float, false>(a, ws, ws_bytes, lb, stream);
    case HX_DTYPE_U32: return launch_kind<uint32_t, false>(a, ws, ws_bytes, lb, stream);
    case HX_DTYPE_I32: return launch_kind<int32_t, false>(a, ws, ws_bytes, lb, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)a.dtype);
}

} // namespace hx

extern "C" uint32_t hx_debug_tagged_word_hi(uint32_t kind, uint32_t tag, uint32_t flag) {
    return hx::tagged_word_hi(kind, tag, flag);
}
