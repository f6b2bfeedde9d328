// Map-reductions for gfx950: dot products, traces and norms
// (crates/hephaestus-rocm/src/application/linalg/norms.rs:32-490 with its
// maps IdentityMap, DotMap, AbsMap, SquareMap and MaxAbsMap).
//
// The reference maps and reduces one element per thread in a 256-wide LDS
// halving tree, one launch per tree pass, and takes the L2 square root in a
// further elementwise launch (norms.rs:466-477).  Here the map is fused into
// the same single-launch grid reduction as the full reduce:
//   * every block grid-strides over the operand(s) with 16-byte loads
//     (both operands of a dot when their alignment agrees), maps each
//     element, accumulates (f32 sums in f64: products and squares of f32
//     values are exact in f64) and publishes one partial as tagged slot
//     words (PartialSlot);
//   * the last block gathers the partials (gather_partials), folds them in
//     index order and writes the scalar, taking the square root of an L2
//     norm in the same launch.
// Integer sums and products wrap mod 2^32; |INT_MIN| is INT_MIN, as abs()
// on a two's-complement int.
#include "hx_device.hpp"
#include "hx_internal.hpp"

#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxBlocks = 768; // as the full reduce: 3 blocks per CU

enum MapKind { kMapSum = 0, kMapDot = 1, kMapAbsSum = 2, kMapSquareSum = 3, kMapAbsMax = 4 };

template <typename T> struct MapSumAcc { using type = uint32_t; };
template <> struct MapSumAcc<float> { using type = double; };

template <typename T> __device__ __forceinline__ uint32_t wrap_abs(T x) {
    if constexpr (std::is_same<T, int32_t>::value) return x < 0 ? 0u - (uint32_t)x : (uint32_t)x;
    else return (uint32_t)x;
}

// Element map and accumulation of each kind.
template <typename T, int M> struct MapPolicy {
    using Acc = typename MapSumAcc<T>::type;
    __device__ static Acc identity() { return Acc(0); }
    __device__ static Acc elem(T x, T y) {
        if constexpr (std::is_same<T, float>::value) {
            if constexpr (M == kMapSum) return (double)x;
            else if constexpr (M == kMapDot) return (double)x * (double)y;
            else if constexpr (M == kMapAbsSum) return (double)__builtin_fabsf(x);
            else return (double)x * (double)x;
        } else {
            if constexpr (M == kMapSum) return (uint32_t)x;
            else if constexpr (M == kMapDot) return (uint32_t)x * (uint32_t)y;
            else if constexpr (M == kMapAbsSum) return wrap_abs(x);
            else return (uint32_t)x * (uint32_t)x;
        }
    }
    __device__ static Acc combine(Acc a, Acc b) { return a + b; }
    __device__ static Acc wave(Acc a) { return wave_sum(a); }
};
// max |x| on order-preserving keys (NaN never wins, as HIP fmaxf); the
// MaxOp identity f32::MIN / i32::MIN / 0 is the empty result.
template <typename T> struct MapPolicy<T, kMapAbsMax> {
    using Acc = uint32_t;
    __device__ static Acc identity() { return Key<T>::max_identity(); }
    __device__ static Acc elem(T x, T) {
        if constexpr (std::is_same<T, float>::value) return f32_key_max(__builtin_fabsf(x));
        else return Key<T>::max_key((T)wrap_abs(x));
    }
    __device__ static Acc combine(Acc a, Acc b) { return a > b ? a : b; }
    __device__ static Acc wave(Acc a) { return wave_umax(a); }
};

struct MapParams {
    const void *a, *b;
    uint64_t n;
    uint64_t a_off, b_off; // element offsets (layout offsets)
    uint32_t rank;
    uint64_t shape[4];
    int64_t a_strides[4], b_strides[4];
    void *out;
    uint64_t *slots; // partial slots (PartialSlot), 16 bytes per block
    uint32_t tag;        // this launch's tag
    uint32_t poll_limit; // gather polls per partial before recomputing it
};

__device__ __forceinline__ void strided_pair(const MapParams &p, uint64_t i, int64_t &oa, int64_t &ob) {
    oa = (int64_t)p.a_off;
    ob = (int64_t)p.b_off;
    for (int d = (int)p.rank - 1; d >= 0; --d) {
        const uint64_t s = p.shape[d];
        const uint64_t q = i / s;
        const int64_t r = (int64_t)(i - q * s);
        oa += r * p.a_strides[d];
        ob += r * p.b_strides[d];
        i = q;
    }
}

template <typename P> __device__ __forceinline__ typename P::Acc block_reduce(typename P::Acc v, typename P::Acc *lds) {
    v = P::wave(v);
    if (lane_id() == 0) lds[threadIdx.x / kWave] = v;
    __syncthreads();
    typename P::Acc r = lds[0];
#pragma unroll
    for (int k = 1; k < kBlock / kWave; ++k) r = P::combine(r, lds[k]);
    __syncthreads(); // lds is reused by the next reduction
    return r;
}

// FLAT: both operands are the contiguous ranges [a_off, +n) and [b_off, +n)
// (b is ignored for one-operand maps).  The head peel aligns a; b's vectors
// need only 4-byte alignment (Vec4A4), so the operands may sit at any element
// offsets from each other.
// map_thread_fold: the fold of thread threadIdx.x of "block" vb of a
// G-block grid (the last block calls it with another block's index to
// recompute a missing partial).
template <typename T, int M, bool FLAT>
__device__ __forceinline__ typename MapPolicy<T, M>::Acc map_thread_fold(const MapParams &p, uint32_t vb, uint32_t G) {
    using P = MapPolicy<T, M>;
    using Acc = typename P::Acc;
    using V = typename Vec4A4<T>::type;
    constexpr bool kTwo = M == kMapDot;
    const uint64_t n = p.n;
    const uint64_t tid = (uint64_t)vb * kBlock + threadIdx.x;
    const uint64_t nthreads = (uint64_t)G * kBlock;
    Acc acc = P::identity();
    if constexpr (FLAT) {
        const T *a = (const T *)p.a + p.a_off;
        const T *b = kTwo ? (const T *)p.b + p.b_off : a;
        const uint64_t mis = ((uintptr_t)a >> 2) & 3u;
        uint64_t head = mis ? 4 - mis : 0;
        if (head > n) head = n;
        if (tid < head) acc = P::combine(acc, P::elem(a[tid], b[tid]));
        const uint64_t nvec = (n - head) >> 2;
        const V *va = (const V *)(a + head);
        const V *vb = (const V *)(b + head);
        uint64_t vi = tid;
        for (; vi + nthreads < nvec; vi += 2 * nthreads) {
            const V x0 = load_a4<true>(&va[vi]), x1 = load_a4<true>(&va[vi + nthreads]);
            V y0 = x0, y1 = x1;
            if constexpr (kTwo) {
                y0 = load_a4<true>(&vb[vi]);
                y1 = load_a4<true>(&vb[vi + nthreads]);
            }
            acc = P::combine(acc, P::combine(P::combine(P::elem(x0.x, y0.x), P::elem(x0.y, y0.y)),
                                             P::combine(P::elem(x0.z, y0.z), P::elem(x0.w, y0.w))));
            acc = P::combine(acc, P::combine(P::combine(P::elem(x1.x, y1.x), P::elem(x1.y, y1.y)),
                                             P::combine(P::elem(x1.z, y1.z), P::elem(x1.w, y1.w))));
        }
        if (vi < nvec) {
            const V x0 = load_a4<true>(&va[vi]);
            V y0 = x0;
            if constexpr (kTwo) y0 = load_a4<true>(&vb[vi]);
            acc = P::combine(acc, P::combine(P::combine(P::elem(x0.x, y0.x), P::elem(x0.y, y0.y)),
                                             P::combine(P::elem(x0.z, y0.z), P::elem(x0.w, y0.w))));
        }
        const uint64_t tail0 = head + 4 * nvec;
        if (tail0 + tid < n) acc = P::combine(acc, P::elem(a[tail0 + tid], b[tail0 + tid]));
    } else {
        const T *a = (const T *)p.a;
        const T *b = kTwo ? (const T *)p.b : a;
        for (uint64_t i = tid; i < n; i += nthreads) {
            int64_t oa, ob;
            strided_pair(p, i, oa, ob);
            acc = P::combine(acc, P::elem(a[oa], kTwo ? b[ob] : a[oa]));
        }
    }
    return acc;
}

template <typename T, int M> __device__ __forceinline__ void write_map_result(const MapParams &p, typename MapPolicy<T, M>::Acc r) {
    if constexpr (M == kMapAbsMax) {
        *(T *)p.out = Key<T>::decode(r);
    } else if constexpr (M == kMapSquareSum && std::is_same<T, float>::value) {
        *(float *)p.out = (float)__builtin_sqrt(r); // sqrt of the f64 sum, rounded once more to f32
    } else {
        *(T *)p.out = (T)r;
    }
}

template <typename T, int M, bool FLAT>
__global__ __launch_bounds__(kBlock) void map_reduce_kernel(MapParams p) {
    using P = MapPolicy<T, M>;
    using Acc = typename P::Acc;
    using Slot = PartialSlot<Acc>;
    __shared__ Acc lds[kBlock / kWave];
    __shared__ Acc vals[kMaxBlocks];
    __shared__ uint32_t missing[kMaxBlocks / 32];
    const uint32_t G = gridDim.x;
    const Acc part = block_reduce<P>(map_thread_fold<T, M, FLAT>(p, blockIdx.x, G), lds);
    if (blockIdx.x + 1 != G) {
        if (threadIdx.x == 0) Slot::publish(p.slots + (uint64_t)blockIdx.x * Slot::kWords, p.tag, part);
        return;
    }
    gather_partials<kBlock, kMaxBlocks>(p.slots, p.tag, p.poll_limit, G, part, vals, missing, [&](uint32_t k) {
        return block_reduce<P>(map_thread_fold<T, M, FLAT>(p, k, G), lds);
    });
    Acc r = P::identity();
    for (uint32_t k = threadIdx.x; k < G; k += kBlock) r = P::combine(r, vals[k]);
    r = block_reduce<P>(r, lds);
    if (threadIdx.x == 0) write_map_result<T, M>(p, r);
}

template <typename T, int M> __global__ void map_reduce_empty_kernel(MapParams p) {
    if (threadIdx.x == 0 && blockIdx.x == 0) write_map_result<T, M>(p, MapPolicy<T, M>::identity());
}

uint32_t map_blocks(uint64_t n) {
    uint64_t blocks = ceil_div(n, 2048);
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    return blocks < 1 ? 1u : (uint32_t)blocks;
}

template <typename T, int M>
hx_status launch_typed(const MapReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    MapParams p{};
    p.a = a.a;
    p.b = a.b;
    p.n = a.n;
    p.a_off = a.a_layout.offset;
    p.b_off = a.b_layout.offset;
    p.rank = a.a_layout.rank;
    for (uint32_t d = 0; d < 4; ++d) {
        p.shape[d] = d < a.a_layout.rank ? a.a_layout.shape[d] : 1;
        p.a_strides[d] = d < a.a_layout.rank ? a.a_layout.strides[d] : 0;
        p.b_strides[d] = d < a.b_layout.rank ? a.b_layout.strides[d] : 0;
    }
    p.out = a.out;
    p.slots = (uint64_t *)((char *)ws + kLookbackOffset);
    p.poll_limit = gather_poll_limit();
    if (a.n == 0) {
        hipLaunchKernelGGL((map_reduce_empty_kernel<T, M>), dim3(1), dim3(64), 0, stream, p);
        return check_launch("map_reduce_empty_kernel");
    }
    const uint32_t blocks = map_blocks(a.n);
    if (ws_bytes < map_reduce_workspace_bytes(a.n))
        return fail(HX_ERR_DISPATCH_FAILED, "map-reduction workspace of %llu bytes is below %llu",
                    (unsigned long long)ws_bytes, (unsigned long long)map_reduce_workspace_bytes(a.n));
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    if (a.flat)
        hipLaunchKernelGGL((map_reduce_kernel<T, M, true>), dim3(blocks), dim3(kBlock), 0, stream, p);
    else
        hipLaunchKernelGGL((map_reduce_kernel<T, M, false>), dim3(blocks), dim3(kBlock), 0, stream, p);
    HX_TRY(check_launch("map_reduce_kernel"));
    commit_lookback_launch(lb);
    return HX_OK;
}

template <typename T>
hx_status launch_kind(const MapReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    switch (a.map) {
    case HX_MAP_SUM: return launch_typed<T, kMapSum>(a, ws, ws_bytes, lb, stream);
    case HX_MAP_DOT: return launch_typed<T, kMapDot>(a, ws, ws_bytes, lb, stream);
    case HX_MAP_NORM_L1: return launch_typed<T, kMapAbsSum>(a, ws, ws_bytes, lb, stream);
    case HX_MAP_NORM_L2: return launch_typed<T, kMapSquareSum>(a, ws, ws_bytes, lb, stream);
    case HX_MAP_NORM_MAX: return launch_typed<T, kMapAbsMax>(a, ws, ws_bytes, lb, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown map-reduction %d", (int)a.map);
}

} // namespace

// Two 64-bit slot words per block after the header, where every tagged
// status word of a workspace lives.
uint64_t map_reduce_workspace_bytes(uint64_t n) { return kLookbackOffset + (uint64_t)map_blocks(n) * 16; }

hx_status launch_map_reduce(const MapReduceArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb,
                            hipStream_t stream) {
    switch (a.dtype) {
    case HX_DTYPE_F32: return launch_kind<float>(a, ws, ws_bytes, lb, stream);
    case HX_DTYPE_U32: return launch_kind<uint32_t>(a, ws, ws_bytes, lb, stream);
    case HX_DTYPE_I32: return launch_kind<int32_t>(a, ws, ws_bytes, lb, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)a.dtype);
}

} // namespace hx
