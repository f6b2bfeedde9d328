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
#include "rows_walk.hpp"

#include <type_traits>
#include <utility>

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
    RowsGeom g;            // non-flat views: rows of a, form 2 walks b
    // kPairTile: a is contiguous along the rows, (k, i, j) at a_off + k *
    // col_bs + i + j * col_ld; b along the columns, (k, i, j) at b_off + k *
    // row_bs + i * row_ld + j, for matrices k of a batch.
    uint64_t rows, cols, tiles, tiles_c, tiles_m;
    int64_t col_ld, row_ld, col_bs, row_bs;
    void *out;
    uint64_t *slots;     // partial slots (PartialSlot), 16 bytes per block
    uint32_t tag;        // this launch's tag
    uint32_t poll_limit; // gather polls per partial before recomputing it
};
// How the operands are walked: flat element ranges, or rows (RowsGeom) of
// 16-byte vector units (both operands' rows contiguous) or of single
// elements, or (a dot of a transposed matrix with a row-major one) 64 x 64
// tiles, the transposed operand's tile turned through LDS.
enum Mode { kFlat = 0, kRowsVec = 1, kRowsScalar = 2, kPairTile = 3 };
// Tile edge of kPairTile and the LDS pitch of its staged tile: column j of
// the tile at j * 65, so the 16 columns a wave reads at one row fall in
// distinct banks.
constexpr int kPairEdge = 64;
constexpr int kPairPitch = kPairEdge + 1;
// Units in flight per thread in the row modes: two for a dot (two loads per
// unit; four walkers took 113 VGPRs against 80 and stride-2 dots 195 us
// against 185 at 2^27 pairs), four for one-operand maps.
template <bool TWO> struct MapWalkers { static constexpr int value = TWO ? 2 : 4; };

// Unit of walker `w` of operand a (and b): elements in x, y[0..count).
template <typename T, int MODE, bool TWO>
__device__ __forceinline__ uint32_t load_pair(const RowsGeom &g, const T *a, const T *b, const RowWalker &w,
                                              T (&x)[4], T (&y)[4]) {
    if constexpr (MODE == kRowsVec) {
        using V = typename Vec4A4<T>::type;
        const uint64_t c0 = 4 * w.unit;
        if (c0 + 4 <= g.cols) {
            const V q = load_a4<true>((const V *)(a + w.off));
            x[0] = (T)q.x;
            x[1] = (T)q.y;
            x[2] = (T)q.z;
            x[3] = (T)q.w;
            if constexpr (TWO) {
                const V r = load_a4<true>((const V *)(b + w.off2));
                y[0] = (T)r.x;
                y[1] = (T)r.y;
                y[2] = (T)r.z;
                y[3] = (T)r.w;
            }
            return 4;
        }
        // Every slot is written on both paths: stores of some slots only
        // get merged into one store at a run-time index, which keeps the
        // arrays in scratch memory.
        const uint32_t cnt = (uint32_t)(g.cols - c0);
#pragma unroll
        for (uint32_t c = 0; c < 4; ++c) {
            x[c] = c < cnt ? a[w.off + c] : T(0);
            if constexpr (TWO) y[c] = c < cnt ? b[w.off2 + c] : T(0);
        }
        return cnt;
    } else {
        x[0] = a[w.off];
        if constexpr (TWO) y[0] = b[w.off2];
        return 1;
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

// map_thread_fold: the fold of thread threadIdx.x of "block" vb of a
// G-block grid (the last block calls it with another block's index to
// recompute a missing partial).
// kFlat: both operands are the contiguous ranges [a_off, +n) and
// [b_off, +n) (b is ignored for one-operand maps).  The head peel aligns a;
// b's vectors need only 4-byte alignment (Vec4A4), so the operands may sit
// at any element offsets from each other.
// Row modes: a's rows walked with b's offsets as the second form
// (layout_rows_pair), MapWalkers units in flight.
// kPairTile: block vb takes tiles vb, vb + G, ... (the tiles of matrix k of
// a batch follow those of matrix k - 1); each thread loads four
// 16-byte vectors of the tile's columns of a (16 lanes a column) and four of
// its rows of b (16 lanes a row), parks a's vectors in `tile` (column j at
// j * kPairPitch) and pairs each element of b with the tile's (i, j).  Tiles
// on the right or bottom edge load and pair only elements inside the
// matrix.
template <typename T, int M, int MODE>
__device__ __forceinline__ typename MapPolicy<T, M>::Acc map_thread_fold(const MapParams &p, uint32_t vb, uint32_t G,
                                                                        T *tile) {
    using P = MapPolicy<T, M>;
    using Acc = typename P::Acc;
    using V = typename Vec4A4<T>::type;
    constexpr bool kTwo = M == kMapDot;
    const uint64_t n = p.n;
    const uint64_t tid = (uint64_t)vb * kBlock + threadIdx.x;
    const uint64_t nthreads = (uint64_t)G * kBlock;
    Acc acc = P::identity();
    if constexpr (MODE == kFlat) {
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
    } else if constexpr (MODE == kPairTile) {
        const T *a0 = (const T *)p.a + p.a_off;
        const T *b0 = (const T *)p.b + p.b_off;
        const uint32_t q4 = 4 * (threadIdx.x & 15), r16 = threadIdx.x >> 4;
        for (uint64_t tb = vb; tb < p.tiles; tb += G) {
            const uint64_t mk = tb / p.tiles_m, tm = tb - mk * p.tiles_m;
            const T *a = a0 + (int64_t)mk * p.col_bs;
            const T *b = b0 + (int64_t)mk * p.row_bs;
            const uint64_t i0 = tm / p.tiles_c * kPairEdge, j0 = tm % p.tiles_c * kPairEdge;
            const bool full = i0 + kPairEdge <= p.rows && j0 + kPairEdge <= p.cols;
            T x[4][4], y[4][4];
            if (full) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const V u = load_a4<true>((const V *)(a + (i0 + q4) + (j0 + r16 + 16 * k) * p.col_ld));
                    const V w = load_a4<true>((const V *)(b + (i0 + r16 + 16 * k) * p.row_ld + j0 + q4));
                    x[k][0] = (T)u.x, x[k][1] = (T)u.y, x[k][2] = (T)u.z, x[k][3] = (T)u.w;
                    y[k][0] = (T)w.x, y[k][1] = (T)w.y, y[k][2] = (T)w.z, y[k][3] = (T)w.w;
                }
            } else {
                // Edge tiles.  Every lane issues its vector loads, so they
                // are in flight together as in a full tile: a vector not
                // wholly inside the matrix is read as the matrix's first
                // vector (elements (0..3, 0) of a, (0, 0..3) of b: inside,
                // as both extents are at least kPairMinEdge) and dropped.
                // The vector of a line that straddles the matrix's edge is
                // then read element by element.
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint64_t jc = j0 + r16 + 16 * k, ir = i0 + r16 + 16 * k;
                    const bool wa = jc < p.cols && i0 + q4 + 4 <= p.rows;
                    const bool wb = ir < p.rows && j0 + q4 + 4 <= p.cols;
                    const V u = load_a4<true>((const V *)(wa ? a + (i0 + q4) + jc * p.col_ld : a));
                    const V w = load_a4<true>((const V *)(wb ? b + ir * p.row_ld + j0 + q4 : b));
                    x[k][0] = wa ? (T)u.x : T(0), x[k][1] = wa ? (T)u.y : T(0);
                    x[k][2] = wa ? (T)u.z : T(0), x[k][3] = wa ? (T)u.w : T(0);
                    y[k][0] = wb ? (T)w.x : T(0), y[k][1] = wb ? (T)w.y : T(0);
                    y[k][2] = wb ? (T)w.z : T(0), y[k][3] = wb ? (T)w.w : T(0);
                }
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint64_t jc = j0 + r16 + 16 * k, ir = i0 + r16 + 16 * k;
                    if (jc < p.cols && i0 + q4 < p.rows && i0 + q4 + 4 > p.rows) {
                        const T *pa = a + (i0 + q4) + jc * p.col_ld;
#pragma unroll
                        for (int c = 0; c < 3; ++c) x[k][c] = i0 + q4 + c < p.rows ? pa[c] : T(0);
                    }
                    if (ir < p.rows && j0 + q4 < p.cols && j0 + q4 + 4 > p.cols) {
                        const T *pb = b + ir * p.row_ld + j0 + q4;
#pragma unroll
                        for (int c = 0; c < 3; ++c) y[k][c] = j0 + q4 + c < p.cols ? pb[c] : T(0);
                    }
                }
            }
            __syncthreads(); // the previous tile's reads of `tile` are done
#pragma unroll
            for (int k = 0; k < 4; ++k)
#pragma unroll
                for (int c = 0; c < 4; ++c) tile[(r16 + 16 * k) * kPairPitch + q4 + c] = x[k][c];
            __syncthreads();
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t il = r16 + 16 * k;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const T t = tile[(q4 + c) * kPairPitch + il];
                    if (full || (i0 + il < p.rows && j0 + q4 + c < p.cols)) acc = P::combine(acc, P::elem(t, y[k][c]));
                }
            }
        }
    } else {
        // Rows (RowsGeom): kWalkers walkers, each stepping kWalkers * nthreads units.
        const RowsGeom &g = p.g;
        const T *a = (const T *)p.a;
        const T *b = kTwo ? (const T *)p.b : a;
        const uint64_t items = g.rows * g.units;
        constexpr int kWalkers = MapWalkers<kTwo>::value;
        RowWalker w[kWalkers];
#pragma unroll
        for (int k = 0; k < kWalkers; ++k)
            w[k].init(g, (int64_t)p.a_off, (int64_t)p.b_off, tid + (uint64_t)k * nthreads);
        for (uint64_t j = tid; j < items; j += (uint64_t)kWalkers * nthreads) {
            T x[kWalkers][4], y[kWalkers][4];
            uint32_t cnt[kWalkers];
#pragma unroll
            for (int k = 0; k < kWalkers; ++k)
                cnt[k] = (j + (uint64_t)k * nthreads < items) ? load_pair<T, MODE, kTwo>(g, a, b, w[k], x[k], y[k])
                                                                : 0u;
#pragma unroll
            for (int k = 0; k < kWalkers; ++k) {
#pragma unroll
                for (uint32_t c = 0; c < 4; ++c)
                    if (c < cnt[k]) acc = P::combine(acc, P::elem(x[k][c], kTwo ? y[k][c] : x[k][c]));
                w[k].advance(g);
            }
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

template <typename T, int M, int MODE>
__global__ __launch_bounds__(kBlock) void map_reduce_kernel(MapParams p) {
    using P = MapPolicy<T, M>;
    using Acc = typename P::Acc;
    using Slot = PartialSlot<Acc>;
    __shared__ Acc lds[kBlock / kWave];
    __shared__ Acc vals[kMaxBlocks];
    __shared__ uint32_t missing[kMaxBlocks / 32];
    __shared__ T tile[MODE == kPairTile ? kPairEdge * kPairPitch : 1];
    const uint32_t G = gridDim.x;
    const Acc part = block_reduce<P>(map_thread_fold<T, M, MODE>(p, blockIdx.x, G, tile), lds);
    if (blockIdx.x + 1 != G) {
        if (threadIdx.x == 0) Slot::publish(p.slots + (uint64_t)blockIdx.x * Slot::kWords, p.tag, part);
        return;
    }
    gather_partials<kBlock, kMaxBlocks>(p.slots, p.tag, p.poll_limit, G, part, vals, missing, [&](uint32_t k) {
        return block_reduce<P>(map_thread_fold<T, M, MODE>(p, k, G, tile), lds);
    });
    Acc r = P::identity();
    for (uint32_t k = threadIdx.x; k < G; k += kBlock) r = P::combine(r, vals[k]);
    r = block_reduce<P>(r, lds);
    if (threadIdx.x == 0) write_map_result<T, M>(p, r);
}

template <typename T, int M> __global__ void map_reduce_empty_kernel(MapParams p) {
    if (threadIdx.x == 0 && blockIdx.x == 0) write_map_result<T, M>(p, MapPolicy<T, M>::identity());
}

// Smallest extent the tiled pairing takes (narrower matrices are walked as
// rows).
constexpr uint64_t kPairMinEdge = 16;

// One block per 4096 elements up to 768 (the full reduction's grid rule).
uint32_t map_blocks(uint64_t n) {
    uint64_t blocks = ceil_div(n, 4096);
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
    PairTranspose pt;
    if (a.flat) {
        hipLaunchKernelGGL((map_reduce_kernel<T, M, kFlat>), dim3(blocks), dim3(kBlock), 0, stream, p);
    } else if (M == kMapDot && layout_pair_transposed(a.a_layout, a.b_layout, &pt) && pt.rows >= kPairMinEdge &&
               pt.cols >= kPairMinEdge) {
        // The product is symmetric, so the operand contiguous along the
        // rows goes first.
        if (!pt.a_is_col) {
            std::swap(p.a, p.b);
            std::swap(p.a_off, p.b_off);
        }
        p.rows = pt.rows;
        p.cols = pt.cols;
        p.tiles_c = ceil_div(pt.cols, (uint64_t)kPairEdge);
        p.tiles_m = ceil_div(pt.rows, (uint64_t)kPairEdge) * p.tiles_c;
        p.tiles = pt.batch * p.tiles_m;
        p.col_bs = pt.col_bs;
        p.row_bs = pt.row_bs;
        p.col_ld = pt.col_ld;
        p.row_ld = pt.row_ld;
        hipLaunchKernelGGL((map_reduce_kernel<T, M, M == kMapDot ? kPairTile : kRowsScalar>), dim3(blocks),
                           dim3(kBlock), 0, stream, p);
    } else {
        const RowsView rv = layout_rows_pair(a.a_layout, M == kMapDot ? a.b_layout : a.a_layout);
        const bool vec = rv.cstride == 1 && rv.cstride2 == 1 && rv.cols >= 4;
        p.g = rows_geom(rv, vec, (uint64_t)MapWalkers<M == kMapDot>::value * blocks * kBlock);
        if (vec)
            hipLaunchKernelGGL((map_reduce_kernel<T, M, kRowsVec>), dim3(blocks), dim3(kBlock), 0, stream, p);
        else
            hipLaunchKernelGGL((map_reduce_kernel<T, M, kRowsScalar>), dim3(blocks), dim3(kBlock), 0, stream, p);
    }
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
