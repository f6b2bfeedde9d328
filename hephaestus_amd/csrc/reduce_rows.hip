// Row-wise and axis reductions for gfx950: AxisReductionOps
// (crates/hephaestus-core/src/domain/reduction.rs:74-223) plus the fused
// row reduce: sum, max and argmax of y = fmaf(a, x, b) out of ONE read of
// each row.
//
// The reference runs one thread per output with a serial loop along the
// axis (crates/hephaestus-rocm/src/application/axis_reduction.rs:16-65): for
// a row-major matrix reduced along axis 1, neighbouring lanes are a whole
// row apart, so no load is coalesced, and sum and max are two full passes.
// Here:
//   rows_kernel        a group of G lanes per row (4 to 256, about four
//                      16-byte vectors per lane): lane l of the group reads
//                      vectors l, l+G, ... of the row, keeps every requested
//                      statistic in registers, then the group combines them
//                      with DPP reductions (and LDS across waves).  Rows that
//                      do not start on a 16-byte boundary take their 0-3
//                      leading and trailing elements one per lane.  Used
//                      whenever the reduced axis has unit stride (or no
//                      stride is unit).
//   rows_split_kernel  the same for few long rows: one wave per (row, chunk),
//                      chunk statistics to partial planes.
//   rows_tile_kernel   rows of 1 to 255 elements, back to back or a little
//                      apart: a block stages a tile of whole rows in LDS
//                      with 16-byte loads, then folds each row with one
//                      thread or a group of 2 to 8 lanes.
//   cols_tiles_kernel  the outputs are adjacent and the reduced axis strided
//                      (axis-0 reduction of a row-major matrix): a wave owns
//                      256 adjacent outputs (one 16-byte load per lane per
//                      line) and a chunk of the axis, so the chip gets
//                      thousands of waves however tall the matrix is.
//   cols_block_kernel  small column reductions in one launch (slices of the
//                      axis folded through LDS).
//   cols_period_kernel axis 0 of dense matrices with 2 to 95 columns, read
//                      as one contiguous range of 1 KiB wave loads.
//   split_fold_kernel  folds the chunk partials of either split form in a
//                      fixed order, so f32 sums do not depend on scheduling.
#include "hx_device.hpp"
#include "hx_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;

enum Flag : int {
    F_SUM = 1,
    F_MAX = 2,
    F_ARG = 4,
    F_MIN = 8,
    F_PROD = 16,
    F_MEAN = 32,
};

// Waves per fold block (split_fold_kernel, cols_block_kernel), and the most
// statistic planes a reduction keeps (sum or mean, product, max or argmax,
// min).
constexpr int kFoldSlices = 16;
constexpr int kMaxPlanes = 4;

struct RowParams {
    const void *base;
    uint64_t rows, cols;
    int64_t row_stride, col_stride;
    uint64_t offset;
    float a, b;
    void *out_sum;  // SUM or MEAN
    void *out_max;
    uint32_t *out_arg;
    void *out_min;
    void *out_prod;
    int64_t out_stride;
    uint64_t out_offset;
    uint64_t row0 = 0; // rows_kernel: row of block 0's first group (launched in batches)
};

template <typename T, bool AFFINE> __device__ __forceinline__ T prologue(T x, float, float) { return x; }
template <> __device__ __forceinline__ float prologue<float, true>(float x, float a, float b) {
    return __builtin_fmaf(a, x, b);
}

template <typename T> struct Acc;
template <> struct Acc<float> { using sum = double; using prod = double; };
template <> struct Acc<uint32_t> { using sum = uint32_t; using prod = uint32_t; };
template <> struct Acc<int32_t> { using sum = uint32_t; using prod = uint32_t; };

// Running statistics of one lane (or thread).
template <typename T, int FLAGS> struct Stats {
    using S = typename Acc<T>::sum;
    using Pr = typename Acc<T>::prod;
    S sum = S(0);
    Pr prod = Pr(1);
    uint32_t maxk = Key<T>::max_identity();
    uint32_t mink = Key<T>::min_identity();
    uint64_t arg = 0ull;

    __device__ __forceinline__ void visit(T y, uint32_t j) {
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum += (S)(typename Wrap<T>::type)y;
        if constexpr ((FLAGS & F_PROD) != 0) prod *= (Pr)(typename Wrap<T>::type)y;
        if constexpr ((FLAGS & F_ARG) != 0) {
            arg = umax64(arg, pack_arg(Key<T>::max_key(y), j));
        } else if constexpr ((FLAGS & F_MAX) != 0) {
            uint32_t k = Key<T>::max_key(y);
            maxk = maxk > k ? maxk : k;
        }
        if constexpr ((FLAGS & F_MIN) != 0) {
            uint32_t k = Key<T>::min_key(y);
            mink = mink < k ? mink : k;
        }
    }
    // Sixteen elements of one lane's trip through a unit-stride row: y[e]
    // has index jt + 4*(e/4)*G + e%4, so e ascends with the index.
    //  - f32 sums: each vector's four values are added pairwise in f32 (two
    //    roundings, at most 2*eps_f32 of their magnitudes) and the four
    //    vector sums are added in f64.  A trip whose total is not finite is
    //    redone element by element in f64, so f32 overflow inside a pair
    //    never changes a result.
    //  - f32 max/argmax: signed keys (one shift and one bit-op per element)
    //    and a max over the trip, then one equality search for the first
    //    index holding it.  Per element that is about half the VALU work of
    //    a 64-bit (key, index) compare per element.  With the per-element
    //    form, 65536 x 4096 rows started at 155 us per launch and rose to
    //    about 195 us a few milliseconds into a sustained run (the clocks
    //    backing off under the extra VALU power) before settling near 160;
    //    this form holds 151-158 us throughout.
    template <int G> __device__ __forceinline__ void visit_trip(const T (&y)[16], uint32_t jt) {
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) {
            if constexpr (std::is_same<T, float>::value) {
                double q[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) q[u] = (double)((y[4 * u] + y[4 * u + 1]) + (y[4 * u + 2] + y[4 * u + 3]));
                double t = (q[0] + q[1]) + (q[2] + q[3]);
                if (!__builtin_isfinite(t)) {
                    // An f32 pair sum overflowed (or the trip holds inf or
                    // NaN): redo the trip in f64, as the per-element path.
                    t = 0.0;
#pragma unroll
                    for (int e = 0; e < 16; ++e) t += (double)y[e];
                }
                sum += t;
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) sum += (S)(typename Wrap<T>::type)y[e];
            }
        }
        if constexpr ((FLAGS & F_PROD) != 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) prod *= (Pr)(typename Wrap<T>::type)y[e];
        }
        if constexpr ((FLAGS & (F_ARG | F_MAX)) != 0) {
            if constexpr (std::is_same<T, float>::value) {
                int32_t ks[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) ks[e] = signed_key(y[e]);
                int32_t tk = ks[0];
#pragma unroll
                for (int e = 1; e < 16; ++e) tk = tk > ks[e] ? tk : ks[e];
                if (tk > kSignedPosInf) {
                    // A NaN with the sign bit clear: the max of the rest.
                    tk = INT32_MIN;
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int32_t k = ks[e] > kSignedPosInf ? INT32_MIN : ks[e];
                        tk = tk > k ? tk : k;
                    }
                }
                // Below -inf: only NaNs with the sign bit set (or none).
                if (tk >= kSignedNegInf) {
                    const uint32_t k = (uint32_t)tk ^ 0x80000000u;  // max_key of that value
                    if constexpr ((FLAGS & F_ARG) != 0) {
                        uint32_t tl = (uint32_t)(4 * 3 * G + 3);
#pragma unroll
                        for (int e = 14; e >= 0; --e) tl = ks[e] == tk ? (uint32_t)(4 * (e / 4) * G + e % 4) : tl;
                        arg = umax64(arg, pack_arg(k, jt + tl));
                    } else {
                        maxk = maxk > k ? maxk : k;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    if constexpr ((FLAGS & F_ARG) != 0) {
                        arg = umax64(arg, pack_arg(Key<T>::max_key(y[e]), jt + (uint32_t)(4 * (e / 4) * G + e % 4)));
                    } else {
                        const uint32_t k = Key<T>::max_key(y[e]);
                        maxk = maxk > k ? maxk : k;
                    }
                }
            }
        }
        if constexpr ((FLAGS & F_MIN) != 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t k = Key<T>::min_key(y[e]);
                mink = mink < k ? mink : k;
            }
        }
    }
    // f32 bits ^ (sign ? 0x7FFFFFFF : 0): as int32 this orders like the
    // value (-0 < +0), with NaNs above +inf (sign clear) or below -inf (sign
    // set); XOR 0x80000000 turns it into max_key of the same value.
    static constexpr int32_t kSignedPosInf = 0x7F800000;
    static constexpr int32_t kSignedNegInf = (int32_t)0x807FFFFF;
    static __device__ __forceinline__ int32_t signed_key(float y) {
        const int32_t b = __float_as_int(y);
        return b ^ ((b >> 31) & 0x7FFFFFFF);
    }
    // Combine the statistics of each aligned group of G lanes (4, 16 or 64)
    // with DPP reductions; every lane of the wave must be active.
    // G = 1 (a thread per row) has nothing to combine.
    template <int G> __device__ __forceinline__ void group_combine() {
        if constexpr (G > 1) {
            if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum = group_reduce<G>(sum, [](S x, S y) { return x + y; });
            if constexpr ((FLAGS & F_PROD) != 0) prod = group_reduce<G>(prod, [](Pr x, Pr y) { return x * y; });
            if constexpr ((FLAGS & F_ARG) != 0)
                arg = group_reduce<G>(arg, [](uint64_t x, uint64_t y) { return umax64(x, y); });
            else if constexpr ((FLAGS & F_MAX) != 0)
                maxk = group_reduce<G>(maxk, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            if constexpr ((FLAGS & F_MIN) != 0)
                mink = group_reduce<G>(mink, [](uint32_t x, uint32_t y) { return x < y ? x : y; });
        }
    }
    __device__ __forceinline__ void write(const RowParams &p, uint64_t r) const {
        const int64_t o = (int64_t)p.out_offset + (int64_t)r * p.out_stride;
        if constexpr ((FLAGS & F_SUM) != 0) ((T *)p.out_sum)[o] = (T)sum;
        if constexpr ((FLAGS & F_MEAN) != 0) {
            if constexpr (std::is_same<T, float>::value)
                ((float *)p.out_sum)[o] = (float)(sum / (double)p.cols);
            else if constexpr (std::is_same<T, int32_t>::value)
                ((int32_t *)p.out_sum)[o] = (int32_t)sum / (int32_t)p.cols;
            else
                ((uint32_t *)p.out_sum)[o] = (uint32_t)sum / (uint32_t)p.cols;
        }
        if constexpr ((FLAGS & F_PROD) != 0) ((T *)p.out_prod)[o] = (T)prod;
        if constexpr ((FLAGS & F_ARG) != 0) {
            const uint32_t key = (uint32_t)(arg >> 32);
            const bool none = std::is_same<T, float>::value ? (key == 0u) : (arg == 0ull);
            if (p.out_arg) p.out_arg[o] = none ? 0xFFFFFFFFu : arg_index(arg);
            if ((FLAGS & F_MAX) != 0 && p.out_max) {
                uint32_t mk = Key<T>::max_identity();
                if (!none && key > mk) mk = key;
                ((T *)p.out_max)[o] = Key<T>::decode(mk);
            }
        } else if constexpr ((FLAGS & F_MAX) != 0) {
            ((T *)p.out_max)[o] = Key<T>::decode(maxk);
        }
        if constexpr ((FLAGS & F_MIN) != 0) ((T *)p.out_min)[o] = Key<T>::decode(mink);
    }

    // Partial statistics of one chunk of the reduced axis, one 8-byte word
    // per statistic, each statistic in its own plane `plane` words apart.
    template <typename A> static __device__ __forceinline__ uint64_t to_word(A v) {
        if constexpr (std::is_same<A, double>::value) return (uint64_t)__double_as_longlong(v);
        else return (uint64_t)v;
    }
    template <typename A> static __device__ __forceinline__ A from_word(uint64_t w) {
        if constexpr (std::is_same<A, double>::value) return __longlong_as_double((long long)w);
        else return (A)w;
    }
    __device__ __forceinline__ void store_partial(uint64_t *w, uint64_t plane) const {
        int q = 0;
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) w[(q++) * plane] = to_word(sum);
        if constexpr ((FLAGS & F_PROD) != 0) w[(q++) * plane] = to_word(prod);
        if constexpr ((FLAGS & F_ARG) != 0) w[(q++) * plane] = arg;
        else if constexpr ((FLAGS & F_MAX) != 0) w[(q++) * plane] = maxk;
        if constexpr ((FLAGS & F_MIN) != 0) w[(q++) * plane] = mink;
        (void)q;
    }
    // Fold another lane's (or component's) statistics into these.
    __device__ __forceinline__ void merge(const Stats &o) {
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum += o.sum;
        if constexpr ((FLAGS & F_PROD) != 0) prod *= o.prod;
        if constexpr ((FLAGS & F_ARG) != 0) arg = umax64(arg, o.arg);
        else if constexpr ((FLAGS & F_MAX) != 0) maxk = maxk > o.maxk ? maxk : o.maxk;
        if constexpr ((FLAGS & F_MIN) != 0) mink = mink < o.mink ? mink : o.mink;
    }
    // These statistics combined with lane (lane ^ m)'s; both lanes end with
    // the same bits (every combination is commutative).
    __device__ __forceinline__ void merge_xor(int m) {
        Stats o;
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) o.sum = __shfl_xor(sum, m, kWave);
        if constexpr ((FLAGS & F_PROD) != 0) o.prod = __shfl_xor(prod, m, kWave);
        if constexpr ((FLAGS & F_ARG) != 0) o.arg = __shfl_xor(arg, m, kWave);
        else if constexpr ((FLAGS & F_MAX) != 0) o.maxk = __shfl_xor(maxk, m, kWave);
        if constexpr ((FLAGS & F_MIN) != 0) o.mink = __shfl_xor(mink, m, kWave);
        merge(o);
    }
    // The statistics one store_partial wrote.
    static __device__ __forceinline__ Stats from_partial(const uint64_t *w, uint64_t plane) {
        Stats s;
        int q = 0;
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) s.sum = from_word<S>(w[(q++) * plane]);
        if constexpr ((FLAGS & F_PROD) != 0) s.prod = from_word<Pr>(w[(q++) * plane]);
        if constexpr ((FLAGS & F_ARG) != 0) s.arg = w[(q++) * plane];
        else if constexpr ((FLAGS & F_MAX) != 0) s.maxk = (uint32_t)w[(q++) * plane];
        if constexpr ((FLAGS & F_MIN) != 0) s.mink = (uint32_t)w[(q++) * plane];
        (void)q;
        return s;
    }
    // Fold a later chunk's partial into this one.
    __device__ __forceinline__ void merge_partial(const uint64_t *w, uint64_t plane) {
        int q = 0;
        if constexpr ((FLAGS & (F_SUM | F_MEAN)) != 0) sum += from_word<S>(w[(q++) * plane]);
        if constexpr ((FLAGS & F_PROD) != 0) prod *= from_word<Pr>(w[(q++) * plane]);
        if constexpr ((FLAGS & F_ARG) != 0) {
            arg = umax64(arg, w[(q++) * plane]);
        } else if constexpr ((FLAGS & F_MAX) != 0) {
            const uint32_t k = (uint32_t)w[(q++) * plane];
            maxk = maxk > k ? maxk : k;
        }
        if constexpr ((FLAGS & F_MIN) != 0) {
            const uint32_t k = (uint32_t)w[(q++) * plane];
            mink = mink < k ? mink : k;
        }
        (void)q;
    }
};

// Statistics of `len` consecutive elements at `src` (unit stride, 4-byte
// aligned), read by the G lanes of a row group (`gl` = lane within the group)
// and reported with global indices from `j0`.  The 0-3 elements before the
// first 16-byte boundary go one per lane, the aligned body as 16-byte vectors
// (lane gl takes vectors gl, gl+G, ..., four in flight per trip), and the
// 0-3 elements after it one per lane.
// Rows of any length therefore stream at the aligned rate.
template <int G, typename T, bool AFFINE, int FLAGS>
__device__ __forceinline__ void visit_unit_span(Stats<T, FLAGS> &st, const T *src, uint64_t len, uint64_t j0, int gl,
                                                float a, float b) {
    using V = typename Vec4<T>::type;
    auto visit4 = [&](const V &x, uint32_t j) {
        st.visit(prologue<T, AFFINE>((T)x.x, a, b), j);
        st.visit(prologue<T, AFFINE>((T)x.y, a, b), j + 1);
        st.visit(prologue<T, AFFINE>((T)x.z, a, b), j + 2);
        st.visit(prologue<T, AFFINE>((T)x.w, a, b), j + 3);
    };
    uint64_t head = (((uint64_t)0 - (uint64_t)(uintptr_t)src) & 15u) >> 2;
    if (head > len) head = len;
    for (uint64_t h = gl; h < head; h += G) st.visit(prologue<T, AFFINE>(src[h], a, b), (uint32_t)(j0 + h));
    const V *vrow = (const V *)(src + head);
    const uint64_t nvec = (len - head) >> 2;
    const uint32_t jb = (uint32_t)(j0 + head);
    // Whole trips of 4 * G vectors, then at most one trip whose loads are
    // predicated per lane.  The trip count is the same for every lane of the
    // group (and of the wave: all groups of a launch share the row length),
    // so lanes never split into a 4-load path and a remainder path.
    const uint64_t full = nvec / (4 * G);
    uint64_t v = gl;
    for (uint64_t k = 0; k < full; ++k, v += 4 * G) {
        V x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = __builtin_nontemporal_load(&vrow[v + u * G]);
        // All four loads issue before any arithmetic waits on the first.
        __builtin_amdgcn_sched_barrier(0);
        T y[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            y[4 * u] = prologue<T, AFFINE>((T)x[u].x, a, b);
            y[4 * u + 1] = prologue<T, AFFINE>((T)x[u].y, a, b);
            y[4 * u + 2] = prologue<T, AFFINE>((T)x[u].z, a, b);
            y[4 * u + 3] = prologue<T, AFFINE>((T)x[u].w, a, b);
        }
        st.template visit_trip<G>(y, jb + (uint32_t)(4 * v));
    }
    if (full * 4 * G < nvec) {
        V x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (v + u * G < nvec) x[u] = __builtin_nontemporal_load(&vrow[v + u * G]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (v + u * G < nvec) visit4(x[u], jb + (uint32_t)(4 * (v + u * G)));
    }
    for (uint64_t t = head + 4 * nvec + gl; t < len; t += G)
        st.visit(prologue<T, AFFINE>(src[t], a, b), (uint32_t)(j0 + t));
}

// Row groups of G lanes: G = 1 is a thread per row (rows of fewer than 16
// elements), G = 4 or 16 puts 16 or 4 rows in each wave, G = 64 a wave per
// row, G = 128 or 256 two or four waves of the block per row.  Rows of up
// to 255 elements at most a little apart take rows_tile_kernel instead
// (tile_rows_fit).  The
// host picks G so that each lane holds at least three 16-byte vectors of its
// row: fewer leaves a lane too little in flight, and the per-row combine then
// dominates.  Multi-wave groups fold per-lane partials through LDS in wave
// order before one group reduction, so f32 sums stay deterministic.  Blocks
// take their rows in XCD-contiguous order (xcd_contiguous).
// Against one wave per row (the previous form), over 2^28 f32 (sum + max +
// argmax of fmaf(.5,x,.25)), microseconds per launch by row length:
// 4096: 156 (162); 3072: 152 (162); 2048: 160 (162); 1000: 173 (235);
// 768: 178 (225); 512: 162 (255); 256: 171 (360); 128: 203 (680);
// 64: 216 (1338).
// VEC: unit column stride, so lanes issue global_load_dwordx4 over each
// row's 16-byte-aligned body; otherwise G = 64 with one element per lane.
template <typename T, bool AFFINE, int FLAGS, bool VEC, int G>
__global__ __launch_bounds__(kBlock) void rows_kernel(RowParams p) {
    static_assert(kBlock % G == 0, "whole row groups per block");
    constexpr int kRowsPerBlock = kBlock / G;
    constexpr int kParts = G > kWave ? G / kWave : 1;
    __shared__ uint64_t sh[G > kWave ? kMaxPlanes * kBlock : 1];
    const int t = threadIdx.x;
    const int gl = t % G;
    uint32_t rl = (uint32_t)(t / G);
    if constexpr (G >= kWave) rl = (uint32_t)__builtin_amdgcn_readfirstlane(rl);
    const uint64_t r = p.row0 + (uint64_t)xcd_contiguous(blockIdx.x, gridDim.x) * kRowsPerBlock + rl;
    Stats<T, FLAGS> st;
    if (r < p.rows) {
        const T *row = (const T *)p.base + ((int64_t)p.offset + (int64_t)r * p.row_stride);
        if constexpr (VEC) {
            visit_unit_span<G, T, AFFINE, FLAGS>(st, row, p.cols, 0, gl, p.a, p.b);
        } else {
            for (uint64_t j = gl; j < p.cols; j += G)
                st.visit(prologue<T, AFFINE>(row[(int64_t)j * p.col_stride], p.a, p.b), (uint32_t)j);
        }
    }
    if constexpr (G > kWave) {
        // Waves other than the row's first leave right after this barrier.
        st.store_partial(&sh[t], kBlock);
        __syncthreads();
        if (gl >= kWave) return;
#pragma unroll
        for (int k = 1; k < kParts; ++k) st.merge_partial(&sh[t + k * kWave], kBlock);
        st.template group_combine<kWave>();
    } else {
        st.template group_combine<G>();
    }
    if (gl == 0 && r < p.rows) st.write(p, r);
}

// Short rows (1 to kTileRowMaxCols elements at unit stride, rows back to
// back or a little apart: tile_rows_fit).  A thread per row (rows_kernel,
// G = 1) holds only a few elements and reads them with 4-byte loads
// wherever rows start off a 16-byte boundary, so the launch is bound by
// lanes and waves, not bytes; groups of 4 lanes (16 elements and more)
// leave lanes idle in partly filled trips.  Here a block stages a tile of
// whole rows in LDS with 16-byte direct loads (every wave load moves 1 KiB
// of contiguous input), then each row is folded out of LDS by one thread,
// or from 64 elements by a group of G = 2, 4 or 8 lanes (the most that
// keeps the tile's rows times G within the block), each lane taking every
// G-th element (or vector) in index order, the group combined with xor
// shuffles; the group's first lane writes the outputs (adjacent groups,
// adjacent rows).  Padded rows load their padding with them.  Rows whose
// length and start distance are even are read as 8- or 16-byte LDS
// vectors: lanes an even number of words apart would otherwise share
// banks.  Over 2^28 f32 (sum, max, argmax), microseconds per launch, lane
// groups -> tiles: 1: 865 -> 385; 2: 578 -> 269; 3: 451 -> 257; 12: 275 ->
// 189; 20: 235 -> 184; 64: 183 -> 160-163; 100: 272 -> 164-167; 128: 167
// -> 155-157; 160: 185 -> 159-164; 255: 171 -> 154-155; 192: 156 ->
// 159-163 (40 rows a tile, 160 of 256 threads at G = 4).  With a thread
// per row the tiles' argmax had fallen behind from 100 elements (188 us
// at 127, 283 at 255).
constexpr uint32_t kRowsTileElems = 8192;
constexpr uint64_t kTileRowMaxCols = 255;

template <typename T, bool AFFINE, int FLAGS, int G>
__global__ __launch_bounds__(kBlock) void rows_tile_kernel(RowParams p, uint32_t tile_rows) {
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "row groups of 1 to 8 lanes");
    constexpr uint32_t kRowsPerPass = kBlock / G;
    __shared__ __attribute__((aligned(16))) T tile[kRowsTileElems];
    const uint32_t C = (uint32_t)p.cols;
    const uint32_t L = (uint32_t)p.row_stride; // C, or more for padded rows
    const uint64_t r0 = p.row0 + (uint64_t)xcd_contiguous(blockIdx.x, gridDim.x) * tile_rows;
    const uint32_t n = p.rows - r0 < tile_rows ? (uint32_t)(p.rows - r0) : tile_rows;
    tile_load_lds<kBlock, kRowsTileElems / 4 / kBlock>((const T *)p.base + (p.offset + r0 * L), (n - 1) * L + C,
                                                       tile);
    __syncthreads();
    const uint32_t w = C | L; // vector LDS reads where every row start and length allow them
    const uint32_t gl = threadIdx.x % G;
    // The G lanes of a row group share r, so they leave the loop together
    // and their xor shuffles never read a lane that has left.
    for (uint32_t r = threadIdx.x / G; r < n; r += kRowsPerPass) {
        Stats<T, FLAGS> st;
        const T *row = tile + r * L;
        if (w % 4 == 0) {
            using V = typename Vec4<T>::type;
            for (uint32_t j = 4 * gl; j < C; j += 4 * G) {
                const V x = *(const V *)(row + j);
                st.visit(prologue<T, AFFINE>((T)x.x, p.a, p.b), j);
                st.visit(prologue<T, AFFINE>((T)x.y, p.a, p.b), j + 1);
                st.visit(prologue<T, AFFINE>((T)x.z, p.a, p.b), j + 2);
                st.visit(prologue<T, AFFINE>((T)x.w, p.a, p.b), j + 3);
            }
        } else if (w % 2 == 0) {
            typedef T V2 __attribute__((ext_vector_type(2)));
            for (uint32_t j = 2 * gl; j < C; j += 2 * G) {
                const V2 x = *(const V2 *)(row + j);
                st.visit(prologue<T, AFFINE>((T)x.x, p.a, p.b), j);
                st.visit(prologue<T, AFFINE>((T)x.y, p.a, p.b), j + 1);
            }
        } else {
            for (uint32_t j = gl; j < C; j += G) st.visit(prologue<T, AFFINE>(row[j], p.a, p.b), j);
        }
#pragma unroll
        for (int m = 1; m < G; m <<= 1) st.merge_xor(m);
        if (gl == 0) st.write(p, r0 + r);
    }
}

// Statistics of lines [j0, j1) of the 64*V adjacent outputs from o0 (V per
// lane) of a column tile, kU lines in flight per lane: V = 4 gives every
// lane one 16-byte load per line, so each load instruction of a wave covers
// 1 KiB of one line.
template <typename T, bool AFFINE, int FLAGS, int V>
__device__ __forceinline__ void cols_walk(const RowParams &p, uint64_t o0, uint64_t j0, uint64_t j1,
                                          Stats<T, FLAGS> (&st)[V]) {
    constexpr int kU = V == 4 ? 8 : 16;
    const T *base = (const T *)p.base + ((int64_t)p.offset + (int64_t)o0 * p.row_stride);
    uint64_t j = j0;
    if constexpr (V == 4) {
        using Vt = typename Vec4A4<T>::type;
        auto visit = [&](const Vt &x, uint32_t jj) {
            st[0].visit(prologue<T, AFFINE>((T)x.x, p.a, p.b), jj);
            st[1].visit(prologue<T, AFFINE>((T)x.y, p.a, p.b), jj);
            st[2].visit(prologue<T, AFFINE>((T)x.z, p.a, p.b), jj);
            st[3].visit(prologue<T, AFFINE>((T)x.w, p.a, p.b), jj);
        };
        for (; j + kU <= j1; j += kU) {
            Vt x[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u)
                x[u] = __builtin_nontemporal_load((const Vt *)(base + (int64_t)(j + u) * p.col_stride));
#pragma unroll
            for (int u = 0; u < kU; ++u) visit(x[u], (uint32_t)(j + u));
        }
        for (; j < j1; ++j) visit(__builtin_nontemporal_load((const Vt *)(base + (int64_t)j * p.col_stride)), (uint32_t)j);
    } else {
        for (; j + kU <= j1; j += kU) {
            T x[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) x[u] = __builtin_nontemporal_load(base + (int64_t)(j + u) * p.col_stride);
#pragma unroll
            for (int u = 0; u < kU; ++u) st[0].visit(prologue<T, AFFINE>(x[u], p.a, p.b), (uint32_t)(j + u));
        }
        for (; j < j1; ++j)
            st[0].visit(prologue<T, AFFINE>(__builtin_nontemporal_load(base + (int64_t)j * p.col_stride), p.a, p.b),
                        (uint32_t)j);
    }
}

// Column tiles (the reduced axis is strided, the outputs adjacent: axis-0
// reduction of a row-major matrix).  A wave owns 64*V adjacent outputs and
// one chunk of the reduced axis (cols_walk).  Adjacent waves take adjacent
// output groups of the same chunk.  SPLIT: the chunk's statistics go to
// partial planes that split_fold_kernel combines in chunk order; otherwise
// the wave covers the whole axis and writes the outputs.
template <typename T, bool AFFINE, int FLAGS, int V, bool SPLIT>
__global__ __launch_bounds__(kBlock) void cols_tiles_kernel(RowParams p, uint64_t *partials, uint64_t chunk,
                                                            uint32_t nchunks, uint64_t groups) {
    const uint64_t w = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    if (w >= groups * nchunks) return;
    const uint64_t g = w % groups, k = w / groups;
    const uint64_t o0 = (g * kWave + (uint64_t)lane_id()) * V;
    if (o0 >= p.rows) return;
    const uint64_t j0 = k * chunk;
    const uint64_t j1 = j0 + chunk < p.cols ? j0 + chunk : p.cols;
    Stats<T, FLAGS> st[V];
    cols_walk<T, AFFINE, FLAGS, V>(p, o0, j0, j1, st);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        if constexpr (SPLIT)
            st[v].store_partial(partials + k * p.rows + o0 + v, (uint64_t)nchunks * p.rows);
        else
            st[v].write(p, o0 + v);
    }
}

// Small column reductions in one launch, with no workspace: a block of
// kFoldSlices waves per output group, wave s walking slice s of the reduced
// axis (`chunk` lines), then lane o of wave 0 folding the slices' statistics
// through LDS in slice order, one component at a time, and writing the
// outputs.  The order depends only on the shape, so f32 sums are bitwise
// reproducible.  The split form (column tiles into partial planes, then
// split_fold_kernel) takes two launches; on a 256 x 256 f32 axis-0 sum that
// is about 6 us per call, each launch costing a few microseconds of host and
// device time whatever its size.
template <typename T, bool AFFINE, int FLAGS, int V>
__global__ __launch_bounds__(kWave *kFoldSlices) void cols_block_kernel(RowParams p, uint64_t chunk) {
    __shared__ uint64_t sh[kMaxPlanes * kFoldSlices * kWave];
    const int lane = lane_id();
    const int s = threadIdx.x / kWave;
    const uint64_t o0 = ((uint64_t)blockIdx.x * kWave + (uint64_t)lane) * V;
    const bool live = o0 < p.rows; // V = 4 only when rows % 4 == 0: all four outputs exist
    const uint64_t j0 = (uint64_t)s * chunk < p.cols ? (uint64_t)s * chunk : p.cols;
    const uint64_t j1 = j0 + chunk < p.cols ? j0 + chunk : p.cols;
    Stats<T, FLAGS> st[V];
    if (live) cols_walk<T, AFFINE, FLAGS, V>(p, o0, j0, j1, st);
    constexpr uint64_t kPlane = (uint64_t)kFoldSlices * kWave;
#pragma unroll
    for (int v = 0; v < V; ++v) {
        st[v].store_partial(&sh[s * kWave + lane], kPlane);
        __syncthreads();
        if (s == 0 && live) {
            Stats<T, FLAGS> total;
            for (int q = 0; q < kFoldSlices; ++q) total.merge_partial(&sh[q * kWave + lane], kPlane);
            total.write(p, o0 + v);
        }
        __syncthreads();
    }
}

// Statistic planes a flag set keeps (sum or mean, product, max or argmax, min).
template <int FLAGS> constexpr int kPlanes = ((FLAGS & (F_SUM | F_MEAN)) != 0) + ((FLAGS & F_PROD) != 0) +
                                             ((FLAGS & (F_ARG | F_MAX)) != 0) + ((FLAGS & F_MIN) != 0);

constexpr uint64_t kPeriodMaxCols = 95; // the period form's widest matrix

// Narrow column reductions, C from 2 to 95: axis 0 of a dense row-major
// [R, C] matrix.  The matrix is one contiguous range of 1 KiB blocks (256
// elements); component k of lane l's vector in block b holds element
// 256 b + 4 l + k, in column (256 b + 4 l + k) mod C.  Blocks b and b + P,
// P = C / gcd(C, 256), give every lane-component the same column, so wave w
// takes the blocks rho + P m of one residue rho = w mod P for m in its chunk
// (w / P): each lane keeps four statistics and every load is a coalesced
// 1 KiB wave access.  Lane-components that share a column fold through the
// wave's LDS in ascending lane-component order, the block's four waves'
// column statistics fold in wave order, and the block stores them to its
// partial plane, which split_fold_kernel folds in block order, so f32 sums
// depend only on the shape (a single block writes the outputs).  Column
// tiles gave such matrices C live lanes per wave (2^28 f32 with C = 3:
// 2.7 ms).  A plane per wave instead of per block left the fold at 34 us of
// 193 (C = 3); an xor-butterfly form for powers of two up to 32 (the lanes
// of one column folded in registers, a plane per wave) took 180 us against
// 165-170 here.
template <typename T, int FLAGS>
__global__ __launch_bounds__(kBlock) void cols_period_kernel(RowParams p, uint64_t *partials, uint32_t period,
                                                             uint64_t chunk, uint32_t nwaves) {
    using V = typename Vec4A4<T>::type;
    constexpr int kBlockWaves = kBlock / kWave;
    __shared__ uint64_t sh[kBlockWaves][kPlanes<FLAGS> * 4 * kWave];
    __shared__ uint64_t sh_tot[kBlockWaves][kPlanes<FLAGS> * (kPeriodMaxCols + 1)];
    const int lane = lane_id();
    const int wv = threadIdx.x / kWave;
    const uint64_t w = (uint64_t)blockIdx.x * kBlockWaves + wv;
    const bool live = w < nwaves; // uniform across the wave; the others fold identities
    const uint32_t C = (uint32_t)p.rows;
    const uint64_t n = p.cols * C;
    const uint64_t nblk = (n + 4 * kWave - 1) / (4 * kWave);
    const uint64_t full_blk = n / (4 * kWave); // blocks whose 256 elements all exist
    const uint32_t rho = (uint32_t)(w % period);
    const uint64_t mcount = nblk > rho ? (nblk - rho + period - 1) / period : 0;
    const uint64_t m0 = w / period * chunk;
    const uint64_t m1 = live ? (m0 + chunk < mcount ? m0 + chunk : mcount) : m0;
    // Column of lane 0's component 0, the same in every block of the
    // residue, and the rows of this lane's four components in block
    // rho + P m0, which advance by 256 P / C = rstep per block of the residue.
    const uint32_t col0 = (uint32_t)(((uint64_t)rho * (4 * kWave)) % C);
    const uint32_t rstep = (uint32_t)((uint64_t)period * (4 * kWave) / C);
    uint32_t row[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) row[k] = (uint32_t)(((rho + (uint64_t)period * m0) * (4 * kWave) + 4 * lane + k) / C);
    const V *src = (const V *)((const T *)p.base + p.offset);
    Stats<T, FLAGS> st[4];
    auto visit4 = [&](const V &x, uint32_t dr) {
        st[0].visit((T)x.x, row[0] + dr);
        st[1].visit((T)x.y, row[1] + dr);
        st[2].visit((T)x.z, row[2] + dr);
        st[3].visit((T)x.w, row[3] + dr);
    };
    // Trips of four whole blocks, then the rest one block at a time with
    // per-element bounds (the range's last block may be partial).
    uint64_t m = m0;
    for (; m + 4 <= m1 && rho + (uint64_t)period * (m + 3) < full_blk; m += 4) {
        V x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            x[u] = __builtin_nontemporal_load(&src[(rho + (uint64_t)period * (m + u)) * kWave + lane]);
#pragma unroll
        for (int u = 0; u < 4; ++u) visit4(x[u], u * rstep);
#pragma unroll
        for (int k = 0; k < 4; ++k) row[k] += 4 * rstep;
    }
    for (; m < m1; ++m) {
        const uint64_t v = (rho + (uint64_t)period * m) * kWave + lane;
        if (4 * v + 4 <= n) {
            visit4(__builtin_nontemporal_load(&src[v]), 0);
        } else {
            const T *s1 = (const T *)src + 4 * v;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (4 * v + k < n) st[k].visit(__builtin_nontemporal_load(&s1[k]), row[k]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) row[k] += rstep;
    }
    constexpr uint64_t kPlane = 4 * kWave;
#pragma unroll
    for (int k = 0; k < 4; ++k) st[k].store_partial(&sh[wv][4 * lane + k], kPlane);
    __syncthreads();
    // Each wave's column totals (waves past nwaves hold identities), then the
    // block's: the waves' totals in wave order, one partial plane per block.
    constexpr uint64_t kColPlane = kPeriodMaxCols + 1;
    for (uint32_t c = lane; c < C; c += kWave) {
        // Lane-components i = 4 l + k in column c: i = c - col0 (mod C).
        Stats<T, FLAGS> total;
        for (uint32_t i = (c + C - col0) % C; i < 4 * kWave; i += C) total.merge_partial(&sh[wv][i], kPlane);
        total.store_partial(&sh_tot[wv][c], kColPlane);
    }
    __syncthreads();
    if (wv != 0) return;
    const uint32_t nblocks = (nwaves + kBlockWaves - 1) / kBlockWaves;
    for (uint32_t c = lane; c < C; c += kWave) {
        Stats<T, FLAGS> total;
#pragma unroll
        for (int q = 0; q < kBlockWaves; ++q) total.merge_partial(&sh_tot[q][c], kColPlane);
        if (nblocks > 1)
            total.store_partial(partials + (uint64_t)blockIdx.x * C + c, (uint64_t)nblocks * C);
        else
            total.write(p, c);
    }
}

// Few long rows (the reduced axis has unit stride but there are too few rows
// to give every CU work): one wave per (row, chunk of 256-element multiples),
// lanes along the chunk as in rows_kernel, partials to the planes.
template <typename T, bool AFFINE, int FLAGS, bool VEC>
__global__ __launch_bounds__(kBlock) void rows_split_kernel(RowParams p, uint64_t *partials, uint64_t chunk,
                                                            uint32_t nchunks) {
    const int lane = lane_id();
    const uint64_t w = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    if (w >= p.rows * nchunks) return; // uniform across the wave
    const uint64_t r = w / nchunks, k = w % nchunks;
    const T *row = (const T *)p.base + ((int64_t)p.offset + (int64_t)r * p.row_stride);
    const uint64_t c0 = k * chunk;
    const uint64_t c1 = c0 + chunk < p.cols ? c0 + chunk : p.cols;
    Stats<T, FLAGS> st;
    if constexpr (VEC) {
        visit_unit_span<kWave, T, AFFINE, FLAGS>(st, row + c0, c1 - c0, c0, lane, p.a, p.b);
    } else {
        for (uint64_t j = c0 + lane; j < c1; j += kWave)
            st.visit(prologue<T, AFFINE>(row[(int64_t)j * p.col_stride], p.a, p.b), (uint32_t)j);
    }
    st.template group_combine<kWave>();
    if (lane == 0) st.store_partial(partials + k * p.rows + r, (uint64_t)nchunks * p.rows);
}

// Fold the chunk partials: a block owns 64 outputs (lanes) and kFoldSlices
// waves; wave s folds its contiguous range of chunks in order, then lane o of
// wave 0 folds the slice results in slice order.  The order depends only on
// the chunk count, so f32 sums do not depend on scheduling.

template <typename T, int FLAGS>
__global__ __launch_bounds__(kWave *kFoldSlices) void split_fold_kernel(RowParams p, const uint64_t *partials,
                                                                       uint32_t nchunks) {
    __shared__ uint64_t sh[kMaxPlanes * kFoldSlices * kWave];
    const int lane = lane_id();
    const int s = threadIdx.x / kWave;
    const uint64_t o = (uint64_t)blockIdx.x * kWave + lane;
    const uint64_t plane = (uint64_t)nchunks * p.rows;
    const uint32_t per = (nchunks + kFoldSlices - 1) / kFoldSlices;
    const uint32_t k0 = s * per < nchunks ? s * per : nchunks;
    const uint32_t k1 = k0 + per < nchunks ? k0 + per : nchunks;
    Stats<T, FLAGS> st;
    if (o < p.rows) {
        // Eight partials loaded together, then merged in chunk order (one
        // dependent load per chunk left a 3-output fold of 2049 chunks at
        // 34 us).
        uint32_t k = k0;
        for (; k + 8 <= k1; k += 8) {
            Stats<T, FLAGS> b[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                b[u] = Stats<T, FLAGS>::from_partial(partials + (uint64_t)(k + u) * p.rows + o, plane);
#pragma unroll
            for (int u = 0; u < 8; ++u) st.merge(b[u]);
        }
        for (; k < k1; ++k) st.merge_partial(partials + (uint64_t)k * p.rows + o, plane);
    }
    st.store_partial(&sh[s * kWave + lane], (uint64_t)kFoldSlices * kWave);
    __syncthreads();
    if (s != 0 || o >= p.rows) return;
    Stats<T, FLAGS> total;
    for (int q = 0; q < kFoldSlices; ++q) total.merge_partial(&sh[q * kWave + lane], (uint64_t)kFoldSlices * kWave);
    total.write(p, o);
}

// Launch shape, computed identically for workspace sizing and for launch.
// 8 waves per CU: measured on a 65536 x 4096 f32 column sum, 2048 waves of
// 128 lines each ran at 6.7 TB/s with the fold; 4096 waves 6.4; 8192 waves
// 5.0 (a second, mostly idle round of waves).
constexpr uint64_t kTargetWaves = 2048;
constexpr uint64_t kMinColChunk = 32;    // lines per column-tile chunk
constexpr uint64_t kMinRowChunk = 8192;  // elements per split-row chunk
constexpr uint64_t kRowTargetWaves = 4096; // split rows when fewer than half this many

// Column reductions that would split their axis take one launch
// (cols_block_kernel) when the matrix is small: at most kBlockFoldLines lines
// (64 per wave) and kBlockFoldElems elements.
constexpr uint64_t kBlockFoldLines = 64 * kFoldSlices;
constexpr uint64_t kBlockFoldElems = 1ull << 20;

// Axis 0 of a dense row-major matrix with any other column count below 96,
// more than kBlockFoldLines lines (fewer take the one-launch block form) and
// row indices within 32 bits: the period form, cols_period_kernel.  From 96
// columns the column tiles keep enough lanes busy (2^28 f32 sums, period
// form against column tiles: C = 65 212 / 227 us, 80 199 / 212, 96 200 /
// 198, 100 200 / 196, 255 201 / 172).
constexpr uint64_t kMinPeriodChunk = 64; // 1 KiB blocks per period-form wave
bool period_columns(const RowParams &p, uintptr_t base) {
    const uint64_t c = p.rows;
    return c >= 2 && c <= kPeriodMaxCols && p.row_stride == 1 && p.col_stride == (int64_t)c && base % 4 == 0 &&
           p.cols > kBlockFoldLines && p.cols <= 0xFFFFFFFFull;
}

struct Shape {
    bool cols = false, vec = false;
    bool period = false; // cols_period_kernel over residues mod P of 1 KiB blocks
    uint32_t P = 1, waves = 0;
    bool block = false; // cols_block_kernel: one launch, no partials
    bool tile = false;  // rows_tile_kernel: tiles of tile_rows short rows
    uint32_t tile_rows = 0;
    int tile_group = 1; // lanes per row of the tile
    int V = 1;
    int G = kWave; // lanes per row for rows_kernel
    uint64_t groups = 0, chunk = 0;
    uint32_t nchunks = 1;
};

// Lanes per row: the largest group that still gives each lane at least
// three 16-byte vectors of the row, except that a wave per row pays for a
// partly filled last trip more than four rows per wave lose, so 64 lanes
// take only rows of whole 4-vector trips.  Measured over 2^28 f32 (sum, max
// and argmax), microseconds per launch by row length and lanes per row:
//   768: 64 -> 181, 16 -> 162     1024: 64 -> 163, 16 -> 170
//   1280: 64 -> 166, 16 -> 158    1536: 128 -> 159, 64 -> 164
//   3072: 256 -> 152, 128 -> 159  256: 16 -> 167, 4 -> 185
//   192: 16 -> 190, 4 -> 204      128: 16 -> 219, 4 -> 201
int row_group_lanes(uint64_t cols, bool vec) {
    if (!vec) return kWave;
    const uint64_t nvec = cols / 4;
    if (nvec >= 3 * 256) return 256;
    if (nvec >= 3 * 128) return 128;
    if (nvec >= 4 * 64 && nvec % (4 * 64) == 0) return 64;
    if (nvec >= 3 * 16) return 16;
    if (nvec >= 4) return 4;
    return 1;
}

// Rows for rows_tile_kernel: 1 to kTileRowMaxCols elements at unit stride,
// row starts L >= C elements apart with at least 64 rows to a tile.  The
// tile loads the whole span, padding included, so L stays within twice the
// row or within 32 elements (128 bytes, the line any row read fetches).
bool tile_rows_fit(const RowParams &p, uintptr_t base) {
    const uint64_t C = p.cols;
    if (C < 1 || C > kTileRowMaxCols || (p.col_stride != 1 && C != 1) || base % 4 != 0) return false;
    if (p.row_stride < (int64_t)C) return false;
    const uint64_t L = (uint64_t)p.row_stride;
    return L <= kTileRowMaxCols && (L <= 2 * C || L <= 32);
}

Shape plan_shape(const RowParams &p, bool cols_layout) {
    Shape s;
    s.cols = cols_layout;
    const uintptr_t base = (uintptr_t)p.base + 4u * p.offset; // every element type is 4 bytes
    uint64_t k = 1;
    if (cols_layout && period_columns(p, base)) {
        // Chunks of whole 4-block trips, about kTargetWaves waves in all;
        // nchunks counts waves (one partial plane each).
        s.period = true;
        uint64_t g = 4 * kWave;
        for (uint64_t a = p.rows; a != 0;) {
            const uint64_t t = g % a;
            g = a;
            a = t;
        }
        s.P = (uint32_t)(p.rows / g);
        const uint64_t nblk = ceil_div(p.cols * p.rows, 4 * kWave);
        uint64_t chunk = ceil_div(nblk, kTargetWaves);
        if (chunk < kMinPeriodChunk) chunk = kMinPeriodChunk;
        s.chunk = ceil_div(chunk, 4) * 4;
        s.waves = s.P * (uint32_t)ceil_div(ceil_div(nblk, s.P), s.chunk);
        s.nchunks = (uint32_t)ceil_div((uint64_t)s.waves, kBlock / kWave); // one partial plane per block
        return s;
    }
    if (cols_layout) {
        // 16-byte vectors at 4-byte alignment (Vec4A4): any line start.
        s.vec = p.row_stride == 1 && p.rows % 4 == 0 && base % 4 == 0;
        s.V = s.vec ? 4 : 1;
        s.groups = ceil_div(p.rows, (uint64_t)kWave * s.V);
        if (s.groups < kTargetWaves) {
            k = ceil_div(kTargetWaves, s.groups);
            const uint64_t kmax = ceil_div(p.cols, kMinColChunk);
            if (k > kmax) k = kmax;
        }
    } else {
        s.vec = p.col_stride == 1 && base % 4 == 0;
        if (tile_rows_fit(p, base)) {
            s.tile = true;
            s.tile_rows = (uint32_t)(((kRowsTileElems - p.cols) / (uint64_t)p.row_stride + 1) & ~3ull);
            while (s.tile_group < 8 && (uint64_t)s.tile_rows * s.tile_group * 2 <= (uint64_t)kBlock) s.tile_group *= 2;
            return s;
        }
        s.G = row_group_lanes(p.cols, s.vec);
        if (p.rows < kRowTargetWaves / 2 && p.cols >= 2 * kMinRowChunk) {
            k = ceil_div(kRowTargetWaves, p.rows);
            const uint64_t kmax = ceil_div(p.cols, kMinRowChunk);
            if (k > kmax) k = kmax;
        }
    }
    if (k < 1) k = 1;
    if (cols_layout && k > 1 && p.cols <= kBlockFoldLines && p.rows * p.cols <= kBlockFoldElems) {
        s.block = true;
        s.chunk = ceil_div(p.cols, (uint64_t)kFoldSlices);
        s.nchunks = 1;
        return s;
    }
    if (k > 1) {
        uint64_t chunk = ceil_div(p.cols, k);
        if (!cols_layout) chunk = ceil_div(chunk, 256) * 256; // whole 1 KiB wave loads per chunk
        s.chunk = chunk;
        s.nchunks = (uint32_t)ceil_div(p.cols, chunk);
    } else {
        s.chunk = p.cols;
        s.nchunks = 1;
    }
    return s;
}

int planes_of(int flags) {
    return ((flags & (F_SUM | F_MEAN)) != 0) + ((flags & F_PROD) != 0) + ((flags & (F_ARG | F_MAX)) != 0) +
           ((flags & F_MIN) != 0);
}

uint64_t shape_bytes(const RowParams &p, const Shape &s, int flags) {
    if (p.rows == 0 || s.nchunks <= 1) return 0;
    return (uint64_t)planes_of(flags) * s.nchunks * p.rows * 8u;
}

template <typename T, bool AFFINE, int FLAGS>
hx_status launch_rows_typed(const RowParams &p, bool cols_layout, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    if (p.rows == 0) return HX_OK;
    const Shape s = plan_shape(p, cols_layout);
    const bool split = s.nchunks > 1;
    uint64_t *partials = (uint64_t *)ws;
    if (split && ws_bytes < shape_bytes(p, s, FLAGS))
        return fail(HX_ERR_DISPATCH_FAILED, "axis reduction workspace of %llu bytes is too small",
                    (unsigned long long)ws_bytes);
    if (s.period) {
        hipLaunchKernelGGL((cols_period_kernel<T, FLAGS>), dim3(s.nchunks), dim3(kBlock), 0, stream, p, partials, s.P,
                           s.chunk, s.waves);
        HX_TRY(check_launch("cols_period_kernel"));
    } else if (s.block) {
        if (s.groups > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "axis reduction exceeds the grid range");
        const dim3 grid((uint32_t)s.groups), block(kWave * kFoldSlices);
        if (s.vec)
            hipLaunchKernelGGL((cols_block_kernel<T, AFFINE, FLAGS, 4>), grid, block, 0, stream, p, s.chunk);
        else
            hipLaunchKernelGGL((cols_block_kernel<T, AFFINE, FLAGS, 1>), grid, block, 0, stream, p, s.chunk);
        return check_launch("cols_block_kernel");
    } else if (cols_layout) {
        const uint64_t waves = s.groups * s.nchunks;
        const uint64_t blocks = ceil_div(waves, kBlock / kWave);
        if (blocks > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "axis reduction exceeds the grid range");
        const dim3 grid((uint32_t)blocks), block(kBlock);
        if (s.vec) {
            if (split)
                hipLaunchKernelGGL((cols_tiles_kernel<T, AFFINE, FLAGS, 4, true>), grid, block, 0, stream, p, partials,
                                   s.chunk, s.nchunks, s.groups);
            else
                hipLaunchKernelGGL((cols_tiles_kernel<T, AFFINE, FLAGS, 4, false>), grid, block, 0, stream, p, partials,
                                   s.chunk, s.nchunks, s.groups);
        } else {
            if (split)
                hipLaunchKernelGGL((cols_tiles_kernel<T, AFFINE, FLAGS, 1, true>), grid, block, 0, stream, p, partials,
                                   s.chunk, s.nchunks, s.groups);
            else
                hipLaunchKernelGGL((cols_tiles_kernel<T, AFFINE, FLAGS, 1, false>), grid, block, 0, stream, p, partials,
                                   s.chunk, s.nchunks, s.groups);
        }
        HX_TRY(check_launch("cols_tiles_kernel"));
    } else if (s.tile) {
        // Batches of whole tiles below 2^32 work-items per launch.
        const uint64_t max_blocks = 0xFFFFFFFFull / kBlock;
        const uint64_t blocks = ceil_div(p.rows, (uint64_t)s.tile_rows);
        RowParams q = p;
        for (uint64_t b0 = 0; b0 < blocks; b0 += max_blocks) {
            q.row0 = b0 * s.tile_rows;
            const dim3 grid((uint32_t)std::min<uint64_t>(max_blocks, blocks - b0)), block(kBlock);
            if (s.tile_group == 8)
                hipLaunchKernelGGL((rows_tile_kernel<T, AFFINE, FLAGS, 8>), grid, block, 0, stream, q, s.tile_rows);
            else if (s.tile_group == 4)
                hipLaunchKernelGGL((rows_tile_kernel<T, AFFINE, FLAGS, 4>), grid, block, 0, stream, q, s.tile_rows);
            else if (s.tile_group == 2)
                hipLaunchKernelGGL((rows_tile_kernel<T, AFFINE, FLAGS, 2>), grid, block, 0, stream, q, s.tile_rows);
            else
                hipLaunchKernelGGL((rows_tile_kernel<T, AFFINE, FLAGS, 1>), grid, block, 0, stream, q, s.tile_rows);
            HX_TRY(check_launch("rows_tile_kernel"));
        }
        return HX_OK;
    } else if (split) {
        const uint64_t blocks = ceil_div(p.rows * s.nchunks, kBlock / kWave);
        if (blocks > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "axis reduction exceeds the grid range");
        if (s.vec)
            hipLaunchKernelGGL((rows_split_kernel<T, AFFINE, FLAGS, true>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                               stream, p, partials, s.chunk, s.nchunks);
        else
            hipLaunchKernelGGL((rows_split_kernel<T, AFFINE, FLAGS, false>), dim3((uint32_t)blocks), dim3(kBlock), 0,
                               stream, p, partials, s.chunk, s.nchunks);
        HX_TRY(check_launch("rows_split_kernel"));
    } else {
        // A launch's work-items must stay below 2^32: 2^26 rows of 64 lanes
        // (strided rows) or 2^30 of 4 take several launches of whole blocks.
        const uint64_t rows_per_block = kBlock / s.G;
        const uint64_t max_blocks = 0xFFFFFFFFull / kBlock;
        const uint64_t blocks = ceil_div(p.rows, rows_per_block);
        RowParams q = p;
        for (uint64_t b0 = 0; b0 < blocks; b0 += max_blocks) {
            q.row0 = b0 * rows_per_block;
            const dim3 grid((uint32_t)std::min<uint64_t>(max_blocks, blocks - b0)), block(kBlock);
            if (!s.vec)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, false, kWave>), grid, block, 0, stream, q);
            else if (s.G == 256)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 256>), grid, block, 0, stream, q);
            else if (s.G == 128)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 128>), grid, block, 0, stream, q);
            else if (s.G == 64)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 64>), grid, block, 0, stream, q);
            else if (s.G == 16)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 16>), grid, block, 0, stream, q);
            else if (s.G == 4)
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 4>), grid, block, 0, stream, q);
            else
                hipLaunchKernelGGL((rows_kernel<T, AFFINE, FLAGS, true, 1>), grid, block, 0, stream, q);
            HX_TRY(check_launch("rows_kernel"));
        }
        return HX_OK;
    }
    if (!split) return HX_OK;
    hipLaunchKernelGGL((split_fold_kernel<T, FLAGS>), dim3((uint32_t)ceil_div(p.rows, kWave)),
                       dim3(kWave * kFoldSlices), 0, stream, p, (const uint64_t *)partials, s.nchunks);
    return check_launch("split_fold_kernel");
}

template <typename T, bool AFFINE>
hx_status launch_rows_flags(const RowParams &p, int flags, bool cols_layout, void *ws, uint64_t ws_bytes,
                            hipStream_t stream) {
    switch (flags) {
    case F_SUM: return launch_rows_typed<T, AFFINE, F_SUM>(p, cols_layout, ws, ws_bytes, stream);
    case F_MAX: return launch_rows_typed<T, AFFINE, F_MAX>(p, cols_layout, ws, ws_bytes, stream);
    case F_ARG: return launch_rows_typed<T, AFFINE, F_ARG>(p, cols_layout, ws, ws_bytes, stream);
    case F_MIN: return launch_rows_typed<T, AFFINE, F_MIN>(p, cols_layout, ws, ws_bytes, stream);
    case F_PROD: return launch_rows_typed<T, AFFINE, F_PROD>(p, cols_layout, ws, ws_bytes, stream);
    case F_MEAN: return launch_rows_typed<T, AFFINE, F_MEAN>(p, cols_layout, ws, ws_bytes, stream);
    case F_SUM | F_MAX: return launch_rows_typed<T, AFFINE, F_SUM | F_MAX>(p, cols_layout, ws, ws_bytes, stream);
    case F_SUM | F_ARG: return launch_rows_typed<T, AFFINE, F_SUM | F_ARG>(p, cols_layout, ws, ws_bytes, stream);
    case F_MAX | F_ARG: return launch_rows_typed<T, AFFINE, F_MAX | F_ARG>(p, cols_layout, ws, ws_bytes, stream);
    case F_SUM | F_MAX | F_ARG:
        return launch_rows_typed<T, AFFINE, F_SUM | F_MAX | F_ARG>(p, cols_layout, ws, ws_bytes, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unsupported row statistic set %d", flags);
}

hx_status launch_rows_any(const RowParams &p, hx_dtype dtype, bool affine, int flags, bool cols_layout, void *ws,
                          uint64_t ws_bytes, hipStream_t stream) {
    switch (dtype) {
    case HX_DTYPE_F32:
        return affine ? launch_rows_flags<float, true>(p, flags, cols_layout, ws, ws_bytes, stream)
                      : launch_rows_flags<float, false>(p, flags, cols_layout, ws, ws_bytes, stream);
    case HX_DTYPE_U32: return launch_rows_flags<uint32_t, false>(p, flags, cols_layout, ws, ws_bytes, stream);
    case HX_DTYPE_I32: return launch_rows_flags<int32_t, false>(p, flags, cols_layout, ws, ws_bytes, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)dtype);
}

int rows_params(const RowsArgs &a, RowParams *p) {
    *p = RowParams{};
    p->base = a.base;
    p->rows = a.rows;
    p->cols = a.cols;
    p->row_stride = (int64_t)a.row_stride;
    p->col_stride = 1;
    p->offset = a.offset;
    p->a = a.a;
    p->b = a.b;
    p->out_sum = a.out_sum;
    p->out_max = a.out_max;
    p->out_arg = a.out_argmax;
    p->out_stride = 1;
    p->out_offset = 0;
    return (a.out_sum ? F_SUM : 0) | (a.out_argmax ? F_ARG : 0) | (a.out_max ? F_MAX : 0);
}

int axis_params(const AxisArgs &a, RowParams *p, bool *cols_layout) {
    *p = RowParams{};
    p->base = a.in;
    p->rows = a.outer;
    p->cols = a.axis_len;
    p->row_stride = a.in_outer_stride;
    p->col_stride = a.in_axis_stride;
    p->offset = a.in_offset;
    p->out_stride = a.out_stride;
    p->out_offset = a.out_offset;
    int flags = 0;
    switch (a.op) {
    case HX_OP_SUM: flags = F_SUM; p->out_sum = a.out; break;
    case HX_OP_MEAN: flags = F_MEAN; p->out_sum = a.out; break;
    case HX_OP_PROD: flags = F_PROD; p->out_prod = a.out; break;
    case HX_OP_MIN: flags = F_MIN; p->out_min = a.out; break;
    case HX_OP_MAX: flags = F_MAX; p->out_max = a.out; break;
    case HX_OP_ARGMAX: flags = F_ARG; p->out_arg = (uint32_t *)a.out; break;
    }
    // Unit stride along the reduced axis -> lanes along the axis; unit
    // stride across outputs (and not along the axis) -> lanes across outputs.
    const bool axis_unit = a.in_axis_stride == 1 || a.in_axis_stride == -1;
    const bool outer_unit = a.in_outer_stride == 1 || a.in_outer_stride == -1;
    *cols_layout = !axis_unit && outer_unit;
    return flags;
}

} // namespace

uint64_t rows_workspace_bytes(const RowsArgs &a) {
    RowParams p;
    const int flags = rows_params(a, &p);
    return shape_bytes(p, plan_shape(p, false), flags);
}

hx_status launch_rows(const RowsArgs &a, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    RowParams p;
    const int flags = rows_params(a, &p);
    if (flags == 0) return HX_OK;
    return launch_rows_any(p, a.dtype, a.affine, flags, false, ws, ws_bytes, stream);
}

uint64_t axis_reduce_workspace_bytes(const AxisArgs &a) {
    RowParams p;
    bool cols_layout;
    const int flags = axis_params(a, &p, &cols_layout);
    return shape_bytes(p, plan_shape(p, cols_layout), flags);
}

hx_status launch_axis_reduce(const AxisArgs &a, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    RowParams p;
    bool cols_layout;
    const int flags = axis_params(a, &p, &cols_layout);
    return launch_rows_any(p, a.dtype, false, flags, cols_layout, ws, ws_bytes, stream);
}

} // namespace hx
