// Device-side building blocks shared by every gfx950 kernel of the library:
// wave64 reductions and scans, order-preserving keys for max/argmax, the
// combining operators with their identities, and the counter-based
// generator.  Header-only; included by the .hip translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hx {

constexpr int kWave = 64;

// 16-byte vectors (one global_load_dwordx4 per lane).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T> struct Vec4 { using type = u32x4; };
template <> struct Vec4<float> { using type = f32x4; };
// The same 16-byte vectors at 4-byte alignment: global_load_dwordx4 and
// global_store_dwordx4 accept any dword-aligned address (the compiler emits
// the same instruction), so a line that starts off a 16-byte boundary still
// moves one 16-byte vector per lane and instruction.
typedef float f32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
template <typename T> struct Vec4A4 { using type = u32x4_a4; };
template <> struct Vec4A4<float> { using type = f32x4_a4; };

// Vector loads/stores; NT marks them non-temporal (streamed through, not
// retained in the caches).
template <bool NT, typename V> __device__ __forceinline__ V load_vec(const V *ptr) {
    if constexpr (NT) return __builtin_nontemporal_load(ptr);
    else return *ptr;
}
template <bool NT, typename V> __device__ __forceinline__ void store_vec(V v, V *ptr) {
    if constexpr (NT) __builtin_nontemporal_store(v, ptr);
    else *ptr = v;
}
// The same through dword-aligned pointers.  The parameter types name the
// 4-byte-aligned typedefs explicitly: a template parameter deduced from the
// pointer would be the canonical, 16-byte-aligned vector type.
template <bool NT> __device__ __forceinline__ f32x4_a4 load_a4(const f32x4_a4 *ptr) {
    if constexpr (NT) return __builtin_nontemporal_load(ptr);
    else return *ptr;
}
template <bool NT> __device__ __forceinline__ u32x4_a4 load_a4(const u32x4_a4 *ptr) {
    if constexpr (NT) return __builtin_nontemporal_load(ptr);
    else return *ptr;
}
template <bool NT> __device__ __forceinline__ void store_a4(f32x4_a4 v, f32x4_a4 *ptr) {
    if constexpr (NT) __builtin_nontemporal_store(v, ptr);
    else *ptr = v;
}
template <bool NT> __device__ __forceinline__ void store_a4(u32x4_a4 v, u32x4_a4 *ptr) {
    if constexpr (NT) __builtin_nontemporal_store(v, ptr);
    else *ptr = v;
}

// ---------------------------------------------------------- stream stores
// The output side of a read+write stream (scan tiles, copy, vector forms)
// stores through a buffer resource with cache policy nt | sc1: streamed, and
// written through the L2 at device scope instead of being left dirty there
// for a later write-back.  Measured on MI355X copying 1 GiB with nt loads:
// nt stores 349.5 us (6.14 TB/s), nt | sc1 stores 340 us (6.32 TB/s); the
// runtime's own hipMemcpyAsync device-to-device blit 415-422 us.
// `base` must be wave-uniform and `bytes` < 2^32; the hardware range check
// drops any store at or beyond `bytes`.
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferWord3 = 0x00020000;  // raw dword buffer, descriptor word 3 (gfx9 family)
constexpr int kStreamStorePolicy = 2 | 16; // nt | sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, kBufferWord3);
}
template <typename V> __device__ __forceinline__ void stream_store(V v, __amdgpu_buffer_rsrc_t r, uint32_t off) {
    static_assert(sizeof(V) == 16, "16-byte vectors");
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, (int)off, 0, kStreamStorePolicy);
}

// ------------------------------------------------------ direct LDS loads
// ne 4-byte elements from src (dword aligned) into a 16-byte aligned LDS
// tile with global_load_lds_dwordx4: each wave's 64 vectors of a step land
// at its LDS base + 16 * lane, with no register round trip and no LDS write
// instructions.  THREADS threads move up to VPT vectors each (THREADS * VPT
// * 4 >= ne); a partial tile's last ne mod 4 elements move one per thread.
// Every load has landed in LDS when this returns; the caller's barrier
// publishes the tile to the block.
constexpr int kLoadLdsNt = 2; // cache policy of the direct LDS loads: nt (streamed through)
template <int THREADS, int VPT, typename T>
__device__ __forceinline__ void tile_load_lds(const T *src, uint32_t ne, T *tile) {
    static_assert(sizeof(T) == 4, "4-byte elements");
    const uint32_t nv = ne / 4;
    const uint32_t wbase = __builtin_amdgcn_readfirstlane(threadIdx.x & ~(uint32_t)(kWave - 1));
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const uint32_t v = threadIdx.x + (uint32_t)u * THREADS;
        if (v < nv)
            __builtin_amdgcn_global_load_lds(
                (const void *)(src + 4 * v),
                (__attribute__((address_space(3))) void *)(tile + 4 * (wbase + (uint32_t)u * THREADS)), 16, 0,
                kLoadLdsNt);
    }
    const uint32_t e = 4 * nv + threadIdx.x;
    if (e < ne) tile[e] = __builtin_nontemporal_load(src + e);
    __builtin_amdgcn_s_waitcnt(0); // vmcnt(0): the direct loads are in LDS
}

// ----------------------------------------------------------------- lanes

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

// ------------------------------------------------------------ operators
// Combining operators of crates/hephaestus-core/src/domain/ops.rs:735-803
// with the identities of ops.rs:926-983.  `Acc` is the accumulation type:
// f32 sums and products accumulate in f64 so the per-output error of a
// reduction is one final rounding; integer sums and products wrap mod 2^32
// exactly like `unsigned int` / `int` arithmetic in the reference kernels.

template <typename T> struct SumAcc { using type = T; };
template <> struct SumAcc<float> { using type = double; };

struct OpSum {
    template <typename A> __device__ __forceinline__ static A identity() { return A(0); }
    template <typename A> __device__ __forceinline__ static A combine(A a, A b) { return a + b; }
};
struct OpProd {
    template <typename A> __device__ __forceinline__ static A identity() { return A(1); }
    template <typename A> __device__ __forceinline__ static A combine(A a, A b) { return a * b; }
};

// Integer sums and products use unsigned arithmetic so overflow wraps
// (defined behaviour); the bits equal the reference's two's complement.
template <typename T> struct Wrap { using type = T; };
template <> struct Wrap<int32_t> { using type = uint32_t; };

// -------------------------------------------------------- ordered keys
// Max and min are computed on order-preserving 32-bit keys, which makes
// them exact and independent of combination order:
//   f32: key = bits ^ (sign ? 0xFFFFFFFF : 0x80000000), the IEEE total order
//        (-inf < ... < -0 < +0 < ... < +inf); NaN maps to the key that
//        never wins (0 for max, 0xFFFFFFFF for min), so NaN is ignored like
//        HIP fmaxf/fminf, the reference's `max(lhs, rhs)` (ops.rs:902-919).
//   i32: key = bits ^ 0x80000000;  u32: key = value.
// The MaxOp identity f32::MIN (ops.rs:956-958) is folded in by the caller.

__device__ __forceinline__ uint32_t f32_key_max(float x) {
    uint32_t b = __float_as_uint(x);
    uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
    return (x != x) ? 0u : k;
}
__device__ __forceinline__ uint32_t f32_key_min(float x) {
    uint32_t b = __float_as_uint(x);
    uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
    return (x != x) ? 0xFFFFFFFFu : k;
}
__device__ __forceinline__ float f32_from_key(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k ^ 0x80000000u) : ~k;
    return __uint_as_float(b);
}

template <typename T> struct Key;
template <> struct Key<float> {
    __device__ __forceinline__ static uint32_t max_key(float x) { return f32_key_max(x); }
    __device__ __forceinline__ static uint32_t min_key(float x) { return f32_key_min(x); }
    __device__ __forceinline__ static float decode(uint32_t k) { return f32_from_key(k); }
    // key of f32::MIN / f32::MAX (the MaxOp / MinOp identities)
    __device__ __forceinline__ static uint32_t max_identity() { return f32_key_max(-3.40282347e+38f); }
    __device__ __forceinline__ static uint32_t min_identity() { return f32_key_min(3.40282347e+38f); }
};
template <> struct Key<uint32_t> {
    __device__ __forceinline__ static uint32_t max_key(uint32_t x) { return x; }
    __device__ __forceinline__ static uint32_t min_key(uint32_t x) { return x; }
    __device__ __forceinline__ static uint32_t decode(uint32_t k) { return k; }
    __device__ __forceinline__ static uint32_t max_identity() { return 0u; }
    __device__ __forceinline__ static uint32_t min_identity() { return 0xFFFFFFFFu; }
};
template <> struct Key<int32_t> {
    __device__ __forceinline__ static uint32_t max_key(int32_t x) { return (uint32_t)x ^ 0x80000000u; }
    __device__ __forceinline__ static uint32_t min_key(int32_t x) { return (uint32_t)x ^ 0x80000000u; }
    __device__ __forceinline__ static int32_t decode(uint32_t k) { return (int32_t)(k ^ 0x80000000u); }
    __device__ __forceinline__ static uint32_t max_identity() { return 0u; }
    __device__ __forceinline__ static uint32_t min_identity() { return 0xFFFFFFFFu; }
};

// Argmax packs (key, index) into one u64 so that an unsigned max picks the
// largest key and, among equal keys, the LOWEST index:
//   packed = key << 32 | ~index.
// Packed 0 means "no element" (empty input, or only NaN for f32).
__device__ __forceinline__ uint64_t pack_arg(uint32_t key, uint32_t index) {
    return ((uint64_t)key << 32) | (uint64_t)(~index);
}
__device__ __forceinline__ uint32_t arg_index(uint64_t packed) {
    return ~(uint32_t)(packed & 0xFFFFFFFFull);
}
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// ------------------------------------------------------------- XCD order
// The dispatcher hands workgroups to the eight XCDs round robin (block b
// runs on XCD b % 8).  Where blocks may take their ranges in any order,
// xcd_contiguous(b, G) -- a permutation of [0, G) -- gives each XCD one
// contiguous run of ranges.  Measured on MI355X over 1 GiB, against range b
// per block: 256 KiB read-only tiles 157.3 -> 154.4 us, the copy tiles
// 337.5 -> 332 us, 65536 x 4096 fused rows 151.7 -> 149.5 us.  Not a
// general win: 16 KiB axpy tiles slowed 523 -> 539 us, and contiguous
// per-block ranges in the grid-stride full reduction 151 -> 213 us, so
// those keep block order.  Scans cannot use it: a look-back needs every
// tile's predecessors dispatched before it.
constexpr uint32_t kXcds = 8;
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t b, uint32_t G) {
    if (G % kXcds != 0) return b;
    return (b % kXcds) * (G / kXcds) + b / kXcds;
}

// ---------------------------------------------------- wave64 collectives
// Butterfly (xor) reductions: every lane ends with the same bits, and the
// combination tree is fixed, so results are deterministic.

template <typename T> __device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v + __shfl_xor(v, m, kWave);
    return v;
}
template <typename T> __device__ __forceinline__ T wave_prod(T v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = v * __shfl_xor(v, m, kWave);
    return v;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) { uint32_t o = __shfl_xor(v, m, kWave); v = v > o ? v : o; }
    return v;
}
__device__ __forceinline__ uint32_t wave_umin(uint32_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) { uint32_t o = __shfl_xor(v, m, kWave); v = v < o ? v : o; }
    return v;
}
__device__ __forceinline__ uint64_t wave_umax64(uint64_t v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = umax64(v, __shfl_xor(v, m, kWave));
    return v;
}

template <typename Op, typename A> __device__ __forceinline__ A wave_reduce(A v);
template <> __device__ __forceinline__ double wave_reduce<OpSum, double>(double v) { return wave_sum(v); }
template <> __device__ __forceinline__ uint32_t wave_reduce<OpSum, uint32_t>(uint32_t v) { return wave_sum(v); }
template <> __device__ __forceinline__ float wave_reduce<OpSum, float>(float v) { return wave_sum(v); }
template <> __device__ __forceinline__ double wave_reduce<OpProd, double>(double v) { return wave_prod(v); }
template <> __device__ __forceinline__ uint32_t wave_reduce<OpProd, uint32_t>(uint32_t v) { return wave_prod(v); }
template <> __device__ __forceinline__ float wave_reduce<OpProd, float>(float v) { return wave_prod(v); }

// ------------------------------------------------------- DPP lane moves
// GFX9 data-parallel-primitive controls.  A DPP move reads another lane's
// register inside the VALU instruction itself (no LDS round trip, unlike a
// generic shuffle).  Lanes whose source is outside the pattern, and lanes of
// rows masked off, receive `fill`.
constexpr int kDppRowShr1 = 0x111;    // lane l <- l-1 within its row of 16
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;
constexpr int kDppWaveShr1 = 0x138;   // lane l <- l-1 across the wave
constexpr int kDppRowBcast15 = 0x142; // row r <- lane 15 of row r-1
constexpr int kDppRowBcast31 = 0x143; // rows 2,3 <- lane 31

template <int CTRL, int ROW_MASK = 0xf, typename A> __device__ __forceinline__ A dpp_move(A fill, A v) {
    static_assert(sizeof(A) == 4, "DPP moves are 32-bit");
    const int r = __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill), __builtin_bit_cast(int, v), CTRL,
                                              ROW_MASK, 0xf, false);
    return __builtin_bit_cast(A, r);
}

// Value of lane `src` (uniform result).
template <typename A> __device__ __forceinline__ A read_lane(A v, int src) {
    static_assert(sizeof(A) == 4, "32-bit lanes");
    return __builtin_bit_cast(A, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// Lane permutations inside each row of 16 whose sources are always in range:
// quad xor 1 (quad_perm [1,0,3,2]), quad xor 2 ([2,3,0,1]), the 8-lane
// mirror (l <-> 7-l) and the 16-lane mirror (l <-> 15-l).
constexpr int kDppQuadXor1 = 0xB1;
constexpr int kDppQuadXor2 = 0x4E;
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL, typename A> __device__ __forceinline__ A dpp_permute(A v) {
    if constexpr (sizeof(A) == 4) {
        return dpp_move<CTRL>(v, v);
    } else {
        static_assert(sizeof(A) == 8, "4- or 8-byte lanes");
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = dpp_move<CTRL>((uint32_t)b, (uint32_t)b);
        const uint32_t hi = dpp_move<CTRL>((uint32_t)(b >> 32), (uint32_t)(b >> 32));
        return __builtin_bit_cast(A, (uint64_t)lo | ((uint64_t)hi << 32));
    }
}
template <typename A> __device__ __forceinline__ A read_lane_any(A v, int src) {
    if constexpr (sizeof(A) == 4) {
        return read_lane(v, src);
    } else {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = read_lane((uint32_t)b, src), hi = read_lane((uint32_t)(b >> 32), src);
        return __builtin_bit_cast(A, (uint64_t)lo | ((uint64_t)hi << 32));
    }
}

// Reduction over aligned groups of G lanes (G = 4, 16 or 64) with DPP moves
// instead of LDS shuffles: quad xor 1 and 2, then (G >= 16) the 8- and
// 16-lane mirrors, then (G = 64) the four rows of 16 read with readlane and
// combined as (r0 . r1) . (r2 . r3).  After each DPP step every lane of the
// sub-group holds the same bits (f is commutative), so every lane of a group
// ends with the group's value (wave-uniform for G = 64) and the tree is fixed:
// floating-point results are deterministic.  Every lane of the wave must be
// active: DPP reads of disabled lanes return the reader's own value.
template <int G, typename A, typename F> __device__ __forceinline__ A group_reduce(A v, F f) {
    static_assert(G == 4 || G == 16 || G == 64, "groups of 4, 16 or 64 lanes");
    v = f(v, dpp_permute<kDppQuadXor1>(v));
    v = f(v, dpp_permute<kDppQuadXor2>(v));
    if constexpr (G >= 16) {
        v = f(v, dpp_permute<kDppRowHalfMirror>(v));
        v = f(v, dpp_permute<kDppRowMirror>(v));
    }
    if constexpr (G == 64)
        v = f(f(read_lane_any(v, 0), read_lane_any(v, 16)), f(read_lane_any(v, 32), read_lane_any(v, 48)));
    return v;
}

// Inclusive scan across the 64 lanes: Hillis-Steele inside each row of 16
// lanes (shifts 1, 2, 4, 8), then the row totals are carried forward with
// the two row broadcasts (lane 15 into rows 1 and 3, lane 31 into rows 2
// and 3).  Six DPP steps for 32-bit values; other widths use shuffles.
template <typename Op, typename A> __device__ __forceinline__ A wave_inclusive_scan(A v) {
    if constexpr (sizeof(A) == 4) {
        const A id = Op::template identity<A>();
        v = Op::combine(dpp_move<kDppRowShr1>(id, v), v);
        v = Op::combine(dpp_move<kDppRowShr2>(id, v), v);
        v = Op::combine(dpp_move<kDppRowShr4>(id, v), v);
        v = Op::combine(dpp_move<kDppRowShr8>(id, v), v);
        v = Op::combine(dpp_move<kDppRowBcast15, 0xa>(id, v), v);
        v = Op::combine(dpp_move<kDppRowBcast31, 0xc>(id, v), v);
        return v;
    } else {
        const int lane = lane_id();
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            A t = __shfl_up(v, d, kWave);
            if (lane >= d) v = Op::combine(t, v);
        }
        return v;
    }
}

// Exclusive form of an inclusive wave scan: lane l gets lane l-1's value,
// lane 0 the identity.
template <typename Op, typename A> __device__ __forceinline__ A wave_shift_right(A incl) {
    return dpp_move<kDppWaveShr1>(Op::template identity<A>(), incl);
}

template <typename A> __device__ __forceinline__ A wave_broadcast(A v, int src) { return __shfl(v, src, kWave); }

// 64-bit lane masks from wave-wide predicates.
__device__ __forceinline__ uint64_t ballot(bool p) { return (uint64_t)__ballot(p); }

// ---------------------------------------------------- agent-scope atomics
// Look-back status words are read and written with agent-scope atomics so
// every XCD's L2 observes them coherently.

__device__ __forceinline__ uint64_t ld_relaxed(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_acquire(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_relaxed32(const uint32_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed(uint64_t *p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_release32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed32(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fetch_add32(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t fetch_add32_acqrel(uint32_t *p, uint32_t v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed_f64(double *p, double v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ double ld_relaxed_f64(const double *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------- single-launch grid folds
// A grid reduction in one launch: every block but the last publishes its
// partial as self-tagged words with relaxed agent-scope stores; the last
// block -- dispatched last -- gathers them.  A reader accepts a partial only
// when every half carries this launch's tag, so no release/acquire pair
// (which on multi-XCD CDNA writes back and invalidates the L2) is needed.
// Slot words start zeroed and tags are never 0.
//
// A slot word has the layout of a look-back status word -- high half
// (tag << 2) | flag, low half 32 bits of the value -- with flag 3
// (kSlotFlag), which no look-back status uses (they use 1 and 2).  Slots
// and statuses share one workspace region and one tag counter, so a slot
// never reads a status word left by another kernel as a current partial,
// whatever the two launches' tags.
// The look-back statuses (scan.hip, segmented.hip) build their high halves
// with status_word_hi as well.
constexpr uint32_t kSlotFlag = 3;
__host__ __device__ __forceinline__ uint32_t status_word_hi(uint32_t tag, uint32_t flag) { return (tag << 2) | flag; }
__host__ __device__ __forceinline__ uint32_t slot_word_hi(uint32_t tag) { return status_word_hi(tag, kSlotFlag); }

// The 16-byte f64 status slot of the f32 tile scans (scan.hip
// F64QuadStatus): dword i = (check << 16) | bits [63-16i : 48-16i] of the
// value, check = status_word_hi(tag, flag) with tag < 2^14.  decode gives
// flag 0 unless all four checks are equal and carry `tag`, so a read that
// mixes dwords of two writes, or meets words of the 64-bit formats above
// (whose high halves are below 2^16, while a check dword is >= 2^18), reads
// as not ready.
__host__ __device__ __forceinline__ void slot16_encode(uint32_t tag, uint32_t flag, uint64_t b, uint32_t (&q)[4]) {
    const uint32_t c = status_word_hi(tag, flag) << 16;
    q[0] = c | (uint32_t)(b >> 48);
    q[1] = c | ((uint32_t)(b >> 32) & 0xFFFFu);
    q[2] = c | ((uint32_t)(b >> 16) & 0xFFFFu);
    q[3] = c | ((uint32_t)b & 0xFFFFu);
}
__host__ __device__ __forceinline__ uint32_t slot16_decode(uint32_t tag, const uint32_t (&q)[4], uint64_t &b) {
    const uint32_t c = q[0] >> 16;
    const bool same = (((q[0] ^ q[1]) | (q[0] ^ q[2]) | (q[0] ^ q[3])) >> 16) == 0u;
    b = ((uint64_t)(q[0] & 0xFFFFu) << 48) | ((uint64_t)(q[1] & 0xFFFFu) << 32) | ((uint64_t)(q[2] & 0xFFFFu) << 16) |
        (uint64_t)(q[3] & 0xFFFFu);
    return (same && (c >> 2) == tag) ? (c & 3u) : 0u;
}
template <typename Acc> struct PartialSlot {
    static_assert(sizeof(Acc) == 4 || sizeof(Acc) == 8, "partials are 32- or 64-bit");
    static constexpr uint32_t kWords = sizeof(Acc) / 4;
    __device__ __forceinline__ static void publish(uint64_t *w, uint32_t tag, Acc v) {
        const uint64_t t = (uint64_t)slot_word_hi(tag) << 32;
        if constexpr (kWords == 1) {
            st_relaxed(w, t | __builtin_bit_cast(uint32_t, v));
        } else {
            const uint64_t b = __builtin_bit_cast(uint64_t, v);
            st_relaxed(&w[0], t | (b & 0xFFFFFFFFull));
            st_relaxed(&w[1], t | (b >> 32));
        }
    }
    __device__ __forceinline__ static bool read(const uint64_t *w, uint32_t tag, Acc &v) {
        const uint32_t want = slot_word_hi(tag);
        if constexpr (kWords == 1) {
            const uint64_t a = ld_relaxed(w);
            v = __builtin_bit_cast(Acc, (uint32_t)a);
            return (uint32_t)(a >> 32) == want;
        } else {
            const uint64_t a = ld_relaxed(&w[0]), b = ld_relaxed(&w[1]);
            v = __builtin_bit_cast(Acc, (a & 0xFFFFFFFFull) | (b << 32));
            return (uint32_t)(a >> 32) == want && (uint32_t)(b >> 32) == want;
        }
    }
};

// Run by every thread of the last block of a G-block grid (G <= MAXP) once
// its own partial `own` is known: leaves partial k of every block in
// vals[k] (LDS).  Each thread loads its slots (t, t + BLOCK, ...) in one
// round -- one memory round trip in the common case -- then polls those
// still unpublished.  A partial missing after `poll_limit` polls (16384 by
// default: each poll is a memory round trip plus a short sleep, so that is
// milliseconds, while partials normally land within microseconds) is
// recomputed by `recompute(k)`, a block-uniform call that returns block k's
// partial with the streaming code, so the value is bit-identical and the
// launch finishes whatever the dispatch order.  poll_limit 0 skips the
// slots and recomputes every partial (a test of that path).  `missing` is
// MAXP / 32 words of LDS.
template <int BLOCK, int MAXP, typename Acc, typename Recompute>
__device__ __forceinline__ void gather_partials(const uint64_t *slots, uint32_t tag, uint32_t poll_limit, uint32_t G,
                                                Acc own, Acc *vals, uint32_t *missing, Recompute &&recompute) {
    using Slot = PartialSlot<Acc>;
    constexpr int kPer = MAXP / BLOCK;
    static_assert(MAXP % BLOCK == 0 && MAXP % 32 == 0, "whole slots per thread");
    const uint32_t last = G - 1;
    for (uint32_t k = threadIdx.x; k < MAXP / 32; k += BLOCK) missing[k] = 0u;
    __syncthreads();
    Acc v[kPer];
    bool ok[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t k = threadIdx.x + (uint32_t)i * BLOCK;
        ok[i] = k >= last || (poll_limit != 0 && Slot::read(slots + (uint64_t)k * Slot::kWords, tag, v[i]));
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t k = threadIdx.x + (uint32_t)i * BLOCK;
        if (k >= last) continue;
        uint32_t polls = 0;
        while (!ok[i] && polls++ < poll_limit) {
            __builtin_amdgcn_s_sleep(2);
            ok[i] = Slot::read(slots + (uint64_t)k * Slot::kWords, tag, v[i]);
        }
        if (ok[i])
            vals[k] = v[i];
        else
            atomicOr(&missing[k / 32], 1u << (k % 32));
    }
    if (threadIdx.x == 0) vals[last] = own;
    __syncthreads();
    for (uint32_t wd = 0; wd * 32 < last; ++wd) {
        uint32_t m = missing[wd];
        while (m != 0u) {
            const uint32_t k = wd * 32 + (uint32_t)__builtin_ctz(m);
            m &= m - 1u;
            const Acc r = recompute(k);
            if (threadIdx.x == 0) vals[k] = r;
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------ generator
// SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014): output i for seed s is mix(s + (i+1)*gamma).
__host__ __device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

} // namespace hx
