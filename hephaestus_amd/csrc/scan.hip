// Prefix scans for gfx950: ScanOps (crates/hephaestus-core/src/domain/
// scan.rs:197-264), extended with the exclusive form and rank-1 operands.
//
// The reference launches ONE 256-lane block per scan line; each lane walks a
// contiguous chunk serially, lane 0 folds the chunk totals, and a second sweep
// re-reads and re-writes the output (core accelerator/scan.rs:56-155).  A 1-D
// scan of 2^28 elements therefore runs on one CU.  Here every line is cut
// into tiles that all CUs process in a single pass (32768 elements for long
// lines; a line of up to 32768 elements is one tile of the smallest shape
// that holds it, see tile_shape):
//
//   * block b scans tile b.  The tile is loaded with 16-byte vectors,
//     wave-striped: step j of wave w holds 256 contiguous elements, lane l
//     four of them; each step is a 4-element register scan plus a 6-step
//     wave64 scan of the lane totals;
//   * the tile aggregate is published, wave 0 looks back for the tile's
//     exclusive prefix and publishes the tile's inclusive prefix;
//   * every element is read once and written once, 16-byte vectors again.
//
// The look-back has two levels.  Tiles are grouped in superblocks of 64; the
// last tile of a superblock also publishes the superblock's aggregate (as
// soon as its 63 predecessors have published theirs) and later its
// inclusive prefix.  A tile first folds its own superblock's predecessors
// (one poll of 64 lanes) and then whole superblocks, 64 per poll.  With ~2000
// tiles in flight, a flat look-back walks up to ~32 sequential polls to
// reach a published prefix; the two levels need about two.
//
// Forward progress does not depend on the order in which the hardware
// dispatches blocks: when a status stays unpublished for p.spin_limit polls
// (its block may not be running yet), the waiting wave computes the missing
// value itself -- a tile aggregate from the input with the owner's
// arithmetic, a superblock value from its tiles' statuses -- and publishes
// it ("decoupled fallback", Smith, Levien and Owens 2024).  There is no
// tile-ticket counter: one same-address device-scope atomic per tile
// serialises at ~11 ns on MI355X, which alone cost 745 us for 65536 tiles.
//
// Status words carry a 14-bit per-launch tag (set by the host), so a launch
// never clears the status array and needs no end-of-launch bookkeeping.
// Integer scans publish (tag, flag, value) in ONE 64-bit word.  f32 scans
// carry the inter-tile prefix in f64 (every output stays within a few ulp of
// the f32-rounded exact prefix at 2^30 elements) in ONE 16-byte slot, read
// and written with one 16-byte access; each of its four dwords carries the
// tag and flag next to 16 bits of the value.
#include "hx_device.hpp"
#include "hx_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace hx {
namespace {

constexpr int kBlock = 256;                          // column-scan kernels
constexpr int kWaves = 8;                            // waves per tile block (long lines)
constexpr int kSteps = 16;                           // 16-byte vectors per lane (long lines)
constexpr int kSuper = 64;                           // tiles per superblock
constexpr uint32_t kInvalid = 0, kAggregate = 1, kPrefix = 2;

__device__ __forceinline__ uint64_t status_word(uint32_t tag, uint32_t flag, uint32_t v) {
    return ((uint64_t)status_word_hi(tag, flag) << 32) | (uint64_t)v;
}

// Tile statuses sit one per 128-byte line.  Tiles publish their statuses
// at about the same moment from CUs all over the chip, through to memory;
// packed densely, 16 of them shared a line.  Measured on MI355X, 2^28 u32
// exclusive scan, one process: status stride 8 bytes 336.3 us, 16: 334.7,
// 32: 332.6, 64: 331.6, 128: 328.8, 256: 328.5; 2^30 f32 inclusive scan,
// 16-byte slots: 1313.6 us, 128-byte stride 1291.0.  The column look-back
// (lanes across lines, polled as one contiguous run) keeps dense words.
constexpr uint64_t kTileStatusBytes = 128;

// (tag, flag, value) in one 64-bit word: [63:34] tag, [33:32] flag, [31:0]
// value; entry t at word t * STRIDE.
template <uint32_t STRIDE> struct PackedStatusT {
    using C = uint32_t;
    uint64_t *words;
    __device__ __forceinline__ uint64_t *at(uint64_t t) const { return words + t * STRIDE; }
    __device__ __forceinline__ void publish(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        st_relaxed(at(t), status_word(tag, flag, v));
    }
    // Fallback publication: never overwrites a word of this launch (so a
    // published inclusive prefix is never downgraded to an aggregate).
    __device__ __forceinline__ void publish_if_unset(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        uint64_t cur = ld_relaxed(at(t));
        if ((uint32_t)(cur >> 34) == tag) return;
        __hip_atomic_compare_exchange_strong(at(t), &cur, status_word(tag, flag, v), __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Tile-level owner publication (same single store).
    __device__ __forceinline__ void publish_tile(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        publish(t, tag, flag, v);
    }
    __device__ __forceinline__ void read(uint64_t t, uint32_t tag, uint32_t &flag, C &v) const {
        const uint64_t w = ld_relaxed(at(t));
        const uint32_t hi = (uint32_t)(w >> 32);
        flag = ((hi >> 2) == tag) ? (hi & 3u) : kInvalid;
        v = (uint32_t)w;
    }
};
using PackedStatus = PackedStatusT<1>;                             // column look-back
using TilePackedStatus = PackedStatusT<kTileStatusBytes / 8>;      // tile scans

// f64 carries of the tile scans: one 16-byte slot per entry (at the start of
// the entry's 128-byte line; adjacent slots for row-tile columns), overwritten by
// its single writer (aggregate, then inclusive prefix) and read with ONE
// 16-byte load per lane.  Dword i of the slot is (check << 16) | bits
// [63-16i : 48-16i] of the f64, with check = (tag << 2) | flag (tags below
// 2^14; slot16_encode / slot16_decode).  A reader accepts the slot only when the four checks agree with
// each other and carry this launch's tag, so only 32-bit single-copy
// atomicity is assumed: a read that mixes dwords of two writes (aggregate
// and prefix, or an earlier launch's words) never has four equal checks.
// Words of the packed and partial-slot formats left in the same area read as
// not ready: their high halves are below 2^16, a check dword is at least
// 2^18.  Measured against two self-tagged 8-byte words read with two loads,
// 2^30 f32 inclusive scan on MI355X: 1360 -> 1315 us; the number of loads
// per poll, not their cache scope, set the difference (agent and system
// scope both 1360 us).
template <uint32_t STRIDE> struct F64QuadStatusT {
    using C = double;
    typedef uint32_t slot_t __attribute__((ext_vector_type(4)));
    uint64_t *words;
    __device__ __forceinline__ volatile __attribute__((address_space(1))) slot_t *slot(uint64_t t) const {
        return (volatile __attribute__((address_space(1))) slot_t *)(words + t * STRIDE);
    }
    __device__ __forceinline__ void publish(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        uint32_t w[4];
        slot16_encode(tag, flag, __builtin_bit_cast(uint64_t, v), w);
        slot_t q;
        q.x = w[0];
        q.y = w[1];
        q.z = w[2];
        q.w = w[3];
        *slot(t) = q;
    }
    __device__ __forceinline__ void publish_tile(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        publish(t, tag, flag, v);
    }
    // Slots have one writer: waiters that compute a missing value keep it
    // to themselves (SharedFallback).
    __device__ __forceinline__ void publish_if_unset(uint64_t, uint32_t, uint32_t, C) const {}
    __device__ __forceinline__ void read(uint64_t t, uint32_t tag, uint32_t &flag, C &v) const {
        const slot_t q = *slot(t);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
        uint64_t b;
        flag = slot16_decode(tag, w, b);
        v = __builtin_bit_cast(double, b);
    }
};
using F64QuadStatus = F64QuadStatusT<kTileStatusBytes / 8>; // tile scans: one slot per 128-byte line
using F64QuadDense = F64QuadStatusT<2>;                     // row-tile columns: adjacent slots

// f64 values for the single-pass column scan: one slot of two self-tagged
// words (high and low halves) per entry, which the owner writes twice --
// aggregate, then inclusive prefix.  A reader accepts the slot only when both
// halves carry this launch's tag and the same flag; a half-updated slot reads
// as not ready.  Every slot has exactly one writer (waiters that give up
// compute the value themselves and do not publish it), so halves of
// different values can only meet transiently.
struct F64PairStatus {
    using C = double;
    uint64_t *words;
    __device__ __forceinline__ void publish_tile(uint64_t t, uint32_t tag, uint32_t flag, C v) const {
        const uint64_t b = __builtin_bit_cast(uint64_t, v);
        st_relaxed(&words[2 * t], status_word(tag, flag, (uint32_t)(b >> 32)));
        st_relaxed(&words[2 * t + 1], status_word(tag, flag, (uint32_t)b));
    }
    __device__ __forceinline__ void publish_if_unset(uint64_t, uint32_t, uint32_t, C) const {}
    __device__ __forceinline__ void read(uint64_t t, uint32_t tag, uint32_t &flag, C &v) const {
        const uint64_t hi = ld_relaxed(&words[2 * t]), lo = ld_relaxed(&words[2 * t + 1]);
        const uint32_t h = (uint32_t)(hi >> 32), l = (uint32_t)(lo >> 32);
        flag = (h == l && (h >> 2) == tag) ? (h & 3u) : kInvalid;
        v = __builtin_bit_cast(double, (hi << 32) | (lo & 0xFFFFFFFFull));
    }
};

// Whether waiters that compute a missing status publish it for others
// (publish_if_unset, a CAS on a single word) or keep it to themselves.
template <typename S> struct SharedFallback { static constexpr bool value = true; };
template <uint32_t STRIDE> struct SharedFallback<F64QuadStatusT<STRIDE>> { static constexpr bool value = false; };

struct ScanParams {
    const void *in;
    void *out;
    uint64_t lines, len, tiles_per_line, total_tiles, supers_per_line;
    int64_t in_line_stride, in_elem_stride;
    int64_t out_line_stride, out_elem_stride;
    uint64_t in_offset, out_offset;
    uint32_t tag;        // this launch's status tag
    uint32_t spin_limit; // polls before a waiter computes a missing value (64)
    uint64_t tile0;      // tile of block 0 (tile kernels launched in batches)
    uint32_t head;       // tile lines: elements [0, head) of the line are virtual (scan_out_head)
};

// The four elements of one lane and step (logical index e..e+3 of the
// line), identity past the end and, with HEAD, before p.head.
template <typename T, bool VEC, bool REV, bool NT, bool HEAD>
__device__ __forceinline__ void load4(const ScanParams &p, const T *in, int64_t ib, uint64_t e, T ident,
                                      T (&v)[4]) {
    const uint64_t head = HEAD ? p.head : 0u;
    if constexpr (VEC) {
        if (e + 3 < p.len && e >= head) {
            using V = typename Vec4A4<T>::type;
            if constexpr (REV) {
                // Logical e..e+3 are physical len-1-e down to len-4-e.
                const V q = load_a4<NT>((const V *)(in + ib + (int64_t)(p.len - 4 - e)));
                v[0] = (T)q.w;
                v[1] = (T)q.z;
                v[2] = (T)q.y;
                v[3] = (T)q.x;
            } else {
                const V q = load_a4<NT>((const V *)(in + ib + (int64_t)e));
                v[0] = (T)q.x;
                v[1] = (T)q.y;
                v[2] = (T)q.z;
                v[3] = (T)q.w;
            }
            return;
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint64_t i = e + c;
        const uint64_t li = REV ? (p.len - 1 - i) : i;
        v[c] = (i < p.len && i >= head) ? in[ib + (int64_t)li * p.in_elem_stride] : ident;
    }
}

// A lane's left-to-right fold of its four elements; the owner and the
// fallback both build step totals from it the same way.
template <typename T, typename Op>
__device__ __forceinline__ T lane_fold(const T (&v)[4]) {
    return Op::combine(Op::combine(Op::combine(v[0], v[1]), v[2]), v[3]);
}

// Aggregate of tile `u` computed by ONE wave, step by step, with the same
// operations and order as the four owner waves (fallback path).
template <typename T, typename Op, bool VEC, bool REV, bool NT, int STEPS, int WAVES, bool HEAD>
__device__ T tile_aggregate(const ScanParams &p, uint64_t u) {
    constexpr int kWaveElems = kWave * 4 * STEPS;
    constexpr int kTileElems = WAVES * kWaveElems;
    const T ident = Op::template identity<T>();
    const uint64_t line = u / p.tiles_per_line;
    const uint64_t tin = u - line * p.tiles_per_line;
    const int64_t ib = (int64_t)p.in_offset + (int64_t)line * p.in_line_stride;
    const T *in = (const T *)p.in;
    T agg = ident;
    for (int w = 0; w < WAVES; ++w) {
        T carry = ident;
        for (int j = 0; j < STEPS; ++j) {
            T v[4];
            load4<T, VEC, REV, NT, HEAD>(p, in, ib,
                                   tin * kTileElems + (uint64_t)w * kWaveElems + (uint64_t)j * (kWave * 4) +
                                       (uint64_t)lane_id() * 4,
                                   ident, v);
            const T incl = wave_inclusive_scan<Op, T>(lane_fold<T, Op>(v));
            carry = Op::combine(carry, read_lane(incl, kWave - 1));
        }
        agg = Op::combine(agg, carry);
    }
    return agg;
}

// The look-back reaches the tile's own aggregate through a hook: poll() runs
// on every spin, agg() yields the aggregate.  KnownAgg: the aggregate is
// already computed and published when the look-back starts.  (A variant
// whose fifth wave starts looking back while the data waves still load, and
// publishes the aggregate from poll(), measured 19% slower at 2^28 u32: the
// extra wave's registers cut occupancy and its polls span the whole load.)
template <typename C> struct KnownAgg {
    C a;
    __device__ __forceinline__ void poll() {}
    __device__ __forceinline__ C agg() { return a; }
};

// Wave-wide fold of the look-back values.  f64 carries fold with DPP moves
// (no lane-address registers, which the shuffle form keeps live across the
// whole look-back); 32-bit values keep the shuffle butterfly.
template <typename Op, typename C> __device__ __forceinline__ C lookback_reduce(C v) {
    if constexpr (sizeof(C) == 8)
        return group_reduce<64>(v, [](C a, C b) { return Op::combine(a, b); });
    else
        return wave_reduce<Op, C>(v);
}

// Fold of the statuses of the `count` (<= 64) tiles just before tile
// `tile_end`, nearest first, stopping at the first inclusive prefix; `found`
// tells whether one was met.  Lane l reads the tile at distance l.  A tile
// that stays unpublished is computed by tile_aggregate: published for every
// waiter where the status takes shared fallbacks, else kept in the lane that
// reads that tile.
template <typename T, typename Op, typename Status, bool VEC, bool REV, bool NT, int STEPS, int WAVES, bool HEAD,
          typename Hook>
__device__ typename Status::C fold_tiles(const ScanParams &p, const Status &st, uint64_t tile_end, int count,
                                         bool &found, Hook &hook) {
    using C = typename Status::C;
    const int lane = lane_id();
    const C ident = Op::template identity<C>();
    uint32_t flag;
    C val;
    uint32_t spins = 0;
    constexpr bool kShared = SharedFallback<Status>::value;
    bool own = false; // this lane's tile aggregate, computed by this wave
    C own_val = ident;
    for (;;) {
        flag = kAggregate; // lanes past `count`: valid, not a prefix, identity
        val = ident;
        if (lane < count) st.read(tile_end - 1 - lane, p.tag, flag, val);
        if constexpr (!kShared) {
            if (own && flag == kInvalid) {
                flag = kAggregate;
                val = own_val;
            }
        }
        const uint64_t pm = ballot(flag == kPrefix);
        const uint64_t im = ballot(flag == kInvalid);
        // Every status up to and including the nearest prefix is needed.
        const uint64_t need = pm ? (((pm & (~pm + 1ull)) << 1) - 1ull) : ~0ull;
        const uint64_t missing = im & need;
        if (missing == 0ull) break;
        hook.poll();
        if (++spins >= p.spin_limit) {
            const int k = __ffsll((long long)missing) - 1;
            const uint64_t u = tile_end - 1 - (uint64_t)k;
            const T a = tile_aggregate<T, Op, VEC, REV, NT, STEPS, WAVES, HEAD>(p, u);
            if constexpr (kShared) {
                if (lane == 0) st.publish_if_unset(u, p.tag, kAggregate, (C)a);
            } else if (lane == k) {
                own = true;
                own_val = (C)a;
            }
            spins = 0;
            continue;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    const uint64_t pm = ballot(flag == kPrefix);
    const int first = pm ? (__ffsll((long long)pm) - 1) : kWave;
    found = pm != 0ull;
    return lookback_reduce<Op, C>((lane <= first) ? val : ident);
}

// Exclusive prefix of tile `tile` (position `tin` in its line), computed by
// one wave.  The last tile of a superblock publishes the superblock
// aggregate on the way (it needs the tile's own aggregate: hook.agg()).
template <typename T, typename Op, typename Status, bool VEC, bool REV, bool NT, int STEPS, int WAVES, bool HEAD,
          typename Hook>
__device__ typename Status::C lookback(const ScanParams &p, const Status &st, const Status &st1, uint64_t tile,
                                       uint64_t line, uint64_t tin, Hook &hook) {
    using C = typename Status::C;
    const int lane = lane_id();
    const C ident = Op::template identity<C>();
    const int pos = (int)(tin % kSuper);
    const uint64_t sb = tin / kSuper;
    const uint64_t line_super = line * p.supers_per_line;
    const bool last_in_super = pos == kSuper - 1 && tin + 1 < p.tiles_per_line;

    // Level 0: predecessors in the tile's own superblock.
    bool found = false;
    C excl = pos > 0 ? fold_tiles<T, Op, Status, VEC, REV, NT, STEPS, WAVES, HEAD>(p, st, tile, pos, found, hook) : ident;
    if (found) return excl; // superblock 0 always ends here (tile 0 is a prefix)
    if (last_in_super) {
        const C a = hook.agg();
        if (lane == 0) st1.publish(line_super + sb, p.tag, kAggregate, Op::combine(excl, a));
    }

    // Level 1: whole superblocks, nearest first.
    int64_t pred = (int64_t)(line_super + sb) - 1;
    for (;;) {
        const int64_t idx = pred - lane;
        const bool in_line = idx >= (int64_t)line_super;
        uint32_t flag;
        C val;
        uint32_t spins = 0;
        constexpr bool kShared = SharedFallback<Status>::value;
        uint32_t own_flag = kInvalid; // this lane's superblock, rebuilt by this wave
        C own_val = ident;
        for (;;) {
            flag = kPrefix; // before the line's first superblock: identity
            val = ident;
            if (in_line) st1.read((uint64_t)idx, p.tag, flag, val);
            if constexpr (!kShared) {
                if (flag == kInvalid && own_flag != kInvalid) {
                    flag = own_flag;
                    val = own_val;
                }
            }
            const uint64_t pm = ballot(flag == kPrefix);
            const uint64_t im = ballot(flag == kInvalid);
            const uint64_t need = pm ? (((pm & (~pm + 1ull)) << 1) - 1ull) : ~0ull;
            const uint64_t missing = im & need;
            if (missing == 0ull) break;
            hook.poll();
            if (++spins >= p.spin_limit) {
                // Rebuild the missing superblock's value from its 64 tiles:
                // an inclusive prefix if one of them has one, else the sum.
                const int k = __ffsll((long long)missing) - 1;
                const uint64_t s = (uint64_t)(pred - k);
                const uint64_t s_end = line * p.tiles_per_line + (s - line_super + 1) * kSuper;
                bool f = false;
                const C v = fold_tiles<T, Op, Status, VEC, REV, NT, STEPS, WAVES, HEAD>(p, st, s_end, kSuper, f, hook);
                if constexpr (kShared) {
                    if (lane == 0) st1.publish_if_unset(s, p.tag, f ? kPrefix : kAggregate, v);
                } else if (lane == k) {
                    own_flag = f ? kPrefix : kAggregate;
                    own_val = v;
                }
                spins = 0;
                continue;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        const uint64_t pm = ballot(flag == kPrefix);
        const int first = pm ? (__ffsll((long long)pm) - 1) : kWave;
        excl = Op::combine(excl, lookback_reduce<Op, C>((lane <= first) ? val : ident));
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

// The tile's exclusive prefix applied to an element's in-tile prefix.
// Integers: one combine.  f32 with an f64 carry: the carry is split once per
// tile into f32 hi + lo (lo = the f32 rounding of carry - hi, exact to
// ~2^-48 relative) and each output is hi + (within + lo) (sums) or
// fma(hi, within, lo * within) (products), about one ulp from the f64
// combine rounded to f32 and far inside 2 ceil(log2 n) eps sum|x|.  The f64
// form converts every element to f64: the compiler hoists those conversions
// above the store branch and holds 96 extra registers, which kept f32 tiles
// at one block per CU.  A non-finite hi takes lo = 0 (hi + w then gives the
// f64 form's inf or NaN).
template <typename T, typename C, typename Op> struct TileCarry {
    T c;
    __device__ __forceinline__ explicit TileCarry(C v) : c((T)v) {}
    __device__ __forceinline__ T apply(T within) const { return Op::combine(c, within); }
};
template <typename Op> struct TileCarry<float, double, Op> {
    float hi, lo;
    __device__ __forceinline__ explicit TileCarry(double v) {
        hi = (float)v;
        lo = __builtin_isfinite(hi) ? (float)(v - (double)hi) : 0.0f;
    }
    __device__ __forceinline__ float apply(float w) const {
        if constexpr (std::is_same<Op, OpSum>::value) {
            return hi + (w + lo);
        } else {
            // lo * w is not finite only where w is infinite or NaN, or the
            // product overflows; hi * w then gives the f64 form's inf, NaN
            // or sign (fma(hi, w, -inf) would turn +inf into NaN or -inf).
            const float lw = lo * w;
            return __builtin_isfinite(lw) ? __builtin_fmaf(hi, w, lw) : hi * w;
        }
    }
};

// Full tiles of unit-stride lines (every tile but a line's ragged last one;
// the vectors need only 4-byte alignment): a block-uniform base pointer plus one 32-bit lane offset,
// so each step is a single base + offset + immediate vector access with no
// bounds check and no per-step 64-bit address held in registers.
// A whole tile of a reverse scan is a mirrored block of memory: logical
// elements e..e+3 of a lane's step are one 16-byte vector in reversed order,
// at byte (tile_bytes - 16 - lane_off - j * 1024) from the block's lowest
// address (always >= 0).
// Tiles are held to 128 VGPRs, two 8-wave blocks per CU: the integer
// inclusive forms (131 VGPRs unconstrained, one block per CU) spill a few
// words of look-back state and still gain ~3% (2^28 u32 inclusive 0.388 ->
// 0.378 ms).  f32 tiles fit in 121 with no spill through three changes: the
// split carry (TileCarry), the DPP look-back fold (lookback_reduce), and wave
// 0's 64 data registers parked in LDS while it looks back (ParkTile), with
// the wave's exclusive offset read only after the look-back.  Before them
// f32 tiles needed ~150 and ran one 12-wave block per CU.
template <typename T> struct ScanWavesPerEu { static constexpr int value = 4; };

// f32 tiles park wave 0's data in LDS during the look-back (16 KiB per
// block).  Integer tiles fit without it (116 VGPRs); parking measured 0.4%
// slower there.
template <typename T> struct ParkTile { static constexpr bool value = false; };
template <> struct ParkTile<float> { static constexpr bool value = true; };

// Paced tiles (integer scans).  Two blocks share each CU, and the memory
// instructions of all their waves queue through the CU's one vector-memory
// path in issue order.  A block that has its carry issues its 16 stores per
// wave back to back, and the other block's loads -- the next tile's, which
// set the pace of the whole stream -- wait behind them.  So:
//   * a block whose tile has predecessors (it will look back) runs at wave
//     priority 3 from its start and drops to 0 for its stores: when waves of
//     both blocks are ready to issue, the loads go first;
//   * stores leave 32 idle cycles (four s_nop 7) between each other, so a
//     load that becomes ready during a block's store phase is issued at the
//     next gap instead of after the whole burst.
// Measured on MI355X, 2^28 u32 exclusive scan, one process: burst stores
// 356.9 us; gaps only 350.7-353.8; priority only 344.9; both 335.6 (gaps of
// s_sleep 1: 336.4, two or three s_nop 7: 336.5-336.8, six or eight: 335.7-
// 335.8, every second store only: 339.2; priority 3 for the loads and 1 for
// the look-back: 338.6).  At 2^30: 1405.5 -> 1323.2 us.  Lines of one tile
// (row-wise scans) never look back; for them the gaps alone pay (the same
// kernel without look-back: burst 363.9 us, gaps 341.1; with the priority as
// well 349.5), so they keep the default priority.  f32 tiles, two blocks
// per CU as well, gain the same way (2^30 f32: 1382.8 us unpaced, 1315.6
// paced).

__device__ __forceinline__ void store_gap() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

template <typename T, bool NT, int STEPS>
__device__ __forceinline__ void load_full_tile_rev(const T *base, uint32_t rev_off, T (&x)[STEPS][4]) {
    using V = typename Vec4A4<T>::type;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const V q = load_a4<NT>((const V *)((const char *)base + rev_off - (uint32_t)j * (kWave * 16)));
        x[j][0] = (T)q.w;
        x[j][1] = (T)q.z;
        x[j][2] = (T)q.y;
        x[j][3] = (T)q.x;
    }
}

template <typename T, bool NT, int STEPS>
__device__ __forceinline__ void load_full_tile(const T *base, uint32_t lane_off, T (&x)[STEPS][4]) {
    using V = typename Vec4A4<T>::type;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const V q = load_a4<NT>((const V *)((const char *)base + lane_off + (uint32_t)j * (kWave * 16)));
        x[j][0] = (T)q.x;
        x[j][1] = (T)q.y;
        x[j][2] = (T)q.z;
        x[j][3] = (T)q.w;
    }
}

// STEPS vectors per lane: a tile is 4 waves * 64 lanes * 4 * STEPS elements.
// VEC: unit-stride lines (16-byte vector loads and stores at any 4-byte
// aligned start).  REV:
// suffix scan (logical element i is physical len-1-i).  NT: non-temporal
// vector accesses.
template <typename T, typename Op, typename Status, bool EXCL, bool VEC, bool REV, int STEPS = kSteps,
          bool NT = true, int WAVES = kWaves, bool HEAD = false>
__global__ __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(ScanWavesPerEu<T>::value)))
void scan_tiles_kernel(ScanParams p, Status st, Status st1) {
    using C = typename Status::C;
    constexpr int kWaveElems = kWave * 4 * STEPS;
    constexpr int kTileElems = WAVES * kWaveElems;
    __shared__ T s_wave_tot[WAVES];
    __shared__ C s_excl;
    constexpr bool kPark = ParkTile<T>::value;
    __shared__ T s_park[kPark ? STEPS * 4 * kWave : 1];

    const bool looks_back = p.tiles_per_line > 1;
    if (looks_back) __builtin_amdgcn_s_setprio(3);

    const uint64_t tile = p.tile0 + blockIdx.x;
    const uint64_t line = tile / p.tiles_per_line;
    const uint64_t tin = tile - line * p.tiles_per_line;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = lane_id();
    const int64_t ib = (int64_t)p.in_offset + (int64_t)line * p.in_line_stride;
    const int64_t ob = (int64_t)p.out_offset + (int64_t)line * p.out_line_stride;
    const uint64_t e0 = tin * kTileElems + (uint64_t)w * kWaveElems + (uint64_t)lane * 4;
    const T *in = (const T *)p.in;
    T *out = (T *)p.out;
    const T ident = Op::template identity<T>();

    // Wave index made explicitly uniform so lane offsets stay 32-bit.
    const uint32_t lane_off =
        ((uint32_t)__builtin_amdgcn_readfirstlane(w) * kWaveElems + (uint32_t)lane * 4) * (uint32_t)sizeof(T);
    const bool full = VEC && (tin + 1) * kTileElems <= p.len && (!HEAD || tin > 0);
    // Reverse: the tile's lowest physical element, and the mirrored offset.
    const int64_t rev_tile = REV ? (int64_t)(p.len - (tin + 1) * kTileElems) : 0;
    const uint32_t rev_off = (uint32_t)(kTileElems - 4) * (uint32_t)sizeof(T) - lane_off;
    T x[STEPS][4];
    if (full) {
        if constexpr (REV)
            load_full_tile_rev<T, NT, STEPS>(in + ib + rev_tile, rev_off, x);
        else
            load_full_tile<T, NT, STEPS>(in + ib + (int64_t)(tin * kTileElems), lane_off, x);
        // All STEPS loads are issued before any arithmetic is scheduled.
        __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
        for (int j = 0; j < STEPS; ++j)
            load4<T, VEC, REV, NT, HEAD>(p, in, ib, e0 + (uint64_t)j * (kWave * 4), ident, x[j]);
    }

    // Per step: register scan of 4, wave scan of lane totals, running carry.
    T carry = ident;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const T p0 = x[j][0];
        const T p1 = Op::combine(p0, x[j][1]);
        const T p2 = Op::combine(p1, x[j][2]);
        const T p3 = Op::combine(p2, x[j][3]);
        const T incl = wave_inclusive_scan<Op, T>(p3);
        const T lex = wave_shift_right<Op, T>(incl);
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
        carry = Op::combine(carry, read_lane(incl, kWave - 1));
    }
    if (lane == 0) s_wave_tot[w] = carry;
    __syncthreads();
    // Wave totals are combined in wave order for the tile aggregate and each
    // wave's exclusive offset.  f32 tiles read the offset after the look-back
    // (nothing of it is held across the look-back) and park wave 0's data in
    // LDS meanwhile, so its registers are free for the look-back; the empty
    // asm statements keep the compiler from forwarding the parked values.
    T wave_excl = ident;
    T tile_agg = ident;
    if constexpr (!kPark) {
#pragma unroll
        for (int k = 0; k < WAVES; ++k) {
            if (k < w) wave_excl = Op::combine(wave_excl, s_wave_tot[k]);
            tile_agg = Op::combine(tile_agg, s_wave_tot[k]);
        }
    }

    if (w == 0) {
        if constexpr (kPark) {
#pragma unroll
            for (int k = 0; k < WAVES; ++k) tile_agg = Op::combine(tile_agg, s_wave_tot[k]);
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                using V = typename Vec4A4<T>::type;
                V v;
                v.x = x[j][0];
                v.y = x[j][1];
                v.z = x[j][2];
                v.w = x[j][3];
                *(V *)&s_park[(j * kWave + lane) * 4] = v;
            }
            asm volatile("" ::: "memory");
        }
        const C agg = (C)tile_agg;
        C excl = Op::template identity<C>();
        if (tin == 0) {
            // A line of one tile has no successor to read it (its status
            // area is not even allocated: scan_bytes).
            if (lane == 0 && looks_back) st.publish_tile(tile, p.tag, kPrefix, agg);
        } else {
            if (lane == 0) st.publish_tile(tile, p.tag, kAggregate, agg);
            KnownAgg<C> hook{agg};
            excl = lookback<T, Op, Status, VEC, REV, NT, STEPS, WAVES, HEAD>(p, st, st1, tile, line, tin, hook);
            if (lane == 0) st.publish_tile(tile, p.tag, kPrefix, Op::combine(excl, agg));
        }
        if (lane == 0 && tin % kSuper == kSuper - 1 && tin + 1 < p.tiles_per_line)
            st1.publish(line * p.supers_per_line + tin / kSuper, p.tag, kPrefix, Op::combine(excl, agg));
        if (lane == 0) s_excl = excl;
        if constexpr (kPark) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                using V = typename Vec4A4<T>::type;
                const V v = *(const V *)&s_park[(j * kWave + lane) * 4];
                x[j][0] = v.x;
                x[j][1] = v.y;
                x[j][2] = v.z;
                x[j][3] = v.w;
            }
        }
    }
    __syncthreads();
    const TileCarry<T, C, Op> tile_carry(s_excl);
    if constexpr (kPark) {
#pragma unroll
        for (int k = 0; k < WAVES; ++k)
            if (k < w) wave_excl = Op::combine(wave_excl, s_wave_tot[k]);
    }
    if (looks_back) __builtin_amdgcn_s_setprio(0);

    if (full) {
        using V = typename Vec4A4<T>::type;
        if constexpr (REV) {
            const auto orsrc = stream_rsrc(out + ob + rev_tile, kTileElems * (uint32_t)sizeof(T));
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                V v;
                v.w = tile_carry.apply(Op::combine(wave_excl, x[j][0]));
                v.z = tile_carry.apply(Op::combine(wave_excl, x[j][1]));
                v.y = tile_carry.apply(Op::combine(wave_excl, x[j][2]));
                v.x = tile_carry.apply(Op::combine(wave_excl, x[j][3]));
                stream_store(v, orsrc, rev_off - (uint32_t)j * (kWave * 16));
                store_gap();
            }
        } else {
            const auto orsrc = stream_rsrc(out + ob + (int64_t)(tin * kTileElems), kTileElems * (uint32_t)sizeof(T));
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                V v;
                v.x = tile_carry.apply(Op::combine(wave_excl, x[j][0]));
                v.y = tile_carry.apply(Op::combine(wave_excl, x[j][1]));
                v.z = tile_carry.apply(Op::combine(wave_excl, x[j][2]));
                v.w = tile_carry.apply(Op::combine(wave_excl, x[j][3]));
                stream_store(v, orsrc, lane_off + (uint32_t)j * (kWave * 16));
                store_gap();
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
        T r[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // Opaque to the optimizer: the ragged tile's outputs are not
            // merged with the whole-tile path's and hoisted above the branch
            // (which kept every output of the tile live at once).
            T xv = x[j][c];
            asm volatile("" : "+v"(xv));
            r[c] = tile_carry.apply(Op::combine(wave_excl, xv));
        }
        if constexpr (VEC) {
            if (e + 3 < p.len && e >= (HEAD ? p.head : 0u)) {
                using V = typename Vec4A4<T>::type;
                V v;
                if constexpr (REV) {
                    v.w = r[0];
                    v.z = r[1];
                    v.y = r[2];
                    v.x = r[3];
                    store_a4<NT>(v, (V *)(out + ob + (int64_t)(p.len - 4 - e)));
                } else {
                    v.x = r[0];
                    v.y = r[1];
                    v.z = r[2];
                    v.w = r[3];
                    store_a4<NT>(v, (V *)(out + ob + (int64_t)e));
                }
                continue;
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint64_t i = e + c;
            const uint64_t li = REV ? (p.len - 1 - i) : i;
            if (i < p.len && i >= (HEAD ? p.head : 0u)) out[ob + (int64_t)li * p.out_elem_stride] = r[c];
        }
    }
}

// Short dense lines: a scan along lines of fewer than 256 elements packed
// back to back (line stride = length, element stride 1, input and output).
// One tile per line (scan_tiles_kernel) left most of a block idle and made
// the launch block-bound: [2^24, 4] u32 along axis 1 took 4.0 ms.  Here the
// operand is one flat range of lines x len elements, cut into tiles of
// WAVES x 64 x 4 x STEPS elements in logical order (a reverse scan mirrors
// the range), loaded and stored as 16-byte vectors exactly like a 1-D scan,
// and scanned with a segmented scan that restarts at every line start
// (logical index k with k % len == 0):
//
//   * per lane, the four elements' running values restart at a line start;
//   * across the wave, (flag, value) pairs -- flag: a line starts in the
//     span -- take a six-step DPP scan under the segmented combine
//     (f1, v1) . (f2, v2) = (f1 | f2, f2 ? v2 : v1 + v2), which is
//     associative; across steps a register carry, across waves LDS;
//   * the line open at the tile start takes the fold of its elements in the
//     previous tile (at most len - 1 < 255 of them), which wave 0 re-reads,
//     so no tile waits for another: no look-back and no status words.
//
// Line starts are tracked with an incremental remainder, no division per
// element.  f32 lines scan in f32 (a line holds fewer than 256 elements).
// Tiles of 8 waves x 16 steps with gaps between stores (as the paced
// integer tiles): 2^28 u32 along lines of 4 / 100 / 255 elements, 357.9 /
// 355.5 / 365.6 us without gaps, 354.9 / 357.2 / 358.9 with; 8 steps
// 406.7 / 417.0 / 419.6 (one tile per line took 16 ms at 4 elements).  f32
// lines at 16 steps spill a few registers under the 128-VGPR cap and still
// beat 12 steps, which fit (355.3 / 359.1 / 362.6 against 368.9 / 366.8 /
// 368.4 us) and 8 steps (395.7 / 404.4 / 410.5).
struct ShortParams {
    const void *in;
    void *out;
    uint64_t n;      // lines * len
    uint64_t in_offset, out_offset;
    uint64_t tile0;  // tile of block 0 (launched in batches)
    uint32_t len;    // elements per line, 1..255
};

// The segmented combine on (flag, value) pairs.
template <typename Op, typename T>
__device__ __forceinline__ void seg_combine(uint32_t fa, T va, uint32_t &fb, T &vb) {
    vb = fb ? vb : Op::combine(va, vb);
    fb |= fa;
}

// Inclusive segmented scan across the 64 lanes (Hillis-Steele on DPP moves,
// as wave_inclusive_scan; lanes with no source take (0, identity)).
template <typename Op, typename T> __device__ __forceinline__ void wave_seg_scan(uint32_t &f, T &v) {
    const T id = Op::template identity<T>();
#define HX_SEG_STEP(CTRL, MASK)                                                                                      \
    {                                                                                                                \
        const T vs = dpp_move<CTRL, MASK>(id, v);                                                                    \
        const uint32_t fs = dpp_move<CTRL, MASK>(0u, f);                                                             \
        seg_combine<Op, T>(fs, vs, f, v);                                                                            \
    }
    HX_SEG_STEP(kDppRowShr1, 0xf)
    HX_SEG_STEP(kDppRowShr2, 0xf)
    HX_SEG_STEP(kDppRowShr4, 0xf)
    HX_SEG_STEP(kDppRowShr8, 0xf)
    HX_SEG_STEP(kDppRowBcast15, 0xa)
    HX_SEG_STEP(kDppRowBcast31, 0xc)
#undef HX_SEG_STEP
}

template <typename T, typename Op, bool EXCL, bool REV, int STEPS, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(4)))
void scan_short_lines_kernel(ShortParams p) {
    constexpr uint32_t kWaveElems = kWave * 4 * STEPS;
    constexpr uint32_t kTileElems = WAVES * kWaveElems;
    __shared__ uint32_t s_wf[WAVES];
    __shared__ T s_wv[WAVES];
    __shared__ T s_carry;

    const T ident = Op::template identity<T>();
    const uint64_t tile = p.tile0 + blockIdx.x;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = lane_id();
    const uint32_t L = p.len;
    const T *in = (const T *)p.in + p.in_offset;
    T *out = (T *)p.out + p.out_offset;
    const uint64_t k0 = tile * kTileElems;                                // tile's first logical element
    const uint64_t wbase = k0 + (uint64_t)w * kWaveElems;
    const bool full = k0 + kTileElems <= p.n;
    // Logical element k lives at in[k] (forward) or in[n - 1 - k] (reverse).
    const uint32_t lane_off = ((uint32_t)w * kWaveElems + (uint32_t)lane * 4) * (uint32_t)sizeof(T);

    T x[STEPS][4];
    if (full) {
        using V = typename Vec4A4<T>::type;
        if constexpr (REV) {
            const char *base = (const char *)(in + (p.n - k0 - kTileElems));
            const uint32_t rev = (kTileElems - 4) * (uint32_t)sizeof(T) - lane_off;
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                const V q = load_a4<true>((const V *)(base + rev - (uint32_t)j * (kWave * 16)));
                x[j][0] = (T)q.w;
                x[j][1] = (T)q.z;
                x[j][2] = (T)q.y;
                x[j][3] = (T)q.x;
            }
        } else {
            const char *base = (const char *)(in + k0);
#pragma unroll
            for (int j = 0; j < STEPS; ++j) {
                const V q = load_a4<true>((const V *)(base + lane_off + (uint32_t)j * (kWave * 16)));
                x[j][0] = (T)q.x;
                x[j][1] = (T)q.y;
                x[j][2] = (T)q.z;
                x[j][3] = (T)q.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
        for (int j = 0; j < STEPS; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint64_t k = wbase + (uint64_t)j * (kWave * 4) + (uint64_t)lane * 4 + c;
                x[j][c] = k < p.n ? in[REV ? p.n - 1 - k : k] : ident;
            }
    }

    // The line open at the tile start: the fold of its elements before k0.
    const uint32_t m = (uint32_t)(k0 % L);
    if (w == 0) {
        T a = ident;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t i = (uint32_t)lane + 64u * q;
            if (i < m) {
                const uint64_t k = k0 - m + i;
                a = Op::combine(a, in[REV ? p.n - 1 - k : k]);
            }
        }
        a = wave_reduce<Op, T>(a);
        if (lane == 0) s_carry = a;
    }

    // Remainder of this lane's first element modulo L, then per step.
    const uint32_t wrem = (uint32_t)(wbase % L);
    uint32_t r = (wrem + (uint32_t)lane * 4u) % L;
    const uint32_t step_inc = (kWave * 4u) % L;
    uint32_t fs = 0u; // step carry: (flag, value)
    T vs = ident;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        // flags of the four elements: remainder 0 marks a line start
        uint32_t rc = r, f[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            f[c] = rc == 0u;
            rc += 1u;
            rc = rc >= L ? rc - L : rc;
        }
        T pl[4];
        pl[0] = x[j][0];
#pragma unroll
        for (int c = 1; c < 4; ++c) pl[c] = f[c] ? x[j][c] : Op::combine(pl[c - 1], x[j][c]);
        uint32_t fl = f[0] | f[1] | f[2] | f[3];
        T vl = pl[3];
        wave_seg_scan<Op, T>(fl, vl); // lane inclusive over the wave's step
        // lane exclusive: the previous lane's inclusive value
        uint32_t fe = dpp_move<kDppWaveShr1>(0u, fl);
        T ve = dpp_move<kDppWaveShr1>(ident, vl);
        // this lane's incoming value within the wave: step carry, then lanes before
        const T vin = fe ? ve : Op::combine(vs, ve);
        uint32_t seen = 0u; // a line start at or before element c in this lane
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            seen |= f[c];
            x[j][c] = seen ? pl[c] : Op::combine(vin, pl[c]);
        }
        if constexpr (EXCL) {
            // exclusive: identity at a line start, else the inclusive value
            // of the element before (the lane's incoming value for c = 0)
#pragma unroll
            for (int c = 3; c >= 1; --c) x[j][c] = f[c] ? ident : x[j][c - 1];
            x[j][0] = f[0] ? ident : vin;
        }
        // carry to the next step: the wave's inclusive (flag, value) at lane 63
        const uint32_t f63 = read_lane(fl, kWave - 1);
        const T v63 = read_lane(vl, kWave - 1);
        vs = f63 ? v63 : Op::combine(vs, v63);
        fs |= f63;
        r += step_inc;
        r = r >= L ? r - L : r;
        // One step at a time: interleaving steps' scans (the scheduler's
        // choice) spilled the f32 forms at 16 steps.
        __builtin_amdgcn_sched_barrier(0);
    }
    if (lane == 0) {
        s_wf[w] = fs;
        s_wv[w] = vs;
    }
    __syncthreads();
    // This wave's incoming value: the open line's carry, then waves before.
    T win = s_carry;
    for (int q = 0; q < w; ++q) win = s_wf[q] ? s_wv[q] : Op::combine(win, s_wv[q]);
    // Elements before the wave's first line start take win.
    const uint64_t first_start = wbase + (uint64_t)((L - wrem) % L);

    if (full) {
        using V = typename Vec4A4<T>::type;
        const auto orsrc = stream_rsrc(REV ? (void *)(out + (p.n - k0 - kTileElems)) : (void *)(out + k0),
                                       kTileElems * (uint32_t)sizeof(T));
        const uint32_t rev = (kTileElems - 4) * (uint32_t)sizeof(T) - lane_off;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const uint64_t k = wbase + (uint64_t)j * (kWave * 4) + (uint64_t)lane * 4;
            T y[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) y[c] = k + c >= first_start ? x[j][c] : Op::combine(win, x[j][c]);
            V v;
            if constexpr (REV) {
                v.w = y[0];
                v.z = y[1];
                v.y = y[2];
                v.x = y[3];
                stream_store(v, orsrc, rev - (uint32_t)j * (kWave * 16));
            } else {
                v.x = y[0];
                v.y = y[1];
                v.z = y[2];
                v.w = y[3];
                stream_store(v, orsrc, lane_off + (uint32_t)j * (kWave * 16));
            }
            store_gap();
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < STEPS; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint64_t k = wbase + (uint64_t)j * (kWave * 4) + (uint64_t)lane * 4 + c;
            T xv = x[j][c];
            asm volatile("" : "+v"(xv)); // not merged with the whole-tile stores (see scan_tiles_kernel)
            if (k < p.n) out[REV ? p.n - 1 - k : k] = k >= first_start ? xv : Op::combine(win, xv);
        }
}

// Column scans: many strided lines whose starts are adjacent in memory
// (axis-0 scan of a row-major matrix).  From 256 lines up they take the
// single-pass col_lookback_kernel below; narrower matrices take this chunked
// reduce-then-scan.  Lanes run across lines -- a wave owns 64*V adjacent
// lines, V = 4 giving every lane one 16-byte load per step -- and the scan
// axis is cut into chunks so that thousands of waves share the work however
// tall the matrix is:
//   col_totals_kernel  chunk totals of every line (one read of the input);
//   col_carry_kernel   per line, an exclusive scan of its chunk totals in
//                      place (chunks x lines words, a thread per line);
//   col_scan_kernel    every chunk rescanned from its carry, outputs written.
// With one chunk only col_scan_kernel runs (carry = identity).  Each lane
// walks its lines serially; f32 accumulates in f64, integers wrap in u32.
template <typename T> struct ColAcc { using type = uint32_t; };
template <> struct ColAcc<float> { using type = double; };

struct ColShape {
    int V = 1;
    uint64_t groups = 0, chunk = 0;
    uint32_t nchunks = 1;
};

template <typename T, int V> struct ColIO;
template <typename T> struct ColIO<T, 1> {
    using A = typename ColAcc<T>::type;
    static __device__ __forceinline__ void load(const T *p, A (&x)[1]) { x[0] = (A)__builtin_nontemporal_load(p); }
    static __device__ __forceinline__ void store(T *p, const A (&y)[1]) { __builtin_nontemporal_store((T)y[0], p); }
    static __device__ __forceinline__ void load_n(const T *p, uint32_t, A, A (&x)[1]) { load(p, x); }
    static __device__ __forceinline__ void store_n(T *p, uint32_t, const A (&y)[1]) { store(p, y); }
};
template <typename T> struct ColIO<T, 4> {
    using A = typename ColAcc<T>::type;
    using Vt = typename Vec4A4<T>::type;
    static __device__ __forceinline__ void load(const T *p, A (&x)[4]) {
        const Vt v = __builtin_nontemporal_load((const Vt *)p);
        x[0] = (A)v.x;
        x[1] = (A)v.y;
        x[2] = (A)v.z;
        x[3] = (A)v.w;
    }
    static __device__ __forceinline__ void store(T *p, const A (&y)[4]) {
        Vt v;
        v.x = (T)y[0];
        v.y = (T)y[1];
        v.z = (T)y[2];
        v.w = (T)y[3];
        __builtin_nontemporal_store(v, (Vt *)p);
    }
    // The lane of a partial group (the last nv < 4 lines, when the line
    // count is not a multiple of 4) moves its lines one by one; the others
    // read as `ident` and are never stored.
    static __device__ __forceinline__ void load_n(const T *p, uint32_t nv, A ident, A (&x)[4]) {
        if (nv >= 4) {
            load(p, x);
            return;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) x[v] = (uint32_t)v < nv ? (A)__builtin_nontemporal_load(p + v) : ident;
    }
    static __device__ __forceinline__ void store_n(T *p, uint32_t nv, const A (&y)[4]) {
        if (nv >= 4) {
            store(p, y);
            return;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
            if ((uint32_t)v < nv) __builtin_nontemporal_store((T)y[v], p + v);
    }
};

// Lines of this lane's group that exist (V, or fewer in the last group).
__device__ __forceinline__ uint32_t col_valid_lines(uint64_t lines, uint64_t line0, int V) {
    return lines - line0 < (uint64_t)V ? (uint32_t)(lines - line0) : (uint32_t)V;
}

// Wave w -> (line group g, chunk k); adjacent waves take adjacent groups of
// the same chunk.  Returns false for lanes with no line.
struct ColWork {
    uint64_t line0, k, i0, i1;
};
__device__ __forceinline__ bool col_work(const ScanParams &p, uint64_t chunk, uint32_t nchunks, uint64_t groups,
                                         int V, ColWork *w) {
    const uint64_t wave = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    if (wave >= groups * nchunks) return false;
    const uint64_t g = wave % groups;
    w->k = wave / groups;
    w->line0 = (g * kWave + (uint64_t)lane_id()) * V;
    if (w->line0 >= p.lines) return false;
    w->i0 = w->k * chunk;
    w->i1 = w->i0 + chunk < p.len ? w->i0 + chunk : p.len;
    return true;
}

template <typename T, typename Op, int V, bool REV>
__global__ __launch_bounds__(kBlock) void col_totals_kernel(ScanParams p, typename ColAcc<T>::type *totals,
                                                            uint64_t chunk, uint32_t nchunks, uint64_t groups) {
    using A = typename ColAcc<T>::type;
    constexpr int kU = V == 4 ? 8 : 16;
    ColWork w;
    if (!col_work(p, chunk, nchunks, groups, V, &w)) return;
    const T *in = (const T *)p.in + ((int64_t)p.in_offset + (int64_t)w.line0 * p.in_line_stride);
    const uint32_t nv = col_valid_lines(p.lines, w.line0, V);
    const A aid = Op::template identity<A>();
    A acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = aid;
    uint64_t i = w.i0;
    for (; i + kU <= w.i1; i += kU) {
        A x[kU][V];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const uint64_t li = REV ? p.len - 1 - (i + u) : i + u;
            ColIO<T, V>::load_n(in + (int64_t)li * p.in_elem_stride, nv, aid, x[u]);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int v = 0; v < V; ++v) acc[v] = Op::combine(acc[v], x[u][v]);
    }
    for (; i < w.i1; ++i) {
        const uint64_t li = REV ? p.len - 1 - i : i;
        A x[V];
        ColIO<T, V>::load_n(in + (int64_t)li * p.in_elem_stride, nv, aid, x);
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = Op::combine(acc[v], x[v]);
    }
#pragma unroll
    for (int v = 0; v < V; ++v)
        if ((uint32_t)v < nv) totals[w.k * p.lines + w.line0 + v] = acc[v];
}

// Exclusive scan of each line's chunk totals, in place.  A block owns 64
// lines (lanes) and kCarrySlices waves; wave s totals its contiguous range of
// chunks, the slice totals are scanned through LDS, and each wave rewrites
// its range from its slice carry.
constexpr int kCarrySlices = 16;

template <typename A, typename Op>
__global__ __launch_bounds__(kWave *kCarrySlices) void col_carry_kernel(A *totals, uint64_t lines,
                                                                        uint32_t nchunks) {
    __shared__ A sh[kCarrySlices * kWave];
    const int lane = lane_id();
    const int s = threadIdx.x / kWave;
    const uint64_t line = (uint64_t)blockIdx.x * kWave + lane;
    const uint32_t per = (nchunks + kCarrySlices - 1) / kCarrySlices;
    const uint32_t k0 = s * per < nchunks ? s * per : nchunks;
    const uint32_t k1 = k0 + per < nchunks ? k0 + per : nchunks;
    A t = Op::template identity<A>();
    if (line < lines)
        for (uint32_t k = k0; k < k1; ++k) t = Op::combine(t, totals[(uint64_t)k * lines + line]);
    sh[s * kWave + lane] = t;
    __syncthreads();
    if (line >= lines) return;
    A acc = Op::template identity<A>();
    for (int q = 0; q < s; ++q) acc = Op::combine(acc, sh[q * kWave + lane]);
    for (uint32_t k = k0; k < k1; ++k) {
        const A v = totals[(uint64_t)k * lines + line];
        totals[(uint64_t)k * lines + line] = acc;
        acc = Op::combine(acc, v);
    }
}

template <typename T, typename Op, int V, bool EXCL, bool REV, bool CARRY>
__global__ __launch_bounds__(kBlock) void col_scan_kernel(ScanParams p, const typename ColAcc<T>::type *carries,
                                                          uint64_t chunk, uint32_t nchunks, uint64_t groups) {
    using A = typename ColAcc<T>::type;
    constexpr int kU = V == 4 ? 8 : 16;
    ColWork w;
    if (!col_work(p, chunk, nchunks, groups, V, &w)) return;
    const T *in = (const T *)p.in + ((int64_t)p.in_offset + (int64_t)w.line0 * p.in_line_stride);
    T *out = (T *)p.out + ((int64_t)p.out_offset + (int64_t)w.line0 * p.out_line_stride);
    const uint32_t nv = col_valid_lines(p.lines, w.line0, V);
    const A aid = Op::template identity<A>();
    A acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = CARRY && (uint32_t)v < nv ? carries[w.k * p.lines + w.line0 + v] : aid;
    auto step = [&](uint64_t li, const A (&x)[V]) {
        A y[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if constexpr (EXCL) {
                y[v] = acc[v];
                acc[v] = Op::combine(acc[v], x[v]);
            } else {
                acc[v] = Op::combine(acc[v], x[v]);
                y[v] = acc[v];
            }
        }
        ColIO<T, V>::store_n(out + (int64_t)li * p.out_elem_stride, nv, y);
    };
    uint64_t i = w.i0;
    for (; i + kU <= w.i1; i += kU) {
        A x[kU][V];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const uint64_t li = REV ? p.len - 1 - (i + u) : i + u;
            ColIO<T, V>::load_n(in + (int64_t)li * p.in_elem_stride, nv, aid, x[u]);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) step(REV ? p.len - 1 - (i + u) : i + u, x[u]);
    }
    for (; i < w.i1; ++i) {
        const uint64_t li = REV ? p.len - 1 - i : i;
        A x[V];
        ColIO<T, V>::load_n(in + (int64_t)li * p.in_elem_stride, nv, aid, x);
        step(li, x);
    }
}

// Narrow column scans: axis 0 of a dense row-major [R, C] matrix, C a power
// of two from 32 to 128, read as the one contiguous range of 16-byte vectors
// it is.  Component k of vector g holds column (4g + k) mod C, and since C
// divides 256 that is column (4l + k) mod C for lane l of every step: a lane
// always holds the same four columns, and the lanes of one column in a step
// are l, l + s, l + 2s, ... with s = C / 4 (a "class").  A reverse scan
// mirrors the range (logical vector g is physical vector nvec - 1 - g, its
// components reversed), so every pass works in logical order and logical
// columns.  Tiles are the scan's own: 8 waves x 16 steps of 64 vectors
// (128 KiB, two blocks per CU), each wave streaming its own 16 KiB run with
// all 16 loads in flight.  Three launches:
//   col_narrow_totals_kernel  per tile and column, the total (one read);
//   col_narrow_carry_kernel   per column, an exclusive scan of its totals;
//   col_narrow_scan_kernel    every tile rescanned from its carries (one
//                             read, one write).
// f32 steps scan in f32 and add f64 carries; integers wrap.  The column-tile
// forms gave such matrices one live lane in 64/C.  Narrower powers of two
// take the single-pass row tiles (2^28 u32 at C = 4 / 8 / 16: 515 / 522 /
// 525 us here, 439 / 450 / 455 there).
constexpr int kNarrowWaves = 8, kNarrowSteps = 16;
constexpr int kNarrowWavesPerEu = 4; // two 8-wave blocks per CU: at most 128 VGPRs
constexpr uint64_t kNarrowTileVecs = (uint64_t)kNarrowWaves * kNarrowSteps * kWave;

// Lane permutes for the class scans: lane l reads lane src(l), src given as
// a byte address (4 * lane), 32-bit values.
template <typename A> __device__ __forceinline__ A lane_permute(A v, int addr) {
    static_assert(sizeof(A) == 4, "32-bit lanes");
    return __builtin_bit_cast(A, __builtin_amdgcn_ds_bpermute(addr, __builtin_bit_cast(int, v)));
}

// Byte addresses of the lanes a class scan reads, per lane (S = C / 4 >= 2):
// its class's last lane in the row below and in row 1 (S <= 16) or the lane
// 32 below (S = 32), its class's last lane in the wave, and the lane S below.
struct ClassLanes {
    int below, row1, last, prev;
    template <int S> __device__ __forceinline__ void init(int lane) {
        const int c = lane & (S - 1);
        if constexpr (S <= 16) {
            below = 4 * (((lane & ~15) - S + c) & (kWave - 1));
            row1 = 4 * (32 - S + c);
        } else {
            below = 4 * (lane & 31);
            row1 = 0;
        }
        last = 4 * (kWave - S + c);
        prev = 4 * ((lane - S) & (kWave - 1));
    }
};

// Inclusive scan over the lanes of each class l mod S (S = 1, 2, 4, ..., 32):
// lane l ends with the combination, in lane order, of the lanes l' <= l with
// l' = l (mod S).  Distances S..8 inside each row of 16 lanes are DPP row
// shifts; the class totals of lower rows then come in with two lane permutes
// (rows 1 and 3 take their class's last lane of the row below; rows 2 and 3
// then take its last lane of row 1).  S = 1 is the plain wave scan.  32-bit
// values.
template <int S, typename Op, typename A>
__device__ __forceinline__ A class_inclusive_scan(A v, int lane, const ClassLanes &cl) {
    if constexpr (S == 1) {
        return wave_inclusive_scan<Op, A>(v);
    } else {
        const A id = Op::template identity<A>();
        if constexpr (S <= 2) v = Op::combine(dpp_move<kDppRowShr2>(id, v), v);
        if constexpr (S <= 4) v = Op::combine(dpp_move<kDppRowShr4>(id, v), v);
        if constexpr (S <= 8) v = Op::combine(dpp_move<kDppRowShr8>(id, v), v);
        if constexpr (S <= 16) {
            const A below = lane_permute(v, cl.below);
            v = (lane & 16) ? Op::combine(below, v) : v;
            const A row1 = lane_permute(v, cl.row1);
            v = lane >= 32 ? Op::combine(row1, v) : v;
        } else {
            const A half = lane_permute(v, cl.below);
            v = lane >= 32 ? Op::combine(half, v) : v;
        }
        return v;
    }
}
// The class total (the inclusive value of the class's last lane).
template <int S, typename A> __device__ __forceinline__ A class_total(A incl, const ClassLanes &cl) {
    if constexpr (S == 1) return read_lane(incl, kWave - 1);
    else return lane_permute(incl, cl.last);
}
// Exclusive form: lane l takes lane l - S's inclusive value, the first S
// lanes the identity.
template <int S, typename Op, typename A>
__device__ __forceinline__ A class_shift(A incl, int lane, const ClassLanes &cl) {
    if constexpr (S == 1) {
        return wave_shift_right<Op, A>(incl);
    } else {
        const A t = lane_permute(incl, cl.prev);
        return lane >= S ? t : Op::template identity<A>();
    }
}

// The rescan's in-wave part for class stride S, once the carries into the
// wave are known (`outer`, per component): each step's components scanned
// over their classes, and each output -- the carry, then the lane's running
// class total before the step, then its (inclusive or exclusive) class
// prefix -- handed to store(j, y) as soon as the step is scanned, so no
// output is held in registers.  The running totals are in T: an f32 wave
// prefix covers at most 16 steps of 64 values, and the carry is f64.
template <int S, typename T, typename Op, bool EXCL, typename Store>
__device__ __forceinline__ void narrow_wave_scan(const T (&x)[16][4], const typename ColAcc<T>::type (&outer)[4],
                                                 int lane, Store &&store) {
    using A = typename ColAcc<T>::type;
    ClassLanes cl;
    if constexpr (S > 1) cl.template init<S>(lane);
    T run[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) run[k] = Op::template identity<T>();
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        T y[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const T incl = class_inclusive_scan<S, Op, T>(x[j][k], lane, cl);
            const T tot = class_total<S, T>(incl, cl);
            const T pre = EXCL ? class_shift<S, Op, T>(incl, lane, cl) : incl;
            y[k] = (T)Op::combine(outer[k], (A)Op::combine(run[k], pre));
            run[k] = Op::combine(run[k], tot);
        }
        store(j, y);
    }
}

// Lane `lane`, wave `w` of tile `t`: its 16 logical vectors (steps j), whole
// tiles through one block-uniform base and a 32-bit lane offset, the last
// tile checked (identity past the end).
template <typename T, bool REV>
__device__ __forceinline__ void narrow_tile_load(const T *in, uint64_t nvec, uint64_t t, int w, int lane, T ident,
                                                 T (&x)[kNarrowSteps][4]) {
    using V = typename Vec4A4<T>::type;
    const uint64_t g0 = t * kNarrowTileVecs + (uint64_t)w * (kNarrowSteps * kWave) + (uint64_t)lane;
    if ((t + 1) * kNarrowTileVecs <= nvec) {
        const uint32_t lane_off = ((uint32_t)__builtin_amdgcn_readfirstlane(w) * (kNarrowSteps * kWave) +
                                   (uint32_t)lane) * 16u;
        if constexpr (REV) {
            const char *base = (const char *)(in + 4 * (nvec - (t + 1) * kNarrowTileVecs));
            const uint32_t rev_off = (uint32_t)(kNarrowTileVecs * 16 - 16) - lane_off;
#pragma unroll
            for (int j = 0; j < kNarrowSteps; ++j) {
                const V q = load_a4<true>((const V *)(base + rev_off - (uint32_t)j * (kWave * 16)));
                x[j][0] = (T)q.w;
                x[j][1] = (T)q.z;
                x[j][2] = (T)q.y;
                x[j][3] = (T)q.x;
            }
        } else {
            const char *base = (const char *)(in + 4 * t * kNarrowTileVecs);
#pragma unroll
            for (int j = 0; j < kNarrowSteps; ++j) {
                const V q = load_a4<true>((const V *)(base + lane_off + (uint32_t)j * (kWave * 16)));
                x[j][0] = (T)q.x;
                x[j][1] = (T)q.y;
                x[j][2] = (T)q.z;
                x[j][3] = (T)q.w;
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        return;
    }
#pragma unroll
    for (int j = 0; j < kNarrowSteps; ++j) {
        const uint64_t g = g0 + (uint64_t)j * kWave;
        if (g < nvec) {
            const V q = load_a4<true>((const V *)(in + 4 * (REV ? nvec - 1 - g : g)));
            x[j][0] = (T)(REV ? q.w : q.x);
            x[j][1] = (T)(REV ? q.z : q.y);
            x[j][2] = (T)(REV ? q.y : q.z);
            x[j][3] = (T)(REV ? q.x : q.w);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) x[j][k] = ident;
        }
    }
}

// Pass 1: the totals of tile t, one per logical column, at totals[t * C + c].
// Each lane folds its 16 steps per component, the lanes of a class fold with
// xor butterflies from 32 down to s, and the waves' totals fold in wave
// order: a fixed order, so f32 totals (accumulated in f64) are reproducible.
template <typename T, typename Op, bool REV>
__global__ __launch_bounds__(kNarrowWaves *kWave) void col_narrow_totals_kernel(ScanParams p,
                                                                                typename ColAcc<T>::type *totals) {
    using A = typename ColAcc<T>::type;
    __shared__ A sh[kNarrowWaves][kBlock / 2]; // C <= 128 columns
    const int lane = lane_id();
    const int w = threadIdx.x / kWave;
    const uint32_t C = (uint32_t)p.lines;
    const uint32_t s = C / 4;
    const uint64_t nvec = (p.len * C) >> 2;
    const uint64_t t = xcd_contiguous(blockIdx.x, gridDim.x); // no look-back: any tile order
    T x[kNarrowSteps][4];
    narrow_tile_load<T, REV>((const T *)p.in + p.in_offset, nvec, t, w, lane, Op::template identity<T>(), x);
    A acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        acc[k] = Op::template identity<A>();
#pragma unroll
        for (int j = 0; j < kNarrowSteps; ++j) acc[k] = Op::combine(acc[k], (A)x[j][k]);
    }
    for (int m = kWave / 2; m >= (int)s; m >>= 1)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = Op::combine(acc[k], __shfl_xor(acc[k], m, kWave));
    if (lane < (int)s)
#pragma unroll
        for (int k = 0; k < 4; ++k) sh[w][4 * lane + k] = acc[k];
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < C; c += kNarrowWaves * kWave) {
        A tot = Op::template identity<A>();
#pragma unroll
        for (int q = 0; q < kNarrowWaves; ++q) tot = Op::combine(tot, sh[q][c]);
        totals[t * C + c] = tot;
    }
}

// Pass 2: per column, the exclusive scan of the tile totals in place.  A
// block per column; thread i owns a contiguous range of tiles, loaded 8 at a
// time with the loads of a batch in flight together (one batch, held in
// registers, for up to 8192 tiles), its range total scanned across the block
// in thread order, and its range rewritten.  The order depends only on the
// tile count, so f32 carries are reproducible.  (Re-reading each value in the
// rewrite loop made every iteration a dependent memory round trip: 17-25 us
// per launch.)
constexpr int kNarrowCarryThreads = 1024;
constexpr int kNarrowCarryBatch = 8;
// Entry (tile k, column c) is totals[k * ks + c * cs]: row-major (ks = C,
// cs = 1) for the narrow form, column-major (ks = 1, cs = tiles) for the row
// tiles, whose carry launch read row-major totals C words apart (2^28 u32 at
// C = 100 and 255, about 16400 tiles: 76 us per launch).
template <typename A, typename Op>
__global__ __launch_bounds__(kNarrowCarryThreads) void col_narrow_carry_kernel(A *totals, uint64_t ks, uint64_t cs,
                                                                               uint64_t ntiles) {
    __shared__ A sh[kNarrowCarryThreads / kWave];
    A *col = totals + (uint64_t)blockIdx.x * cs;
    const int lane = lane_id();
    const int w = threadIdx.x / kWave;
    const uint64_t per = (ntiles + kNarrowCarryThreads - 1) / kNarrowCarryThreads;
    const uint64_t k0 = (uint64_t)threadIdx.x * per < ntiles ? (uint64_t)threadIdx.x * per : ntiles;
    const uint64_t k1 = k0 + per < ntiles ? k0 + per : ntiles;
    const A id = Op::template identity<A>();
    A v[kNarrowCarryBatch];
    A sum = id;
    for (uint64_t k = k0; k < k1; k += kNarrowCarryBatch) {
#pragma unroll
        for (int u = 0; u < kNarrowCarryBatch; ++u) v[u] = k + u < k1 ? col[(k + u) * ks] : id;
#pragma unroll
        for (int u = 0; u < kNarrowCarryBatch; ++u) sum = Op::combine(sum, v[u]);
    }
    // Exclusive scan of the range totals in thread order: within each wave,
    // then the wave totals through LDS.
    A incl = sum;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const A t = __shfl_up(incl, d, kWave);
        if (lane >= d) incl = Op::combine(t, incl);
    }
    if (lane == kWave - 1) sh[w] = incl;
    __syncthreads();
    A acc = id;
    for (int q = 0; q < w; ++q) acc = Op::combine(acc, sh[q]);
    const A prev = __shfl_up(incl, 1, kWave);
    if (lane > 0) acc = Op::combine(acc, prev);
    for (uint64_t k = k0; k < k1; k += kNarrowCarryBatch) {
        if (per > kNarrowCarryBatch) { // the range spans several batches: reload this one
#pragma unroll
            for (int u = 0; u < kNarrowCarryBatch; ++u) v[u] = k + u < k1 ? col[(k + u) * ks] : id;
        }
#pragma unroll
        for (int u = 0; u < kNarrowCarryBatch; ++u) {
            if (k + u < k1) col[(k + u) * ks] = acc;
            acc = Op::combine(acc, v[u]);
        }
    }
}

// Pass 3: tile t rescanned from its columns' carries (pass 2), or from the
// identity for a single tile.  Each wave first folds its column totals (per
// lane over its 16 steps, then across the lanes of a class), the waves'
// totals combine with the tile's carries through LDS in wave order, and only
// then are the steps scanned (narrow_wave_scan), every step stored as soon as
// it is scanned: holding the outputs until the carries were known took
// 140-145 VGPRs, one block per CU.  Whole tiles store through the
// stream-store path, the last tile element by element.
template <typename T, typename Op, bool EXCL, bool REV, bool CARRY>
__global__ __launch_bounds__(kNarrowWaves *kWave) __attribute__((amdgpu_waves_per_eu(kNarrowWavesPerEu)))
void col_narrow_scan_kernel(ScanParams p, const typename ColAcc<T>::type *carries) {
    using A = typename ColAcc<T>::type;
    using V = typename Vec4A4<T>::type;
    __shared__ A sh[kNarrowWaves][kBlock / 2]; // C <= 128 columns
    const int lane = lane_id();
    const int w = threadIdx.x / kWave;
    const uint32_t C = (uint32_t)p.lines;
    const uint32_t s = C / 4;
    const uint64_t nvec = (p.len * C) >> 2;
    const uint64_t t = xcd_contiguous(blockIdx.x, gridDim.x); // no look-back: any tile order
    T x[kNarrowSteps][4];
    narrow_tile_load<T, REV>((const T *)p.in + p.in_offset, nvec, t, w, lane, Op::template identity<T>(), x);

    // The wave's column totals, then per column the carry into each wave.
    A acc[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        acc[k] = Op::template identity<A>();
#pragma unroll
        for (int j = 0; j < kNarrowSteps; ++j) acc[k] = Op::combine(acc[k], (A)x[j][k]);
    }
    for (int m = kWave / 2; m >= (int)s; m >>= 1)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[k] = Op::combine(acc[k], __shfl_xor(acc[k], m, kWave));
    if (lane < (int)s)
#pragma unroll
        for (int k = 0; k < 4; ++k) sh[w][4 * lane + k] = acc[k];
    __syncthreads();
    if (threadIdx.x < C) {
        A c = CARRY ? carries[t * C + threadIdx.x] : Op::template identity<A>();
#pragma unroll
        for (int q = 0; q < kNarrowWaves; ++q) {
            const A v = sh[q][threadIdx.x];
            sh[q][threadIdx.x] = c;
            c = Op::combine(c, v);
        }
    }
    __syncthreads();
    A outer[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) outer[k] = sh[w][(uint32_t)(4 * lane + k) & (C - 1)];

    T *out = (T *)p.out + p.out_offset;
    const bool full = (t + 1) * kNarrowTileVecs <= nvec;
    const uint32_t lane_off =
        ((uint32_t)__builtin_amdgcn_readfirstlane(w) * (kNarrowSteps * kWave) + (uint32_t)lane) * 16u;
    const uint32_t rev_off = (uint32_t)(kNarrowTileVecs * 16 - 16) - lane_off;
    const auto orsrc = stream_rsrc(out + 4 * (REV ? (full ? nvec - (t + 1) * kNarrowTileVecs : 0)
                                                   : t * kNarrowTileVecs),
                                   (uint32_t)(kNarrowTileVecs * 16));
    const uint64_t g0 = t * kNarrowTileVecs + (uint64_t)w * (kNarrowSteps * kWave) + (uint64_t)lane;
    auto store = [&](int j, const T (&y)[4]) {
        V v;
        v.x = REV ? y[3] : y[0];
        v.y = REV ? y[2] : y[1];
        v.z = REV ? y[1] : y[2];
        v.w = REV ? y[0] : y[3];
        if (full) {
            stream_store(v, orsrc, REV ? rev_off - (uint32_t)j * (kWave * 16) : lane_off + (uint32_t)j * (kWave * 16));
        } else {
            const uint64_t g = g0 + (uint64_t)j * kWave;
            if (g < nvec) store_a4<true>(v, (V *)(out + 4 * (REV ? nvec - 1 - g : g)));
        }
    };
    switch (s) { // wave-uniform: C is a launch parameter
    case 8: narrow_wave_scan<8, T, Op, EXCL>(x, outer, lane, store); break;
    case 16: narrow_wave_scan<16, T, Op, EXCL>(x, outer, lane, store); break;
    default: narrow_wave_scan<32, T, Op, EXCL>(x, outer, lane, store); break;
    }
}

// Row-tile column scans: axis 0 of a dense row-major [R, C] matrix for the
// other column counts from 2 to 255 (every C but 32, 64 and 128).  Unless C
// divides 256 the 16-byte lanes of the narrow form would not see fixed
// columns.  Up to kRowTileLbMaxCols columns the tiles look back in one pass
// (col_rowtile_lookback_kernel, below); wider matrices take three.  A tile
// of `rows` whole rows (a multiple of 4, at most kRowTileElems elements)
// moves between HBM and LDS as coalesced 16-byte vectors.  In LDS, thread j
// owns column j mod C over row group j / C, one of G = 512 / C contiguous
// groups of `rpg` rows: pass 1 (col_rowtile_totals_kernel) folds each group,
// then scans the group totals along the groups (row_group_scan), whose last
// group holds the tile's column totals; pass 2 is
// col_narrow_carry_kernel; pass 3 (col_rowtile_scan_kernel) folds the
// groups again, then rescans each group's rows in place from the tile's
// carry and the earlier groups' totals before the tile is stored.  Every
// combination runs in ColAcc (f64 for f32) in an order fixed by the shape,
// so f32 results are reproducible.  Mirrored scans take tiles from row R - 1
// down and walk each tile's rows upwards in LDS.  The strided per-line path
// gave these shapes one lane per line (2^28 u32, C = 3: 2.3 ms; C = 12:
// 10 ms).  Tiles of 16384 elements and 512 threads (two blocks per CU by
// LDS) measured best: 2^28 u32 at C = 3 / 12 / 100 / 255 took 597 / 586 /
// 592 / 638 us, against 614 / 594 / 656 / 712 with 8192 elements and 256
// threads and 651 / 682 / 820 / 906 with 4096.
constexpr int kRowTileThreads = 512;
constexpr uint32_t kRowTileElems = 16384;
constexpr int kRowTileVecsPerThread = (int)(kRowTileElems / 4 / kRowTileThreads);

struct RowTileShape {
    uint64_t R = 0, tiles = 0;
    uint32_t C = 0;
    uint32_t rows = 0;   // rows per tile
    uint32_t groups = 0; // row groups (threads) per column
    uint32_t rpg = 0;    // rows per group
};

RowTileShape row_tile_shape(uint64_t C, uint64_t R) {
    RowTileShape s;
    s.R = R;
    s.C = (uint32_t)C;
    // Whole 128-byte lines per tile (rows * C a multiple of 32), so every
    // tile of an aligned matrix starts on a line: 2^28 u32, C = 3 / 5 / 7 /
    // 10: 465 / 452 / 472 / 472 us -> 453 / 447 / 456 / 466.
    uint32_t m = 32;
    while (m > 4 && C % (32 / m * 2) == 0) m /= 2;
    s.rows = (uint32_t)(kRowTileElems / C) / m * m; // C < 256: at least 64
    s.groups = (uint32_t)(kRowTileThreads / C);
    // An odd group length keeps the lanes of one wave (64 / C groups, C * rpg
    // elements apart in LDS) off a common bank: with C = 2 and 32 rows per
    // group every lane of a wave hit one bank (2^28 u32: 1081 us).
    s.rpg = ((s.rows + s.groups - 1) / s.groups) | 1u;
    s.tiles = ceil_div(R, (uint64_t)s.rows);
    return s;
}

// Tile t's physical rows [r0, r0 + n).
template <bool REV>
__device__ __forceinline__ void row_tile_span(const RowTileShape &s, uint64_t t, uint64_t &r0, uint32_t &n) {
    const uint64_t a = t * s.rows;
    const uint64_t b = a + s.rows < s.R ? a + s.rows : s.R;
    n = (uint32_t)(b - a);
    r0 = REV ? s.R - b : a;
}

// ne elements from src (4-byte aligned) straight into the 16-byte aligned LDS
// tile (tile_load_lds): no register round trip and no LDS write
// instructions (2^28 u32 scans, 2-4% faster than loads into registers and
// 16-byte LDS writes: C = 4 437 -> 422 us, C = 24 514 -> 502).
template <typename T> __device__ __forceinline__ void row_tile_load(const T *src, uint32_t ne, T *tile) {
    tile_load_lds<kRowTileThreads, kRowTileVecsPerThread>(src, ne, tile);
}

template <typename T> __device__ __forceinline__ void row_tile_store(const T *tile, uint32_t ne, T *dst) {
    using VA = typename Vec4A4<T>::type;
    using VL = typename Vec4<T>::type;
    const uint32_t nv = ne / 4;
#pragma unroll
    for (int u = 0; u < kRowTileVecsPerThread; ++u) {
        const uint32_t v = threadIdx.x + (uint32_t)u * kRowTileThreads;
        if (v < nv) store_a4<true>((VA)(*(const VL *)(tile + 4 * v)), (VA *)(dst + 4 * v));
    }
    const uint32_t e = 4 * nv + threadIdx.x;
    if (e < ne) __builtin_nontemporal_store(tile[e], dst + e);
}

// Fold of column c over logical rows [lo, hi) of a tile of n rows (logical
// row i is physical row n - 1 - i when mirrored), eight LDS reads in flight.
template <typename T, typename Op, bool REV>
__device__ __forceinline__ typename ColAcc<T>::type row_group_fold(const T *tile, uint32_t n, uint32_t C, uint32_t c,
                                                                  uint32_t lo, uint32_t hi) {
    using A = typename ColAcc<T>::type;
    A acc = Op::template identity<A>();
    uint32_t i = lo;
    for (; i + 8 <= hi; i += 8) {
        T x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = tile[(REV ? n - 1 - (i + u) : i + u) * C + c];
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = Op::combine(acc, (A)x[u]);
    }
    for (; i < hi; ++i) acc = Op::combine(acc, (A)tile[(REV ? n - 1 - i : i) * C + c]);
    return acc;
}

// Inclusive scan of the group totals gtot[g * C + c] along the groups of
// each column, in place: Hillis-Steele steps over LDS, two barriers each,
// in an order fixed by the shape.  Folding the earlier groups one LDS read
// at a time took a thread up to 169 dependent reads (C = 3) per tile.  Every
// thread of the block calls it.
template <typename A, typename Op>
__device__ __forceinline__ void row_group_scan(A *gtot, uint32_t groups, uint32_t C, uint32_t j, bool owner,
                                               uint32_t g) {
    for (uint32_t d = 1; d < groups; d <<= 1) {
        const bool take = owner && g >= d;
        A o = Op::template identity<A>();
        if (take) o = gtot[j - d * C];
        __syncthreads();
        if (take) gtot[j] = Op::combine(o, gtot[j]);
        __syncthreads();
    }
}

// Rescan of column c over logical rows [lo, hi) in place from `pre` (the
// carry into the group), eight rows read before they are rewritten.
template <typename T, typename Op, bool EXCL, bool REV>
__device__ __forceinline__ void row_group_rescan(T *tile, uint32_t n, uint32_t C, uint32_t c, uint32_t lo,
                                                 uint32_t hi, typename ColAcc<T>::type pre) {
    using A = typename ColAcc<T>::type;
    auto step = [&](T &slot, T x) {
        if constexpr (EXCL) {
            slot = (T)pre;
            pre = Op::combine(pre, (A)x);
        } else {
            pre = Op::combine(pre, (A)x);
            slot = (T)pre;
        }
    };
    uint32_t i = lo;
    for (; i + 8 <= hi; i += 8) {
        T x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = tile[(REV ? n - 1 - (i + u) : i + u) * C + c];
#pragma unroll
        for (int u = 0; u < 8; ++u) step(tile[(REV ? n - 1 - (i + u) : i + u) * C + c], x[u]);
    }
    for (; i < hi; ++i) {
        T &slot = tile[(REV ? n - 1 - i : i) * C + c];
        step(slot, slot);
    }
}

template <typename T, typename Op, bool REV>
__global__ __launch_bounds__(kRowTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void col_rowtile_totals_kernel(ScanParams p, RowTileShape s,
                                                                             typename ColAcc<T>::type *totals) {
    using A = typename ColAcc<T>::type;
    __shared__ __attribute__((aligned(16))) T tile[kRowTileElems];
    __shared__ A gtot[kRowTileThreads];
    const uint64_t t = xcd_contiguous(blockIdx.x, gridDim.x); // no look-back: any tile order
    const uint32_t C = s.C;
    uint64_t r0;
    uint32_t n;
    row_tile_span<REV>(s, t, r0, n);
    row_tile_load<T>((const T *)p.in + p.in_offset + r0 * C, n * C, tile);
    __syncthreads();
    const uint32_t j = threadIdx.x, g = j / C, c = j - g * C;
    const bool owner = g < s.groups;
    if (owner) {
        const uint32_t lo = g * s.rpg < n ? g * s.rpg : n;
        const uint32_t hi = lo + s.rpg < n ? lo + s.rpg : n;
        gtot[j] = row_group_fold<T, Op, REV>(tile, n, C, c, lo, hi);
    }
    __syncthreads();
    row_group_scan<A, Op>(gtot, s.groups, C, j, owner, g);
    if (j < C) totals[(uint64_t)j * s.tiles + t] = gtot[(s.groups - 1) * C + j]; // column-major
}

template <typename T, typename Op, bool EXCL, bool REV, bool CARRY>
__global__ __launch_bounds__(kRowTileThreads) __attribute__((amdgpu_waves_per_eu(4))) void col_rowtile_scan_kernel(ScanParams p, RowTileShape s,
                                                                           const typename ColAcc<T>::type *carries) {
    using A = typename ColAcc<T>::type;
    __shared__ __attribute__((aligned(16))) T tile[kRowTileElems];
    __shared__ A gtot[kRowTileThreads];
    const uint64_t t = xcd_contiguous(blockIdx.x, gridDim.x); // no look-back: any tile order
    const uint32_t C = s.C;
    uint64_t r0;
    uint32_t n;
    row_tile_span<REV>(s, t, r0, n);
    row_tile_load<T>((const T *)p.in + p.in_offset + r0 * C, n * C, tile);
    __syncthreads();
    const uint32_t j = threadIdx.x, g = j / C, c = j - g * C;
    const bool owner = g < s.groups;
    const uint32_t lo = g * s.rpg < n ? g * s.rpg : n;
    const uint32_t hi = lo + s.rpg < n ? lo + s.rpg : n;
    if (owner) gtot[j] = row_group_fold<T, Op, REV>(tile, n, C, c, lo, hi);
    __syncthreads();
    row_group_scan<A, Op>(gtot, s.groups, C, j, owner, g);
    if (owner) {
        A pre = CARRY ? carries[(uint64_t)c * s.tiles + t] : Op::template identity<A>();
        if (g > 0) pre = Op::combine(pre, gtot[j - C]);
        row_group_rescan<T, Op, EXCL, REV>(tile, n, C, c, lo, hi, pre);
    }
    __syncthreads();
    row_tile_store<T>(tile, n * C, (T *)p.out + p.out_offset + r0 * C);
}

// Single-pass row-tile column scan: the row tiles above with a decoupled
// look-back over C-wide carries, so every element is read once and written
// once.  Status entry (tile u, column c) is u * C + c.  After its groups'
// totals, tile t publishes its column aggregates (threads c < C), and the
// whole block looks back in rounds: thread j reads predecessor k = j / C
// (tile t - 1 - base - k) in column c = j mod C, so a round covers 512 / C
// predecessors; per column the nearest inclusive prefix of the round is an
// LDS atomicMin of k; entries up to it that are not ready are polled again,
// and after p.spin_limit polls the waiter rebuilds that predecessor's column
// aggregate from the input (rowtile_column_aggregate: the same group sums,
// folded in group order, so integers match the owner's bits and f32 its value
// to rounding) and uses it, so progress never depends on dispatch order.  The round's needed values fold over k through an LDS tree
// into the column carry, which is published with the tile's aggregate as the
// inclusive prefix.  Tile 0's value is always its prefix.  f32 carries are
// f64 in 16-byte slots (F64QuadDense), integers packed words.  Unlike the
// three-pass form, an f32 carry's f64 rounding depends on which predecessors
// had published prefixes: results agree with the f64 scan to within its
// bound, not bit for bit across runs.  2^28 u32, us, three passes -> one:
// C = 2 556 -> 474, 3 599 -> 471, 7 608 -> 473, 12 606 -> 468, 24 579 ->
// 514; at C = 48 / 100 / 255 (a round covering 10 / 5 / 2 predecessors)
// one pass took 622 / 800 / 1093, and several statuses per thread and
// round (up to 8) 572 / 687 / 909 against 578 / 585 / 635 in three passes.
template <typename T, typename Op, bool REV>
__device__ __forceinline__ typename ColAcc<T>::type rowtile_column_aggregate(const ScanParams &p, const RowTileShape &s,
                                                                         uint64_t u, uint32_t c) {
    using A = typename ColAcc<T>::type;
    const uint32_t C = s.C;
    uint64_t r0;
    uint32_t n;
    row_tile_span<REV>(s, u, r0, n);
    const T *base = (const T *)p.in + p.in_offset + r0 * C + c;
    A tot = Op::template identity<A>();
    for (uint32_t g = 0; g < s.groups; ++g) {
        const uint32_t lo = g * s.rpg < n ? g * s.rpg : n;
        const uint32_t hi = lo + s.rpg < n ? lo + s.rpg : n;
        A acc = Op::template identity<A>();
        for (uint32_t i = lo; i < hi; ++i) acc = Op::combine(acc, (A)base[(uint64_t)(REV ? n - 1 - i : i) * C]);
        tot = Op::combine(tot, acc);
    }
    return tot;
}

template <typename T, typename Op, typename Status, bool EXCL, bool REV>
__global__ __launch_bounds__(kRowTileThreads) __attribute__((amdgpu_waves_per_eu(4)))
void col_rowtile_lookback_kernel(ScanParams p, RowTileShape s, Status st) {
    using A = typename ColAcc<T>::type;
    __shared__ __attribute__((aligned(16))) T tile[kRowTileElems];
    __shared__ A gtot[kRowTileThreads];
    __shared__ A lb_val[kRowTileThreads];
    __shared__ A s_agg[256], s_carry[256];
    __shared__ uint32_t s_first[256], s_done[256];
    __shared__ uint32_t s_rows;
    const uint64_t t = p.tile0 + blockIdx.x; // scan order: the look-back needs dispatch order
    const uint32_t C = s.C;
    const A aid = Op::template identity<A>();
    uint64_t r0;
    uint32_t n;
    row_tile_span<REV>(s, t, r0, n);
    row_tile_load<T>((const T *)p.in + p.in_offset + r0 * C, n * C, tile);
    __syncthreads();
    const uint32_t j = threadIdx.x, g = j / C, c = j - g * C;
    const bool owner = g < s.groups;
    const uint32_t lo = g * s.rpg < n ? g * s.rpg : n;
    const uint32_t hi = lo + s.rpg < n ? lo + s.rpg : n;
    if (owner) gtot[j] = row_group_fold<T, Op, REV>(tile, n, C, c, lo, hi);
    __syncthreads();
    row_group_scan<A, Op>(gtot, s.groups, C, j, owner, g);
    if (j < C) {
        const A tot = gtot[(s.groups - 1) * C + j];
        s_agg[j] = tot;
        st.publish_tile(t * C + j, p.tag, t == 0 ? kPrefix : kAggregate, tot);
        s_carry[j] = aid;
        s_done[j] = t == 0 ? 1u : 0u;
    }
    __syncthreads();
    if (t > 0) {
        const uint32_t KP = kRowTileThreads / C; // predecessors per round
        const uint32_t k = j / C, kc = j - k * C;
        // Lanes of this wave below this one in the same column (l - C,
        // l - 2C, ...): of a wave's prefix flags in one column only the
        // lowest lane's goes to LDS, so the atomics on a column's word stay
        // at one per wave (one per thread took C = 3 scans from 456 to
        // about 580 us).
        const int lane = lane_id();
        uint64_t below = 0;
        for (int l = lane - (int)C; l >= 0; l -= (int)C) below |= 1ull << l;
        uint64_t base = 0;
        for (;;) {
            const bool item = k < KP && base + k < t && s_done[kc] == 0u;
            const uint64_t u = t - 1 - base - k;
            uint32_t flag = kInvalid;
            A val = aid;
            if (item) st.read(u * C + kc, p.tag, flag, val);
            uint32_t spins = 0;
            bool need;
            for (;;) {
                if (j < C) s_first[j] = KP;
                if (j == 0) s_rows = 0;
                __syncthreads();
                const bool pre = item && flag == kPrefix;
                const uint64_t pm = ballot(pre);
                if (pre && (pm & below) == 0ull) atomicMin(&s_first[kc], k);
                __syncthreads();
                need = item && k <= s_first[kc];
                const bool missing = need && flag == kInvalid;
                if (!__syncthreads_or(missing)) break;
                if (++spins >= p.spin_limit) {
                    if (missing) {
                        val = rowtile_column_aggregate<T, Op, REV>(p, s, u, kc);
                        flag = u == 0 ? kPrefix : kAggregate; // tile 0's aggregate is its prefix
                    }
                    spins = 0;
                } else {
                    __builtin_amdgcn_s_sleep(1);
                    if (missing) st.read(u * C + kc, p.tag, flag, val);
                }
            }
            // Fold the round's needed values over k (rows of a [KP][C]
            // array) in a fixed tree as deep as the deepest needed row, then
            // into the column carries.
            lb_val[j] = need ? val : aid;
            const uint32_t deep =
                group_reduce<64>(need ? k + 1 : 0u, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
            if (lane == 0 && deep > 0) atomicMax(&s_rows, deep);
            __syncthreads();
            for (uint32_t cur = s_rows; cur > 1;) {
                const uint32_t half = (cur + 1) / 2;
                if (j < (cur - half) * C) lb_val[j] = Op::combine(lb_val[j], lb_val[j + half * C]);
                __syncthreads();
                cur = half;
            }
            bool pending = false;
            if (j < C && s_done[j] == 0u) {
                s_carry[j] = Op::combine(s_carry[j], lb_val[j]);
                if (s_first[j] < KP) s_done[j] = 1u;
                else pending = true;
            }
            if (!__syncthreads_or(pending)) break;
            base += KP;
        }
        if (j < C) st.publish_tile(t * C + j, p.tag, kPrefix, Op::combine(s_carry[j], s_agg[j]));
        __syncthreads();
    }
    if (owner) {
        A pre = s_carry[c];
        if (g > 0) pre = Op::combine(pre, gtot[j - C]);
        row_group_rescan<T, Op, EXCL, REV>(tile, n, C, c, lo, hi, pre);
    }
    __syncthreads();
    row_tile_store<T>(tile, n * C, (T *)p.out + p.out_offset + r0 * C);
}

// Single-pass column scan.  A block owns a tile of kColTileRows scan steps x
// 64*V adjacent lines.  Its kColDataWaves data waves each hold kColRows
// steps of the tile in registers (lane l: lines 64*V*g + V*l .. +V-1), scan
// them per line, and combine their totals through LDS.  The block's last
// wave holds no data: it runs the decoupled look-back, lane l for its V
// lines, polling kColPoll earlier chunks of the same line group per round
// trip and folding aggregates until each line meets an inclusive prefix.
// Integer scans publish one packed word per line and chunk; f32 scans an
// f64 carry in a two-word slot (F64PairStatus), with the tile's steps
// scanned in f32 and the carries and outputs formed in f64.
// Data and look-back waves run separate code paths (wave-uniform), so the
// tile's registers are not live during the look-back.  Status entry of
// (chunk c, line j) is c * lpad + j.  Every element is read once and written
// once.  A predecessor that stays unpublished for p.spin_limit rounds has its
// aggregate rebuilt from the input by the waiter with the owner's arithmetic
// (f32: per-wave f32 prefix from the identity, then f64 over the waves in
// order) and used directly, so progress never depends on dispatch order.
constexpr int kColWaves = 16;
constexpr int kColDataWaves = kColWaves - 1;
constexpr int kColRows = 16;
constexpr uint64_t kColTileRows = (uint64_t)kColDataWaves * kColRows;
// Predecessor chunks polled per round trip.  Status reads are device-scope
// and uncached, and wider polls cost more than the round trips they save
// (u32, 65536 x 4096 / 1048576 x 256: 1 chunk 0.352 / 0.462 ms; 2: 0.354 /
// 0.491; 4: 0.361 / 0.568; 8: 0.384 / 0.762).
constexpr int kColPoll = 1;

template <typename T, int V>
__device__ __forceinline__ void col_load_t(const T *p, T (&x)[V]) {
    if constexpr (V == 4) {
        using Vt = typename Vec4A4<T>::type;
        const Vt v = __builtin_nontemporal_load((const Vt *)p);
        x[0] = (T)v.x;
        x[1] = (T)v.y;
        x[2] = (T)v.z;
        x[3] = (T)v.w;
    } else {
        x[0] = __builtin_nontemporal_load(p);
    }
}

template <typename T, int V>
__device__ __forceinline__ void col_store_t(T *p, const T (&y)[V]) {
    if constexpr (V == 4) {
        using Vt = typename Vec4A4<T>::type;
        Vt v;
        v.x = y[0];
        v.y = y[1];
        v.z = y[2];
        v.w = y[3];
        __builtin_nontemporal_store(v, (Vt *)p);
    } else {
        __builtin_nontemporal_store(y[0], p);
    }
}

// The same for the lane of a partial group: its nv < V lines one by one,
// the others read as `ident` and never stored.
template <typename T, int V>
__device__ __forceinline__ void col_load_n(const T *p, uint32_t nv, T ident, T (&x)[V]) {
    if (V == 1 || nv >= (uint32_t)V) {
        col_load_t<T, V>(p, x);
        return;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) x[v] = (uint32_t)v < nv ? __builtin_nontemporal_load(p + v) : ident;
}

template <typename T, int V>
__device__ __forceinline__ void col_store_n(T *p, uint32_t nv, const T (&y)[V]) {
    if (V == 1 || nv >= (uint32_t)V) {
        col_store_t<T, V>(p, y);
        return;
    }
#pragma unroll
    for (int v = 0; v < V; ++v)
        if ((uint32_t)v < nv) __builtin_nontemporal_store(y[v], p + v);
}

// Aggregate of chunk c for the V lines starting at line0, exactly as the
// owner computes it (the decoupled fallback).
template <typename T, typename Op, int V, bool REV>
__device__ void col_tile_aggregate(const ScanParams &p, uint64_t c, uint64_t line0,
                                   typename ColAcc<T>::type (&agg)[V]) {
    using A = typename ColAcc<T>::type;
    const T *in = (const T *)p.in + ((int64_t)p.in_offset + (int64_t)line0 * p.in_line_stride);
    const uint32_t nv = col_valid_lines(p.lines, line0, V);
#pragma unroll
    for (int v = 0; v < V; ++v) agg[v] = Op::template identity<A>();
    // Rolled loops: this rare path must not add register pressure to the
    // kernel, whose tile stays live in registers across the look-back.
#pragma unroll 1
    for (int q = 0; q < kColDataWaves; ++q) {
        T run[V];
#pragma unroll
        for (int v = 0; v < V; ++v) run[v] = Op::template identity<T>();
#pragma unroll 1
        for (int r = 0; r < kColRows; ++r) {
            const uint64_t i = c * kColTileRows + (uint64_t)q * kColRows + r;
            if (i >= p.len) break;
            const uint64_t li = REV ? p.len - 1 - i : i;
            T x[V];
            col_load_n<T, V>(in + (int64_t)li * p.in_elem_stride, nv, Op::template identity<T>(), x);
#pragma unroll
            for (int v = 0; v < V; ++v) run[v] = Op::combine(run[v], x[v]);
        }
#pragma unroll
        for (int v = 0; v < V; ++v) agg[v] = Op::combine(agg[v], (A)run[v]);
    }
}

// Addressing of a line group: a wave-uniform element base (the group's
// lowest address on every step) and one 32-bit byte offset per lane, so each
// access is a scalar base plus a vector offset and no per-step 64-bit address
// stays live across the look-back.
struct ColGroupAddr {
    int64_t base;      // element offset of the group's lowest line, step 0
    uint32_t lane_off; // bytes from there to this lane's first line
};

template <int V, typename T>
__device__ __forceinline__ ColGroupAddr col_group_addr(uint64_t g, int lane, int64_t line_stride, uint64_t offset) {
    constexpr int64_t kGroup = (int64_t)kWave * V;
    ColGroupAddr a;
    if (line_stride > 0) {
        a.base = (int64_t)offset + (int64_t)g * kGroup;
        a.lane_off = (uint32_t)(lane * V) * (uint32_t)sizeof(T);
    } else { // -1: lines run downwards in memory (one line per lane)
        a.base = (int64_t)offset - ((int64_t)g * kGroup + kGroup - 1);
        a.lane_off = (uint32_t)(kGroup - 1 - lane * V) * (uint32_t)sizeof(T);
    }
    return a;
}

// The look-back wave: publishes the tile's aggregate, folds its
// predecessors' statuses per line (kColPoll chunks per round trip, consumed
// in order and in step for all of the lane's lines, so no status is counted
// twice), publishes the inclusive prefix and leaves the carry in s_carry.
template <typename T, typename Op, typename Status, int V, bool REV>
__device__ void col_lookback_wave(const ScanParams &p, const Status &st, uint64_t c, uint64_t lpad, uint64_t line0,
                                  bool active, const typename ColAcc<T>::type (&agg)[V],
                                  typename ColAcc<T>::type (&excl)[V]) {
    using A = typename ColAcc<T>::type;
    constexpr int P = kColPoll;
    const A aid = Op::template identity<A>();
#pragma unroll
    for (int v = 0; v < V; ++v) excl[v] = aid;
    if (!active) return;
    const uint64_t e = c * lpad + line0;
    if (c == 0) {
#pragma unroll
        for (int v = 0; v < V; ++v) st.publish_tile(e + v, p.tag, kPrefix, agg[v]);
        return;
    }
#pragma unroll
    for (int v = 0; v < V; ++v) st.publish_tile(e + v, p.tag, kAggregate, agg[v]);
    bool done[V];
#pragma unroll
    for (int v = 0; v < V; ++v) done[v] = false;
    uint64_t pos = c - 1; // next predecessor to consume
    uint32_t spins = 0;
    for (;;) {
        uint32_t flag[P][V];
        A val[P][V];
#pragma unroll
        for (int k = 0; k < P; ++k)
#pragma unroll
            for (int v = 0; v < V; ++v) {
                flag[k][v] = kInvalid;
                val[k][v] = aid;
                if (!done[v] && (uint64_t)k <= pos) st.read((pos - k) * lpad + line0 + v, p.tag, flag[k][v], val[k][v]);
            }
        // The next predecessor not ready for some line: wait, and after
        // p.spin_limit polls take its aggregate from the input (the owner's
        // arithmetic) and use it directly -- so progress never depends on
        // dispatch order.  Publishing it is only a courtesy to other
        // waiters, and is skipped where a status slot must keep one writer.
        bool ready0 = true;
#pragma unroll
        for (int v = 0; v < V; ++v) ready0 = ready0 && (done[v] || flag[0][v] != kInvalid);
        if (!ready0) {
            if (++spins < p.spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                continue;
            }
            A fb[V];
            col_tile_aggregate<T, Op, V, REV>(p, pos, line0, fb);
#pragma unroll
            for (int v = 0; v < V; ++v)
                if (!done[v] && flag[0][v] == kInvalid) {
                    st.publish_if_unset(pos * lpad + line0 + v, p.tag, kAggregate, fb[v]);
                    flag[0][v] = kAggregate;
                    val[0][v] = fb[v];
                }
        }
        spins = 0;
        int used = 0;
        bool finished = false;
#pragma unroll
        for (int k = 0; k < P; ++k) {
            if (finished || used < k || (uint64_t)k > pos) break;
            bool ready = true;
#pragma unroll
            for (int v = 0; v < V; ++v) ready = ready && (done[v] || flag[k][v] != kInvalid);
            if (!ready) break;
            // Chunk 0's aggregate is its inclusive prefix: a fallback may
            // have published it as an aggregate, and consuming it still
            // finishes the line.
            const bool first_chunk = (uint64_t)k == pos;
            bool all = true;
#pragma unroll
            for (int v = 0; v < V; ++v) {
                if (done[v]) continue;
                excl[v] = Op::combine(val[k][v], excl[v]);
                if (flag[k][v] == kPrefix || first_chunk) done[v] = true;
                else all = false;
            }
            used = k + 1;
            finished = all;
        }
        if (finished) break;
        pos -= (uint64_t)used; // used >= 1 (entry pos was ready); chunk 0 finishes every line
    }
#pragma unroll
    for (int v = 0; v < V; ++v) st.publish_tile(e + v, p.tag, kPrefix, Op::combine(excl[v], agg[v]));
}

template <typename T, typename Op, typename Status, int V, bool EXCL, bool REV>
__global__ __launch_bounds__(kColWaves *kWave) void col_lookback_kernel(ScanParams p, Status st, uint64_t groups,
                                                                        uint64_t lpad) {
    using A = typename ColAcc<T>::type;
    constexpr int kLines = kWave * V;
    __shared__ A s_agg[kColDataWaves][kLines];
    __shared__ A s_carry[kLines];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = lane_id();
    const uint64_t tile = blockIdx.x;
    const uint64_t g = tile % groups, c = tile / groups;
    const uint64_t line0 = (g * kWave + (uint64_t)lane) * V;
    const bool active = line0 < p.lines;
    const uint32_t nv = active ? col_valid_lines(p.lines, line0, V) : 0u;
    const A aid = Op::template identity<A>();

    if (w == kColDataWaves) {
        __syncthreads(); // the data waves' totals
        A agg[V], excl[V];
#pragma unroll
        for (int v = 0; v < V; ++v) agg[v] = aid;
#pragma unroll 1
        for (int q = 0; q < kColDataWaves; ++q)
#pragma unroll
            for (int v = 0; v < V; ++v) agg[v] = Op::combine(agg[v], s_agg[q][lane * V + v]);
        col_lookback_wave<T, Op, Status, V, REV>(p, st, c, lpad, line0, active, agg, excl);
#pragma unroll
        for (int v = 0; v < V; ++v) s_carry[lane * V + v] = excl[v];
        __syncthreads(); // the carry
        return;
    }

    const uint64_t i0 = c * kColTileRows + (uint64_t)w * kColRows;
    const ColGroupAddr ia = col_group_addr<V, T>(g, lane, p.in_line_stride, p.in_offset);
    const ColGroupAddr oa = col_group_addr<V, T>(g, lane, p.out_line_stride, p.out_offset);
    const T tid = Op::template identity<T>();

    // The wave's steps, scanned per line from the identity.
    T x[kColRows][V];
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        const uint64_t i = i0 + r;
        if (active && i < p.len) {
            const int64_t li = (int64_t)(REV ? p.len - 1 - i : i);
            const char *row = (const char *)((const T *)p.in + (ia.base + li * p.in_elem_stride));
            col_load_n<T, V>((const T *)(row + ia.lane_off), nv, tid, x[r]);
        } else {
#pragma unroll
            for (int v = 0; v < V; ++v) x[r][v] = tid;
        }
    }
#pragma unroll
    for (int r = 0; r < kColRows; ++r)
#pragma unroll
        for (int v = 0; v < V; ++v) x[r][v] = Op::combine(r == 0 ? tid : x[r - 1][v], x[r][v]);
#pragma unroll
    for (int v = 0; v < V; ++v) s_agg[w][lane * V + v] = (A)x[kColRows - 1][v];
    __syncthreads(); // totals to the look-back wave
    __syncthreads(); // its carry
    if (!active) return;

    A carry[V];
#pragma unroll
    for (int v = 0; v < V; ++v) carry[v] = s_carry[lane * V + v];
#pragma unroll 1
    for (int q = 0; q < w; ++q)
#pragma unroll
        for (int v = 0; v < V; ++v) carry[v] = Op::combine(carry[v], s_agg[q][lane * V + v]);
#pragma unroll
    for (int r = 0; r < kColRows; ++r) {
        const uint64_t i = i0 + r;
        if (i >= p.len) break;
        T y[V];
#pragma unroll
        for (int v = 0; v < V; ++v) {
            if constexpr (EXCL)
                y[v] = r == 0 ? finalize<T, A, Op>(carry[v], tid) : finalize<T, A, Op>(carry[v], x[r - 1][v]);
            else
                y[v] = finalize<T, A, Op>(carry[v], x[r][v]);
        }
        const int64_t li = (int64_t)(REV ? p.len - 1 - i : i);
        char *row = (char *)((T *)p.out + (oa.base + li * p.out_elem_stride));
        col_store_n<T, V>((T *)(row + oa.lane_off), nv, y);
    }
}

// 16 waves per CU: on a 65536 x 4096 u32 column scan 4096 waves of 256 steps
// took 164 + 12 + 386 us (totals, carry, rescan); 8192 waves 202 + 23 + 512.
constexpr uint64_t kColTargetWaves = 4096;
constexpr uint64_t kColMinChunk = 32;      // scan steps per chunk

bool column_mode(const ScanArgs &a) {
    const bool contiguous = a.in_elem_stride == 1 && a.out_elem_stride == 1;
    const bool adjacent = (a.in_line_stride == 1 || a.in_line_stride == -1) &&
                          (a.out_line_stride == 1 || a.out_line_stride == -1);
    return !contiguous && adjacent && a.lines >= 16;
}

ColShape column_shape(const ScanArgs &a) {
    ColShape s;
    const uintptr_t ibase = (uintptr_t)a.in + 4u * a.in_offset; // every element type is 4 bytes
    const uintptr_t obase = (uintptr_t)a.out + 4u * a.out_offset;
    // A lane's four adjacent lines are one 16-byte vector per step; the
    // vectors need only 4-byte alignment (Vec4A4), so any element stride and
    // start qualify.  When the line count is not a multiple of 4, the lane
    // of the last group moves its 1-3 lines one by one (col_load_n,
    // ColIO::load_n): u32 [8191, 8191] and [1023, 65537] along axis 0 took
    // 189 and 293 us with one line per lane everywhere.
    const bool vec = a.in_line_stride == 1 && a.out_line_stride == 1 && ibase % 4 == 0 && obase % 4 == 0;
    s.V = vec ? 4 : 1;
    s.groups = ceil_div(a.lines, (uint64_t)kWave * s.V);
    uint64_t k = 1;
    if (s.groups < kColTargetWaves) {
        k = ceil_div(kColTargetWaves, s.groups);
        const uint64_t kmax = ceil_div(a.len, kColMinChunk);
        if (k > kmax) k = kmax;
    }
    if (k <= 1) {
        s.chunk = a.len;
        s.nchunks = 1;
    } else {
        s.chunk = ceil_div(a.len, k);
        s.nchunks = (uint32_t)ceil_div(a.len, s.chunk);
    }
    return s;
}

// Single-pass column scans (col_lookback_kernel): line groups, padded line
// count of the status array, chunks of kColTileRows steps.
struct ColLbShape {
    int V = 1;
    uint64_t groups = 0, lpad = 0, chunks = 0;
};

ColLbShape col_lb_shape(const ScanArgs &a) {
    ColLbShape s;
    s.V = column_shape(a).V;
    s.groups = ceil_div(a.lines, (uint64_t)kWave * s.V);
    s.lpad = s.groups * kWave * s.V;
    s.chunks = ceil_div(a.len, kColTileRows);
    return s;
}

// The single pass needs whole line groups: with fewer than 256 lines every
// tile leaves lanes idle and all tiles form one long look-back chain
// (measured, u32: 4194304 x 64 1.63 ms single-pass against 0.75 ms chunked;
// 1048576 x 256 0.46 against 0.71; 65536 x 4096 0.35 against 0.54; f32
// 65536 x 4096 0.48 against 0.56).
constexpr uint64_t kSinglePassMinLines = 256;
// Many short lines: a scan of at most kColShortMaxLen steps whose chunked
// form needs one chunk over at least kColShortMinGroups line groups reads and
// writes each element once in col_scan_kernel, with no carries and no
// look-back.  The single pass's tiles hold 240 steps, so at 4 steps a
// sixteenth of its waves had data: u32 [4, 2^24] along axis 0 took 760 us
// single-pass and takes 85 this way ([16, 2^22] 207 -> 131, [64, 2^20] 109
// -> 100).  Longer lines keep the single pass ([240, 2^20]: 373 us against
// 435), and so do fewer groups, which leave the chip too few waves for
// serial steps ([32, 2^16]: 5.3 us against 7.5).
constexpr uint64_t kColShortMaxLen = 64;
constexpr uint64_t kColShortMinGroups = 1024;
bool column_single_pass(const ScanArgs &a) {
    if (!column_mode(a) || a.lines < kSinglePassMinLines) return false;
    const ColShape s = column_shape(a);
    return !(s.nchunks == 1 && a.len <= kColShortMaxLen && s.groups >= kColShortMinGroups);
}

uint64_t column_bytes(const ScanArgs &a) {
    const ColShape s = column_shape(a);
    if (s.nchunks <= 1 || a.lines == 0) return 0;
    return (uint64_t)s.nchunks * a.lines * (a.dtype == HX_DTYPE_F32 ? 8u : 4u);
}

template <typename T, typename Op, int V, bool EXCL, bool REV>
hx_status launch_column_v(const ScanParams &p, const ColShape &s, void *ws, hipStream_t stream) {
    using A = typename ColAcc<T>::type;
    A *totals = (A *)ws;
    const uint64_t blocks = ceil_div(s.groups * s.nchunks, kBlock / kWave);
    if (blocks > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "column scan exceeds the grid range");
    const dim3 grid((uint32_t)blocks), block(kBlock);
    if (s.nchunks <= 1) {
        hipLaunchKernelGGL((col_scan_kernel<T, Op, V, EXCL, REV, false>), grid, block, 0, stream, p,
                           (const A *)nullptr, s.chunk, s.nchunks, s.groups);
        return check_launch("col_scan_kernel");
    }
    hipLaunchKernelGGL((col_totals_kernel<T, Op, V, REV>), grid, block, 0, stream, p, totals, s.chunk, s.nchunks,
                       s.groups);
    HX_TRY(check_launch("col_totals_kernel"));
    hipLaunchKernelGGL((col_carry_kernel<A, Op>), dim3((uint32_t)ceil_div(p.lines, kWave)), dim3(kWave * kCarrySlices),
                       0, stream, totals, p.lines, s.nchunks);
    HX_TRY(check_launch("col_carry_kernel"));
    hipLaunchKernelGGL((col_scan_kernel<T, Op, V, EXCL, REV, true>), grid, block, 0, stream, p, (const A *)totals,
                       s.chunk, s.nchunks, s.groups);
    return check_launch("col_scan_kernel");
}

template <typename T, typename Op, typename Status, int V, bool EXCL, bool REV>
hx_status launch_col_lookback_v(const ScanParams &p, const ColLbShape &s, const Status &st, hipStream_t stream) {
    hipLaunchKernelGGL((col_lookback_kernel<T, Op, Status, V, EXCL, REV>), dim3((uint32_t)(s.groups * s.chunks)),
                       dim3(kColWaves * kWave), 0, stream, p, st, s.groups, s.lpad);
    return check_launch("col_lookback_kernel");
}

template <typename T, typename Op, typename Status, int V>
hx_status launch_col_lookback_s(const ScanParams &p, const ColLbShape &s, const Status &st, bool excl, bool rev,
                                hipStream_t stream) {
    if (excl)
        return rev ? launch_col_lookback_v<T, Op, Status, V, true, true>(p, s, st, stream)
                   : launch_col_lookback_v<T, Op, Status, V, true, false>(p, s, st, stream);
    return rev ? launch_col_lookback_v<T, Op, Status, V, false, true>(p, s, st, stream)
               : launch_col_lookback_v<T, Op, Status, V, false, false>(p, s, st, stream);
}

template <typename T, typename Op>
hx_status launch_col_lookback(const ScanParams &p, const ColLbShape &s, bool excl, bool rev, void *status,
                              hipStream_t stream) {
    if constexpr (std::is_same<T, float>::value) {
        const F64PairStatus st{(uint64_t *)status};
        return s.V == 4 ? launch_col_lookback_s<T, Op, F64PairStatus, 4>(p, s, st, excl, rev, stream)
                        : launch_col_lookback_s<T, Op, F64PairStatus, 1>(p, s, st, excl, rev, stream);
    } else {
        const PackedStatus st{(uint64_t *)status};
        return s.V == 4 ? launch_col_lookback_s<T, Op, PackedStatus, 4>(p, s, st, excl, rev, stream)
                        : launch_col_lookback_s<T, Op, PackedStatus, 1>(p, s, st, excl, rev, stream);
    }
}

template <typename T, typename Op, bool EXCL>
hx_status launch_column(const ScanParams &p, const ColShape &s, bool rev, void *ws, hipStream_t stream) {
    if (s.V == 4)
        return rev ? launch_column_v<T, Op, 4, EXCL, true>(p, s, ws, stream)
                   : launch_column_v<T, Op, 4, EXCL, false>(p, s, ws, stream);
    return rev ? launch_column_v<T, Op, 1, EXCL, true>(p, s, ws, stream)
               : launch_column_v<T, Op, 1, EXCL, false>(p, s, ws, stream);
}

// One 128-byte line per tile or superblock entry (a packed u32 word or a
// 16-byte f64 slot at its start).
uint64_t status_bytes(uint64_t entries) { return entries * kTileStatusBytes; }

// Tile shapes (waves x 16-byte steps per lane).  A line up to 32768
// elements is one tile: the smallest shape that holds it, so a block never
// carries idle waves and a row-wise scan needs no look-back.  Longer lines
// take 8 x 16 tiles chained by the look-back.  Measured on 2^28 u32 (f32)
// inclusive scans as 65536 x 4096: 1316 us (2329) with 8 x 16 tiles, whose
// waves 1-7 held no elements, against 334 (333) with 4 x 4; 262144 x 1024:
// 3404 (6047) against 331 (339) with 2 x 2; 16384 x 16384: 4 x 16 360 us,
// 8 x 8 410; 1048576 x 256: 1 x 1 351 us, 2 x 2 636; 524288 x 512: 1 x 2
// 339, 2 x 2 434.
struct TileShape {
    int waves, steps;
    uint64_t elems() const { return (uint64_t)waves * kWave * 4 * steps; }
};
// Lines longer than one 8 x 16 tile: the tiles chained by the look-back.
// f32 lines took 12 x 16 tiles (one block per CU) before f32 tiles fit in
// 128 VGPRs; 8 x 16 at two blocks per CU: 2^30 f32 1373.1 -> 1315.6 us.
constexpr int kLongWaves = 8, kLongSteps = 16;
inline TileShape tile_shape(uint64_t len) {
    if (len <= 256) return {1, 1};
    if (len <= 512) return {1, 2};
    if (len <= 1024) return {2, 2};
    if (len <= 2048) return {2, 4};
    if (len <= 4096) return {4, 4};
    if (len <= 8192) return {4, 8};
    if (len <= 16384) return {4, 16};
    if (len <= 32768) return {kWaves, kSteps};
    return TileShape{kLongWaves, kLongSteps};
}

// A launch's work-items (blocks x block size) must stay below 2^32, so many
// short lines (2^26 lines of at most 512 elements, 2^24 of at most 8192)
// take several launches of consecutive tiles, in order.  A later batch's
// look-back reads an earlier batch's statuses, published under the same tag
// before that launch ended; lines of one tile publish none.
template <typename T, typename Op, typename Status, bool EXCL, int STEPS, int WAVES>
hx_status launch_tiles_shaped(ScanParams p, const Status &st, const Status &st1, bool vec, bool rev,
                              hipStream_t stream) {
    const uint64_t max_blocks = std::min<uint64_t>(0x7FFFFFFFull, 0xFFFFFFFFull / (WAVES * kWave));
    const uint64_t total = p.total_tiles;
    for (uint64_t t0 = 0; t0 < total; t0 += max_blocks) {
        p.tile0 = t0;
        const dim3 grid((uint32_t)std::min<uint64_t>(max_blocks, total - t0)), block(WAVES * kWave);
        if (p.head != 0) {
            // Only long lines of 16-byte accesses run on virtual lines
            // (scan_out_head); the bounds cost the other launches registers,
            // so they have kernels of their own.
            if constexpr (STEPS == kSteps && WAVES == kWaves) {
                if (!vec) return fail(HX_ERR_DISPATCH_FAILED, "virtual line heads need 16-byte accesses");
                if (rev)
                    hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, true, true, STEPS, true, WAVES, true>),
                                       grid, block, 0, stream, p, st, st1);
                else
                    hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, true, false, STEPS, true, WAVES, true>),
                                       grid, block, 0, stream, p, st, st1);
                HX_TRY(check_launch("scan_tiles_kernel"));
                continue;
            } else {
                return fail(HX_ERR_DISPATCH_FAILED, "virtual line heads need the long-line tiles");
            }
        }
        if (vec && rev)
            hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, true, true, STEPS, true, WAVES>), grid, block,
                               0, stream, p, st, st1);
        else if (vec)
            hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, true, false, STEPS, true, WAVES>), grid, block,
                               0, stream, p, st, st1);
        else if (rev)
            hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, false, true, STEPS, true, WAVES>), grid, block,
                               0, stream, p, st, st1);
        else
            hipLaunchKernelGGL((scan_tiles_kernel<T, Op, Status, EXCL, false, false, STEPS, true, WAVES>), grid, block,
                               0, stream, p, st, st1);
        HX_TRY(check_launch("scan_tiles_kernel"));
    }
    return HX_OK;
}

template <typename T, typename Op, typename Status, bool EXCL>
hx_status launch_tiles(const ScanParams &p, const Status &st, const Status &st1, bool vec, bool rev,
                       const TileShape &shape, hipStream_t stream) {
    switch (shape.waves * 100 + shape.steps) {
    case 101: return launch_tiles_shaped<T, Op, Status, EXCL, 1, 1>(p, st, st1, vec, rev, stream);
    case 102: return launch_tiles_shaped<T, Op, Status, EXCL, 2, 1>(p, st, st1, vec, rev, stream);
    case 202: return launch_tiles_shaped<T, Op, Status, EXCL, 2, 2>(p, st, st1, vec, rev, stream);
    case 204: return launch_tiles_shaped<T, Op, Status, EXCL, 4, 2>(p, st, st1, vec, rev, stream);
    case 404: return launch_tiles_shaped<T, Op, Status, EXCL, 4, 4>(p, st, st1, vec, rev, stream);
    case 408: return launch_tiles_shaped<T, Op, Status, EXCL, 8, 4>(p, st, st1, vec, rev, stream);
    case 416: return launch_tiles_shaped<T, Op, Status, EXCL, 16, 4>(p, st, st1, vec, rev, stream);
    default: break;
    }
    static_assert(kLongWaves == kWaves && kLongSteps == kSteps, "long lines take the 32768-element tile");
    return launch_tiles_shaped<T, Op, Status, EXCL, kSteps, kWaves>(p, st, st1, vec, rev, stream);
}

// Short dense lines (scan_short_lines_kernel): fewer than 256 elements per
// line, lines packed back to back in input and output.
constexpr uint64_t kShortLineMax = 256;
constexpr int kShortWaves = 8, kShortSteps = 16;
bool short_line_scan(const ScanArgs &a) {
    return a.len >= 1 && a.len < kShortLineMax && a.lines >= 2 && a.in_elem_stride == 1 &&
           a.out_elem_stride == 1 && a.in_line_stride == (int64_t)a.len && a.out_line_stride == (int64_t)a.len;
}

template <typename T, typename Op, bool EXCL, bool REV>
hx_status launch_short_dir(ShortParams p, hipStream_t stream) {
    constexpr uint64_t kTile = (uint64_t)kShortWaves * kWave * 4 * kShortSteps;
    const uint64_t tiles = ceil_div(p.n, kTile);
    const uint64_t max_blocks = std::min<uint64_t>(0x7FFFFFFFull, 0xFFFFFFFFull / (kShortWaves * kWave));
    for (uint64_t t0 = 0; t0 < tiles; t0 += max_blocks) {
        p.tile0 = t0;
        hipLaunchKernelGGL((scan_short_lines_kernel<T, Op, EXCL, REV, kShortSteps, kShortWaves>),
                           dim3((uint32_t)std::min<uint64_t>(max_blocks, tiles - t0)), dim3(kShortWaves * kWave), 0,
                           stream, p);
        HX_TRY(check_launch("scan_short_lines_kernel"));
    }
    return HX_OK;
}

template <typename T, typename Op>
hx_status launch_short(const ScanArgs &a, hipStream_t stream) {
    ShortParams p{};
    p.in = a.in;
    p.out = a.out;
    p.n = a.lines * a.len;
    p.in_offset = a.in_offset;
    p.out_offset = a.out_offset;
    p.len = (uint32_t)a.len;
    if (a.exclusive)
        return a.reverse ? launch_short_dir<T, Op, true, true>(p, stream) : launch_short_dir<T, Op, true, false>(p, stream);
    return a.reverse ? launch_short_dir<T, Op, false, true>(p, stream) : launch_short_dir<T, Op, false, false>(p, stream);
}

// Narrow column scans (col_narrow_*): see the kernels' comment.
bool narrow_column_scan(const ScanArgs &a) {
    const uint64_t c = a.lines;
    const uintptr_t ibase = (uintptr_t)a.in + 4u * a.in_offset; // every element type is 4 bytes
    const uintptr_t obase = (uintptr_t)a.out + 4u * a.out_offset;
    return c >= 32 && c < kSinglePassMinLines && (c & (c - 1)) == 0 && a.in_line_stride == 1 &&
           a.out_line_stride == 1 && a.in_elem_stride == (int64_t)c && a.out_elem_stride == (int64_t)c &&
           ibase % 4 == 0 && obase % 4 == 0;
}

uint64_t narrow_tiles(const ScanArgs &a) { return ceil_div((a.len * a.lines) >> 2, kNarrowTileVecs); }
uint64_t narrow_bytes(const ScanArgs &a) {
    const uint64_t tiles = narrow_tiles(a);
    if (tiles <= 1) return 0;
    return tiles * a.lines * (a.dtype == HX_DTYPE_F32 ? 8u : 4u);
}

template <typename T, typename Op, bool EXCL, bool REV>
hx_status launch_narrow_dir(const ScanParams &p, uint64_t tiles, void *ws, hipStream_t stream) {
    using A = typename ColAcc<T>::type;
    if (tiles > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "column scan exceeds the grid range");
    const dim3 grid((uint32_t)tiles), block(kNarrowWaves * kWave);
    A *totals = (A *)ws;
    if (tiles > 1) {
        hipLaunchKernelGGL((col_narrow_totals_kernel<T, Op, REV>), grid, block, 0, stream, p, totals);
        HX_TRY(check_launch("col_narrow_totals_kernel"));
        hipLaunchKernelGGL((col_narrow_carry_kernel<A, Op>), dim3((uint32_t)p.lines), dim3(kNarrowCarryThreads), 0,
                           stream, totals, p.lines, (uint64_t)1, tiles);
        HX_TRY(check_launch("col_narrow_carry_kernel"));
        hipLaunchKernelGGL((col_narrow_scan_kernel<T, Op, EXCL, REV, true>), grid, block, 0, stream, p,
                           (const A *)totals);
    } else {
        hipLaunchKernelGGL((col_narrow_scan_kernel<T, Op, EXCL, REV, false>), grid, block, 0, stream, p,
                           (const A *)totals);
    }
    return check_launch("col_narrow_scan_kernel");
}

template <typename T, typename Op>
hx_status launch_narrow(const ScanArgs &a, const ScanParams &p, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    const uint64_t tiles = narrow_tiles(a);
    if (tiles > 1 && ws_bytes < narrow_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small", (unsigned long long)ws_bytes);
    if (a.exclusive)
        return a.reverse ? launch_narrow_dir<T, Op, true, true>(p, tiles, ws, stream)
                         : launch_narrow_dir<T, Op, true, false>(p, tiles, ws, stream);
    return a.reverse ? launch_narrow_dir<T, Op, false, true>(p, tiles, ws, stream)
                     : launch_narrow_dir<T, Op, false, false>(p, tiles, ws, stream);
}

// Row-tile column scans (col_rowtile_*): see the kernels' comment.
bool rowtile_column_scan(const ScanArgs &a) {
    const uint64_t c = a.lines;
    const uintptr_t ibase = (uintptr_t)a.in + 4u * a.in_offset; // every element type is 4 bytes
    const uintptr_t obase = (uintptr_t)a.out + 4u * a.out_offset;
    return c >= 2 && c < kSinglePassMinLines && !narrow_column_scan(a) && a.in_line_stride == 1 &&
           a.out_line_stride == 1 && a.in_elem_stride == (int64_t)c && a.out_elem_stride == (int64_t)c &&
           ibase % 4 == 0 && obase % 4 == 0;
}

// Row-tile scans of more than one tile and at most kRowTileLbMaxCols columns
// look back (col_rowtile_lookback_kernel) instead of taking three passes:
// a look-back round covers 512 / C predecessors, and with fewer the chain of
// tiles falls behind.
constexpr uint64_t kRowTileLbMaxCols = 24;
bool rowtile_single_pass(const ScanArgs &a) {
    return a.lines <= kRowTileLbMaxCols && row_tile_shape(a.lines, a.len).tiles > 1;
}

uint64_t rowtile_bytes(const ScanArgs &a) {
    const RowTileShape s = row_tile_shape(a.lines, a.len);
    if (s.tiles <= 1) return 0;
    return s.tiles * a.lines * (a.dtype == HX_DTYPE_F32 ? 8u : 4u);
}

template <typename T, typename Op, bool EXCL, bool REV>
hx_status launch_rowtile_dir(const ScanParams &p, const RowTileShape &s, void *ws, hipStream_t stream) {
    using A = typename ColAcc<T>::type;
    if (s.tiles > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "column scan exceeds the grid range");
    const dim3 grid((uint32_t)s.tiles), block(kRowTileThreads);
    A *totals = (A *)ws;
    if (s.tiles > 1) {
        hipLaunchKernelGGL((col_rowtile_totals_kernel<T, Op, REV>), grid, block, 0, stream, p, s, totals);
        HX_TRY(check_launch("col_rowtile_totals_kernel"));
        hipLaunchKernelGGL((col_narrow_carry_kernel<A, Op>), dim3(s.C), dim3(kNarrowCarryThreads), 0, stream, totals,
                           (uint64_t)1, s.tiles, s.tiles);
        HX_TRY(check_launch("col_narrow_carry_kernel"));
        hipLaunchKernelGGL((col_rowtile_scan_kernel<T, Op, EXCL, REV, true>), grid, block, 0, stream, p, s,
                           (const A *)totals);
    } else {
        hipLaunchKernelGGL((col_rowtile_scan_kernel<T, Op, EXCL, REV, false>), grid, block, 0, stream, p, s,
                           (const A *)totals);
    }
    return check_launch("col_rowtile_scan_kernel");
}

uint64_t rowtile_lb_bytes(const ScanArgs &a) {
    const RowTileShape s = row_tile_shape(a.lines, a.len);
    return kLookbackOffset + s.tiles * a.lines * (a.dtype == HX_DTYPE_F32 ? 16u : 8u);
}

template <typename T, typename Op, typename Status, bool EXCL>
hx_status launch_rowtile_lb_dir(const ScanParams &p, const RowTileShape &s, const Status &st, bool rev,
                                hipStream_t stream) {
    const dim3 grid((uint32_t)s.tiles), block(kRowTileThreads);
    if (rev)
        hipLaunchKernelGGL((col_rowtile_lookback_kernel<T, Op, Status, EXCL, true>), grid, block, 0, stream, p, s, st);
    else
        hipLaunchKernelGGL((col_rowtile_lookback_kernel<T, Op, Status, EXCL, false>), grid, block, 0, stream, p, s, st);
    return check_launch("col_rowtile_lookback_kernel");
}

template <typename T, typename Op>
hx_status launch_rowtile_lb(const ScanArgs &a, ScanParams p, void *ws, uint64_t ws_bytes, LookbackState &lb,
                            hipStream_t stream) {
    const RowTileShape s = row_tile_shape(a.lines, a.len);
    if (s.tiles > 0x7FFFFFFFull) return fail(HX_ERR_DISPATCH_FAILED, "column scan exceeds the grid range");
    if (ws_bytes < rowtile_lb_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small", (unsigned long long)ws_bytes);
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    p.tile0 = 0;
    uint64_t *words = (uint64_t *)((char *)ws + kLookbackOffset);
    hx_status r;
    if constexpr (std::is_same<T, float>::value) {
        const F64QuadDense st{words};
        r = a.exclusive ? launch_rowtile_lb_dir<T, Op, F64QuadDense, true>(p, s, st, a.reverse, stream)
                        : launch_rowtile_lb_dir<T, Op, F64QuadDense, false>(p, s, st, a.reverse, stream);
    } else {
        const PackedStatus st{words};
        r = a.exclusive ? launch_rowtile_lb_dir<T, Op, PackedStatus, true>(p, s, st, a.reverse, stream)
                        : launch_rowtile_lb_dir<T, Op, PackedStatus, false>(p, s, st, a.reverse, stream);
    }
    if (r == HX_OK) commit_lookback_launch(lb);
    return r;
}

template <typename T, typename Op>
hx_status launch_rowtile(const ScanArgs &a, const ScanParams &p, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    const RowTileShape s = row_tile_shape(a.lines, a.len);
    if (s.tiles > 1 && ws_bytes < rowtile_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small", (unsigned long long)ws_bytes);
    if (a.exclusive)
        return a.reverse ? launch_rowtile_dir<T, Op, true, true>(p, s, ws, stream)
                         : launch_rowtile_dir<T, Op, true, false>(p, s, ws, stream);
    return a.reverse ? launch_rowtile_dir<T, Op, false, true>(p, s, ws, stream)
                     : launch_rowtile_dir<T, Op, false, false>(p, s, ws, stream);
}

// 16-byte scans of lines longer than one tile whose outputs start off a
// 128-byte boundary (by the same amount on every line) run on virtual lines
// `head` (1-31) elements longer, the virtual elements (logical [0, head))
// read as the identity and never stored, so that every whole tile's stores
// cover whole lines.  Forward lines gain the elements before their start
// (both offsets move back by head), reverse lines after their end (logical
// index 0 is the physical last).  2^28 u32 exclusive scans, output (and
// input) at element offset k, tiles on the line's own grid: k = 0, 16, 32:
// 331-336 us; k = 1, 4, 5, 8: 418-428.  Stores that start 16 or 32 bytes
// into a 64-byte segment cost as much as unaligned ones; misaligned loads
// cost nothing measurable (input offset 1, output aligned: 333 us).
constexpr uint64_t kOutGrid = 32; // elements: 128 bytes
uint32_t scan_out_head(const ScanArgs &a) {
    if (a.len <= 32768 || a.in_elem_stride != 1 || a.out_elem_stride != 1) return 0;
    if (a.lines > 1 && a.out_line_stride % (int64_t)kOutGrid != 0) return 0;
    const uintptr_t ibase = (uintptr_t)a.in + 4u * a.in_offset; // every element type is 4 bytes
    const uintptr_t obase = (uintptr_t)a.out + 4u * a.out_offset;
    if (ibase % 4 != 0 || obase % 4 != 0) return 0;
    const uint64_t first = obase / 4;
    return a.reverse ? (uint32_t)((kOutGrid - (first + a.len) % kOutGrid) % kOutGrid)
                     : (uint32_t)(first % kOutGrid);
}

uint64_t scan_bytes(const ScanArgs &a) {
    if (short_line_scan(a)) return 0;
    if (narrow_column_scan(a)) return narrow_bytes(a);
    if (rowtile_column_scan(a)) return rowtile_single_pass(a) ? rowtile_lb_bytes(a) : rowtile_bytes(a);
    if (column_mode(a) && column_single_pass(a)) {
        const ColLbShape c = col_lb_shape(a);
        return kLookbackOffset + c.chunks * c.lpad * (a.dtype == HX_DTYPE_F32 ? 16u : 8u);
    }
    if (column_mode(a)) return column_bytes(a);
    const uint64_t vlen = a.len + scan_out_head(a);
    const uint64_t tpl = ceil_div(vlen, tile_shape(vlen).elems());
    // Lines of one tile never look back and publish no status.
    if (tpl <= 1) return kLookbackOffset;
    return kLookbackOffset + status_bytes(tpl * a.lines) + status_bytes(ceil_div(tpl, kSuper) * a.lines);
}

template <typename T, typename Op>
hx_status launch_op(const ScanArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    ScanParams p{};
    p.in = a.in;
    p.out = a.out;
    p.lines = a.lines;
    p.len = a.len;
    const TileShape shape = tile_shape(a.len);
    p.tiles_per_line = ceil_div(a.len, shape.elems());
    p.total_tiles = p.tiles_per_line * a.lines;
    p.supers_per_line = ceil_div(p.tiles_per_line, kSuper);
    p.in_line_stride = a.in_line_stride;
    p.in_elem_stride = a.in_elem_stride;
    p.out_line_stride = a.out_line_stride;
    p.out_elem_stride = a.out_elem_stride;
    p.in_offset = a.in_offset;
    p.out_offset = a.out_offset;
    p.spin_limit = lookback_poll_limit();
    if (a.lines == 0 || a.len == 0) return HX_OK;

    if (short_line_scan(a)) return launch_short<T, Op>(a, stream);
    if (narrow_column_scan(a)) return launch_narrow<T, Op>(a, p, ws, ws_bytes, stream);
    if (rowtile_column_scan(a))
        return rowtile_single_pass(a) ? launch_rowtile_lb<T, Op>(a, p, ws, ws_bytes, lb, stream)
                                      : launch_rowtile<T, Op>(a, p, ws, ws_bytes, stream);
    if (column_mode(a) && column_single_pass(a)) {
        const ColLbShape cs = col_lb_shape(a);
        if (cs.groups * cs.chunks > 0x7FFFFFFFull)
            return fail(HX_ERR_DISPATCH_FAILED, "column scan exceeds the grid range");
        if (ws_bytes < scan_bytes(a))
            return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small",
                        (unsigned long long)ws_bytes);
        HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
        hx_status s = launch_col_lookback<T, Op>(p, cs, a.exclusive, a.reverse, (char *)ws + kLookbackOffset, stream);
        if (s == HX_OK) commit_lookback_launch(lb);
        return s;
    }
    if (column_mode(a)) {
        const ColShape cs = column_shape(a);
        if (cs.nchunks > 1 && ws_bytes < column_bytes(a))
            return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small",
                        (unsigned long long)ws_bytes);
        return a.exclusive ? launch_column<T, Op, true>(p, cs, a.reverse, ws, stream)
                           : launch_column<T, Op, false>(p, cs, a.reverse, ws, stream);
    }
    if (ws_bytes < scan_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "scan workspace of %llu bytes is too small", (unsigned long long)ws_bytes);
    const uint32_t head = scan_out_head(a);
    if (head != 0) {
        // Virtual lines head elements longer.  Forward: both offsets move
        // back by head, so virtual element head is each line's first.
        // Reverse: the virtual elements lie past the line's physical end.
        p.head = head;
        p.len = a.len + head;
        if (!a.reverse) {
            p.in_offset = a.in_offset - head;
            p.out_offset = a.out_offset - head;
        }
        p.tiles_per_line = ceil_div(p.len, shape.elems());
        p.total_tiles = p.tiles_per_line * a.lines;
        p.supers_per_line = ceil_div(p.tiles_per_line, kSuper);
    }
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    const bool contiguous = a.in_elem_stride == 1 && a.out_elem_stride == 1;
    const uintptr_t ibase = (uintptr_t)((const T *)a.in + a.in_offset);
    const uintptr_t obase = (uintptr_t)((T *)a.out + a.out_offset);
    // Vector accesses need only 4-byte alignment (Vec4A4), which every
    // 4-byte element has: contiguous lines take the vector path wherever
    // they start, forward or mirrored.
    const bool vec = contiguous && ibase % 4 == 0 && obase % 4 == 0;
    uint64_t *level0 = (uint64_t *)((char *)ws + kLookbackOffset);
    uint64_t *level1 = (uint64_t *)((char *)level0 + status_bytes(p.total_tiles));
    hx_status s;
    if constexpr (std::is_same<T, float>::value) {
        F64QuadStatus st{level0}, st1{level1};
        s = a.exclusive ? launch_tiles<T, Op, F64QuadStatus, true>(p, st, st1, vec, a.reverse, shape, stream)
                        : launch_tiles<T, Op, F64QuadStatus, false>(p, st, st1, vec, a.reverse, shape, stream);
    } else {
        TilePackedStatus st{level0}, st1{level1};
        s = a.exclusive ? launch_tiles<T, Op, TilePackedStatus, true>(p, st, st1, vec, a.reverse, shape, stream)
                        : launch_tiles<T, Op, TilePackedStatus, false>(p, st, st1, vec, a.reverse, shape, stream);
    }
    if (s == HX_OK) commit_lookback_launch(lb);
    return s;
}

} // namespace

uint64_t scan_workspace_bytes(const ScanArgs &a) { return scan_bytes(a); }

bool scan_uses_lookback(const ScanArgs &a) {
    if (rowtile_column_scan(a)) return rowtile_single_pass(a);
    if (short_line_scan(a) || narrow_column_scan(a)) return false;
    return !column_mode(a) || column_single_pass(a);
}

hx_status launch_scan(const ScanArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb, hipStream_t stream) {
    const bool prod = a.op == HX_OP_PROD;
    switch (a.dtype) {
    case HX_DTYPE_F32:
        return prod ? launch_op<float, OpProd>(a, ws, ws_bytes, lb, stream)
                    : launch_op<float, OpSum>(a, ws, ws_bytes, lb, stream);
    case HX_DTYPE_U32:
    case HX_DTYPE_I32:
        // Two's complement: i32 sums and products have the bits of u32 ones.
        return prod ? launch_op<uint32_t, OpProd>(a, ws, ws_bytes, lb, stream)
                    : launch_op<uint32_t, OpSum>(a, ws, ws_bytes, lb, stream);
    }
    return fail(HX_ERR_INVALID_CONFIGURATION, "unknown dtype %d", (int)a.dtype);
}

} // namespace hx

// Host-side checks of the f32 scan slot codec (the device code uses the same
// inline functions).
extern "C" void hx_debug_slot16_encode(uint32_t tag, uint32_t flag, uint64_t bits, uint32_t *dwords) {
    uint32_t q[4];
    hx::slot16_encode(tag, flag, bits, q);
    for (int i = 0; i < 4; ++i) dwords[i] = q[i];
}
extern "C" uint32_t hx_debug_slot16_decode(uint32_t tag, const uint32_t *dwords, uint64_t *bits) {
    const uint32_t q[4] = {dwords[0], dwords[1], dwords[2], dwords[3]};
    uint64_t b = 0;
    const uint32_t flag = hx::slot16_decode(tag, q, b);
    *bits = b;
    return flag;
}
