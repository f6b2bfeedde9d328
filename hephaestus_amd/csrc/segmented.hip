// Segmented sum for gfx950.  Offsets follow the CSR
// row_ptr convention (crates/hephaestus-core/src/domain/sparse.rs:179-220):
// S+1 entries, offsets[0] = 0, offsets[S] = n, non-decreasing, and
//   out[s] = sum of values[offsets[s] .. offsets[s+1])   (mod 2^32).
//
// The reference's nearest kernel is CSR SpMV with one thread per row and a
// serial inner loop (crates/hephaestus-rocm/src/application/sparse/
// spmv.rs:17-42), which leaves neighbouring lanes hundreds of elements
// apart.  Here the work is cut by ELEMENTS, not by segments, so every block
// streams the same 32 KiB with 16-byte loads whatever the segment lengths.
// Two launches:
//
//   1. seg_tile_map_kernel: one coalesced pass over the offsets records, for
//      every tile edge, the offset indices around it (upper and lower bound),
//      so no block searches the offsets;
//   2. segmented_sum_kernel: block b loads tile b (4 waves x 8 vectors per
//      lane = 8192 values; 8 waves, 16384 values, when segments average
//      4096 values or more) and the offsets that end in it, scans the values
//      in registers, marks segment ends in an LDS bitmask and writes every
//      segment that ends in the tile.  The segment open at the tile start
//      takes the sum of earlier tiles from a segmented decoupled look-back:
//      a tile that holds a segment start publishes its tail at once as a
//      prefix, so a look-back almost always stops at the nearest
//      predecessor.
//
// Segments averaging at most 29 values take a segment-parallel path instead
// (seg_short_kernel below), which needs no look-back.
//
// Integer addition mod 2^32 is associative, so every output is bit-exact.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {
namespace {

constexpr int kBlock = 256; // helper kernels
// Tile geometry of segmented_sum_kernel: WAVES waves, each lane holding
// STEPS 16-byte vectors of values in registers.
template <int WAVES, int STEPS> struct SegTile {
    static constexpr int kWaveElems = kWave * 4 * STEPS;
    static constexpr int kElems = WAVES * kWaveElems;
};
// 4 x 8 measured best at 2^27 (8192-value tiles, seven blocks per CU): larger
// tiles leave fewer blocks per CU to overlap one block's barriers with
// another's loads (4 x 8: 89.5 us; 2 x 8: 90.5-92; 8 x 8: 107; an earlier
// form of the kernel: 8 x 16 230 us).
constexpr int kSegWaves = 4, kSegSteps = 8;
constexpr int kTile = SegTile<kSegWaves, kSegSteps>::kElems;
// Long segments (mean n / S of kLongMean or more) take 16384-value tiles,
// 8 waves x 8 steps: half the look-backs per byte, which is what long
// segments pay for (their tiles rarely hold a segment start).  At 2^27
// values, us per launch with 8192- against 16384-value tiles: mean 300
// 85.4 / 106.0, 3000 96.0 / 98.2, 4000 99.8 / 99.6, 8000 106.2 / 99.0,
// 10^5 119.5 / 114.7, 10^6 137.2 / 125.3, 10^7 147.8 / 129.6.  (4 x 16
// tiles spill: about 400 us everywhere.)
constexpr int kLongWaves = 8;
constexpr int kLongTile = SegTile<kLongWaves, kSegSteps>::kElems;
constexpr uint64_t kLongMean = 4096;
// Mean segment length from which look-backs walk tiles only (one level):
// segments of thousands of tiles leave few superblocks resolved when a
// look-back reaches them (see seg_lookback).
constexpr uint64_t kTwoLevelMaxMean = 1ull << 18;
constexpr int kSlots = 2048; // segment values compacted per round
constexpr uint32_t kInvalid = 0, kAggregate = 1, kPrefix = 2;

struct SegParams {
    const uint32_t *values;
    uint64_t n;
    const uint32_t *offsets;
    uint64_t segments; // S
    uint32_t *out;
    uint64_t total_tiles;
    uint64_t *status;          // look-back words, one per tile (16 bytes apart)
    uint64_t *sstatus;         // then one per 64-tile superblock
    uint32_t *ub_map, *lb_map; // tile edges -> offset indices (total_tiles + 1 each)
    uint32_t tag;              // this launch's status tag
    uint32_t spin_limit;       // polls before computing a predecessor (64)
};
// A tile whose segment ends number more than kEndCap (only possible with runs
// of empty segments) handles the first kEndCap itself; seg_tile_map_kernel
// sums the rest beforehand.  Every such excess segment lies inside its tile,
// after the tile's first end, so its sum needs neither the tile's prefixes
// nor its marks.
constexpr uint64_t kEndCap = 4096;

// Offsets clamped into [0, n]: malformed offsets can never address values
// out of bounds.
__device__ __forceinline__ uint64_t off_at(const SegParams &p, uint64_t k) {
    const uint64_t o = p.offsets[k];
    return o < p.n ? o : p.n;
}

__device__ __forceinline__ uint64_t status_word(uint32_t tag, uint32_t flag, uint32_t v) {
    return ((uint64_t)status_word_hi(tag, flag) << 32) | (uint64_t)v;
}

// Status words 16 bytes apart (tile and superblock statuses alike): tiles
// publish at about the same moment from CUs all over the chip, and dense
// words put 16 publishers on one 128-byte line.  The scans, whose tiles are
// four times larger, take a whole line per status; here a 64-lane poll
// over 64 lines costs more than it saves.  Measured at 2^27 values, us per
// launch with 8 / 16 / 32 / 128-byte strides: mean 300 84.6 / 84.4 / 85.0 /
// 88.3; segmented_long workload 111.2 / 105.9 / 105.2 / 107.1.
constexpr uint64_t kSegStatusStride = 2; // 64-bit words
__device__ __forceinline__ uint64_t *seg_word(uint64_t *base, uint64_t i) { return base + i * kSegStatusStride; }

// The status tile u's owner publishes, computed by ONE wave (fallback path):
// a prefix (the sum from the last segment start in the tile to its end) when
// the tile holds a segment start, else an aggregate (the tile total).
template <int TILE>
__device__ void seg_tile_status(const SegParams &p, uint64_t u, uint32_t &flag, uint32_t &value) {
    const uint64_t t0 = u * TILE;
    const uint64_t t1 = (t0 + TILE < p.n) ? t0 + TILE : p.n;
    uint64_t k_star = p.lb_map[u + 1];
    k_star = k_star < p.segments + 1 ? k_star : p.segments + 1;
    uint64_t h = k_star >= 1 ? off_at(p, k_star - 1) : 0;
    if (h > t1 - 1) h = t1 - 1;
    const bool has_head = h >= t0;
    uint32_t s = 0;
    for (uint64_t i = (has_head ? h : t0) + lane_id(); i < t1; i += kWave) s += p.values[i];
    value = wave_sum(s);
    flag = has_head ? kPrefix : kAggregate;
}

// Fallback publication: never overwrites a word of this launch.
__device__ __forceinline__ void publish_if_unset(uint64_t *word, uint32_t tag, uint32_t flag, uint32_t v) {
    uint64_t cur = ld_relaxed(word);
    if ((uint32_t)(cur >> 34) == tag) return;
    __hip_atomic_compare_exchange_strong(word, &cur, status_word(tag, flag, v), __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
}

// Tiles per superblock.  The last tile of each superblock also publishes
// the superblock's carry out, as a prefix, when the tile holds a segment
// start (at once) or once its own look-back resolves.  A two-level look-back
// folds the tiles of its own superblock, then whole superblocks (scan.hip has
// the same two levels), so where superblocks have resolved it skips 64 tiles
// a step.  The superblock statuses are published in both forms.
constexpr int kSegSuper = 64;

// Fold of the statuses of the `count` (<= 64) tiles just before tile `end`,
// nearest first, stopping at the first prefix; `found` tells whether one was
// met.  Lane l reads the tile at distance l.  A status that stays
// unpublished is computed by the waiter (decoupled fallback).  One wave.
template <int TILE>
__device__ uint32_t seg_fold_tiles(const SegParams &p, uint64_t end, int count, uint32_t tag, bool &found) {
    const int lane = lane_id();
    uint32_t flag, val;
    uint32_t spins = 0;
    for (;;) {
        flag = kAggregate; // lanes past `count`: valid, not a prefix, 0
        val = 0;
        if (lane < count) {
            const uint64_t wd = ld_relaxed(seg_word(p.status, end - 1 - (uint64_t)lane));
            const uint32_t hi = (uint32_t)(wd >> 32);
            flag = ((hi >> 2) == tag) ? (hi & 3u) : kInvalid;
            val = (uint32_t)wd;
        }
        const uint64_t pm = ballot(flag == kPrefix);
        const uint64_t im = ballot(flag == kInvalid);
        // Every status up to and including the nearest prefix is needed.
        const uint64_t need = pm ? (((pm & (~pm + 1ull)) << 1) - 1ull) : ~0ull;
        const uint64_t missing = im & need;
        if (missing == 0ull) break;
        if (++spins >= p.spin_limit) {
            const uint64_t u = end - 1 - (uint64_t)(__ffsll((long long)missing) - 1);
            uint32_t fflag, fval;
            seg_tile_status<TILE>(p, u, fflag, fval);
            if (lane == 0) publish_if_unset(seg_word(p.status, u), tag, fflag, fval);
            spins = 0;
            continue;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    const uint64_t pm = ballot(flag == kPrefix);
    const int first = pm ? (__ffsll((long long)pm) - 1) : kWave;
    found = pm != 0ull;
    return wave_sum((lane <= first) ? val : 0u);
}

// Exclusive prefix of segment sums carried in from earlier tiles: folds
// predecessor statuses until one is a prefix (a tile that holds a segment
// start, or that already resolved its own carry).  TWO_LEVEL: the tiles of
// the tile's superblock, then whole superblocks; otherwise tiles only, 64
// per round trip.  One wave.
//
// Measured at 2^27 values, geometric segment lengths (us per launch, one
// level / two levels): mean 300 85 / 84.4, 3000 96 / 86.4, 10^5 114 /
// 102.9, 10^6 125 / 138, 10^7 130 / 188.  When segments span thousands of
// tiles, few superblocks have resolved when a look-back reaches them, and
// the second level only adds round trips; the host picks the form by mean
// segment length (kTwoLevelMaxMean).
template <int TILE, bool TWO_LEVEL> __device__ uint32_t seg_lookback(const SegParams &p, uint64_t tile, uint32_t tag) {
    const int lane = lane_id();
    if constexpr (!TWO_LEVEL) {
        uint32_t c_in = 0;
        for (uint64_t end = tile;; end -= kWave) {
            const int count = end < (uint64_t)kWave ? (int)end : kWave;
            bool found = false;
            c_in += seg_fold_tiles<TILE>(p, end, count, tag, found);
            if (found || end <= (uint64_t)kWave) return c_in; // tile 0 always holds a segment start
        }
    } else {
        const int pos = (int)(tile % kSegSuper);
        const uint64_t sb = tile / kSegSuper;
        bool found = false;
        uint32_t c_in = pos > 0 ? seg_fold_tiles<TILE>(p, tile, pos, tag, found) : 0u;
        if (found) return c_in;
        // Level 1: windows of 64 superblocks, nearest first.  A superblock
        // status is only ever a prefix (its carry out), published by its last
        // tile once that tile's carry is known, or by a waiter that found a
        // prefix among its tiles; a superblock without one is folded from its
        // 64 tiles (one round trip).  Publishing aggregates as well made
        // look-backs skip tiles that had resolved since and walk further
        // back (10^6: 186 us, 10^7: 279).
        int64_t pred = (int64_t)sb - 1;
        for (;;) {
            const int64_t idx = pred - lane;
            uint32_t flag = kPrefix, val = 0; // before superblock 0: the identity
            if (idx >= 0) {
                const uint64_t wd = ld_relaxed(seg_word(p.sstatus, (uint64_t)idx));
                const uint32_t hi = (uint32_t)(wd >> 32);
                flag = ((hi >> 2) == tag) ? (hi & 3u) : kInvalid;
                val = (uint32_t)wd;
            }
            const uint64_t pm = ballot(flag == kPrefix);
            const int stop = pm ? (__ffsll((long long)pm) - 1) : kWave;
            // Superblocks nearer than the nearest published prefix, from their
            // tiles, nearest first.
            for (int q = 0; q < stop; ++q) {
                const uint64_t s = (uint64_t)(pred - q);
                bool f = false;
                const uint32_t v = seg_fold_tiles<TILE>(p, (s + 1) * kSegSuper, kSegSuper, tag, f);
                c_in += v;
                if (f) {
                    if (lane == 0) publish_if_unset(seg_word(p.sstatus, s), tag, kPrefix, v);
                    return c_in;
                }
            }
            if (pm) return c_in + read_lane(val, stop);
            pred -= kWave;
        }
    }
}

// Block b processes tile b; see scan.hip for why there is no ticket counter
// and how the fallback guarantees progress in any dispatch order.
//
// Per tile, LDS holds only segment bookkeeping (about 0.5 byte per value
// plus kSlots words), never the values themselves:
//   s_mask   bit q set when tile element q is the LAST element of a segment
//            (q + 1 + t0 is an offset in (t0, t1]);
//   s_wrank  per mask word, the popcount of the earlier words of its wave,
//            so a set bit's rank among all set bits is a few LDS reads;
//   s_val    x at the set bits, compacted by rank, kSlots per round.
// Each lane keeps its elements' tile-local inclusive prefixes x in
// registers and stores x at its set bits.  Set bits are segment ends, so
// the bit before a segment's end bit is the end of the previous segment: the
// thread assigned to offset k reads x at its end's rank and subtracts x at
// the rank before (mod 2^32).  A segment that began before the tile start
// takes its x alone plus the look-back carry; one that begins exactly at the
// tile start takes its x alone.
//
// The tile's offset range comes from the map built by seg_tile_map_kernel,
// so the offsets a block needs are loaded once, right after its values,
// with no search on the critical path.  Only the segment already open at the
// tile start needs the carry from earlier tiles: every other output is
// written first, and wave 0 looks back last, when the rest of the block is
// done (polling earlier, between two barriers, held every wave of the block
// and cost ~15% at 2^27 values).
// Register budget: 72 VGPRs gives 7 waves per SIMD.  For the 4 x 8 tiles
// (one wave per SIMD per block) that is seven blocks per CU (the compiler's
// own choice, 74, allows six: 92 us at 2^27 against 89.5; a 64 cap spills to
// scratch and takes 156 us).  The 8 x 8 long-segment tiles take two waves
// per SIMD per block, so the same budget fits three of them per CU (six
// waves per SIMD).
template <int WAVES, int STEPS, bool TWO_LEVEL = true>
__global__ __launch_bounds__(WAVES * kWave) __attribute__((amdgpu_waves_per_eu(7, 7))) void segmented_sum_kernel(
    SegParams p) {
    static_assert(STEPS % 8 == 0, "each lane ranks whole mask words");
    constexpr int kWaveElems = SegTile<WAVES, STEPS>::kWaveElems;
    constexpr int kTile = SegTile<WAVES, STEPS>::kElems;
    constexpr int kThreads = WAVES * kWave;
    constexpr int kWords = kTile / 32;
    constexpr int kWaveWords = kWaveElems / 32;
    constexpr int kLaneWords = kWaveWords / kWave;
    __shared__ uint32_t s_wave_tot[WAVES];
    __shared__ uint32_t s_wave_pop[WAVES];
    __shared__ uint32_t s_hpref;
    __shared__ uint32_t s_open; // in-tile part of the open segment
    __shared__ uint32_t s_mask[kWords];
    __shared__ uint32_t s_wrank[kWords];
    __shared__ uint32_t s_val[kSlots + 1]; // slot 0: the rank before the round

    const uint64_t tile = blockIdx.x;
    const uint32_t tag = p.tag;
    const int w = threadIdx.x / kWave;
    const int lane = lane_id();
    const uint64_t t0 = tile * kTile;
    const uint64_t t1 = (t0 + kTile < p.n) ? t0 + kTile : p.n;
    const uint64_t tlen = t1 - t0;
    const uint64_t e0 = t0 + (uint64_t)w * kWaveElems + (uint64_t)lane * 4;
    const uint64_t kmax = p.segments + 1;

    // Offsets of the tile: k_lo = ub(t0) (segment of t0 is k_lo - 1),
    // k_hi1 = ub(t1), k_star = lb(t1) = ub(t1 - 1) (segment of t1-1 is
    // k_star - 1).  Clamped so malformed offsets stay in bounds.
    uint64_t k_lo = p.ub_map[tile], k_hi1 = p.ub_map[tile + 1], k_star = p.lb_map[tile + 1];
    k_lo = k_lo < kmax ? k_lo : kmax;
    k_hi1 = k_hi1 < k_lo ? k_lo : (k_hi1 < kmax ? k_hi1 : kmax);
    k_star = k_star < kmax ? k_star : kmax;
    // Ends handled here: the first kEndCap.  Later ends lie after all of
    // these, so the ranks of these need no mark of theirs.
    const uint64_t k_end = k_hi1 - k_lo > kEndCap ? k_lo + kEndCap : k_hi1;

    for (int i = threadIdx.x; i < kWords; i += kThreads) s_mask[i] = 0u;
    if (threadIdx.x == 0) s_open = 0u;

    // Values first, with a block-uniform base for whole tiles.
    uint32_t x[STEPS][4];
    if (tlen == (uint64_t)kTile) {
        const char *base = (const char *)(p.values + t0);
        const uint32_t lane_off =
            ((uint32_t)__builtin_amdgcn_readfirstlane(w) * kWaveElems + (uint32_t)lane * 4) * 4u;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const u32x4_a4 v = load_a4<true>((const u32x4_a4 *)(base + lane_off + (uint32_t)j * (kWave * 16)));
            x[j][0] = v.x;
            x[j][1] = v.y;
            x[j][2] = v.z;
            x[j][3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
            if (e + 3 < p.n) {
                const u32x4_a4 v = __builtin_nontemporal_load((const u32x4_a4 *)(p.values + e));
                x[j][0] = v.x;
                x[j][1] = v.y;
                x[j][2] = v.z;
                x[j][3] = v.w;
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) x[j][c] = (e + c < p.n) ? p.values[e + c] : 0u;
            }
        }
    }
    // Then the first kThreads segment ends of the tile (k = k_lo + thread)
    // and their starts, plus the starts of the segments holding t0 and t1-1.
    const uint64_t kq = k_lo + threadIdx.x;
    const bool have_q = kq < k_end && kq >= 1;
    const uint64_t ob_q = have_q ? off_at(p, kq) : 0, oa_q = have_q ? off_at(p, kq - 1) : 0;
    const uint64_t first_start = k_lo >= 1 ? off_at(p, k_lo - 1) : 0;
    uint64_t h = k_star >= 1 ? off_at(p, k_star - 1) : 0;
    if (h > t1 - 1) h = t1 - 1; // only reachable with malformed offsets

    // Wave-local inclusive prefix of the values (mod 2^32).
    uint32_t carry = 0;
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const uint32_t p0 = x[j][0];
        const uint32_t p1 = p0 + x[j][1];
        const uint32_t p2 = p1 + x[j][2];
        const uint32_t p3 = p2 + x[j][3];
        const uint32_t incl = wave_inclusive_scan<OpSum, uint32_t>(p3);
        const uint32_t lex = wave_shift_right<OpSum, uint32_t>(incl);
        const uint32_t step_tot = read_lane(incl, kWave - 1);
        const uint32_t base = carry + lex;
        x[j][0] = base + p0;
        x[j][1] = base + p1;
        x[j][2] = base + p2;
        x[j][3] = base + p3;
        carry += step_tot;
    }
    if (lane == 0) s_wave_tot[w] = carry;
    __syncthreads();

    // Tile-local prefixes, and the segment-end marks.
    uint32_t wave_excl = 0, total = 0;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) {
        const uint32_t t = s_wave_tot[k];
        if (k < w) wave_excl += t;
        total += t;
    }
#pragma unroll
    for (int j = 0; j < STEPS; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) x[j][c] += wave_excl;
    for (uint64_t k = kq; k < k_end; k += kThreads) {
        const uint64_t b = k == kq ? ob_q : off_at(p, k);
        if (b > t0 && b <= t1) {
            const uint32_t q = (uint32_t)(b - 1 - t0);
            atomicOr(&s_mask[q >> 5], 1u << (q & 31));
        }
    }
    // The segment holding t1-1 starts at h; its tile-local start prefix
    // x(h - 1) is published with the tile's status.
    if (h > t0) {
        const uint32_t q = (uint32_t)(h - 1 - t0);
        if ((int)(q / kWaveElems) == w && (int)((q % (kWave * 4)) / 4) == lane) {
            const int jq = (int)((q % kWaveElems) / (kWave * 4)), cq = (int)(q % 4);
#pragma unroll
            for (int j = 0; j < STEPS; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    if (j == jq && c == cq) s_hpref = x[j][c];
        }
    }
    __syncthreads();

    const bool has_head = h >= t0;
    const bool needs_carry = tile > 0 && first_start < t0;
    const bool last_in_super = tile % kSegSuper == kSegSuper - 1;
    if (w == 0 && lane == 0) {
        if (has_head) {
            const uint32_t carry_out = total - (h > t0 ? s_hpref : 0u);
            st_relaxed(seg_word(p.status, tile), status_word(tag, kPrefix, carry_out));
            if (last_in_super) st_relaxed(seg_word(p.sstatus, tile / kSegSuper), status_word(tag, kPrefix, carry_out));
        } else if (tile > 0) {
            st_relaxed(seg_word(p.status, tile), status_word(tag, kAggregate, total));
        }
    }

    // Per wave: popcounts for ranking.
    {
        uint32_t words[kLaneWords];
        uint32_t lane_pop = 0;
#pragma unroll
        for (int i = 0; i < kLaneWords; ++i) {
            words[i] = s_mask[w * kWaveWords + lane * kLaneWords + i];
            lane_pop += __builtin_popcount(words[i]);
        }
        const uint32_t pop_incl = wave_inclusive_scan<OpSum, uint32_t>(lane_pop);
        uint32_t run = pop_incl - lane_pop;
#pragma unroll
        for (int i = 0; i < kLaneWords; ++i) {
            s_wrank[w * kWaveWords + lane * kLaneWords + i] = run;
            run += __builtin_popcount(words[i]);
        }
        if (lane == kWave - 1) s_wave_pop[w] = pop_incl;
    }
    __syncthreads();

    // This wave's rank base.
    uint32_t rank_base = 0, marks = 0;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) {
        const uint32_t pk = s_wave_pop[k];
        if (k < w) rank_base += pk;
        marks += pk;
    }


    // Marked positions are segment ends, so the tile-local prefix at a
    // segment's start is the value at the previous mark: a segment's sum is
    // the difference of two consecutive ranks (mod 2^32).  Round r holds
    // ranks [r*kSlots - 1, (r+1)*kSlots - 1) in slots 0..kSlots.
    const uint32_t rounds = marks == 0 ? 1u : (marks + kSlots - 1) / kSlots;
    for (uint32_t round = 0; round < rounds; ++round) {
        const uint32_t r0 = round * kSlots;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const int word = w * kWaveWords + j * (kWave * 4 / 32) + (lane >> 3);
            const uint32_t mw = s_mask[word];
            const int sh = (lane & 7) * 4;
            const uint32_t nib = (mw >> sh) & 0xFu;
            if (nib) {
                const uint32_t rb = rank_base + s_wrank[word];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    if (nib & (1u << c)) {
                        const uint32_t slot = rb + __builtin_popcount(mw & ((1u << (sh + c)) - 1u)) + 1u - r0;
                        if (slot <= (uint32_t)kSlots) s_val[slot] = x[j][c];
                    }
                }
            }
        }
        __syncthreads();
        // Segments s = k-1 whose end offset off(k) lies in (t0, t1].
        for (uint64_t k = kq; k < k_end; k += kThreads) {
            if (k == 0) continue;
            const uint64_t b = k == kq ? ob_q : off_at(p, k);
            uint64_t a = k == kq ? oa_q : off_at(p, k - 1);
            if (a > b) a = b; // malformed: treat as empty
            if (b <= t0 || b > t1) continue; // malformed (non-monotonic) offsets
            if (a == b) {
                if (round == 0) p.out[k - 1] = 0u;
                continue;
            }
            const uint32_t q = (uint32_t)(b - 1 - t0);
            const int qw = (int)(q / kWaveElems);
            uint32_t rank = s_wrank[q >> 5] + __builtin_popcount(s_mask[q >> 5] & ((1u << (q & 31)) - 1u));
            for (int k2 = 0; k2 < qw; ++k2) rank += s_wave_pop[k2];
            if (rank < r0 || rank - r0 >= (uint32_t)kSlots) continue;
            uint32_t v = s_val[rank - r0 + 1];
            if (a > t0) v -= s_val[rank - r0]; // prefix at a - 1, the previous mark
            if (a < t0)
                s_open = v; // written after the look-back
            else
                p.out[k - 1] = v;
        }
        if (round + 1 < rounds) __syncthreads();
    }

    // The carry into the open segment, and the final status of a tile with
    // no segment start (so later look-backs stop here).
    if (needs_carry || (!has_head && tile > 0)) {
        __syncthreads(); // s_open
        if (w == 0) {
            const bool publish_super = last_in_super && !has_head;
            const uint32_t c_in = seg_lookback<kTile, TWO_LEVEL>(p, tile, tag);
            if (lane == 0) {
                if (!has_head) st_relaxed(seg_word(p.status, tile), status_word(tag, kPrefix, c_in + total));
                if (publish_super) st_relaxed(seg_word(p.sstatus, tile / kSegSuper), status_word(tag, kPrefix, c_in + total));
                if (needs_carry && k_lo < k_hi1 && k_lo >= 1 && k_lo <= p.segments) p.out[k_lo - 1] = s_open + c_in;
            }
        }
    }
}

// The tile map: for every tile edge B_t = t * TILE (t < tiles) and for
// B_tiles = n, ub_map[t] = #{k : off(k) <= B_t} and lb_map[t] =
// #{k : off(k) < B_t}.  With sorted offsets, the edges with ub = k are those
// in [off(k-1), off(k)) and those with lb = k are in (off(k-1), off(k)]
// (off(-1) = 0 resp. -1, off(S+1) = infinity): one coalesced pass over the
// offsets instead of a search per tile.  Lane j of a wave takes k = base + j;
// an interval of at most kDirectEdges edges is written by its lane, and the
// wave writes the longer ones together, one interval at a time (64 edges per
// store), so a long segment's many edges do not fall to one thread (15
// segments over 2^27 values: 238 us with a thread per interval).
constexpr uint32_t kDirectEdges = 8;

__device__ __forceinline__ void map_write_edges(uint32_t *map, uint32_t first, uint32_t count, uint32_t k) {
    const int lane = lane_id();
    const bool big = count > kDirectEdges;
    if (!big)
        for (uint32_t i = 0; i < count; ++i) map[first + i] = k;
    uint64_t pending = ballot(big);
    while (pending) { // wave-uniform
        const int j = __ffsll((long long)pending) - 1;
        pending &= pending - 1;
        const uint32_t f = read_lane(first, j), c = read_lane(count, j), kj = read_lane(k, j);
        for (uint32_t i = (uint32_t)lane; i < c; i += kWave) map[f + i] = kj;
    }
}

// Segment k - 1 = [lo, hi) ends in the tile of element hi - 1, starting at
// t0.  It is an excess end of that tile (beyond the first kEndCap ends,
// which the tile's block handles) exactly when off(k - kEndCap) > t0, since
// the tile's first end is the first k' with off(k') > t0.  Such a segment
// lies inside the tile: a lane sums up to kWave values itself, the wave sums
// longer ones together, one at a time.  Called wave-uniformly.
template <int TILE>
__device__ __forceinline__ void excess_sums(const SegParams &p, uint64_t k, uint64_t lo, uint64_t hi) {
    const int lane = lane_id();
    uint64_t a = 0;
    uint32_t len = 0;
    bool mine = false;
    if (k >= kEndCap && k <= p.segments && hi > 0) {
        const uint64_t t0 = (hi - 1) / TILE * TILE;
        if (off_at(p, k - kEndCap) > t0) {
            mine = true;
            a = lo < t0 ? t0 : (lo > hi ? hi : lo); // clamps only malformed offsets
            len = (uint32_t)(hi - a);
        }
    }
    uint32_t sum = 0;
    if (len <= (uint32_t)kWave)
        for (uint32_t j = 0; j < len; ++j) sum += p.values[a + j];
    uint64_t pending = ballot(len > (uint32_t)kWave);
    while (pending) { // wave-uniform
        const int j = __ffsll((long long)pending) - 1;
        pending &= pending - 1;
        const uint64_t aj = ((uint64_t)read_lane((uint32_t)(a >> 32), j) << 32) | read_lane((uint32_t)a, j);
        const uint32_t lj = read_lane(len, j);
        uint32_t part = 0;
        for (uint32_t q = (uint32_t)lane; q < lj; q += kWave) part += p.values[aj + q];
        part = wave_sum(part);
        if (lane == j) sum = part;
    }
    if (mine) p.out[k - 1] = sum;
}

template <int TILE>
__global__ __launch_bounds__(kBlock) void seg_tile_map_kernel(SegParams p) {
    const uint64_t tiles = p.total_tiles;
    const uint64_t S = p.segments;
    const int lane = lane_id();
    const uint64_t wave = ((uint64_t)blockIdx.x * kBlock + threadIdx.x) / kWave;
    const uint64_t nwaves = (uint64_t)gridDim.x * (kBlock / kWave);
    for (uint64_t base = wave * kWave; base <= S + 1; base += nwaves * kWave) { // wave-uniform
        const uint64_t k = base + (uint64_t)lane;
        uint32_t ua = 0, un = 0, la = 0, ln = 0;
        uint64_t ex_lo = 0, ex_hi = 0; // segment k - 1, for k in [1, S]
        if (k <= S + 1) {
            const uint64_t lo = k == 0 ? 0 : off_at(p, k - 1);
            const uint64_t hi = k <= S ? off_at(p, k) : p.n + 1; // off_at clamps into [0, n]
            // ub: edges t with lo <= t * TILE < hi (lo for k == 0 is 0).
            const uint64_t u0 = (lo + TILE - 1) / TILE;
            uint64_t u1 = (hi + TILE - 1) / TILE;
            if (u1 > tiles) u1 = tiles;
            if (u1 > u0) {
                ua = (uint32_t)u0;
                un = (uint32_t)(u1 - u0);
            }
            if (lo <= p.n && p.n < hi) p.ub_map[tiles] = (uint32_t)k;
            // lb: edges t with lo' < t * TILE <= hi, lo' = off(k-1) or -1 for k == 0.
            const uint64_t l0 = k == 0 ? 0 : lo / TILE + 1;
            uint64_t l1 = hi / TILE + 1;
            if (l1 > tiles) l1 = tiles;
            if (l1 > l0) {
                la = (uint32_t)l0;
                ln = (uint32_t)(l1 - l0);
            }
            if ((k == 0 || lo < p.n) && p.n <= hi) p.lb_map[tiles] = (uint32_t)k;
            // Segments that end at offset 0 are empty and end in no tile.
            if (k >= 1 && k <= S && hi == 0) p.out[k - 1] = 0u;
            if (k >= 1 && k <= S) {
                ex_lo = lo;
                ex_hi = hi;
            }
        }
        map_write_edges(p.ub_map, ua, un, (uint32_t)k);
        map_write_edges(p.lb_map, la, ln, (uint32_t)k);
        excess_sums<TILE>(p, k, ex_lo, ex_hi);
    }
}

// ---------------------------------------------------------------------------
// Short segments (mean length n / S of at most kShortSpan / 256).  Cut by
// elements, a tile of 8192 values holds hundreds to thousands of segment
// ends, and segmented_sum_kernel spends its time ranking them in rounds of
// kSlots.  Here the work is cut by SEGMENTS instead: block b takes the
// SB <= 256 * J consecutive segments [s0, s1), whose values are the one
// contiguous span [off(s0), off(s1)).  The block loads the span's first
// chunk (up to 8192 values, 16-byte loads from the 4-aligned element at or
// below off(s0)), writes the chunk's inclusive prefix sums to LDS, and
// thread t forms out[s] = P(end - 1) - P(start - 1) for s = s0 + t + 256 j:
// offsets are read and outputs written coalesced, and no segment needs a
// carry from another block.  SB is the most segments (up to 16 per thread)
// whose expected span, SB n / S values, stays within kShortSpan.
//
// A span longer than one chunk (a long segment among short ones) is not
// walked by one block: the block stores the first chunk's part of each of
// its outputs (0 for segments that start later) and appends one worklist
// entry per further chunk -- the segment that holds the chunk's first
// element and that element's index -- and seg_short_drain_kernel adds each
// chunk's part to its outputs with 32-bit atomics (exact: the sum is mod
// 2^32 in any order).
constexpr int kShortWaves = 4, kShortSteps = 8;
constexpr int kShortThreads = kShortWaves * kWave;
constexpr int kShortChunk = SegTile<kShortWaves, kShortSteps>::kElems; // values per chunk
// Most values a block's expected span may hold: 8192 less about 2.4 standard
// deviations of 512 geometric lengths of mean 14, so spans rarely overflow.
constexpr uint64_t kShortSpan = 7424;
constexpr int kShortMaxJ = 16;
constexpr uint64_t kWorkHeader = 256; // worklist count, then entries
constexpr uint32_t kDrainBlocks = 1280; // five 32 KiB-LDS blocks per CU

struct ShortParams {
    const uint32_t *values;
    uint64_t n;
    const uint32_t *offsets;
    uint64_t segments; // S
    uint32_t *out;
    uint64_t seg_per_block;        // SB
    unsigned long long *work_count; // entries appended this launch
    uint2 *work;                    // (segment holding the chunk start, chunk start)
    uint64_t work_cap;
};

__device__ __forceinline__ uint64_t short_off(const ShortParams &p, uint64_t k) {
    const uint64_t o = p.offsets[k];
    return o < p.n ? o : p.n;
}

// Values [lo, hi) of the chunk that starts at element `base` (base <= lo,
// hi <= base + kShortChunk), zero elsewhere.  Each wave writes the inclusive
// prefix sums (mod 2^32) of its 2048 values to s_p; after the barrier the
// last word of each wave's quarter is that wave's total, so no other LDS is
// needed (which keeps the block at exactly 32 KiB, five blocks per CU).
struct ChunkCarry {
    uint32_t w1, w2, w3; // sums of the chunk before waves 1, 2, 3
};
constexpr int kShortWaveElems = SegTile<kShortWaves, kShortSteps>::kWaveElems;
static_assert(kShortWaves == 4 && kShortWaveElems == 2048, "chunk_prefix_at selects among four quarters");

__device__ __forceinline__ ChunkCarry short_chunk_prefix(const uint32_t *values, uint64_t base, uint64_t lo,
                                                         uint64_t hi, uint32_t *s_p) {
    const int w = threadIdx.x / kWave;
    const int lane = lane_id();
    const uint64_t e0 = base + (uint64_t)w * kShortWaveElems + (uint64_t)lane * 4;
    uint32_t x[kShortSteps][4];
#pragma unroll
    for (int j = 0; j < kShortSteps; ++j) {
        const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
        if (e >= lo && e + 4 <= hi) {
            const u32x4_a4 v = load_a4<true>((const u32x4_a4 *)(values + e));
            x[j][0] = v.x;
            x[j][1] = v.y;
            x[j][2] = v.z;
            x[j][3] = v.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) x[j][c] = (e + c >= lo && e + c < hi) ? values[e + c] : 0u;
        }
    }
    uint32_t carry = 0;
#pragma unroll
    for (int j = 0; j < kShortSteps; ++j) {
        const uint32_t p0 = x[j][0];
        const uint32_t p1 = p0 + x[j][1];
        const uint32_t p2 = p1 + x[j][2];
        const uint32_t p3 = p2 + x[j][3];
        const uint32_t incl = wave_inclusive_scan<OpSum, uint32_t>(p3);
        const uint32_t base_j = carry + wave_shift_right<OpSum, uint32_t>(incl);
        u32x4 v;
        v.x = base_j + p0;
        v.y = base_j + p1;
        v.z = base_j + p2;
        v.w = base_j + p3;
        *(u32x4 *)&s_p[w * kShortWaveElems + j * (kWave * 4) + lane * 4] = v;
        carry += read_lane(incl, kWave - 1);
    }
    __syncthreads();
    const uint32_t t0 = s_p[kShortWaveElems - 1], t1 = s_p[2 * kShortWaveElems - 1],
                   t2 = s_p[3 * kShortWaveElems - 1];
    return ChunkCarry{t0, t0 + t1, t0 + t1 + t2};
}

// Inclusive prefix of the chunk at local index i.
__device__ __forceinline__ uint32_t chunk_prefix_at(const uint32_t *s_p, const ChunkCarry &c, uint32_t i) {
    const uint32_t q = i / kShortWaveElems;
    const uint32_t add = q == 0 ? 0u : (q == 1 ? c.w1 : (q == 2 ? c.w2 : c.w3));
    return s_p[i] + add;
}

// Sum of chunk-local elements [l, h), 0 <= l <= h <= kShortChunk.
__device__ __forceinline__ uint32_t chunk_range_sum(const uint32_t *s_p, const ChunkCarry &c, uint32_t l, uint32_t h) {
    if (h <= l) return 0u;
    uint32_t v = chunk_prefix_at(s_p, c, h - 1);
    if (l > 0) v -= chunk_prefix_at(s_p, c, l - 1);
    return v;
}

// Chunks [c_lo, c_lo + count) of segment s go to worklist entries
// [slot, slot + count); chunk c starts at element base + c * kShortChunk.
// `base` is block-uniform.  Short ranges are written by their lane; the wave
// writes longer ones together, one range at a time.
__device__ __forceinline__ void short_write_entries(const ShortParams &p, uint64_t slot, uint64_t base, uint32_t s,
                                                    uint32_t c_lo, uint32_t count) {
    const int lane = lane_id();
    const bool big = count > kDirectEdges;
    if (!big)
        for (uint32_t i = 0; i < count; ++i)
            if (slot + i < p.work_cap)
                p.work[slot + i] = make_uint2(s, (uint32_t)(base + (uint64_t)(c_lo + i) * kShortChunk));
    uint64_t pending = ballot(big);
    while (pending) { // wave-uniform
        const int j = __ffsll((long long)pending) - 1;
        pending &= pending - 1;
        const uint32_t lo = read_lane(c_lo, j), cnt = read_lane(count, j), sj = read_lane(s, j);
        const uint64_t sl = ((uint64_t)read_lane((uint32_t)(slot >> 32), j) << 32) | read_lane((uint32_t)slot, j);
        for (uint32_t i = (uint32_t)lane; i < cnt; i += kWave)
            if (sl + i < p.work_cap)
                p.work[sl + i] = make_uint2(sj, (uint32_t)(base + (uint64_t)(lo + i) * kShortChunk));
    }
}

__global__ void seg_short_init_kernel(unsigned long long *work_count) { *work_count = 0ull; }

// Chunks of the span [a0, a1) whose first element lies in the segment part
// [l, h): c in [ceil((l - base) / chunk), ceil((h - base) / chunk)), from 1.
__device__ __forceinline__ void short_chunk_range(uint64_t base, uint64_t l, uint64_t h, uint64_t chunks,
                                                  uint32_t &c_lo, uint32_t &count) {
    c_lo = 1;
    count = 0;
    if (h <= l) return;
    uint64_t c0 = (l - base + kShortChunk - 1) / kShortChunk, c1 = (h - base + kShortChunk - 1) / kShortChunk;
    if (c0 < 1) c0 = 1;
    if (c1 > chunks) c1 = chunks;
    if (c1 > c0) {
        c_lo = (uint32_t)c0;
        count = (uint32_t)(c1 - c0);
    }
}

template <int J>
__global__ __launch_bounds__(kShortThreads) void seg_short_kernel(ShortParams p) {
    __shared__ __align__(16) uint32_t s_p[kShortChunk];
    const uint64_t SB = p.seg_per_block; // at most J * kShortThreads
    const int lane = lane_id();
    const uint64_t s0 = (uint64_t)blockIdx.x * SB;
    const uint64_t s1 = s0 + SB < p.segments ? s0 + SB : p.segments;
    const uint64_t a0 = short_off(p, s0);
    uint64_t a1 = short_off(p, s1);
    if (a1 < a0) a1 = a0; // only reachable with malformed offsets
    if (a1 == a0) { // block-uniform: every segment of the block is empty
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const uint64_t s = s0 + threadIdx.x + (uint64_t)j * kShortThreads;
            if (s < s1) p.out[s] = 0u;
        }
        return;
    }
    const uint64_t base = a0 & ~3ull;
    const uint64_t c1 = a1 < base + kShortChunk ? a1 : base + kShortChunk;

    // This thread's segments s0 + t + 256 j.  Their offsets are loaded here
    // but first used after the value loads are issued, so both arrive in one
    // memory round trip.
    // A segment's end is the next lane's start; the end of lane 63's segment
    // in group j is loaded by lane j of the wave into one register.
    uint32_t lo[J];
    const uint64_t wave_s = s0 + (threadIdx.x & ~(kWave - 1));
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint64_t s = s0 + threadIdx.x + (uint64_t)j * kShortThreads;
        lo[j] = s <= s1 ? p.offsets[s] : 0u; // s == s1: the last segment's end
    }
    const uint64_t edge_k = wave_s + (uint64_t)lane * kShortThreads + kWave;
    const uint32_t edge = (lane < J && edge_k <= s1) ? p.offsets[edge_k] : 0u;
    const ChunkCarry cc = short_chunk_prefix(p.values, base, a0, c1, s_p);
    // Segment j's bounds, clamped into the span (only malformed offsets are
    // changed); recomputed where needed rather than held, which took J = 16
    // from 115 to 102 VGPRs (J = 15 and 16 run four waves per SIMD; J <= 14,
    // at 94, five).
    auto bounds = [&](int j, uint64_t &st, uint64_t &en) {
        const uint32_t next = __shfl_down(lo[j], 1);
        const uint32_t e = lane == kWave - 1 ? read_lane(edge, j) : next;
        const uint64_t s = s0 + threadIdx.x + (uint64_t)j * kShortThreads;
        st = lo[j] < a0 ? a0 : (lo[j] > a1 ? a1 : lo[j]);
        en = (s >= s1 || e < st) ? st : (e > a1 ? a1 : e);
    };
#pragma unroll
    for (int j = 0; j < J; ++j) {
        uint64_t st, en;
        bounds(j, st, en);
        const uint64_t s = s0 + threadIdx.x + (uint64_t)j * kShortThreads;
        if (s < s1) {
            const uint64_t h = en < c1 ? en : c1;
            const uint64_t l = st < h ? st : h;
            p.out[s] = chunk_range_sum(s_p, cc, (uint32_t)(l - base), (uint32_t)(h - base));
        }
    }
    if (a1 <= base + kShortChunk) return; // block-uniform
    // Chunks 1 .. chunks-1 go to the worklist: the entry of the chunk that
    // starts at element e is written by the lane whose segment holds e, at
    // slots each wave reserves with one atomic.
    const uint64_t chunks = (a1 - base + kShortChunk - 1) / kShortChunk;
    uint32_t lane_total = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        uint64_t st, en;
        bounds(j, st, en);
        uint32_t c_lo, count;
        short_chunk_range(base, st, en, chunks, c_lo, count);
        lane_total += count;
    }
    const uint32_t incl = wave_inclusive_scan<OpSum, uint32_t>(lane_total);
    const uint32_t wave_total = read_lane(incl, kWave - 1);
    if (wave_total == 0) return; // wave-uniform
    unsigned long long first = 0;
    if (lane == 0) first = atomicAdd(p.work_count, (unsigned long long)wave_total);
    first = ((uint64_t)read_lane((uint32_t)(first >> 32), 0) << 32) | read_lane((uint32_t)first, 0);
    uint64_t slot = first + (incl - lane_total);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        uint64_t st, en;
        bounds(j, st, en);
        uint32_t c_lo, count;
        short_chunk_range(base, st, en, chunks, c_lo, count);
        const uint64_t s = s0 + threadIdx.x + (uint64_t)j * kShortThreads;
        short_write_entries(p, slot, base, (uint32_t)s, c_lo, count);
        slot += count;
    }
}

// Sum (mod 2^32) of this wave's share of values [c0, c1), c1 - c0 <=
// kShortChunk, laid out as in short_chunk_prefix.
__device__ __forceinline__ uint32_t short_chunk_wave_sum(const uint32_t *values, uint64_t c0, uint64_t c1) {
    const int w = threadIdx.x / kWave;
    const uint64_t e0 = c0 + (uint64_t)w * kShortWaveElems + (uint64_t)lane_id() * 4;
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kShortSteps; ++j) {
        const uint64_t e = e0 + (uint64_t)j * (kWave * 4);
        if (e + 4 <= c1) {
            const u32x4_a4 v = load_a4<true>((const u32x4_a4 *)(values + e));
            sum += v.x + v.y + v.z + v.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) sum += (e + c < c1) ? values[e + c] : 0u;
        }
    }
    return wave_sum(sum);
}

// Adds each deferred chunk's part to the outputs of the segments that
// overlap it.  Grid-strided over the entries, so every block reaches the end
// whatever the count; entries beyond the workspace (possible only with
// malformed offsets) are dropped.
__global__ __launch_bounds__(kShortThreads) void seg_short_drain_kernel(ShortParams p) {
    __shared__ __align__(16) uint32_t s_p[kShortChunk];
    uint64_t count = *p.work_count;
    if (count > p.work_cap) count = p.work_cap;
    uint2 next = blockIdx.x < count ? p.work[blockIdx.x] : make_uint2(0u, 0u);
    // Each wave accumulates its whole-chunk sums per segment and adds them
    // once the segment changes: many chunks of one long segment would
    // otherwise serialise on one output word.
    uint64_t acc_s = ~0ull;
    uint32_t acc_v = 0;
    for (uint64_t i = blockIdx.x; i < count; i += gridDim.x) { // block-uniform
        const uint2 e = next; // the next entry is loaded while this one runs
        if (i + gridDim.x < count) next = p.work[i + gridDim.x];
        if (e.x >= p.segments) continue;
        const uint64_t sf = e.x, c0 = e.y;
        const uint64_t s1b = (sf / p.seg_per_block + 1) * p.seg_per_block;
        const uint64_t s1 = s1b < p.segments ? s1b : p.segments;
        const uint64_t a1 = short_off(p, s1);
        const uint64_t c1 = c0 + kShortChunk < a1 ? c0 + kShortChunk : a1;
        if (c0 >= c1) continue;
        // A chunk inside one segment (the usual case: a long segment's
        // middle) needs only its sum: no LDS and no barrier.
        if (short_off(p, sf + 1) >= c1) {
            const uint32_t v = short_chunk_wave_sum(p.values, c0, c1);
            if (sf != acc_s) {
                if (lane_id() == 0 && acc_s != ~0ull && acc_v) atomicAdd(&p.out[acc_s], acc_v);
                acc_s = sf;
                acc_v = 0;
            }
            acc_v += v;
            continue;
        }
        const ChunkCarry cc = short_chunk_prefix(p.values, c0, c0, c1, s_p);
        for (uint64_t s = sf + threadIdx.x; s < s1; s += kShortThreads) {
            const uint64_t st = short_off(p, s);
            if (st >= c1) break; // offsets are sorted: so do all later segments
            const uint64_t en = short_off(p, s + 1);
            const uint64_t l = st > c0 ? st : c0, h = en < c1 ? en : c1;
            if (h > l) {
                const uint32_t v = chunk_range_sum(s_p, cc, (uint32_t)(l - c0), (uint32_t)(h - c0));
                if (v) atomicAdd(&p.out[s], v);
            }
        }
        __syncthreads(); // s_p is rewritten by the next entry
    }
    if (lane_id() == 0 && acc_s != ~0ull && acc_v) atomicAdd(&p.out[acc_s], acc_v);
}

// n == 0: every segment is empty.
__global__ void segmented_zero_kernel(uint32_t *out, uint64_t s) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < s;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = 0u;
}

// Bit 0: offsets[0] != 0 or offsets[S] != n.  Bit 1: a decrease.
__global__ void validate_offsets_kernel(const uint32_t *offsets, uint64_t count, uint64_t n,
                                        uint32_t *flags) {
    const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < count; k += nthreads) {
        const uint32_t o = offsets[k];
        if ((k == 0 && o != 0u) || (k == count - 1 && (uint64_t)o != n)) atomicOr(&flags[0], 1u);
        if (k + 1 < count && offsets[k + 1] < o) atomicOr(&flags[0], 2u);
    }
}

} // namespace

namespace {

// Segments per block: as many as keep the block's expected span (SB n / S
// values) within kShortSpan, at most kShortMaxJ per thread, rounded down to
// whole groups of 256 (one segment per thread each) when that keeps 80% of
// them.  A partly filled last group costs a whole j step; too few segments
// leave blocks short of work.  2^27 values, us with the exact count against
// whole groups: mean 2 236 / 237, 4 156 / 149, 8 129 / 131, 14 120 / 115,
// 16 115 / 149 (464 segments against 256), 20 115 / 128, 24 114 / 107,
// 28 114 / 105.
uint64_t short_seg_per_block(const SegmentedArgs &a) {
    const uint64_t cap = (uint64_t)kShortMaxJ * kShortThreads;
    if (a.n == 0) return cap;
    uint64_t sb = kShortSpan * a.num_segments / a.n;
    if (sb > cap) sb = cap;
    const uint64_t whole = sb / kShortThreads * kShortThreads;
    return 5 * whole >= 4 * sb ? whole : sb;
}

// Taken when a block holds at least one segment per thread, mean n / S up
// to kShortSpan / 256 = 29.  At 2^27 values it beats the element tiles from
// 4.5x (mean 1) to 1.4x (mean 12), and at 2^26 values, mean 16 / 20 / 24 /
// 28, 83.5 / 75.8 / 72.8 / 68.9 us on the tiles against 60.6 / 59.3 / 56.1
// / 54.7 here.  From mean 30 the tiles hold their own (67 us either way;
// mean 40 59 against 61).
bool short_path(const SegmentedArgs &a) {
    return a.num_segments > 0 && a.n > 0 && short_seg_per_block(a) >= (uint64_t)kShortThreads;
}

// Segments per thread: J covers the block's segments, the last group of 256
// partly filled.
int short_j(const SegmentedArgs &a) {
    return (int)ceil_div(short_seg_per_block(a), (uint64_t)kShortThreads);
}

uint64_t short_blocks(const SegmentedArgs &a) { return ceil_div(a.num_segments, short_seg_per_block(a)); }

// Every block defers at most ceil((span + 3) / chunk) - 1 < (span + 3) / chunk
// chunks, and the spans of sorted offsets add up to n.
uint64_t short_work_cap(const SegmentedArgs &a) {
    return (a.n + 3 * short_blocks(a)) / kShortChunk + 1;
}

template <int J> hx_status launch_short_j(int j, const ShortParams &p, uint64_t blocks, hipStream_t stream) {
    if constexpr (J > kShortMaxJ) {
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce: no kernel for %d segments per thread", j);
    } else {
        if (j != J) return launch_short_j<J + 1>(j, p, blocks, stream);
        hipLaunchKernelGGL((seg_short_kernel<J>), dim3((uint32_t)blocks), dim3(kShortThreads), 0, stream, p);
        return check_launch("seg_short_kernel");
    }
}

hx_status launch_short(const SegmentedArgs &a, void *ws, uint64_t ws_bytes, hipStream_t stream) {
    ShortParams p{};
    p.values = (const uint32_t *)a.values;
    p.n = a.n;
    p.offsets = a.offsets;
    p.segments = a.num_segments;
    p.out = (uint32_t *)a.out;
    const int j = short_j(a);
    p.seg_per_block = short_seg_per_block(a);
    p.work_count = (unsigned long long *)ws;
    p.work = (uint2 *)((char *)ws + kWorkHeader);
    p.work_cap = short_work_cap(a);
    if (ws_bytes < kWorkHeader + p.work_cap * sizeof(uint2))
        return fail(HX_ERR_DISPATCH_FAILED, "segmented workspace of %llu bytes is too small",
                    (unsigned long long)ws_bytes);
    const uint64_t blocks = short_blocks(a);
    hipLaunchKernelGGL(seg_short_init_kernel, dim3(1), dim3(1), 0, stream, p.work_count);
    HX_TRY(check_launch("seg_short_init_kernel"));
    HX_TRY(launch_short_j<1>(j, p, blocks, stream));
    const uint64_t drain = p.work_cap < kDrainBlocks ? p.work_cap : kDrainBlocks;
    hipLaunchKernelGGL(seg_short_drain_kernel, dim3((uint32_t)drain), dim3(kShortThreads), 0, stream, p);
    return check_launch("seg_short_drain_kernel");
}

} // namespace

namespace {
uint64_t align256(uint64_t b) { return (b + 255) & ~255ull; }
bool long_tiles(const SegmentedArgs &a) { return a.n >= kLongMean * a.num_segments; }
uint64_t seg_tile_elems(const SegmentedArgs &a) { return long_tiles(a) ? kLongTile : kTile; }
uint64_t tile_map_bytes(uint64_t tiles) { return align256(2 * (tiles + 1) * 4); }
} // namespace

// Look-back status words: 8 bytes per tile and per 64-tile superblock on the
// element-tile path, none on the short path.
uint64_t segmented_lookback_bytes(const SegmentedArgs &a) {
    if (a.n == 0 || a.num_segments == 0 || short_path(a)) return 0;
    const uint64_t tiles = ceil_div(a.n, seg_tile_elems(a));
    return kLookbackOffset + (tiles + ceil_div(tiles, kSegSuper)) * 8 * kSegStatusStride;
}

// Everything else, which must never share memory with status words: the
// tile maps, or the short path's chunk worklist.
uint64_t segmented_aux_bytes(const SegmentedArgs &a) {
    if (a.n == 0 || a.num_segments == 0) return 0;
    if (short_path(a)) return kWorkHeader + short_work_cap(a) * sizeof(uint2);
    const uint64_t tiles = ceil_div(a.n, seg_tile_elems(a));
    return tile_map_bytes(tiles);
}

// A prepared plan's one workspace: the status words, then the rest.  Its
// layout never changes, so the status words always stay where they were.
uint64_t segmented_workspace_bytes(const SegmentedArgs &a) {
    return align256(segmented_lookback_bytes(a)) + segmented_aux_bytes(a);
}

hx_status launch_segmented(const SegmentedArgs &a, void *ws, uint64_t ws_bytes, void *aux, uint64_t aux_bytes,
                           LookbackState &lb, hipStream_t stream) {
    if (a.num_segments == 0) return HX_OK;
    if (a.n == 0) {
        uint64_t blocks = ceil_div(a.num_segments, kBlock);
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(segmented_zero_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (uint32_t *)a.out, a.num_segments);
        return check_launch("segmented_zero_kernel");
    }
    if (a.num_segments >= 0xFFFFFFFFull)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce of %llu segments exceeds the u32 offset range",
                    (unsigned long long)a.num_segments);
    if (((uintptr_t)a.values) % 4 != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce values must be 4-byte aligned");
    if (!aux) { // one workspace (a prepared plan): status words, then the rest
        const uint64_t at = align256(segmented_lookback_bytes(a));
        if (!ws || ws_bytes < at)
            return fail(HX_ERR_DISPATCH_FAILED, "segmented workspace of %llu bytes is too small",
                        (unsigned long long)ws_bytes);
        aux = (char *)ws + at;
        aux_bytes = ws_bytes - at;
        ws_bytes = at;
    }
    if (aux_bytes < segmented_aux_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "segmented scratch of %llu bytes is too small",
                    (unsigned long long)aux_bytes);
    if (short_path(a)) return launch_short(a, aux, aux_bytes, stream);
    SegParams p{};
    p.values = (const uint32_t *)a.values;
    p.n = a.n;
    p.offsets = a.offsets;
    p.segments = a.num_segments;
    p.out = (uint32_t *)a.out;
    const bool long_tile = long_tiles(a);
    p.total_tiles = ceil_div(a.n, seg_tile_elems(a));
    p.status = (uint64_t *)((char *)ws + kLookbackOffset);
    p.sstatus = p.status + p.total_tiles * kSegStatusStride;
    p.ub_map = (uint32_t *)aux;
    p.lb_map = p.ub_map + p.total_tiles + 1;
    if (p.total_tiles >= 0x80000000ull)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce of %llu tiles exceeds the grid range",
                    (unsigned long long)p.total_tiles);
    if (ws_bytes < segmented_lookback_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "segmented workspace of %llu bytes is too small",
                    (unsigned long long)ws_bytes);
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    p.spin_limit = lookback_poll_limit();
    uint64_t map_blocks = ceil_div(a.num_segments + 2, kBlock);
    if (map_blocks > 2048) map_blocks = 2048;
    if (long_tile) {
        hipLaunchKernelGGL((seg_tile_map_kernel<kLongTile>), dim3((uint32_t)map_blocks), dim3(kBlock), 0, stream,
                           p);
        HX_TRY(check_launch("seg_tile_map_kernel"));
        if (a.n < kTwoLevelMaxMean * a.num_segments)
            hipLaunchKernelGGL((segmented_sum_kernel<kLongWaves, kSegSteps, true>), dim3((uint32_t)p.total_tiles),
                               dim3(kLongWaves * kWave), 0, stream, p);
        else
            hipLaunchKernelGGL((segmented_sum_kernel<kLongWaves, kSegSteps, false>), dim3((uint32_t)p.total_tiles),
                               dim3(kLongWaves * kWave), 0, stream, p);
    } else {
        hipLaunchKernelGGL((seg_tile_map_kernel<kTile>), dim3((uint32_t)map_blocks), dim3(kBlock), 0, stream, p);
        HX_TRY(check_launch("seg_tile_map_kernel"));
        hipLaunchKernelGGL((segmented_sum_kernel<kSegWaves, kSegSteps>), dim3((uint32_t)p.total_tiles),
                           dim3(kSegWaves * kWave), 0, stream, p);
    }
    HX_TRY(check_launch("segmented_sum_kernel"));
    commit_lookback_launch(lb);
    return HX_OK;
}

hx_status validate_offsets_on_device(hx_device *dev, const uint32_t *offsets, uint64_t count,
                                     uint64_t n) {
    uint32_t *flags = nullptr;
    HX_HIP(hipMalloc(&flags, 4), HX_ERR_ALLOCATION_FAILED, "validation flag hipMalloc");
    hipError_t err = hipMemsetAsync(flags, 0, 4, dev->stream);
    if (err == hipSuccess) {
        uint64_t blocks = ceil_div(count, kBlock);
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(validate_offsets_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0,
                           dev->stream, offsets, count, n, flags);
        err = hipGetLastError();
    }
    uint32_t host = 0;
    if (err == hipSuccess) err = hipMemcpyAsync(&host, flags, 4, hipMemcpyDeviceToHost, dev->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(dev->stream);
    (void)hipFree(flags);
    if (err != hipSuccess) return hip_fail(HX_ERR_DISPATCH_FAILED, err, "offset validation");
    // Messages follow validate_csr (core sparse.rs:186-212).
    if (host & 1u)
        return fail(HX_ERR_DISPATCH_FAILED,
                    "invalid segment offsets: offsets must start at 0 and end at the element count");
    if (host & 2u)
        return fail(HX_ERR_DISPATCH_FAILED, "invalid segment offsets: offsets must be non-decreasing");
    return HX_OK;
}

} // namespace hx
