// Segmented sum for gfx950.  Offsets follow the CSR
// row_ptr convention (crates/hephaestus-core/src/domain/sparse.rs:179-220):
// S+1 entries, offsets[0] = 0, offsets[S] = n, non-decreasing, and
//   out[s] = sum of values[offsets[s] .. offsets[s+1])   (mod 2^32).
//
// The reference's nearest kernel is CSR SpMV with one thread per row and a
// serial inner loop (crates/hephaestus-rocm/src/application/sparse/
// spmv.rs:17-42), which leaves neighbouring lanes hundreds of elements
// apart.  Here the work is cut by ELEMENTS, not by segments, so every block
// streams the same 64 KiB with 16-byte loads whatever the segment lengths:
//
//   * block b takes tile b (no ticket counter) and loads its 16384 values
//     (8 waves x 8 vectors per lane), wave-striped like the scan;
//   * while those loads are in flight, three waves run 64-ary searches over
//     the offsets for the segment boundaries the tile touches;
//   * the tile's inclusive prefix goes to LDS; every segment that ENDS in the
//     tile gets E[end] - E[start] (plus the carry for the segment that began
//     in an earlier tile);
//   * the carry is a segmented decoupled look-back: a tile that contains a
//     segment start publishes its carry-out at once as a "prefix", so the
//     look-back almost always stops at the nearest predecessor.
// The 64 KiB LDS prefix caps residency at two blocks per CU; at 2^27 values
// the 8x8 tile ran 151 us against 187 us for 4 waves x 4 vectors (4096-value
// tiles).
// Integer addition mod 2^32 is associative, so every output is bit-exact.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {
namespace {

constexpr int kBlock = 256; // helper kernels
// Tile geometry of segmented_sum_kernel: WAVES waves, each lane holding
// STEPS 16-byte vectors; the tile's inclusive prefix lives in LDS.
template <int WAVES, int STEPS> struct SegTile {
    static constexpr int kWaveElems = kWave * 4 * STEPS;
    static constexpr int kElems = WAVES * kWaveElems;
};
constexpr int kSegWaves = 8, kSegSteps = 8; // 16384-element tiles (64 KiB of LDS prefix)
constexpr int kTile = SegTile<kSegWaves, kSegSteps>::kElems;
constexpr uint32_t kInvalid = 0, kAggregate = 1, kPrefix = 2;
constexpr uint32_t kSpinLimit = 64; // polls before computing a predecessor

struct SegParams {
    const uint32_t *values;
    uint64_t n;
    const uint32_t *offsets;
    uint64_t segments; // S
    uint32_t *out;
    uint64_t total_tiles;
    WorkspaceHeader *hdr;
    uint64_t *status;
    uint32_t tag;         // this launch's status tag
};

// Offsets clamped into [0, n]: malformed offsets can never address values
// out of bounds.
__device__ __forceinline__ uint64_t off_at(const SegParams &p, uint64_t k) {
    const uint64_t o = p.offsets[k];
    return o < p.n ? o : p.n;
}

// First k in [0, S] with off(k) > v, or S+1 if none (upper bound).  Each
// round probes 64 evenly spaced positions, one per lane, and keeps the gap
// between the last "<= v" and the first "> v" probe.  Terminates for any
// offset contents because the range strictly shrinks.
__device__ uint64_t wave_upper_bound(const SegParams &p, uint64_t v) {
    const int lane = lane_id();
    uint64_t lo = 0, hi = p.segments + 1;
    while (hi > lo) {
        const uint64_t len = hi - lo;
        const uint64_t step = (len + kWave - 1) / kWave;
        uint64_t pos = lo + (uint64_t)(lane + 1) * step - 1;
        if (pos > hi - 1) pos = hi - 1;
        const bool pred = off_at(p, pos) > v;
        const uint64_t m = ballot(pred);
        if (m == 0ull) return hi;
        const int f = __ffsll((long long)m) - 1;
        const uint64_t pf = __shfl(pos, f, kWave);
        if (step == 1) return pf; // every position in the range was probed
        const uint64_t pprev = f > 0 ? __shfl(pos, f - 1, kWave) : 0;
        lo = f > 0 ? pprev + 1 : lo;
        hi = pf + 1;
        if (hi - lo == 1) return lo;
    }
    return lo;
}

__device__ __forceinline__ uint64_t status_word(uint32_t tag, uint32_t flag, uint32_t v) {
    return ((uint64_t)((tag << 2) | flag) << 32) | (uint64_t)v;
}

// The status tile u's owner publishes, computed by ONE wave (fallback path):
// a prefix (the sum from the last segment start in the tile to its end) when
// the tile holds a segment start, else an aggregate (the tile total).
template <int TILE>
__device__ void seg_tile_status(const SegParams &p, uint64_t u, uint32_t &flag, uint32_t &value) {
    const uint64_t t0 = u * TILE;
    const uint64_t t1 = (t0 + TILE < p.n) ? t0 + TILE : p.n;
    const uint64_t k_star = wave_upper_bound(p, t1 - 1);
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

// Block b processes tile b; see scan.hip for why there is no ticket counter
// and how the fallback guarantees progress in any dispatch order.
template <int WAVES, int STEPS>
__global__ __launch_bounds__(WAVES * kWave) void segmented_sum_kernel(SegParams p) {
    static_assert(WAVES >= 4, "waves 1-3 run the boundary searches");
    constexpr int kWaveElems = SegTile<WAVES, STEPS>::kWaveElems;
    constexpr int kTile = SegTile<WAVES, STEPS>::kElems;
    constexpr int kThreads = WAVES * kWave;
    __shared__ uint64_t s_bound[3];
    __shared__ uint32_t s_wave_tot[WAVES];
    __shared__ uint32_t s_carry;
    // Eb[4 + i] = tile-local inclusive prefix at element i, Eb[3] = 0, so
    // the exclusive prefix at i is Eb[3 + i].  The 4-word offset keeps every
    // lane's four prefixes one aligned 16-byte LDS store (conflict-free;
    // four scalar stores at a 4-word lane stride conflicted 4-way).
    __shared__ __attribute__((aligned(16))) uint32_t Eb[kTile + 4];

    const uint64_t tile = blockIdx.x;
    const uint32_t tag = p.tag;
    const int w = threadIdx.x / kWave;
    const int lane = lane_id();
    const uint64_t t0 = tile * kTile;
    const uint64_t t1 = (t0 + kTile < p.n) ? t0 + kTile : p.n;
    const uint64_t e0 = t0 + (uint64_t)w * kWaveElems + (uint64_t)lane * 4;

    // Issue the value loads first; the searches below overlap them.  Whole
    // tiles use a block-uniform base and one 32-bit lane offset.
    uint32_t x[STEPS][4];
    if (t1 - t0 == (uint64_t)kTile) {
        const char *base = (const char *)(p.values + t0);
        const uint32_t lane_off =
            ((uint32_t)__builtin_amdgcn_readfirstlane(w) * kWaveElems + (uint32_t)lane * 4) * 4u;
#pragma unroll
        for (int j = 0; j < STEPS; ++j) {
            const u32x4 v = load_vec<true>((const u32x4 *)(base + lane_off + (uint32_t)j * (kWave * 16)));
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
                const u32x4 v = __builtin_nontemporal_load((const u32x4 *)(p.values + e));
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

    // k_lo = ub(t0): first offset past the tile start (segment of t0 is
    // k_lo - 1); k_hi1 = ub(t1); k_star = ub(t1 - 1) (segment of t1-1 is
    // k_star - 1).
    if (w >= 1) {
        const uint64_t v = (w == 1) ? t0 : (w == 2) ? t1 : t1 - 1;
        const uint64_t r = wave_upper_bound(p, v);
        if (lane == 0) s_bound[w - 1] = r;
    }

    // Tile-local inclusive prefix of the values (mod 2^32).
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
    uint32_t wave_excl = 0;
#pragma unroll
    for (int k = 0; k < WAVES; ++k)
        if (k < w) wave_excl += s_wave_tot[k];
#pragma unroll
    for (int j = 0; j < STEPS; ++j) {
        const int le = w * kWaveElems + j * (kWave * 4) + lane * 4;
        u32x4 v;
        v.x = wave_excl + x[j][0];
        v.y = wave_excl + x[j][1];
        v.z = wave_excl + x[j][2];
        v.w = wave_excl + x[j][3];
        *(u32x4 *)&Eb[4 + le] = v;
    }
    if (threadIdx.x == 0) Eb[3] = 0;
    __syncthreads();
    const uint32_t *E = Eb + 3; // E[i]: exclusive prefix at element i

    const uint64_t k_lo = s_bound[0];
    const uint64_t k_hi1 = s_bound[1];
    const uint64_t k_star = s_bound[2];
    const uint64_t tlen = t1 - t0;
    const uint32_t total = E[tlen];

    if (w == 0) {
        // Start of the segment holding t1-1, and of the one holding t0.
        uint64_t h = k_star >= 1 ? off_at(p, k_star - 1) : 0;
        if (h > t1 - 1) h = t1 - 1; // only reachable with malformed offsets
        const uint64_t first_start = k_lo >= 1 ? off_at(p, k_lo - 1) : 0;
        const bool has_head = h >= t0;
        const bool needs_carry = tile > 0 && first_start < t0;
        uint32_t c_in = 0;
        if (has_head) {
            if (lane == 0) st_relaxed(&p.status[tile], status_word(tag, kPrefix, total - E[h - t0]));
        } else if (tile > 0 && lane == 0) {
            st_relaxed(&p.status[tile], status_word(tag, kAggregate, total));
        }
        if (needs_carry || (!has_head && tile > 0)) {
            // Look back over predecessors until a prefix (a tile holding a
            // segment start, or one that already resolved its carry).
            int64_t pred = (int64_t)tile - 1;
            for (;;) {
                const int64_t idx = pred - lane;
                uint32_t flag, val;
                uint32_t spins = 0;
                for (;;) {
                    flag = kPrefix;
                    val = 0;
                    if (idx >= 0) {
                        const uint64_t wd = ld_relaxed(&p.status[idx]);
                        const uint32_t hi = (uint32_t)(wd >> 32);
                        flag = ((hi >> 2) == tag) ? (hi & 3u) : kInvalid;
                        val = (uint32_t)wd;
                    }
                    const uint64_t pm = ballot(flag == kPrefix);
                    const uint64_t im = ballot(flag == kInvalid);
                    const uint64_t need = pm ? (((pm & (~pm + 1ull)) << 1) - 1ull) : ~0ull;
                    const uint64_t missing = im & need;
                    if (missing == 0ull) break;
                    if (++spins >= kSpinLimit) {
                        const uint64_t u = (uint64_t)(pred - (__ffsll((long long)missing) - 1));
                        uint32_t fflag, fval;
                        seg_tile_status<kTile>(p, u, fflag, fval);
                        if (lane == 0) publish_if_unset(&p.status[u], tag, fflag, fval);
                        spins = 0;
                        continue;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                const uint64_t pm = ballot(flag == kPrefix);
                const int first = pm ? (__ffsll((long long)pm) - 1) : kWave;
                c_in += wave_sum((lane <= first) ? val : 0u);
                if (pm) break;
                pred -= kWave;
            }
        }
        if (!has_head && tile > 0 && lane == 0) st_relaxed(&p.status[tile], status_word(tag, kPrefix, c_in + total));
        if (lane == 0) s_carry = c_in;
    }
    __syncthreads();
    const uint32_t c_in = s_carry;

    // Segments s = k-1 whose end offset off(k) lies in (t0, t1]; tile 0 also
    // owns the empty segments that end at 0.
    uint64_t k_first = tile == 0 ? 1 : (k_lo > 1 ? k_lo : 1);
    uint64_t k_last = k_hi1 >= 1 ? k_hi1 - 1 : 0;
    if (k_last > p.segments) k_last = p.segments;
    for (uint64_t k = k_first + threadIdx.x; k <= k_last; k += kThreads) {
        const uint64_t b = off_at(p, k);
        uint64_t a = off_at(p, k - 1);
        if (a > b) a = b; // malformed: treat as empty
        if (b < t0 || b > t1) continue; // malformed (non-monotonic) offsets
        const uint64_t a_loc = (a > t0 ? a : t0) - t0;
        uint32_t v = E[b - t0] - E[a_loc];
        if (a < t0) v += c_in;
        p.out[k - 1] = v;
    }
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

uint64_t segmented_workspace_bytes(const SegmentedArgs &a) {
    return kLookbackOffset + ceil_div(a.n, kTile) * 8;
}

hx_status launch_segmented(const SegmentedArgs &a, void *ws, uint64_t ws_bytes, LookbackState &lb,
                           hipStream_t stream) {
    if (a.num_segments == 0) return HX_OK;
    if (a.n == 0) {
        uint64_t blocks = ceil_div(a.num_segments, kBlock);
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(segmented_zero_kernel, dim3((uint32_t)blocks), dim3(kBlock), 0, stream,
                           (uint32_t *)a.out, a.num_segments);
        return check_launch("segmented_zero_kernel");
    }
    SegParams p{};
    p.values = (const uint32_t *)a.values;
    p.n = a.n;
    p.offsets = a.offsets;
    p.segments = a.num_segments;
    p.out = (uint32_t *)a.out;
    p.total_tiles = ceil_div(a.n, kTile);
    p.hdr = (WorkspaceHeader *)ws;
    p.status = (uint64_t *)((char *)ws + kLookbackOffset);
    if (p.total_tiles >= 0x80000000ull)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce of %llu tiles exceeds the grid range",
                    (unsigned long long)p.total_tiles);
    if (((uintptr_t)a.values) % 16 != 0)
        return fail(HX_ERR_DISPATCH_FAILED, "segmented reduce values must be 16-byte aligned");
    if (ws_bytes < segmented_workspace_bytes(a))
        return fail(HX_ERR_DISPATCH_FAILED, "segmented workspace of %llu bytes is too small",
                    (unsigned long long)ws_bytes);
    HX_TRY(next_lookback_launch(lb, ws, ws_bytes, stream, &p.tag));
    hipLaunchKernelGGL((segmented_sum_kernel<kSegWaves, kSegSteps>), dim3((uint32_t)p.total_tiles),
                       dim3(kSegWaves * kWave), 0, stream, p);
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
