/*
 * hx_oracle.h — CPU oracle for the reduction / scan path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (hephaestus_amd/) links,
 * loads or calls this library; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker or as the
 * timed CPU baseline.
 *
 * It restates, as sequential folds over host memory, what the reference's
 * CPU oracles compute for this path (the `iter().sum()/min()/max()/scan()`
 * folds of crates/hephaestus-rocm/tests/contract.rs:829-831,1673-1680) and
 * what the reference's seams promise (crates/hephaestus-core/src/domain/
 * reduction.rs, scan.rs, ops.rs:735-983), plus the additions
 * (argmax, exclusive scan, segmented sum, affine prologue).  The reference
 * itself is Rust and cannot be built in this image (no cargo/rustc), so
 * there is no oracle/_ref build.
 *
 * Semantics fixed here (each checked by tests/test_oracle.py):
 *   - u32/i32 sums, products and scans wrap mod 2^32 (two's complement).
 *   - f32 sums and scans are returned as the f64 value of a compensated
 *     (Neumaier) f64 accumulation, together with the matching prefix of
 *     sum |y| so a caller can apply the bound 2*ceil(log2 n)*eps_f32*sum|y|.
 *   - MaxOp folds the identity f32::MIN / 0u / i32::MIN (ops.rs:956-958)
 *     with every non-NaN element under the IEEE total order (-0 < +0);
 *     MinOp likewise with f32::MAX / u32::MAX / i32::MAX.
 *   - argmax is the lowest index attaining the maximum of the non-NaN
 *     elements under the same order; UINT32_MAX when there is none.
 *   - The prologue is y = fmaf(a, x, b) (C99 fmaf, correctly rounded).
 *   - Inputs: SplitMix64 output i for `seed` (Steele, Lea, Flood 2014).
 */
#ifndef HX_ORACLE_H
#define HX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hxo_affine {
    float a;
    float b;
    int32_t enabled;
} hxo_affine;

/* ---- generator ---- */
uint64_t hxo_splitmix64_at(uint64_t seed, uint64_t i);
void hxo_fill_uniform_int(uint32_t *dst, uint64_t n, uint64_t seed, int64_t lo, int64_t hi);
void hxo_fill_uniform_real(float *dst, uint64_t n, uint64_t seed, float lo, float hi);
void hxo_fill_normal(float *dst, uint64_t n, uint64_t seed, double mean, double stddev);

/* ---- full reductions ---- */
uint32_t hxo_sum_u32(const uint32_t *x, uint64_t n);
uint32_t hxo_prod_u32(const uint32_t *x, uint64_t n);
/* f64 (compensated) sum of y; *abs_sum gets sum |y|. */
double hxo_sum_f32(const float *x, uint64_t n, const hxo_affine *pro, double *abs_sum);
uint32_t hxo_max_u32(const uint32_t *x, uint64_t n);
int32_t hxo_max_i32(const int32_t *x, uint64_t n);
float hxo_max_f32(const float *x, uint64_t n, const hxo_affine *pro);
uint32_t hxo_min_u32(const uint32_t *x, uint64_t n);
int32_t hxo_min_i32(const int32_t *x, uint64_t n);
float hxo_min_f32(const float *x, uint64_t n, const hxo_affine *pro);
uint32_t hxo_argmax_u32(const uint32_t *x, uint64_t n);
uint32_t hxo_argmax_i32(const int32_t *x, uint64_t n);
uint32_t hxo_argmax_f32(const float *x, uint64_t n, const hxo_affine *pro);

/* ---- row-wise (row r = x + r*ld, cols elements) ---- */
void hxo_rows_f32(const float *x, uint64_t rows, uint64_t cols, uint64_t ld,
                  const hxo_affine *pro, double *sum, double *abs_sum,
                  float *max, uint32_t *argmax);
void hxo_rows_u32(const uint32_t *x, uint64_t rows, uint64_t cols, uint64_t ld,
                  uint32_t *sum, uint32_t *max, uint32_t *argmax);
void hxo_rows_i32(const int32_t *x, uint64_t rows, uint64_t cols, uint64_t ld,
                  int32_t *sum, int32_t *max, uint32_t *argmax);

/* ---- scans (in logical order; reverse = suffix scan) ---- */
void hxo_scan_sum_u32(const uint32_t *x, uint64_t n, int exclusive, int reverse, uint32_t *out);
void hxo_scan_prod_u32(const uint32_t *x, uint64_t n, int exclusive, int reverse, uint32_t *out);
/* f64 compensated prefix of x into ref[], matching prefix of |x| into abs[]. */
void hxo_scan_sum_f32(const float *x, uint64_t n, int exclusive, int reverse, double *ref,
                      double *abs_prefix);
/* Count outputs violating |got - ref| <= 2*ceil(log2 n)*eps_f32*abs (eps_f32
 * = 2^-23); *worst gets the largest |got-ref| / (eps_f32*abs) seen. */
uint64_t hxo_check_f32_bound(const float *got, const double *ref, const double *abs_prefix,
                             uint64_t m, uint64_t n_for_log, double *worst);
uint32_t hxo_ceil_log2(uint64_t n);
/* Streaming form for operands too large to hold an f64 reference: runs the
 * compensated forward prefix of x and checks got[] against the same bound
 * on the fly. Returns the number of violations. */
uint64_t hxo_check_scan_f32(const float *x, const float *got, uint64_t n, int exclusive,
                            uint64_t n_for_log, double *worst);

/* ---- segmented sum (offsets: S+1 entries, CSR row_ptr convention) ---- */
void hxo_segmented_sum_u32(const uint32_t *x, uint64_t n, const uint32_t *offsets, uint64_t segments,
                           uint32_t *out);
/* Synthetic geometric segment lengths (mean `mean`, min 1) drawn from
 * SplitMix64(seed, s) until they cover n; returns S and fills offsets
 * (capacity `cap` >= S+1 entries). */
uint64_t hxo_geometric_offsets(uint64_t n, double mean, uint64_t seed, uint32_t *offsets, uint64_t cap);

/* ---- map-reductions (dot, norms) ---- */
uint32_t hxo_dot_u32(const uint32_t *a, const uint32_t *b, uint64_t n);
double hxo_dot_f32(const float *a, const float *b, uint64_t n, double *abs_sum);
uint32_t hxo_norm_l1_i32(const int32_t *x, uint64_t n);
double hxo_norm_l1_f32(const float *x, uint64_t n);
double hxo_sum_squares_f32(const float *x, uint64_t n);
int32_t hxo_norm_max_i32(const int32_t *x, uint64_t n);
float hxo_norm_max_f32(const float *x, uint64_t n);
void hxo_fma_arrays(const float *x, const float *y, float f, uint64_t n, float *out);

/* ---- CPU baselines on all cores (timed, not checkers; each pinned against
 * the sequential functions above by tests/test_oracle.py) ----
 * f32 sum: plain f64 partial per thread, partials added in thread order. */
double hxo_sum_f32_threads(const float *x, uint64_t n, int threads);
/* u32 exclusive scan: chunk totals, then each chunk rescanned from its carry. */
void hxo_scan_excl_u32_threads(const uint32_t *x, uint64_t n, uint32_t *out, int threads);
/* hxo_rows_f32 over contiguous row ranges (bit-identical to it). */
void hxo_rows_f32_threads(const float *x, uint64_t rows, uint64_t cols, uint64_t ld, const hxo_affine *pro,
                          double *sum, double *abs_sum, float *max, uint32_t *argmax, int threads);
/* hxo_segmented_sum_u32 over contiguous segment ranges (bit-identical). */
void hxo_segmented_sum_u32_threads(const uint32_t *x, uint64_t n, const uint32_t *offsets, uint64_t segments,
                                   uint32_t *out, int threads);
/* Forward inclusive f32 scan: f64 chunk totals and carries, f64 running sum
 * rounded to f32 per element. */
void hxo_scan_incl_f32_threads(const float *x, uint64_t n, float *out, int threads);

#ifdef __cplusplus
}
#endif

#endif /* HX_ORACLE_H */
