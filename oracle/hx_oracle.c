/*
 * hx_oracle.c — CPU oracle for the reduction / scan path (TEST
 * INFRASTRUCTURE ONLY; see hx_oracle.h).  Plain sequential folds, written
 * directly from the semantics rather than from the GPU kernels: floats are
 * compared with C relational operators (not the kernels' integer keys),
 * sums use compensated f64 accumulation, and integer arithmetic is done in
 * uint32_t so it wraps mod 2^32.
 */
#define _GNU_SOURCE
#include "hx_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------ generator */

/* SplitMix64 (Steele, Lea, Flood, OOPSLA 2014; Vigna's splitmix64.c):
 * output i of the stream seeded with `seed`. */
uint64_t hxo_splitmix64_at(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1u) * UINT64_C(0x9E3779B97F4A7C15);
    z = (z ^ (z >> 30)) * UINT64_C(0xBF58476D1CE4E5B9);
    z = (z ^ (z >> 27)) * UINT64_C(0x94D049BB133111EB);
    return z ^ (z >> 31);
}

void hxo_fill_uniform_int(uint32_t *dst, uint64_t n, uint64_t seed, int64_t lo, int64_t hi) {
    const uint64_t range = (uint64_t)(hi - lo) + 1u;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t h = hxo_splitmix64_at(seed, i);
        dst[i] = (uint32_t)(lo + (int64_t)(((h >> 32) * range) >> 32));
    }
}

void hxo_fill_uniform_real(float *dst, uint64_t n, uint64_t seed, float lo, float hi) {
    const float width = (float)((double)hi - (double)lo);
    for (uint64_t i = 0; i < n; ++i) {
        const float u = (float)(hxo_splitmix64_at(seed, i) >> 40) * 0x1.0p-24f;
        dst[i] = fmaf(width, u, lo);
    }
}

void hxo_fill_normal(float *dst, uint64_t n, uint64_t seed, double mean, double stddev) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t h1 = hxo_splitmix64_at(seed, 2 * i);
        const uint64_t h2 = hxo_splitmix64_at(seed, 2 * i + 1);
        const double u1 = (double)((h1 >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(h2 >> 11) * 0x1.0p-53;
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = (float)(mean + stddev * z);
    }
}

/* ------------------------------------------------------------- helpers */

static float apply(const hxo_affine *pro, float x) {
    return (pro && pro->enabled) ? fmaf(pro->a, x, pro->b) : x;
}

/* IEEE total order on non-NaN floats: a > b, or both zero with a = +0 and
 * b = -0. */
static int f_greater(float a, float b) {
    if (a > b) return 1;
    if (a == b && a == 0.0f && signbit(b) && !signbit(a)) return 1;
    return 0;
}

/* Neumaier compensated accumulator.  Terms here are f32 values (or exact
 * products of two), so a finite set of them never overflows the f64 running
 * sum: a non-finite running sum means an infinity or a NaN among the terms,
 * and is then the IEEE sum itself (+inf, -inf, or NaN for a NaN or for
 * infinities of both signs).  The compensation is NaN from the first
 * infinity on (inf - inf) and is not added then. */
typedef struct {
    double s, c;
} kacc;
static void kadd(kacc *k, double v) {
    const double t = k->s + v;
    if (fabs(k->s) >= fabs(v)) k->c += (k->s - t) + v;
    else k->c += (v - t) + k->s;
    k->s = t;
}
static double kval(const kacc *k) { return isfinite(k->s) ? k->s + k->c : k->s; }

/* --------------------------------------------------- map-reductions
 * crates/hephaestus-rocm/src/application/linalg/norms.rs:32-490: DotMap
 * "lhs * rhs", AbsMap "abs(lhs)", SquareMap + sqrt, MaxAbsMap with MaxOp.
 * Integer forms wrap mod 2^32 (abs(INT_MIN) = INT_MIN as in C); f32 forms
 * return the compensated f64 value of the exact mapped terms, together with
 * the sum of their magnitudes for the error bound. */

uint32_t hxo_dot_u32(const uint32_t *a, const uint32_t *b, uint64_t n) {
    uint32_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

double hxo_dot_f32(const float *a, const float *b, uint64_t n, double *abs_sum) {
    kacc s = {0, 0}, m = {0, 0};
    for (uint64_t i = 0; i < n; ++i) {
        const double t = (double)a[i] * (double)b[i]; /* exact in f64 */
        kadd(&s, t);
        kadd(&m, fabs(t));
    }
    if (abs_sum) *abs_sum = kval(&m);
    return kval(&s);
}

static uint32_t wrap_abs_i32(int32_t x) { return x < 0 ? 0u - (uint32_t)x : (uint32_t)x; }

uint32_t hxo_norm_l1_i32(const int32_t *x, uint64_t n) {
    uint32_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += wrap_abs_i32(x[i]);
    return s;
}

double hxo_norm_l1_f32(const float *x, uint64_t n) {
    kacc s = {0, 0};
    for (uint64_t i = 0; i < n; ++i) kadd(&s, fabs((double)x[i]));
    return kval(&s);
}

/* sum of squares (exact terms), compensated; the caller takes the root. */
double hxo_sum_squares_f32(const float *x, uint64_t n) {
    kacc s = {0, 0};
    for (uint64_t i = 0; i < n; ++i) kadd(&s, (double)x[i] * (double)x[i]);
    return kval(&s);
}

int32_t hxo_norm_max_i32(const int32_t *x, uint64_t n) {
    int32_t m = INT32_MIN; /* MaxOp identity */
    for (uint64_t i = 0; i < n; ++i) {
        const int32_t a = (int32_t)wrap_abs_i32(x[i]);
        if (a > m) m = a;
    }
    return m;
}

float hxo_norm_max_f32(const float *x, uint64_t n) {
    float m = -FLT_MAX; /* f32::MIN */
    for (uint64_t i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (!isnan(a) && a > m) m = a;
    }
    return m;
}

/* out[i] = fmaf(f, x[i], y[i]) (C99 fmaf, one rounding): axpy is
 * (x, y) = (source, target), xpay (target, source); rocm vector.rs:36-72. */
void hxo_fma_arrays(const float *x, const float *y, float f, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = fmaf(f, x[i], y[i]);
}

/* ------------------------------------------------------ full reductions */

uint32_t hxo_sum_u32(const uint32_t *x, uint64_t n) {
    uint32_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += x[i];
    return s;
}

uint32_t hxo_prod_u32(const uint32_t *x, uint64_t n) {
    uint32_t p = 1;
    for (uint64_t i = 0; i < n; ++i) p *= x[i];
    return p;
}

double hxo_sum_f32(const float *x, uint64_t n, const hxo_affine *pro, double *abs_sum) {
    kacc s = {0, 0}, a = {0, 0};
    for (uint64_t i = 0; i < n; ++i) {
        const double y = (double)apply(pro, x[i]);
        kadd(&s, y);
        kadd(&a, fabs(y));
    }
    if (abs_sum) *abs_sum = kval(&a);
    return kval(&s);
}

uint32_t hxo_max_u32(const uint32_t *x, uint64_t n) {
    uint32_t m = 0;
    for (uint64_t i = 0; i < n; ++i)
        if (x[i] > m) m = x[i];
    return m;
}

int32_t hxo_max_i32(const int32_t *x, uint64_t n) {
    int32_t m = INT32_MIN;
    for (uint64_t i = 0; i < n; ++i)
        if (x[i] > m) m = x[i];
    return m;
}

float hxo_max_f32(const float *x, uint64_t n, const hxo_affine *pro) {
    float m = -FLT_MAX; /* f32::MIN */
    for (uint64_t i = 0; i < n; ++i) {
        const float y = apply(pro, x[i]);
        if (!isnan(y) && f_greater(y, m)) m = y;
    }
    return m;
}

uint32_t hxo_min_u32(const uint32_t *x, uint64_t n) {
    uint32_t m = UINT32_MAX;
    for (uint64_t i = 0; i < n; ++i)
        if (x[i] < m) m = x[i];
    return m;
}

int32_t hxo_min_i32(const int32_t *x, uint64_t n) {
    int32_t m = INT32_MAX;
    for (uint64_t i = 0; i < n; ++i)
        if (x[i] < m) m = x[i];
    return m;
}

float hxo_min_f32(const float *x, uint64_t n, const hxo_affine *pro) {
    float m = FLT_MAX;
    for (uint64_t i = 0; i < n; ++i) {
        const float y = apply(pro, x[i]);
        if (!isnan(y) && f_greater(m, y)) m = y;
    }
    return m;
}

uint32_t hxo_argmax_u32(const uint32_t *x, uint64_t n) {
    uint32_t best = UINT32_MAX;
    for (uint64_t i = 0; i < n; ++i)
        if (best == UINT32_MAX || x[i] > x[best]) best = (uint32_t)i;
    return best;
}

uint32_t hxo_argmax_i32(const int32_t *x, uint64_t n) {
    uint32_t best = UINT32_MAX;
    for (uint64_t i = 0; i < n; ++i)
        if (best == UINT32_MAX || x[i] > x[best]) best = (uint32_t)i;
    return best;
}

uint32_t hxo_argmax_f32(const float *x, uint64_t n, const hxo_affine *pro) {
    uint32_t best = UINT32_MAX;
    float bv = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        const float y = apply(pro, x[i]);
        if (isnan(y)) continue;
        if (best == UINT32_MAX || f_greater(y, bv)) {
            best = (uint32_t)i;
            bv = y;
        }
    }
    return best;
}

/* ------------------------------------------------------------ row-wise */

void hxo_rows_f32(const float *x, uint64_t rows, uint64_t cols, uint64_t ld, const hxo_affine *pro,
                  double *sum, double *abs_sum, float *max, uint32_t *argmax) {
    for (uint64_t r = 0; r < rows; ++r) {
        const float *row = x + r * ld;
        double as = 0.0;
        const double s = hxo_sum_f32(row, cols, pro, &as);
        if (sum) sum[r] = s;
        if (abs_sum) abs_sum[r] = as;
        if (max) max[r] = hxo_max_f32(row, cols, pro);
        if (argmax) argmax[r] = hxo_argmax_f32(row, cols, pro);
    }
}

void hxo_rows_u32(const uint32_t *x, uint64_t rows, uint64_t cols, uint64_t ld, uint32_t *sum,
                  uint32_t *max, uint32_t *argmax) {
    for (uint64_t r = 0; r < rows; ++r) {
        const uint32_t *row = x + r * ld;
        if (sum) sum[r] = hxo_sum_u32(row, cols);
        if (max) max[r] = hxo_max_u32(row, cols);
        if (argmax) argmax[r] = hxo_argmax_u32(row, cols);
    }
}

void hxo_rows_i32(const int32_t *x, uint64_t rows, uint64_t cols, uint64_t ld, int32_t *sum,
                  int32_t *max, uint32_t *argmax) {
    for (uint64_t r = 0; r < rows; ++r) {
        const int32_t *row = x + r * ld;
        if (sum) sum[r] = (int32_t)hxo_sum_u32((const uint32_t *)row, cols);
        if (max) max[r] = hxo_max_i32(row, cols);
        if (argmax) argmax[r] = hxo_argmax_i32(row, cols);
    }
}

/* --------------------------------------------------------------- scans */

void hxo_scan_sum_u32(const uint32_t *x, uint64_t n, int exclusive, int reverse, uint32_t *out) {
    uint32_t acc = 0;
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t i = reverse ? n - 1 - k : k;
        if (exclusive) {
            out[i] = acc;
            acc += x[i];
        } else {
            acc += x[i];
            out[i] = acc;
        }
    }
}

void hxo_scan_prod_u32(const uint32_t *x, uint64_t n, int exclusive, int reverse, uint32_t *out) {
    uint32_t acc = 1;
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t i = reverse ? n - 1 - k : k;
        if (exclusive) {
            out[i] = acc;
            acc *= x[i];
        } else {
            acc *= x[i];
            out[i] = acc;
        }
    }
}

void hxo_scan_sum_f32(const float *x, uint64_t n, int exclusive, int reverse, double *ref,
                      double *abs_prefix) {
    kacc s = {0, 0}, a = {0, 0};
    for (uint64_t k = 0; k < n; ++k) {
        const uint64_t i = reverse ? n - 1 - k : k;
        if (exclusive) {
            ref[i] = kval(&s);
            if (abs_prefix) abs_prefix[i] = kval(&a);
        }
        kadd(&s, (double)x[i]);
        kadd(&a, fabs((double)x[i]));
        if (!exclusive) {
            ref[i] = kval(&s);
            if (abs_prefix) abs_prefix[i] = kval(&a);
        }
    }
}

uint32_t hxo_ceil_log2(uint64_t n) {
    uint32_t l = 0;
    while (l < 64 && (UINT64_C(1) << l) < n) ++l;
    return l;
}

uint64_t hxo_check_f32_bound(const float *got, const double *ref, const double *abs_prefix, uint64_t m,
                             uint64_t n_for_log, double *worst) {
    const double eps = 0x1.0p-23;
    const double k = 2.0 * (double)hxo_ceil_log2(n_for_log) * eps;
    uint64_t bad = 0;
    double w = 0.0;
    for (uint64_t i = 0; i < m; ++i) {
        const double err = fabs((double)got[i] - ref[i]);
        if (!(err <= k * abs_prefix[i])) ++bad; /* NaN counts as a violation */
        if (abs_prefix[i] > 0) {
            const double r = err / (eps * abs_prefix[i]);
            if (r > w) w = r;
        } else if (err > 0) {
            w = INFINITY;
        }
    }
    if (worst) *worst = w;
    return bad;
}

uint64_t hxo_check_scan_f32(const float *x, const float *got, uint64_t n, int exclusive,
                            uint64_t n_for_log, double *worst) {
    const double eps = 0x1.0p-23;
    const double k = 2.0 * (double)hxo_ceil_log2(n_for_log) * eps;
    kacc s = {0, 0}, a = {0, 0};
    uint64_t bad = 0;
    double w = 0.0;
    for (uint64_t i = 0; i < n; ++i) {
        if (!exclusive) {
            kadd(&s, (double)x[i]);
            kadd(&a, fabs((double)x[i]));
        }
        const double ref = kval(&s), ab = kval(&a);
        const double err = fabs((double)got[i] - ref);
        if (!(err <= k * ab)) ++bad;
        if (ab > 0) {
            const double r = err / (eps * ab);
            if (r > w) w = r;
        } else if (err > 0) {
            w = INFINITY;
        }
        if (exclusive) {
            kadd(&s, (double)x[i]);
            kadd(&a, fabs((double)x[i]));
        }
    }
    if (worst) *worst = w;
    return bad;
}

/* ------------------------------------------------------- segmented sum */

void hxo_segmented_sum_u32(const uint32_t *x, uint64_t n, const uint32_t *offsets, uint64_t segments,
                           uint32_t *out) {
    for (uint64_t s = 0; s < segments; ++s) {
        uint64_t a = offsets[s], b = offsets[s + 1];
        if (a > n) a = n;
        if (b > n) b = n;
        uint32_t acc = 0;
        for (uint64_t k = a; k < b; ++k) acc += x[k];
        out[s] = acc;
    }
}

uint64_t hxo_geometric_offsets(uint64_t n, double mean, uint64_t seed, uint32_t *offsets, uint64_t cap) {
    /* length = 1 + floor(ln u / ln(1 - 1/mean)), u in (0, 1]: a geometric
     * number of failures plus one, so min 1 and mean `mean`. */
    const double lq = log1p(-1.0 / mean);
    uint64_t s = 0, pos = 0;
    if (cap == 0) return 0;
    offsets[0] = 0;
    while (pos < n && s + 1 < cap) {
        const uint64_t h = hxo_splitmix64_at(seed, s);
        const double u = (double)((h >> 11) + 1) * 0x1.0p-53;
        uint64_t len = 1 + (uint64_t)floor(log(u) / lq);
        if (len > n - pos) len = n - pos;
        pos += len;
        offsets[++s] = (uint32_t)pos;
    }
    return s;
}

/* ------------------------------------------------------- CPU baselines */

typedef struct {
    const float *xf;
    const uint32_t *xu;
    uint32_t *out;
    uint64_t lo, hi;
    double dsum;
    uint32_t usum, offset;
} job_t;

static void *sum_job(void *arg) {
    job_t *j = (job_t *)arg;
    double s = 0.0;
    for (uint64_t i = j->lo; i < j->hi; ++i) s += (double)j->xf[i];
    j->dsum = s;
    return NULL;
}

double hxo_sum_f32_threads(const float *x, uint64_t n, int threads) {
    if (threads < 1) threads = 1;
    job_t *jobs = calloc((size_t)threads, sizeof(job_t));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        jobs[t].xf = x;
        jobs[t].lo = n * (uint64_t)t / (uint64_t)threads;
        jobs[t].hi = n * (uint64_t)(t + 1) / (uint64_t)threads;
        pthread_create(&tid[t], NULL, sum_job, &jobs[t]);
    }
    double s = 0.0;
    for (int t = 0; t < threads; ++t) {
        pthread_join(tid[t], NULL);
        s += jobs[t].dsum;
    }
    free(jobs);
    free(tid);
    return s;
}

static void *usum_job(void *arg) {
    job_t *j = (job_t *)arg;
    uint32_t s = 0;
    for (uint64_t i = j->lo; i < j->hi; ++i) s += j->xu[i];
    j->usum = s;
    return NULL;
}

static void *uscan_job(void *arg) {
    job_t *j = (job_t *)arg;
    uint32_t acc = j->offset;
    for (uint64_t i = j->lo; i < j->hi; ++i) {
        j->out[i] = acc;
        acc += j->xu[i];
    }
    return NULL;
}

void hxo_scan_excl_u32_threads(const uint32_t *x, uint64_t n, uint32_t *out, int threads) {
    if (threads < 1) threads = 1;
    job_t *jobs = calloc((size_t)threads, sizeof(job_t));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        jobs[t].xu = x;
        jobs[t].out = out;
        jobs[t].lo = n * (uint64_t)t / (uint64_t)threads;
        jobs[t].hi = n * (uint64_t)(t + 1) / (uint64_t)threads;
        pthread_create(&tid[t], NULL, usum_job, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    uint32_t run = 0;
    for (int t = 0; t < threads; ++t) {
        jobs[t].offset = run;
        run += jobs[t].usum;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tid[t], NULL, uscan_job, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
}

/* All-core forms of the remaining baselines: the same per-element
 * arithmetic as the sequential functions above, split over `threads`
 * pthreads by contiguous ranges. */

typedef struct {
    const float *x;
    uint64_t rows, cols, ld;
    const hxo_affine *pro;
    double *sum, *abs_sum;
    float *max;
    uint32_t *argmax;
    uint64_t lo, hi;
} rows_job_t;

static void *rows_job(void *arg) {
    rows_job_t *j = (rows_job_t *)arg;
    hxo_rows_f32(j->x + j->lo * j->ld, j->hi - j->lo, j->cols, j->ld, j->pro, j->sum ? j->sum + j->lo : NULL,
                 j->abs_sum ? j->abs_sum + j->lo : NULL, j->max ? j->max + j->lo : NULL,
                 j->argmax ? j->argmax + j->lo : NULL);
    return NULL;
}

void hxo_rows_f32_threads(const float *x, uint64_t rows, uint64_t cols, uint64_t ld, const hxo_affine *pro,
                          double *sum, double *abs_sum, float *max, uint32_t *argmax, int threads) {
    if (threads < 1) threads = 1;
    rows_job_t *jobs = calloc((size_t)threads, sizeof(rows_job_t));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (rows_job_t){x, rows, cols, ld, pro, sum, abs_sum, max, argmax,
                               rows * (uint64_t)t / (uint64_t)threads, rows * (uint64_t)(t + 1) / (uint64_t)threads};
        pthread_create(&tid[t], NULL, rows_job, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
}

typedef struct {
    const uint32_t *x;
    uint64_t n;
    const uint32_t *offsets;
    uint32_t *out;
    uint64_t lo, hi; /* segment range */
} seg_job_t;

static void *seg_job(void *arg) {
    seg_job_t *j = (seg_job_t *)arg;
    hxo_segmented_sum_u32(j->x, j->n, j->offsets + j->lo, j->hi - j->lo, j->out + j->lo);
    return NULL;
}

void hxo_segmented_sum_u32_threads(const uint32_t *x, uint64_t n, const uint32_t *offsets, uint64_t segments,
                                   uint32_t *out, int threads) {
    if (threads < 1) threads = 1;
    seg_job_t *jobs = calloc((size_t)threads, sizeof(seg_job_t));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        jobs[t] = (seg_job_t){x, n, offsets, out, segments * (uint64_t)t / (uint64_t)threads,
                              segments * (uint64_t)(t + 1) / (uint64_t)threads};
        pthread_create(&tid[t], NULL, seg_job, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
}

typedef struct {
    const float *x;
    float *out;
    uint64_t lo, hi;
    double total, carry;
} fscan_job_t;

static void *fsum_job(void *arg) {
    fscan_job_t *j = (fscan_job_t *)arg;
    double s = 0.0;
    for (uint64_t i = j->lo; i < j->hi; ++i) s += (double)j->x[i];
    j->total = s;
    return NULL;
}

static void *fscan_job(void *arg) {
    fscan_job_t *j = (fscan_job_t *)arg;
    double run = j->carry;
    for (uint64_t i = j->lo; i < j->hi; ++i) {
        run += (double)j->x[i];
        j->out[i] = (float)run;
    }
    return NULL;
}

/* Forward inclusive f32 scan on all cores: chunk totals in f64, their
 * exclusive prefix as each chunk's carry, then each chunk's running f64 sum
 * rounded to f32 per element (a reduce-then-scan, the usual CPU form). */
void hxo_scan_incl_f32_threads(const float *x, uint64_t n, float *out, int threads) {
    if (threads < 1) threads = 1;
    fscan_job_t *jobs = calloc((size_t)threads, sizeof(fscan_job_t));
    pthread_t *tid = calloc((size_t)threads, sizeof(pthread_t));
    for (int t = 0; t < threads; ++t) {
        jobs[t].x = x;
        jobs[t].out = out;
        jobs[t].lo = n * (uint64_t)t / (uint64_t)threads;
        jobs[t].hi = n * (uint64_t)(t + 1) / (uint64_t)threads;
        pthread_create(&tid[t], NULL, fsum_job, &jobs[t]);
    }
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    double run = 0.0;
    for (int t = 0; t < threads; ++t) {
        jobs[t].carry = run;
        run += jobs[t].total;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tid[t], NULL, fscan_job, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
    free(jobs);
    free(tid);
}
