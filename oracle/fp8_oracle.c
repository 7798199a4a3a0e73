/*
 * fp8_oracle.c - CPU restatement of reng-fp8 (crates/reng-fp8/src/lib.rs).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the CPU baseline
 * of bench.py. Nothing in the product library calls it. See fp8_oracle.h.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no -ffast-math, x86-64
 * baseline ISA so no FMA can be formed).
 */
#include "fp8_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* lib.rs:35-37 */
float orc_bf16_to_f32(uint16_t x) { return u2f((uint32_t)x << 16); }

/* lib.rs:41-48: RNE via +0x7fff+lsb, NaN -> 0x7fc0. */
uint16_t orc_f32_to_bf16(float x) {
    uint32_t bits = f2u(x);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    uint32_t round_bias = 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)((bits + round_bias) >> 16);
}

/* lib.rs:63-68 */
uint32_t orc_mantissa_bits(int fmt) { return fmt == ORC_E4M3 ? 3u : 2u; }
/* lib.rs:72-74 */
static uint32_t exponent_bits(int fmt) { return 8u - 1u - orc_mantissa_bits(fmt); }
/* lib.rs:79-84 */
uint32_t orc_exponent_bias(int fmt) { return fmt == ORC_E4M3 ? 7u : 15u; }
/* lib.rs:90-94 */
uint8_t orc_max_finite_code(int fmt) {
    uint32_t mbits = orc_mantissa_bits(fmt);
    uint32_t exp_field = ((1u << exponent_bits(fmt)) - 2u) << mbits;
    return (uint8_t)(exp_field | ((1u << mbits) - 1u));
}
/* lib.rs:98-100 */
float orc_max_finite(int fmt) { return orc_decode(orc_max_finite_code(fmt), fmt); }

/* lib.rs:229-236: exact 2^e for -149..=127. */
float orc_pow2(int e) {
    if (e >= -126) return u2f((uint32_t)(e + 127) << 23);
    return u2f(1u << (e + 149));
}

/* lib.rs:154-201 */
uint8_t orc_encode(float x, int fmt) {
    uint8_t sign = (f2u(x) >> 31) ? 0x80 : 0x00;          /* is_sign_negative, :155 */
    if (isnan(x)) return sign | 0x7f;                      /* :156-158 */
    uint32_t bits = f2u(x) & 0x7fffffffu;                  /* :159 */
    if ((bits >> 23) == 0) return sign;                    /* zero and f32 subnormal, :162-164 */
    float a = u2f(bits);
    int mbits = (int)orc_mantissa_bits(fmt);
    int bias = (int)orc_exponent_bias(fmt);
    int emin = 1 - bias;                                   /* :171 */
    int emax = ((1 << exponent_bits(fmt)) - 2) - bias;     /* :172 */
    int e = (int)(bits >> 23) - 127;                       /* :173 */
    if (e > emax) return sign | orc_max_finite_code(fmt);  /* :174-177 */
    int emx = e > emin ? e : emin;
    int quantum_exp = emx - mbits;                         /* :178 */
    /* :181, exact quotient then round_ties_even (rintf under FE_TONEAREST). */
    uint32_t n = (uint32_t)rintf(a / orc_pow2(quantum_exp));
    int e_eff = emx;                                       /* :182 */
    if (n >= (2u << mbits)) {                              /* :185-188 */
        n >>= 1;
        e_eff += 1;
    }
    if (e_eff > emax) return sign | orc_max_finite_code(fmt); /* :189-191 */
    uint32_t code;
    if (e < emin)                                          /* :192-199 */
        code = n;
    else
        code = ((uint32_t)(e_eff + bias) << mbits) | (n - (1u << mbits));
    return (uint8_t)(sign | (uint8_t)code);
}

/* lib.rs:206-225 */
float orc_decode(uint8_t code, int fmt) {
    uint32_t mbits = orc_mantissa_bits(fmt);
    int bias = (int)orc_exponent_bias(fmt);
    float sign = (code & 0x80) == 0 ? 1.0f : -1.0f;
    uint32_t mant = (uint32_t)code & ((1u << mbits) - 1u);
    uint32_t exp_field = ((uint32_t)code & 0x7fu) >> mbits;
    if (exp_field == (1u << exponent_bits(fmt)) - 1u) {
        return mant == 0 ? sign * INFINITY : NAN;
    }
    float frac = (float)mant / (float)(1u << mbits);
    if (exp_field == 0) return sign * frac * orc_pow2(1 - bias);
    return sign * (1.0f + frac) * orc_pow2((int)exp_field - bias);
}

/* lib.rs:122-127 */
static const uint32_t HW_E4M3[4] = {15, 11, 7, 3};
static const uint32_t HW_E5M2[1] = {15};

/* lib.rs:466-475 */
uint32_t orc_choose_exp_bias(float absmax, int fmt) {
    const uint32_t *biases = fmt == ORC_E4M3 ? HW_E4M3 : HW_E5M2;
    size_t nb = fmt == ORC_E4M3 ? 4 : 1;
    int def = (int)orc_exponent_bias(fmt);
    for (size_t i = 0; i < nb; i++) {
        if (absmax <= orc_max_finite(fmt) * orc_pow2(def - (int)biases[i])) return biases[i];
    }
    return biases[nb - 1];
}

/* lib.rs:567-572, with the thread cap as a parameter (8 in the reference). */
static int split_cap(size_t rows, size_t cols, int cap) {
    const size_t PER_THREAD = (size_t)1 << 20;
    size_t by_size = (rows * cols + PER_THREAD - 1) / PER_THREAD;
    if (by_size < 1) by_size = 1;
    size_t t = by_size < (size_t)cap ? by_size : (size_t)cap;
    if (t > rows) t = rows;
    return (int)t;
}
int orc_split(size_t rows, size_t cols) { return split_cap(rows, cols, 8); }

/* ---- a tiny scoped-thread helper (std::thread::scope in the reference) ---- */
typedef void (*range_fn)(void *ctx, size_t r0, size_t r1);
typedef struct { range_fn fn; void *ctx; size_t r0, r1; } job_t;
static void *job_main(void *p) { job_t *j = (job_t *)p; j->fn(j->ctx, j->r0, j->r1); return NULL; }

/* Chunks of ceil(rows / threads) rows, the last one ragged (lib.rs:581-587). */
static void run_chunks(size_t rows, int threads, range_fn fn, void *ctx) {
    if (threads <= 1) { fn(ctx, 0, rows); return; }
    size_t chunk = (rows + (size_t)threads - 1) / (size_t)threads;
    size_t nparts = (rows + chunk - 1) / chunk;
    pthread_t *tid = (pthread_t *)calloc(nparts, sizeof(pthread_t));
    job_t *jobs = (job_t *)calloc(nparts, sizeof(job_t));
    for (size_t i = 0; i < nparts; i++) {
        size_t r0 = i * chunk, r1 = r0 + chunk < rows ? r0 + chunk : rows;
        jobs[i] = (job_t){fn, ctx, r0, r1};
        if (pthread_create(&tid[i], NULL, job_main, &jobs[i]) != 0) {
            job_main(&jobs[i]);
            tid[i] = 0;
        }
    }
    for (size_t i = 0; i < nparts; i++) if (tid[i]) pthread_join(tid[i], NULL);
    free(tid);
    free(jobs);
}

/* ---- element loaders: bf16 (the reference) or f32 (C1's input) ---- */
typedef struct {
    const void *w; int is_f32; size_t cols; int fmt;
    float *absmax; const float *scales; uint8_t *codes;
} qctx_t;

static inline float elem(const qctx_t *c, size_t i) {
    return c->is_f32 ? ((const float *)c->w)[i] : orc_bf16_to_f32(((const uint16_t *)c->w)[i]);
}

/* lib.rs:447-458: `v > m` ignores NaN, counts inf. */
static void absmax_range(void *p, size_t r0, size_t r1) {
    qctx_t *c = (qctx_t *)p;
    for (size_t r = r0; r < r1; r++) {
        float m = 0.0f;
        for (size_t j = 0; j < c->cols; j++) {
            float v = fabsf(elem(c, r * c->cols + j));
            if (v > m) m = v;
        }
        c->absmax[r] = m;
    }
}

/* lib.rs:591-601: division, not a reciprocal multiply. */
static void encode_range(void *p, size_t r0, size_t r1) {
    qctx_t *c = (qctx_t *)p;
    for (size_t r = r0; r < r1; r++) {
        float s = c->scales[r];
        for (size_t j = 0; j < c->cols; j++) {
            size_t i = r * c->cols + j;
            c->codes[i] = orc_encode(elem(c, i) / s, c->fmt);
        }
    }
}

void orc_row_absmax(const uint16_t *w, size_t rows, size_t cols, float *out) {
    qctx_t c = {w, 0, cols, 0, out, NULL, NULL};
    absmax_range(&c, 0, rows);   /* lib.rs:439-444 is serial */
}

/* lib.rs:519-563 */
static uint32_t quantize_impl(const void *w, int is_f32, size_t rows, size_t cols, int fmt,
                              int scaling, float backoff, uint8_t *codes, float *scales,
                              int thread_cap) {
    if (thread_cap < 1) thread_cap = 1;
    float *absmax = (float *)calloc(rows, sizeof(float));
    qctx_t c = {w, is_f32, cols, fmt, absmax, scales, codes};
    int threads = split_cap(rows, cols, thread_cap);
    run_chunks(rows, threads, absmax_range, &c);           /* :533-534 */
    float full = orc_max_finite(fmt) * backoff;            /* :535 */
    float tensor_absmax = 0.0f;                            /* :536, fold(0.0, f32::max) */
    for (size_t r = 0; r < rows; r++) tensor_absmax = fmaxf(tensor_absmax, absmax[r]);
    uint32_t exp_bias = orc_exponent_bias(fmt);
    if (scaling == ORC_PCS) {                              /* :538-544 */
        for (size_t r = 0; r < rows; r++) scales[r] = absmax[r] > 0.0f ? absmax[r] / full : 1.0f;
    } else if (scaling == ORC_HW) {                        /* :545-549 */
        uint32_t b = orc_choose_exp_bias(tensor_absmax / backoff, fmt);
        float s = orc_pow2((int)orc_exponent_bias(fmt) - (int)b);
        for (size_t r = 0; r < rows; r++) scales[r] = s;
        exp_bias = b;
    } else {                                               /* :550 */
        for (size_t r = 0; r < rows; r++) scales[r] = 1.0f;
    }
    run_chunks(rows, threads, encode_range, &c);           /* :552-553, 604-621 */
    free(absmax);
    return exp_bias;
}

uint32_t orc_quantize_with(const uint16_t *w, size_t rows, size_t cols, int fmt, int scaling,
                           float backoff, uint8_t *codes, float *scales, int thread_cap) {
    return quantize_impl(w, 0, rows, cols, fmt, scaling, backoff, codes, scales, thread_cap);
}

uint32_t orc_quantize_f32_with(const float *w, size_t rows, size_t cols, int fmt, int scaling,
                               float backoff, uint8_t *codes, float *scales, int thread_cap) {
    return quantize_impl(w, 1, rows, cols, fmt, scaling, backoff, codes, scales, thread_cap);
}

/* ---- array helpers for exhaustive checks ---- */
typedef struct { const float *x; uint64_t first; int fmt; uint8_t *out; } ectx_t;
static void enc_arr(void *p, size_t i0, size_t i1) {
    ectx_t *c = (ectx_t *)p;
    for (size_t i = i0; i < i1; i++) c->out[i] = orc_encode(c->x[i], c->fmt);
}
static void enc_bits(void *p, size_t i0, size_t i1) {
    ectx_t *c = (ectx_t *)p;
    for (size_t i = i0; i < i1; i++) c->out[i] = orc_encode(u2f((uint32_t)(c->first + i)), c->fmt);
}
void orc_encode_array(const float *x, size_t n, int fmt, uint8_t *out, int max_threads) {
    ectx_t c = {x, 0, fmt, out};
    run_chunks(n, max_threads < 1 ? 1 : max_threads, enc_arr, &c);
}
void orc_encode_bits_range(uint64_t first, uint64_t count, int fmt, uint8_t *out, int max_threads) {
    ectx_t c = {NULL, first, fmt, out};
    run_chunks((size_t)count, max_threads < 1 ? 1 : max_threads, enc_bits, &c);
}
void orc_decode_array(const uint8_t *c, size_t n, int fmt, float *out) {
    for (size_t i = 0; i < n; i++) out[i] = orc_decode(c[i], fmt);
}

/* lib.rs:328-337 */
void orc_dequantize(const uint8_t *codes, const float *scales, size_t rows, size_t cols, int fmt,
                    float *out) {
    for (size_t r = 0; r < rows; r++) {
        float s = scales[r];
        for (size_t j = 0; j < cols; j++) out[r * cols + j] = orc_decode(codes[r * cols + j], fmt) * s;
    }
}

/* One row of lib.rs:367-386 (shared by row_errors and sample_row_errors). */
static void row_error(const uint16_t *w, const uint8_t *codes, float s, size_t cols, int fmt,
                      float *mean_rel, float *max_rel) {
    double sum = 0.0;
    float mx = 0.0f;
    size_t n = 0;
    for (size_t c = 0; c < cols; c++) {
        float want = orc_bf16_to_f32(w[c]);
        if (want == 0.0f) continue;
        float got = orc_decode(codes[c], fmt) * s;
        float rel = fabsf((got - want) / want);
        sum += (double)rel;
        mx = fmaxf(mx, rel);                /* f32::max ignores NaN */
        n++;
    }
    *mean_rel = n == 0 ? 0.0f : (float)(sum / (double)n);
    *max_rel = mx;
}

/* lib.rs:364-388 */
void orc_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales, size_t rows,
                    size_t cols, int fmt, float *mean_rel, float *max_rel) {
    for (size_t r = 0; r < rows; r++)
        row_error(w + r * cols, codes + r * cols, scales[r], cols, fmt, &mean_rel[r], &max_rel[r]);
}

/* lib.rs:399-431 */
size_t orc_sample_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales,
                             size_t rows, size_t cols, int fmt, size_t max_rows,
                             float *mean_rel, float *max_rel) {
    if (max_rows == 0 || rows == 0) return 0;
    size_t n = max_rows < rows ? max_rows : rows;
    size_t step = (rows + n - 1) / n;
    size_t k = 0;
    for (size_t r = 0; r < rows; r += step, k++)
        row_error(w + r * cols, codes + r * cols, scales[r], cols, fmt, &mean_rel[k], &max_rel[k]);
    return k;
}

/* fp8_probe.rs:55-67, parallel over output rows only (each sum stays sequential). */
typedef struct { const float *a, *b; size_t m, k; const int64_t *idx; size_t ncols; float *c; } gctx_t;
static void gemm_rows(void *p, size_t j0, size_t j1) {
    gctx_t *g = (gctx_t *)p;
    for (size_t row = 0; row < g->m; row++) {
        for (size_t jj = j0; jj < j1; jj++) {
            size_t j = g->idx ? (size_t)g->idx[jj] : jj;
            float acc = 0.0f;
            const float *ar = g->a + row * g->k, *br = g->b + j * g->k;
            for (size_t t = 0; t < g->k; t++) acc += ar[t] * br[t];
            g->c[row * g->ncols + jj] = acc;
        }
    }
}
void orc_gemm(const float *a, const float *b, size_t m, size_t k, size_t n, float *c,
              int max_threads) {
    gctx_t g = {a, b, m, k, NULL, n, c};
    run_chunks(n, max_threads < 1 ? 1 : max_threads, gemm_rows, &g);
}
void orc_gemm_cols(const float *a, const float *b, size_t m, size_t k, const int64_t *cols_idx,
                   size_t ncols, float *c, int max_threads) {
    gctx_t g = {a, b, m, k, cols_idx, ncols, c};
    run_chunks(ncols, max_threads < 1 ? 1 : max_threads, gemm_rows, &g);
}

/* fp8_probe.rs:70-78: the difference is taken in f32, the sums in f64. */
float orc_rel_l2(const float *got, const float *want, size_t n) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < n; i++) {
        double d = (double)(got[i] - want[i]);
        num += d * d;
        den += (double)want[i] * (double)want[i];
    }
    double dd = sqrt(den);
    return (float)(sqrt(num) / (dd > 1e-12 ? dd : 1e-12));
}
