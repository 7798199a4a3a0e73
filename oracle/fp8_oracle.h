/*
 * fp8_oracle.h - CPU restatement of reng-fp8's host quantizer.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
 * compared against, and the CPU baseline that bench.py times beside it. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product library (libreng_hip.so) never links, loads or calls it.
 *
 * Every function restates crates/reng-fp8/src/lib.rs (file:line given on
 * each) or crates/reng-model/src/bin/fp8_probe.rs. It is built with gcc -O2
 * for x86-64 without -ffast-math and with -ffp-contract=off, so an f32
 * division is one IEEE `divss`, exactly as the Rust build of the reference
 * does it (an invalid division such as inf/inf yields x86's negative
 * default NaN).
 *
 * Pinning: every function is checked by tests/test_oracle.py against the
 * reference's golden vectors (tests/golden/fp8_cast.json), its known-answer
 * tests, torch's float8 casts, an independent nearest-value search, and
 * closed forms. See the header of that file for which check pins which
 * function.
 */
#ifndef FP8_ORACLE_H
#define FP8_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Formats and scale schemes use the same integer values as include/reng_hip.h. */
enum { ORC_E4M3 = 0, ORC_E5M2 = 1 };
enum { ORC_PCS = 0, ORC_HW = 1, ORC_UNIT = 2 };

float orc_bf16_to_f32(uint16_t x);
uint16_t orc_f32_to_bf16(float x);
uint32_t orc_mantissa_bits(int fmt);
uint32_t orc_exponent_bias(int fmt);
uint8_t orc_max_finite_code(int fmt);
float orc_max_finite(int fmt);
float orc_pow2(int e);

uint8_t orc_encode(float x, int fmt);
float orc_decode(uint8_t code, int fmt);
uint32_t orc_choose_exp_bias(float absmax, int fmt);
int orc_split(size_t rows, size_t cols);

/* Array helpers (max_threads <= 0 means 1). */
void orc_encode_array(const float *x, size_t n, int fmt, uint8_t *out, int max_threads);
void orc_encode_bits_range(uint64_t first, uint64_t count, int fmt, uint8_t *out, int max_threads);
void orc_decode_array(const uint8_t *c, size_t n, int fmt, float *out);

void orc_row_absmax(const uint16_t *w, size_t rows, size_t cols, float *out);

/* quantize_with: bf16 [rows, cols] row-major -> codes [rows*cols], scales
 * [rows]; returns exp_bias. thread_cap is the reference's 8 (lib.rs:568);
 * a larger cap gives the "all cores" line, which is not reference behaviour. */
uint32_t orc_quantize_with(const uint16_t *w, size_t rows, size_t cols, int fmt, int scaling,
                           float backoff, uint8_t *codes, float *scales, int thread_cap);
/* The same semantics with f32 elements in place of bf16_to_f32(b). */
uint32_t orc_quantize_f32_with(const float *w, size_t rows, size_t cols, int fmt, int scaling,
                               float backoff, uint8_t *codes, float *scales, int thread_cap);

void orc_dequantize(const uint8_t *codes, const float *scales, size_t rows, size_t cols, int fmt,
                    float *out);
void orc_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales, size_t rows,
                    size_t cols, int fmt, float *mean_rel, float *max_rel);
/* Returns the number of sampled rows written. */
size_t orc_sample_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales,
                             size_t rows, size_t cols, int fmt, size_t max_rows,
                             float *mean_rel, float *max_rel);

/* gemm_cpu: c[m, n] = sum_t a[m, t] * b[n, t], f32, sequential in t. */
void orc_gemm(const float *a, const float *b, size_t m, size_t k, size_t n, float *c,
              int max_threads);
/* The same for a subset of output columns (rows of b): c[m, j] for j in cols_idx. */
void orc_gemm_cols(const float *a, const float *b, size_t m, size_t k, const int64_t *cols_idx,
                   size_t ncols, float *c, int max_threads);
float orc_rel_l2(const float *got, const float *want, size_t n);

#ifdef __cplusplus
}
#endif
#endif
