/*
 * reng_hip.h - the C ABI of libreng_hip.so, the MI355X (gfx950) implementation
 * of reng-fp8's per-output-channel FP8 weight quantizer and of the fused
 * fp8-dequant GEMV / GEMM that consumes its codes.
 *
 * Plain C: pointers, sizes and integers only. Every device entry point takes
 * an explicit stream (a hipStream_t passed as void*, NULL = the current
 * device's null stream), is asynchronous on it, and keeps no hidden global
 * stream. Every entry point is callable from any thread. On failure it returns
 * a non-zero status and sets a thread-local message (reng_hip_last_error).
 * There is no CPU fallback: a call that cannot run on the GPU fails.
 *
 * Data layout (the reference's, crates/reng-fp8/src/lib.rs:281-306):
 *   weights  [rows, cols] row-major ([out, in]); bf16 bits or f32; row pitch ld
 *            elements (ld >= cols; ld > cols takes a strided window)
 *   codes    [rows, cols] row-major, one byte per element, pitch cols
 *   scales   [rows] f32, weight[r, c] = decode(codes[r, c]) * scales[r]
 */
#ifndef RENG_HIP_H
#define RENG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RENG_HIP_API __attribute__((visibility("default")))

/* Status codes. */
#define RENG_HIP_OK 0
#define RENG_HIP_EINVAL 1      /* a shape, pointer, enum or backoff the reference would reject */
#define RENG_HIP_EDEVICE 2     /* a HIP runtime error (launch, copy, no device) */
#define RENG_HIP_ENOMEM 3      /* a device or pinned allocation failed */
#define RENG_HIP_EUNSUPPORTED 4

/* Fp8Format (crates/reng-fp8/src/lib.rs:53-58): E4M3 = Gaudi hf8, bias 7, max
 * finite 240 (0x77); E5M2 = f8, bias 15, max finite 57344 (0x7b). */
#define RENG_HIP_E4M3 0
#define RENG_HIP_E5M2 1

/* Scaling (crates/reng-fp8/src/lib.rs:240-256). */
#define RENG_HIP_PCS 0   /* PerChannel: s[r] = absmax[r] / (max_finite * backoff), 1 for a zero row */
#define RENG_HIP_HW 1    /* HwExpBias: one power of two from choose_exp_bias(tensor absmax / backoff) */
#define RENG_HIP_UNIT 2  /* Unit: s = 1 */

/* Element types of weights, activations and outputs. */
#define RENG_HIP_BF16 0
#define RENG_HIP_F32 1

/* Library version string, e.g. "reng-hip 0.1.0 (gfx950)". */
RENG_HIP_API const char *reng_hip_version(void);

/* The message of the last failed call on this thread ("" if none). */
RENG_HIP_API const char *reng_hip_last_error(void);

/* One line describing the current device (name, gfx arch, CUs, HBM bytes,
 * clock) written into buf. */
RENG_HIP_API int reng_hip_device_info(char *buf, size_t len);

/* ---------------------------------------------------------------------------
 * Quantizer
 * ------------------------------------------------------------------------- */

/* reng_fp8::quantize_with (crates/reng-fp8/src/lib.rs:519-563), device-resident.
 * w: dtype [rows, ld] (bf16 bits or f32), the first cols of each row are used.
 * codes: [rows * cols] u8; scales: [rows] f32; exp_bias: optional device u32
 * receiving the exponent bias of the device tensor's metadata (the chosen one
 * for HW, the format's own otherwise). Codes and scales are bit-exact to the
 * reference host quantizer on an x86 host, including NaN (sign | 0x7f), +-inf
 * (saturated; inf inside a per-channel row gives s = inf, so finite entries
 * encode to signed zero and inf/inf to 0xff, x86's negative default NaN) and
 * zero rows (s = 1).
 * Fails with EINVAL where quantize_with panics (lib.rs:527-532): rows or cols
 * zero, backoff not positive and finite; also for ld < cols or NULL pointers. */
RENG_HIP_API int reng_hip_quantize(const void *w, int dtype, size_t rows, size_t cols, size_t ld,
                                   int format, int scaling, float backoff, uint8_t *codes,
                                   float *scales, uint32_t *exp_bias, void *stream);

/* The host-pointer form Rust's `quantize_with` calls: stages through device
 * memory, runs reng_hip_quantize and copies back; synchronous. exp_bias is a
 * host pointer (may be NULL). */
RENG_HIP_API int reng_hip_quantize_host(const void *w, int dtype, size_t rows, size_t cols,
                                        int format, int scaling, float backoff, uint8_t *codes,
                                        float *scales, uint32_t *exp_bias);

/* One matrix of a batch (device pointers); exp_bias may be NULL. */
typedef struct reng_hip_matrix {
    const void *w;
    uint8_t *codes;
    float *scales;
    uint32_t *exp_bias;
    size_t rows, cols, ld;
} reng_hip_matrix;

/* Many matrices, one format / scheme / backoff, as LlamaWeights::quantize_fp8
 * quantizes a layer's seven projections (crates/reng-model/src/lib.rs:1882-1937):
 * each matrix gets exactly what reng_hip_quantize would give it (HW chooses a
 * bias per matrix), in as few launches as the shapes allow. mats is a host
 * array of n descriptors (any n >= 1). */
RENG_HIP_API int reng_hip_quantize_batch(const reng_hip_matrix *mats, size_t n, int dtype,
                                         int format, int scaling, float backoff, void *stream);

/* reng_fp8::row_absmax (lib.rs:439-458): per-row max |w|, NaN ignored, inf counted. */
RENG_HIP_API int reng_hip_row_absmax(const void *w, int dtype, size_t rows, size_t cols, size_t ld,
                                     float *out, void *stream);

/* reng_fp8::choose_exp_bias (lib.rs:466-475), a host function. */
RENG_HIP_API uint32_t reng_hip_choose_exp_bias(float absmax, int format);

/* reng_fp8::encode over an array (lib.rs:154-201): f32 -> code, RNE, saturating,
 * NaN -> sign | 0x7f. */
RENG_HIP_API int reng_hip_encode(const float *x, size_t n, int format, uint8_t *codes, void *stream);

/* reng_fp8::decode over an array (lib.rs:206-225): code -> f32 exactly; the top
 * exponent field is +-inf (mantissa 0) or NaN. */
RENG_HIP_API int reng_hip_decode(const uint8_t *codes, size_t n, int format, float *out, void *stream);

/* Quantized::dequantize / dequantize_bf16 (lib.rs:328-344): out[r, c] =
 * decode(codes[r, c]) * scales[r] as f32, or that rounded to bf16 (RNE). */
RENG_HIP_API int reng_hip_dequantize(const uint8_t *codes, const float *scales, size_t rows,
                                     size_t cols, int format, int out_dtype, void *out, void *stream);

/* reng_fp8::row_errors (max_rows == 0) and sample_row_errors (max_rows > 0)
 * (lib.rs:364-431): mean (f64 sum) and max of |dequant - w| / |w| over the
 * non-zero weights of each (sampled) row; rows sampled every ceil(rows / n),
 * n = min(max_rows, rows). mean_rel and max_rel hold one entry per sampled row. */
RENG_HIP_API int reng_hip_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales,
                                     size_t rows, size_t cols, int format, size_t max_rows,
                                     float *mean_rel, float *max_rel, void *stream);

/* ---------------------------------------------------------------------------
 * Consumer: fused fp8-dequant GEMV / GEMM
 * ------------------------------------------------------------------------- */

/* y[M, N] (bf16, RNE) = x[M, K] (bf16) . (decode(codes[N, K]) * scales[N])^T,
 * f32 accumulation. This is the per-output-channel form of the reference's
 * `fp8_gemm_bf16` complex guid (crates/reng-synapse/src/fp8.rs:278-331) with
 * the bf16 activation the engine wants (the mixed pair gemm_mixed records as
 * refused on Gaudi, fp8.rs:244-276); the CPU semantics are gemm_cpu over
 * Quantized::dequantize (crates/reng-model/src/bin/fp8_probe.rs:55-67).
 * Shapes are row-major: x [M, K], codes [N, K], y [M, N] (the reference's
 * device sizes A [K, m], W [K, N] with transpose_b, out [N, m]).
 * Batches 1..64 use in-register fp8 decode (a GEMV for M = 1, M = 2 with
 * K <= 16384, and M <= 4 when K is not a multiple of 128; bf16 MFMA
 * otherwise); any M is accepted.
 * scales may be NULL (unit scale, the 2-input form).
 * Codes are the quantizer's finite codes; codes of the reserved top exponent
 * field are read as OCP values, not as +-inf/NaN. K must be a multiple of 16. */
RENG_HIP_API int reng_hip_gemm_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales,
                                     size_t M, size_t N, size_t K, int format, uint16_t *y,
                                     void *stream);

/* reng_hip_gemm_w8a16 that allocates nothing: no counterpart in the reference.
 * It is for callers that cannot allocate device memory during the call - code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Same arguments, kernels and results (bit for bit) as
 * reng_hip_gemm_w8a16; the split-K partials of 2 <= M <= 64 products (and of
 * each 64-row tile of a larger M) and the stream-K partials of long-K M > 64
 * products go to a static 32 MiB array in device memory, and the stream-K
 * tile counters to a static array of 4096 counters, that the library holds on
 * each GPU it runs on until the process ends, instead of the grow-only
 * per-stream buffers reng_hip_gemm_w8a16 allocates. A product whose plan needs
 * more is refused (EINVAL); on a 256-CU device the plans need at most 24 MiB.
 * Every call on one GPU shares that GPU's arrays, so calls that overlap on one
 * GPU race: order them on one stream (or otherwise serialize them). */
RENG_HIP_API int reng_hip_gemm_w8a16_noalloc(const uint16_t *x, const uint8_t *codes, const float *scales,
                                             size_t M, size_t N, size_t K, int format, uint16_t *y,
                                             void *stream);

/* gemm_fp8_scaled (crates/reng-synapse/src/fp8.rs:295-331): two fp8 operands
 * and optional f32 scale operands, bf16 out on fp8 MFMA:
 *   out[M, N] = sum_k decode(a[M, k]) * sa[m] * decode(b[N, k]) * sb[n]
 * a [M, K] codes (the activation, e.g. from reng_hip_quantize with PCS over
 * its rows, or UNIT as the reference's probe casts it, fp8_probe.rs:244-247),
 * b [N, K] codes (the weight). scale_a has n_scale_a in {0 (unit), 1, M}
 * entries, scale_b n_scale_b in {0, 1, N}. Both operands must be E4M3 or E5M2
 * finite codes; K must be a multiple of 128. */
RENG_HIP_API int reng_hip_gemm_fp8_scaled(const uint8_t *a, int a_format, const float *scale_a,
                                          size_t n_scale_a, const uint8_t *b, int b_format,
                                          const float *scale_b, size_t n_scale_b, size_t M,
                                          size_t N, size_t K, uint16_t *out, void *stream);

/* ---------------------------------------------------------------------------
 * Decode step of one Llama decoder layer around its fp8 GEMVs
 *
 * The reference's fp8 load path stops at a refusal where the quantized codes
 * would meet a device layer (layer_views, crates/reng-model/src/lib.rs:2636-2649);
 * these entry points are the steps of that layer, one token per call, with the
 * semantics of its CPU decoder layer (layer_cpu, causal, Llama form:
 * crates/reng-synapse/src/model.rs:2903-3100). The seven projections are the
 * GEMV (reng_hip_gemm_w8a16, M = 1) on the layer's codes and scales, or its
 * fused forms below, which take the neighbouring steps into the same pass and
 * are bit-identical to the chain of separate calls. Residual stream f32; GEMV
 * inputs bf16; caches bf16 [positions, n_kv_heads * head_dim].
 * ------------------------------------------------------------------------- */

/* Longest cache an attention call reads: 128Ki rows, Llama 3.1's context. */
#define RENG_HIP_ATTENTION_MAX_LEN 131072

/* out[r, :] = bf16(x[r, :] / sqrt(mean(x[r, :]^2) + eps) * gamma), x f32
 * [rows, cols] (rms_norm_cpu, crates/reng-synapse/src/ops.rs:49-72). */
RENG_HIP_API int reng_hip_rms_norm_bf16(const float *x, const float *gamma, size_t rows, size_t cols, float eps,
                                        uint16_t *out, void *stream);

/* reng_hip_gemm_w8a16 at M = 1 with the residual add as its epilogue:
 * y[n] = residual[n] + bf16(scales[n] * sum_k x[k] * decode(codes[n, k])),
 * f32 residual and y [N] (y may be residual). Bit-identical to
 * reng_hip_gemm_w8a16 (M = 1) then reng_hip_add_bf16_f32. Same argument rules
 * as reng_hip_gemm_w8a16. */
RENG_HIP_API int reng_hip_gemv_w8a16_residual(const uint16_t *x, const uint8_t *codes, const float *scales,
                                              size_t N, size_t K, int format, const float *residual, float *y,
                                              void *stream);

/* A SwiGLU gate and up projection as one GEMV (M = 1) over rows in pairs:
 * row 2i of codes / scales is gate row i, row 2i + 1 up row i (N = 2 *
 * intermediate), and y[i] = bf16(silu(g_i) * u_i) with g_i, u_i the bf16
 * outputs of the two rows, y bf16 [N / 2]. Bit-identical to
 * reng_hip_gemm_w8a16 (M = 1) over each matrix then reng_hip_silu_mul_bf16.
 * N even; otherwise as reng_hip_gemm_w8a16. */
RENG_HIP_API int reng_hip_gemv_w8a16_swiglu(const uint16_t *x, const uint8_t *codes, const float *scales,
                                            size_t N, size_t K, int format, uint16_t *y, void *stream);

/* reng_hip_gemm_w8a16 at M = 1 with the RMSNorm of its input as its prologue:
 * y = bf16(W . bf16(rms_norm(x) * gamma)), x and gamma f32 [K] (4-byte
 * aligned), K % 16 == 0, K <= 32768; every workgroup normalises the row
 * itself. Bit-identical to reng_hip_rms_norm_bf16 (one row) then
 * reng_hip_gemm_w8a16. */
RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm(const float *x, const float *gamma, float eps, const uint8_t *codes,
                                             const float *scales, size_t N, size_t K, int format, uint16_t *y,
                                             void *stream);

/* The same prologue with reng_hip_gemv_w8a16_swiglu's epilogue (rows in (gate,
 * up) pairs, y bf16 [N / 2]): a SwiGLU MLP's norm, gate, up and activation in
 * one pass. */
RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm_swiglu(const float *x, const float *gamma, float eps,
                                                    const uint8_t *codes, const float *scales, size_t N, size_t K,
                                                    int format, uint16_t *y, void *stream);

/* A decode step's first projection in one pass: n = bf16(rms_norm(x) * gamma),
 * [q | k | v] = bf16(n W^T), q and k rotated (rotate-half RoPE with this
 * position's sin_row / cos_row [head_dim] rows of the tables) into q
 * [n_heads * head_dim] and k_row [n_kv_heads * head_dim], v copied into v_row
 * (k_row and v_row: this position's rows of the key and value caches).
 * codes / scales hold the N = (n_heads + 2 n_kv_heads) head_dim rows of
 * [Wq; Wk; Wv] in rotation-pair order: with half = head_dim / 2, row
 * 2 (h half + d) and row 2 (h half + d) + 1 are Wq rows h head_dim + d and
 * h head_dim + d + half (h < n_heads, d < half); the k heads follow the same
 * way from row 2 n_heads half; then the Wv rows in their order. Bit-identical
 * to reng_hip_gemv_w8a16_rmsnorm over [Wq; Wk; Wv] then reng_hip_rope_append.
 * x and gamma f32 [K], K % 16 == 0, K <= 32768; head_dim even. */
RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm_qkv_rope(const float *x, const float *gamma, float eps,
                                                      const uint8_t *codes, const float *scales, size_t n_heads,
                                                      size_t n_kv_heads, size_t head_dim, size_t K, int format,
                                                      const float *sin_row, const float *cos_row, uint16_t *q,
                                                      uint16_t *k_row, uint16_t *v_row, void *stream);

/* h = x + d and out = bf16(rms_norm(h) * gamma) in one pass, x and h f32, d
 * bf16 [rows, cols] (a branch output added to the residual stream, then the
 * next sublayer's RMSNorm; h must not overlap x or d). */
RENG_HIP_API int reng_hip_add_rms_norm_bf16(const float *x, const uint16_t *d, const float *gamma, size_t rows,
                                            size_t cols, float eps, float *h, uint16_t *out, void *stream);

/* Rotate-half RoPE of one position (rope_cpu, ops.rs:118-135) with the row
 * sin_row / cos_row [head_dim] of the tables: q [n_heads * head_dim] bf16 in
 * place; k [n_kv_heads * head_dim] rotated into k_row and v copied into v_row
 * (this position's rows of the key and value caches). head_dim even. */
RENG_HIP_API int reng_hip_rope_append(uint16_t *q, const uint16_t *k, const uint16_t *v, size_t n_heads,
                                      size_t n_kv_heads, size_t head_dim, const float *sin_row, const float *cos_row,
                                      uint16_t *k_row, uint16_t *v_row, void *stream);

/* One query per head over cache rows 0 .. len - 1 (layer_cpu's causal attention,
 * model.rs:3010-3050): out[h] = softmax(scale * q[h] . K[:, g]) V[:, g] with
 * g = h / (n_heads / n_kv_heads), bf16 in and out, f32 inside (online softmax
 * over tiles of 256 rows); 1 <= len <= RENG_HIP_ATTENTION_MAX_LEN; q, k_cache
 * and v_cache 4-byte aligned. One workgroup per query head reads the whole
 * cache: for caches past 512 rows use reng_hip_attention_decode_split. */
RENG_HIP_API int reng_hip_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                           size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t len,
                                           float scale, uint16_t *out, void *stream);

/* Bytes of device workspace reng_hip_attention_decode_split needs for every
 * cache length from 1 to len (0 when all of them take one pass: len <= 512). */
RENG_HIP_API size_t reng_hip_attention_workspace_bytes(size_t n_heads, size_t head_dim, size_t len);

/* reng_hip_attention_decode that, past 512 cache rows, cuts the cache into
 * min(64, ceil(len / 256)) splits, one workgroup per split and group of query
 * heads sharing a key/value head (each split's rows read once for the group);
 * the splits' unnormalised outputs and softmax statistics go to workspace
 * (f32, 4-byte aligned, workspace_bytes >= reng_hip_attention_workspace_bytes(
 * n_heads, head_dim, len)) and a second kernel merges them. Asynchronous on
 * stream; calls that share a workspace must be ordered (one stream). */
RENG_HIP_API int reng_hip_attention_decode_split(const uint16_t *q, const uint16_t *k_cache,
                                                 const uint16_t *v_cache, size_t n_heads, size_t n_kv_heads,
                                                 size_t head_dim, size_t len, float scale, void *workspace,
                                                 size_t workspace_bytes, uint16_t *out, void *stream);

/* out = bf16(silu(gate) * up), silu(g) = g / (1 + exp(-g)) (layer_cpu's
 * Activation::Silu, model.rs:3070-3080). */
RENG_HIP_API int reng_hip_silu_mul_bf16(const uint16_t *gate, const uint16_t *up, size_t n, uint16_t *out,
                                        void *stream);

/* out = x + d, x f32, d bf16 (a branch output added to the residual stream). */
RENG_HIP_API int reng_hip_add_bf16_f32(const float *x, const uint16_t *d, size_t n, float *out, void *stream);

/* ---------------------------------------------------------------------------
 * Self-check (no counterpart in the reference)
 * ------------------------------------------------------------------------- */

/* Runs every non-NaN f32 bit pattern through the hardware conversion the
 * quantizer's fast path uses (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32: after a
 * clamp to +-max finite, and without the clamp below 248 / 61440) and through
 * the exact integer encoder, and counts disagreements. The fast path is only
 * valid on a device where this returns *mismatches == 0;
 * tests/test_gpu_quantize.py requires it. Synchronous. first_mismatch
 * receives the first disagreeing bit pattern. */
RENG_HIP_API int reng_hip_verify_hw_convert(int format, uint64_t *mismatches,
                                            uint32_t *first_mismatch);

/* The read yardstick the GEMV is measured against: reads `bytes` (a positive
 * multiple of 1024, p 16-byte aligned) once, as 1 KB chunks dealt to 32 waves
 * per CU in turn, one chunk per wave in flight (the fastest pattern found for
 * a single read-only launch of GEMV size on MI355X). Computes nothing; sink is
 * device memory of reng_hip_stream_read_sink_bytes() bytes that the kernel
 * writes only if the data's XOR hits a fixed value. Asynchronous. */
RENG_HIP_API size_t reng_hip_stream_read_sink_bytes(void);
RENG_HIP_API int reng_hip_stream_read(const void *p, size_t bytes, void *sink, void *stream);

/* The stream yardstick the quantizer is measured against: reads `elems` bf16
 * values at src (16-byte aligned, elems a positive multiple of 8) and writes
 * the high byte of each to dst (8-byte aligned), i.e. the quantizer's 2 bytes
 * in and 1 byte out per element with no arithmetic, in the quantizer's
 * pattern: 8 KB input chunks per wave, grid-strided over 8 waves per CU, the
 * next chunk requested before this one is stored. No counterpart in the
 * reference: it exists to measure the memory system. Asynchronous. */
RENG_HIP_API int reng_hip_stream_narrow(const void *src, size_t elems, void *dst, void *stream);

/* The copy yardstick the 16 < M <= 64 skinny GEMM is measured against: the
 * data movement of that product's kernel and nothing else - the same grid,
 * LDS ring, global -> LDS copies of the codes [N, K] and the activation
 * x [M, K] (bf16), waits and barriers, with no decode, MFMA or output. x and
 * codes 16-byte aligned, K a positive multiple of 128, 16 < M <= 64; sink is
 * one device word written only by chance. No counterpart in the reference: it
 * exists to measure the kernel's copy floor. Asynchronous. */
RENG_HIP_API int reng_hip_stream_stage(const uint16_t *x, const uint8_t *codes, size_t M, size_t N, size_t K,
                                       void *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* RENG_HIP_H */
