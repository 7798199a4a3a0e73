// api.hip - the extern "C" entry points of libreng_hip.so (include/reng_hip.h):
// argument checks with the reference's refusal semantics, error reporting,
// host-pointer staging, and batching of matrices into launches.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "codec.h"
#include "common.h"
#include "gemm.h"
#include "quantize.h"
#include "staging.h"

namespace reng {

static thread_local char g_err[1024];

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: launch failed: %s", what, hipGetErrorString(e));
        return RENG_HIP_EDEVICE;
    }
    return RENG_HIP_OK;
}

const DeviceProps &device_props() {
    static std::mutex mu;
    static std::map<int, DeviceProps> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    DeviceProps p{};
    hipDeviceProp_t hp;
    if (hipGetDeviceProperties(&hp, dev) == hipSuccess) {
        p.cus = hp.multiProcessorCount;
        p.max_threads_per_cu = hp.maxThreadsPerMultiProcessor;
        p.hbm_bytes = hp.totalGlobalMem;
        p.clock_khz = hp.clockRate;
        snprintf(p.name, sizeof p.name, "%s", hp.name);
        snprintf(p.arch, sizeof p.arch, "%s", hp.gcnArchName);
    } else {
        p.cus = 256;
    }
    if (p.cus < 1) p.cus = 1;
    return cache.emplace(dev, p).first->second;
}

}  // namespace reng

using namespace reng;

namespace {

bool valid_format(int f) { return f == RENG_HIP_E4M3 || f == RENG_HIP_E5M2; }
bool valid_scaling(int s) { return s == RENG_HIP_PCS || s == RENG_HIP_HW || s == RENG_HIP_UNIT; }
bool valid_dtype(int d) { return d == RENG_HIP_BF16 || d == RENG_HIP_F32; }
size_t dtype_bytes(int d) { return d == RENG_HIP_BF16 ? 2 : 4; }
hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

// The checks reng_fp8::quantize_with makes before any work (lib.rs:527-532),
// plus the ones a pointer interface needs.
int check_quantize_args(const void *w, int dtype, size_t rows, size_t cols, size_t ld, int format,
                        int scaling, float backoff, const void *codes, const void *scales) {
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(backoff > 0.0f && isfinite(backoff), "backoff %g is not positive and finite",
                 (double)backoff);
    RENG_REQUIRE(valid_dtype(dtype), "unknown element type %d", dtype);
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(valid_scaling(scaling), "unknown scale scheme %d", scaling);
    RENG_REQUIRE(ld >= cols, "row pitch %zu is smaller than cols %zu", ld, cols);
    RENG_REQUIRE(w && codes && scales, "null weight, code or scale pointer");
    return RENG_HIP_OK;
}

QMat make_qmat(const void *w, size_t cols, size_t ld, uint8_t *codes, float *scales,
               uint32_t *exp_bias, uint64_t row_begin) {
    QMat m;
    m.w = w;
    m.codes = codes;
    m.scales = scales;
    m.exp_bias = exp_bias;
    m.cols = cols;
    m.ld = ld;
    m.row_begin = row_begin;
    return m;
}

}  // namespace

extern "C" {

RENG_HIP_API const char *reng_hip_version(void) { return "reng-hip 0.1.0 (gfx950)"; }

RENG_HIP_API const char *reng_hip_last_error(void) { return g_err; }

RENG_HIP_API int reng_hip_device_info(char *buf, size_t len) {
    clear_error();
    RENG_REQUIRE(buf && len > 0, "null buffer");
    int n = 0;
    RENG_CHECK_HIP(hipGetDeviceCount(&n));
    RENG_REQUIRE(n > 0, "no HIP device");
    const DeviceProps &p = device_props();
    snprintf(buf, len, "%s %s, %d CUs, %zu bytes HBM, %d MHz", p.name, p.arch, p.cus, p.hbm_bytes,
             p.clock_khz / 1000);
    return RENG_HIP_OK;
}

RENG_HIP_API int reng_hip_quantize(const void *w, int dtype, size_t rows, size_t cols, size_t ld,
                                   int format, int scaling, float backoff, uint8_t *codes,
                                   float *scales, uint32_t *exp_bias, void *stream) {
    clear_error();
    int rc = check_quantize_args(w, dtype, rows, cols, ld, format, scaling, backoff, codes, scales);
    if (rc) return rc;
    QBatch b;
    b.n = 1;
    b.total_rows = rows;
    b.m[0] = make_qmat(w, cols, ld, codes, scales, exp_bias, 0);
    return launch_quantize_group(b, dtype, format, scaling, backoff, fast_key(b.m[0], dtype),
                                 as_stream(stream));
}

RENG_HIP_API int reng_hip_quantize_batch(const reng_hip_matrix *mats, size_t n, int dtype,
                                         int format, int scaling, float backoff, void *stream) {
    clear_error();
    RENG_REQUIRE(mats && n > 0, "empty batch");
    for (size_t i = 0; i < n; ++i) {
        const int rc = check_quantize_args(mats[i].w, dtype, mats[i].rows, mats[i].cols, mats[i].ld,
                                           format, scaling, backoff, mats[i].codes, mats[i].scales);
        if (rc) {
            char msg[1024];
            snprintf(msg, sizeof msg, "matrix %zu: %s", i, g_err);
            set_error("%s", msg);
            return rc;
        }
    }
    // Group by kernel configuration, then launch each group in chunks of QBATCH.
    std::map<int, std::vector<size_t>> groups;
    for (size_t i = 0; i < n; ++i) {
        const QMat m = make_qmat(mats[i].w, mats[i].cols, mats[i].ld, mats[i].codes, mats[i].scales,
                                 mats[i].exp_bias, 0);
        groups[fast_key(m, dtype)].push_back(i);
    }
    for (auto &kv : groups) {
        const std::vector<size_t> &idx = kv.second;
        for (size_t c0 = 0; c0 < idx.size(); c0 += QBATCH) {
            QBatch b;
            b.n = 0;
            b.total_rows = 0;
            for (size_t c = c0; c < idx.size() && c < c0 + QBATCH; ++c) {
                const reng_hip_matrix &m = mats[idx[c]];
                b.m[b.n++] = make_qmat(m.w, m.cols, m.ld, m.codes, m.scales, m.exp_bias, b.total_rows);
                b.total_rows += m.rows;
            }
            const int rc = launch_quantize_group(b, dtype, format, scaling, backoff, kv.first,
                                                 as_stream(stream));
            if (rc) return rc;
        }
    }
    return RENG_HIP_OK;
}

RENG_HIP_API int reng_hip_quantize_host(const void *w, int dtype, size_t rows, size_t cols,
                                        int format, int scaling, float backoff, uint8_t *codes,
                                        float *scales, uint32_t *exp_bias) {
    clear_error();
    const int rc = check_quantize_args(w, dtype, rows, cols, cols, format, scaling, backoff, codes, scales);
    if (rc) return rc;
    return quantize_host_staged(w, dtype, rows, cols, format, scaling, backoff, codes, scales, exp_bias);
}

RENG_HIP_API int reng_hip_row_absmax(const void *w, int dtype, size_t rows, size_t cols, size_t ld,
                                     float *out, void *stream) {
    clear_error();
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(valid_dtype(dtype), "unknown element type %d", dtype);
    RENG_REQUIRE(ld >= cols, "row pitch %zu is smaller than cols %zu", ld, cols);
    RENG_REQUIRE(w && out, "null pointer");
    QBatch b;
    b.n = 1;
    b.total_rows = rows;
    b.m[0] = make_qmat(w, cols, ld, nullptr, nullptr, nullptr, 0);
    return launch_row_absmax(b, dtype, out, as_stream(stream));
}

RENG_HIP_API uint32_t reng_hip_choose_exp_bias(float absmax, int format) {
    return format == RENG_HIP_E4M3 ? choose_exp_bias_t<RENG_HIP_E4M3>(absmax)
                                   : choose_exp_bias_t<RENG_HIP_E5M2>(absmax);
}

RENG_HIP_API int reng_hip_encode(const float *x, size_t n, int format, uint8_t *codes, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    if (n == 0) return RENG_HIP_OK;
    RENG_REQUIRE(x && codes, "null pointer");
    return launch_encode(x, n, format, codes, as_stream(stream));
}

RENG_HIP_API int reng_hip_decode(const uint8_t *codes, size_t n, int format, float *out, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    if (n == 0) return RENG_HIP_OK;
    RENG_REQUIRE(codes && out, "null pointer");
    return launch_decode(codes, n, format, out, as_stream(stream));
}

RENG_HIP_API int reng_hip_dequantize(const uint8_t *codes, const float *scales, size_t rows,
                                     size_t cols, int format, int out_dtype, void *out, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(valid_dtype(out_dtype), "unknown output type %d", out_dtype);
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(codes && scales && out, "null pointer");
    return launch_dequantize(codes, scales, rows, cols, format, out_dtype == RENG_HIP_BF16, out,
                             as_stream(stream));
}

RENG_HIP_API int reng_hip_row_errors(const uint16_t *w, const uint8_t *codes, const float *scales,
                                     size_t rows, size_t cols, int format, size_t max_rows,
                                     float *mean_rel, float *max_rel, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(w && codes && scales && mean_rel && max_rel, "null pointer");
    // sample_row_errors (lib.rs:402-405): n = min(max_rows, rows), every ceil(rows / n)
    // rows; max_rows == 0 selects row_errors, every row.
    const size_t n = max_rows == 0 ? rows : (max_rows < rows ? max_rows : rows);
    const size_t step = (rows + n - 1) / n;
    const size_t nsampled = (rows + step - 1) / step;
    return launch_row_errors(w, codes, scales, cols, step, nsampled, format, mean_rel, max_rel,
                             as_stream(stream));
}

namespace {

int w8a16_args(const uint16_t *x, const uint8_t *codes, size_t M, size_t N, size_t K, int format,
               const uint16_t *y) {
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(M > 0 && N > 0 && K > 0, "empty product %zu x %zu x %zu", M, N, K);
    RENG_REQUIRE(K % 16 == 0, "K = %zu is not a multiple of 16", K);
    RENG_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(x && codes && y, "null pointer");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes)) & 15) == 0,
                 "x and codes must be 16-byte aligned");
    return RENG_HIP_OK;
}

}  // namespace

RENG_HIP_API int reng_hip_gemm_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales,
                                     size_t M, size_t N, size_t K, int format, uint16_t *y,
                                     void *stream) {
    clear_error();
    if (int rc = w8a16_args(x, codes, M, N, K, format, y)) return rc;
    return launch_w8a16(x, codes, scales, (uint32_t)M, (uint32_t)N, (uint32_t)K, format, y,
                        as_stream(stream));
}

RENG_HIP_API size_t reng_hip_stream_read_sink_bytes(void) {
    return (size_t)stream_read_sink_words() * sizeof(uint32_t);
}

RENG_HIP_API int reng_hip_stream_read(const void *p, size_t bytes, void *sink, void *stream) {
    clear_error();
    RENG_REQUIRE(p && sink, "null pointer");
    RENG_REQUIRE(bytes >= 1024 && bytes % 1024 == 0, "bytes = %zu is not a positive multiple of 1024", bytes);
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(p) & 15) == 0, "p must be 16-byte aligned");
    return launch_stream_read(p, bytes, static_cast<uint32_t *>(sink), as_stream(stream));
}

RENG_HIP_API int reng_hip_stream_narrow(const void *src, size_t elems, void *dst, void *stream) {
    clear_error();
    RENG_REQUIRE(src && dst, "null pointer");
    RENG_REQUIRE(elems >= 8 && elems % 8 == 0, "elems = %zu is not a positive multiple of 8", elems);
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(src) & 15) == 0, "src must be 16-byte aligned");
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(dst) & 7) == 0, "dst must be 8-byte aligned");
    return launch_stream_narrow(src, elems, dst, as_stream(stream));
}

RENG_HIP_API int reng_hip_stream_stage(const uint16_t *x, const uint8_t *codes, size_t M, size_t N, size_t K,
                                       void *sink, void *stream) {
    clear_error();
    RENG_REQUIRE(x && codes && sink, "null pointer");
    RENG_REQUIRE(M > 16 && M <= 64, "M = %zu outside 17..64", M);
    RENG_REQUIRE(N > 0 && N <= 0xffffffffu, "N = %zu out of range", N);
    RENG_REQUIRE(K >= 128 && K % 128 == 0 && K <= 0xffffffffu, "K = %zu is not a positive multiple of 128", K);
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes)) & 15) == 0,
                 "x and codes must be 16-byte aligned");
    return launch_stage_copy(x, codes, (uint32_t)M, (uint32_t)N, (uint32_t)K, static_cast<uint32_t *>(sink),
                             as_stream(stream));
}

RENG_HIP_API int reng_hip_gemm_w8a16_noalloc(const uint16_t *x, const uint8_t *codes, const float *scales,
                                             size_t M, size_t N, size_t K, int format, uint16_t *y,
                                             void *stream) {
    clear_error();
    if (int rc = w8a16_args(x, codes, M, N, K, format, y)) return rc;
    int rc = RENG_HIP_OK;
    float *p = static_split_scratch(&rc);   // resolved once per device, on its first call there
    if (rc) return rc;
    const SplitScratch fixed{p, STATIC_SCRATCH_FLOATS};
    return launch_w8a16(x, codes, scales, (uint32_t)M, (uint32_t)N, (uint32_t)K, format, y,
                        as_stream(stream), &fixed);
}

namespace {

int gemv_epi_args(const uint16_t *x, const uint8_t *codes, size_t N, size_t K, int format) {
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(N > 0 && K > 0, "empty product 1 x %zu x %zu", N, K);
    RENG_REQUIRE(K % 16 == 0, "K = %zu is not a multiple of 16", K);
    RENG_REQUIRE(N <= 0x7fffffff && K <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(x && codes, "null pointer");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes)) & 15) == 0,
                 "x and codes must be 16-byte aligned");
    return RENG_HIP_OK;
}

}  // namespace

RENG_HIP_API int reng_hip_gemv_w8a16_residual(const uint16_t *x, const uint8_t *codes, const float *scales,
                                              size_t N, size_t K, int format, const float *residual, float *y,
                                              void *stream) {
    clear_error();
    if (int rc = gemv_epi_args(x, codes, N, K, format)) return rc;
    RENG_REQUIRE(residual && y, "null pointer");
    return launch_gemv_residual(x, codes, scales, (uint32_t)N, (uint32_t)K, format, residual, y,
                                as_stream(stream));
}

RENG_HIP_API int reng_hip_gemv_w8a16_swiglu(const uint16_t *x, const uint8_t *codes, const float *scales,
                                            size_t N, size_t K, int format, uint16_t *y, void *stream) {
    clear_error();
    if (int rc = gemv_epi_args(x, codes, N, K, format)) return rc;
    RENG_REQUIRE(N % 2 == 0, "N = %zu rows do not form (gate, up) pairs", N);
    RENG_REQUIRE(y, "null pointer");
    return launch_gemv_swiglu(x, codes, scales, (uint32_t)N, (uint32_t)K, format, y, as_stream(stream));
}

namespace {

int gemv_norm(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales, size_t N,
              size_t K, int format, bool swiglu, uint16_t *y, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(N > 0 && K > 0, "empty product 1 x %zu x %zu", N, K);
    RENG_REQUIRE(K % 16 == 0, "K = %zu is not a multiple of 16", K);
    RENG_REQUIRE(K <= 32768, "K = %zu is past 32768 (the normalised row is staged in 64 KB of LDS)", K);
    RENG_REQUIRE(N <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(!swiglu || N % 2 == 0, "N = %zu rows do not form (gate, up) pairs", N);
    RENG_REQUIRE(eps >= 0.0f, "eps %g is negative", (double)eps);
    RENG_REQUIRE(x && gamma && codes && y, "null pointer");
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(codes) & 15) == 0, "codes must be 16-byte aligned");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 3) == 0,
                 "x and gamma must be 4-byte aligned");
    return launch_gemv_norm(x, gamma, eps, codes, scales, (uint32_t)N, (uint32_t)K, format, swiglu, y,
                            as_stream(stream));
}

}  // namespace

RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm(const float *x, const float *gamma, float eps, const uint8_t *codes,
                                             const float *scales, size_t N, size_t K, int format, uint16_t *y,
                                             void *stream) {
    return gemv_norm(x, gamma, eps, codes, scales, N, K, format, false, y, stream);
}

RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm_swiglu(const float *x, const float *gamma, float eps,
                                                    const uint8_t *codes, const float *scales, size_t N, size_t K,
                                                    int format, uint16_t *y, void *stream) {
    return gemv_norm(x, gamma, eps, codes, scales, N, K, format, true, y, stream);
}

RENG_HIP_API int reng_hip_gemv_w8a16_rmsnorm_qkv_rope(const float *x, const float *gamma, float eps,
                                                      const uint8_t *codes, const float *scales, size_t n_heads,
                                                      size_t n_kv_heads, size_t head_dim, size_t K, int format,
                                                      const float *sin_row, const float *cos_row, uint16_t *q,
                                                      uint16_t *k_row, uint16_t *v_row, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%zu query heads are not a multiple of %zu key/value heads", n_heads, n_kv_heads);
    RENG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim %zu is not even in [2, 1024]",
                 head_dim);
    RENG_REQUIRE(K > 0 && K % 16 == 0, "K = %zu is not a positive multiple of 16", K);
    RENG_REQUIRE(K <= 32768, "K = %zu is past 32768 (the normalised row is staged in 64 KB of LDS)", K);
    RENG_REQUIRE((n_heads + 2 * n_kv_heads) * head_dim <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(eps >= 0.0f, "eps %g is negative", (double)eps);
    RENG_REQUIRE(x && gamma && codes && sin_row && cos_row && q && k_row && v_row, "null pointer");
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(codes) & 15) == 0, "codes must be 16-byte aligned");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 3) == 0,
                 "x and gamma must be 4-byte aligned");
    return launch_gemv_norm_rope(x, gamma, eps, codes, scales, (uint32_t)n_heads, (uint32_t)n_kv_heads,
                                 (uint32_t)head_dim, (uint32_t)K, format, sin_row, cos_row, q, k_row, v_row,
                                 as_stream(stream));
}

RENG_HIP_API int reng_hip_gemm_fp8_scaled(const uint8_t *a, int a_format, const float *scale_a,
                                          size_t n_scale_a, const uint8_t *b, int b_format,
                                          const float *scale_b, size_t n_scale_b, size_t M,
                                          size_t N, size_t K, uint16_t *out, void *stream) {
    clear_error();
    RENG_REQUIRE(valid_format(a_format) && valid_format(b_format), "unknown fp8 format");
    RENG_REQUIRE(M > 0 && N > 0 && K > 0, "empty product %zu x %zu x %zu", M, N, K);
    RENG_REQUIRE(K % 128 == 0, "K = %zu is not a multiple of 128", K);
    RENG_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(n_scale_a == 0 || n_scale_a == 1 || n_scale_a == M,
                 "scale_a has %zu entries; expected 0, 1 or M = %zu", n_scale_a, M);
    RENG_REQUIRE(n_scale_b == 0 || n_scale_b == 1 || n_scale_b == N,
                 "scale_b has %zu entries; expected 0, 1 or N = %zu", n_scale_b, N);
    RENG_REQUIRE((n_scale_a == 0 || scale_a) && (n_scale_b == 0 || scale_b), "null scale pointer");
    RENG_REQUIRE(a && b && out, "null pointer");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0,
                 "a and b must be 16-byte aligned");
    return launch_fp8_gemm(a, a_format, scale_a, (uint32_t)n_scale_a, b, b_format, scale_b,
                           (uint32_t)n_scale_b, (uint32_t)M, (uint32_t)N, (uint32_t)K, out,
                           as_stream(stream));
}

RENG_HIP_API int reng_hip_verify_hw_convert(int format, uint64_t *mismatches, uint32_t *first_mismatch) {
    clear_error();
    RENG_REQUIRE(valid_format(format), "unknown fp8 format %d", format);
    RENG_REQUIRE(mismatches && first_mismatch, "null pointer");
    unsigned long long *d_count = nullptr;
    RENG_CHECK_HIP(hipMalloc(reinterpret_cast<void **>(&d_count), 16));
    uint32_t *d_first = reinterpret_cast<uint32_t *>(d_count + 1);
    const uint32_t init[4] = {0u, 0u, 0xffffffffu, 0u};
    hipError_t e = hipMemcpy(d_count, init, 16, hipMemcpyHostToDevice);
    int rc = RENG_HIP_OK;
    if (e == hipSuccess) rc = run_verify_hw(format, d_count, d_first, nullptr);
    uint32_t back[4] = {0, 0, 0, 0};
    if (e == hipSuccess && rc == RENG_HIP_OK) e = hipMemcpy(back, d_count, 16, hipMemcpyDeviceToHost);
    (void)hipFree(d_count);
    if (rc) return rc;
    if (e != hipSuccess) {
        set_error("verify_hw_convert: %s", hipGetErrorString(e));
        return RENG_HIP_EDEVICE;
    }
    *mismatches = (uint64_t)back[0] | ((uint64_t)back[1] << 32);
    *first_mismatch = back[2];
    return RENG_HIP_OK;
}

}  // extern "C"
