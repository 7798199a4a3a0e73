// layer.hip - the steps of one Llama decoder layer at decode time (one token
// per call) around its seven fp8 GEMVs (csrc/gemm.hip), on device buffers:
//
//   n  = bf16(rms_norm(x, g1))                       reng_hip_rms_norm_bf16
//   q, k, v = n W{q,k,v}^T                           (fp8 GEMV)
//   rotate-half RoPE of q and k at position p; k, v
//   appended to the layer's bf16 cache as row p      reng_hip_rope_append
//   a  = softmax(scale q K^T) V over rows 0..p       reng_hip_attention_decode
//   h  = x + a Wo^T                                  (fp8 GEMV) + reng_hip_add_bf16_f32
//   n2 = bf16(rms_norm(h, g2)); g, u = n2 W{g,u}^T   reng_hip_rms_norm_bf16, (fp8 GEMV)
//   y  = h + (silu(g) * u) Wd^T                      reng_hip_silu_mul_bf16, (fp8 GEMV), add
//
// The semantics are the reference's CPU decoder layer, causal, in its Llama
// form (pre-norm, SiLU gate, GQA, rotate-half RoPE): layer_cpu,
// crates/reng-synapse/src/model.rs:2903-3100, with rms_norm_cpu
// (crates/reng-synapse/src/ops.rs:49-72) and rope_cpu (ops.rs:118-135). The
// residual stream is f32; what feeds a GEMV is bf16 (the w8a16 contract).
// These are latency-bound per token (a few KB each); only the GEMVs stream
// HBM.
#include "common.h"

namespace reng {

namespace layer {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_bf16(float v) { return (uint16_t)f32_to_bf16_bits(v); }

// Sum over the block (blockDim.x a multiple of 64, at most 1024), returned to
// every thread.
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_sum_dpp(v);
    __syncthreads();   // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < waves; ++w) s += red[w];
    return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < waves; ++w) m = fmaxf(m, red[w]);
    return m;
}

// out[r, c] = bf16(x[r, c] * inv_r * g[c]), inv_r = 1 / sqrt(mean_c x[r, c]^2 + eps)
// (rms_norm_cpu, ops.rs:49-72). One block per row.
__global__ __launch_bounds__(256) void rms_norm_bf16(const float *__restrict__ x, const float *__restrict__ g,
                                                     uint32_t cols, float eps, uint16_t *__restrict__ out) {
    __shared__ float red[4];
    const float *xr = x + (size_t)blockIdx.x * cols;
    float ss = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) ss += xr[c] * xr[c];
    const float ms = block_sum(ss, red) / (float)cols;
    const float inv = 1.0f / sqrtf(ms + eps);
    uint16_t *orow = out + (size_t)blockIdx.x * cols;
    for (uint32_t c = threadIdx.x; c < cols; c += blockDim.x) orow[c] = f32_bf16(xr[c] * inv * g[c]);
}

// Rotate-half RoPE of one position (rope_cpu, ops.rs:118-135): for d < half,
// o[d] = x[d] cos[d] - x[d + half] sin[d] and o[d + half] = x[d + half]
// cos[d + half] + x[d] sin[d + half]. Blocks 0 .. nh - 1 rotate the q heads
// in place; blocks nh .. nh + nkv - 1 rotate k head g into k_row and copy v
// head g into v_row (the cache rows of this position).
__global__ __launch_bounds__(64) void rope_append(uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
                                                  const uint16_t *__restrict__ v, uint32_t nh, uint32_t hd,
                                                  const float *__restrict__ sn, const float *__restrict__ cs,
                                                  uint16_t *__restrict__ k_row, uint16_t *__restrict__ v_row) {
    const uint32_t b = blockIdx.x, half = hd / 2;
    const uint16_t *src;
    uint16_t *dst;
    if (b < nh) {
        src = q + (size_t)b * hd;
        dst = q + (size_t)b * hd;
    } else {
        const uint32_t g = b - nh;
        src = k + (size_t)g * hd;
        dst = k_row + (size_t)g * hd;
        for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) v_row[(size_t)g * hd + d] = v[(size_t)g * hd + d];
    }
    for (uint32_t d = threadIdx.x; d < half; d += blockDim.x) {
        const float x0 = bf16_f32(src[d]), x1 = bf16_f32(src[d + half]);
        const float o0 = x0 * cs[d] - x1 * sn[d];
        const float o1 = x1 * cs[d + half] + x0 * sn[d + half];
        dst[d] = f32_bf16(o0);
        dst[d + half] = f32_bf16(o1);
    }
}

// One query per head over cache rows 0 .. len - 1 (the causal row of
// layer_cpu's attention, model.rs:3010-3050): s_j = scale * q_h . k_j[g],
// p = softmax(s), out_h = sum_j p_j v_j[g], with g = h / (nh / nkv). One
// block per head; the scores live in LDS (len floats) and q in f32.
__global__ __launch_bounds__(256) void attention_decode(const uint16_t *__restrict__ q,
                                                        const uint16_t *__restrict__ kc,
                                                        const uint16_t *__restrict__ vc, uint32_t nh,
                                                        uint32_t nkv, uint32_t hd, uint32_t len, float scale,
                                                        uint16_t *__restrict__ out) {
    extern __shared__ float smem[];
    float *qs = smem;            // hd
    float *s = smem + hd;        // len
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, g = h / (nh / nkv), pitch = nkv * hd;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) qs[d] = bf16_f32(q[(size_t)h * hd + d]);
    __syncthreads();
    float mx = -INFINITY;
    for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
        const uint16_t *kr = kc + (size_t)j * pitch + (size_t)g * hd;
        float acc = 0.0f;
        for (uint32_t d = 0; d < hd; d += 2) {
            const uint32_t w = *reinterpret_cast<const uint32_t *>(kr + d);
            acc += qs[d] * __uint_as_float(w << 16) + qs[d + 1] * __uint_as_float(w & 0xffff0000u);
        }
        s[j] = acc * scale;
        mx = fmaxf(mx, s[j]);
    }
    mx = block_max(mx, red);
    float sum = 0.0f;
    for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
        const float e = expf(s[j] - mx);
        s[j] = e;
        sum += e;
    }
    sum = block_sum(sum, red);   // its barriers also publish s[]
    const float inv = 1.0f / sum;
    for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
        float acc = 0.0f;
        for (uint32_t j = 0; j < len; ++j) acc += s[j] * bf16_f32(vc[(size_t)j * pitch + (size_t)g * hd + d]);
        out[(size_t)h * hd + d] = f32_bf16(acc * inv);
    }
}

// out = bf16(silu(g) * u), silu(g) = g / (1 + exp(-g)) (layer_cpu's act,
// model.rs:3070-3080).
__global__ void silu_mul_bf16(const uint16_t *__restrict__ gate, const uint16_t *__restrict__ up, size_t n,
                              uint16_t *__restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float gv = bf16_f32(gate[i]);
        out[i] = f32_bf16(gv / (1.0f + expf(-gv)) * bf16_f32(up[i]));
    }
}

// out = x + d (f32 residual stream plus a bf16 branch output).
__global__ void add_bf16_f32(const float *__restrict__ x, const uint16_t *__restrict__ d, size_t n,
                             float *__restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = x[i] + bf16_f32(d[i]);
}

unsigned grid_for(size_t n, unsigned threads) {
    const size_t cap = (size_t)device_props().cus * 4;
    const size_t b = (n + threads - 1) / threads;
    return (unsigned)(b < 1 ? 1 : b > cap ? cap : b);
}

}  // namespace layer

}  // namespace reng

using namespace reng;
using namespace reng::layer;

namespace {
hipStream_t stream_of(void *s) { return static_cast<hipStream_t>(s); }
}

RENG_HIP_API int reng_hip_rms_norm_bf16(const float *x, const float *gamma, size_t rows, size_t cols, float eps,
                                        uint16_t *out, void *stream) {
    clear_error();
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(rows <= 0x7fffffff && cols <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(x && gamma && out, "null pointer");
    RENG_REQUIRE(eps >= 0.0f, "eps %g is negative", (double)eps);
    hipLaunchKernelGGL(rms_norm_bf16, dim3((unsigned)rows), dim3(256), 0, stream_of(stream), x, gamma,
                       (uint32_t)cols, eps, out);
    return check_launch("rms_norm_bf16");
}

RENG_HIP_API int reng_hip_rope_append(uint16_t *q, const uint16_t *k, const uint16_t *v, size_t n_heads,
                                      size_t n_kv_heads, size_t head_dim, const float *sin_row, const float *cos_row,
                                      uint16_t *k_row, uint16_t *v_row, void *stream) {
    clear_error();
    RENG_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%zu query heads are not a multiple of %zu key/value heads", n_heads, n_kv_heads);
    RENG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim %zu is not even in [2, 1024]",
                 head_dim);
    RENG_REQUIRE(n_heads + n_kv_heads <= 0x7fffffff, "too many heads");
    RENG_REQUIRE(q && k && v && sin_row && cos_row && k_row && v_row, "null pointer");
    hipLaunchKernelGGL(rope_append, dim3((unsigned)(n_heads + n_kv_heads)), dim3(64), 0, stream_of(stream), q, k, v,
                       (uint32_t)n_heads, (uint32_t)head_dim, sin_row, cos_row, k_row, v_row);
    return check_launch("rope_append");
}

RENG_HIP_API int reng_hip_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                           size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t len,
                                           float scale, uint16_t *out, void *stream) {
    clear_error();
    RENG_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%zu query heads are not a multiple of %zu key/value heads", n_heads, n_kv_heads);
    RENG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim %zu is not even in [2, 1024]",
                 head_dim);
    RENG_REQUIRE(len >= 1 && len <= RENG_HIP_ATTENTION_MAX_LEN, "cache length %zu is not in [1, %d]", len,
                 RENG_HIP_ATTENTION_MAX_LEN);
    RENG_REQUIRE(n_heads <= 0x7fffffff, "too many heads");
    RENG_REQUIRE(q && k_cache && v_cache && out, "null pointer");
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(k_cache) & 3) == 0, "k_cache must be 4-byte aligned");
    const size_t lds = (head_dim + len) * sizeof(float);
    hipLaunchKernelGGL(attention_decode, dim3((unsigned)n_heads), dim3(256), lds, stream_of(stream), q, k_cache,
                       v_cache, (uint32_t)n_heads, (uint32_t)n_kv_heads, (uint32_t)head_dim, (uint32_t)len, scale,
                       out);
    return check_launch("attention_decode");
}

RENG_HIP_API int reng_hip_silu_mul_bf16(const uint16_t *gate, const uint16_t *up, size_t n, uint16_t *out,
                                        void *stream) {
    clear_error();
    RENG_REQUIRE(n > 0, "empty vector");
    RENG_REQUIRE(gate && up && out, "null pointer");
    hipLaunchKernelGGL(silu_mul_bf16, dim3(grid_for(n, 256)), dim3(256), 0, stream_of(stream), gate, up, n, out);
    return check_launch("silu_mul_bf16");
}

RENG_HIP_API int reng_hip_add_bf16_f32(const float *x, const uint16_t *d, size_t n, float *out, void *stream) {
    clear_error();
    RENG_REQUIRE(n > 0, "empty vector");
    RENG_REQUIRE(x && d && out, "null pointer");
    hipLaunchKernelGGL(add_bf16_f32, dim3(grid_for(n, 256)), dim3(256), 0, stream_of(stream), x, d, n, out);
    return check_launch("add_bf16_f32");
}
