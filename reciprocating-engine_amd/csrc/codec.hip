// codec.hip - elementwise fp8 kernels: encode / decode over arrays,
// dequantize, the per-row error statistics, and the self-check of the
// hardware conversion the quantizer's fast path relies on.
#include "codec.h"
#include "common.h"

namespace reng {

namespace {

// Grid of at most ~8 blocks per CU for a grid-stride loop over n items.
dim3 stride_grid(uint64_t n, int threads) {
    uint64_t blocks = (n + threads - 1) / threads;
    const uint64_t cap = (uint64_t)device_props().cus * 8;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    return dim3((unsigned)blocks);
}

}  // namespace

// encode (lib.rs:154-201) over an array.
template <int F>
__global__ void encode_kernel(const float *__restrict__ x, uint64_t n, uint8_t *__restrict__ out) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = (uint8_t)encode_exact<F>(x[i]);
}

// decode (lib.rs:206-225) over an array.
template <int F>
__global__ void decode_kernel(const uint8_t *__restrict__ c, uint64_t n, float *__restrict__ out) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = decode_exact<F>(c[i]);
}

// Quantized::dequantize (lib.rs:328-337): decode(code) * scale, one f32
// multiply; dequantize_bf16 (lib.rs:342-344) rounds that to bf16.
template <int F, bool BF16>
__global__ void dequant_kernel(const uint8_t *__restrict__ c, const float *__restrict__ scales,
                               uint64_t rows, uint64_t cols, void *__restrict__ out) {
    const uint64_t n = rows * cols;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float v = decode_exact<F>(c[i]) * scales[i / cols];
        if constexpr (BF16)
            static_cast<uint16_t *>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
        else
            static_cast<float *>(out)[i] = v;
    }
}

// row_errors / sample_row_errors (lib.rs:364-431): one block per sampled row;
// the f64 sum is reduced in a different order than the host's, which moves
// the mean in its last bits only.
template <int F>
__global__ __launch_bounds__(256) void row_errors_kernel(const uint16_t *__restrict__ w,
                                                         const uint8_t *__restrict__ c,
                                                         const float *__restrict__ scales,
                                                         uint64_t cols, uint64_t step,
                                                         uint64_t nsampled,
                                                         float *__restrict__ mean_rel,
                                                         float *__restrict__ max_rel) {
    __shared__ double ssum[4];
    __shared__ float smax[4];
    __shared__ unsigned long long scnt[4];
    for (uint64_t k = blockIdx.x; k < nsampled; k += gridDim.x) {
        const uint64_t r = k * step;
        const float s = scales[r];
        double sum = 0.0;
        float mx = 0.0f;
        unsigned long long cnt = 0;
        for (uint64_t j = threadIdx.x; j < cols; j += 256) {
            const float want = __uint_as_float((uint32_t)w[r * cols + j] << 16);
            if (want == 0.0f) continue;
            const float got = decode_exact<F>(c[r * cols + j]) * s;
            const float rel = __builtin_fabsf((got - want) / want);
            sum += (double)rel;
            mx = __builtin_fmaxf(mx, rel);   // IEEE maxNum: a NaN loses, as f32::max
            ++cnt;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            sum += __shfl_xor(sum, o, 64);
            mx = __builtin_fmaxf(mx, __shfl_xor(mx, o, 64));
            cnt += __shfl_xor(cnt, o, 64);
        }
        const int wv = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) {
            ssum[wv] = sum;
            smax[wv] = mx;
            scnt[wv] = cnt;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            const double ts = ((ssum[0] + ssum[1]) + ssum[2]) + ssum[3];
            const float tm = __builtin_fmaxf(__builtin_fmaxf(smax[0], smax[1]), __builtin_fmaxf(smax[2], smax[3]));
            const unsigned long long tc = scnt[0] + scnt[1] + scnt[2] + scnt[3];
            mean_rel[k] = tc == 0 ? 0.0f : (float)(ts / (double)tc);
            max_rel[k] = tm;
        }
        __syncthreads();
    }
}

// Every non-NaN f32 pattern: the conversion as the fast path uses it (clamped
// into +-max finite, then v_cvt_pk_*) against the exact integer encoder; and,
// below the first midpoint past the largest finite value (248 / 61440), the
// unclamped conversion too.
template <int F>
__global__ void verify_hw_kernel(unsigned long long *__restrict__ count, uint32_t *__restrict__ first) {
    constexpr float UNCLAMPED = F == RENG_HIP_E4M3 ? 248.0f : 61440.0f;
    unsigned long long bad = 0;
    uint32_t fbad = 0xffffffffu;
    const uint64_t total = 1ull << 32;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint32_t u = (uint32_t)i;
        const float x = __uint_as_float(u);
        if (__builtin_isnan(x)) continue;
        const uint32_t ex = encode_exact<F>(x);
        bool ok = (cvt_pk_lo<F>(prep<F, true>(x), 0.0f, 0u) & 0xffu) == ex;
        // Unclamped, below the first midpoint past the largest finite value.
        if (__builtin_fabsf(x) < UNCLAMPED) ok = ok && (cvt_pk_lo<F>(x, 0.0f, 0u) & 0xffu) == ex;
        if (!ok) {
            ++bad;
            fbad = u < fbad ? u : fbad;
        }
    }
    if (bad) {
        atomicAdd(count, bad);
        atomicMin(first, fbad);
    }
}

int launch_encode(const float *x, uint64_t n, int format, uint8_t *out, hipStream_t st) {
    const dim3 g = stride_grid(n, 256);
    if (format == RENG_HIP_E4M3)
        hipLaunchKernelGGL(encode_kernel<RENG_HIP_E4M3>, g, dim3(256), 0, st, x, n, out);
    else
        hipLaunchKernelGGL(encode_kernel<RENG_HIP_E5M2>, g, dim3(256), 0, st, x, n, out);
    return check_launch("encode");
}

int launch_decode(const uint8_t *c, uint64_t n, int format, float *out, hipStream_t st) {
    const dim3 g = stride_grid(n, 256);
    if (format == RENG_HIP_E4M3)
        hipLaunchKernelGGL(decode_kernel<RENG_HIP_E4M3>, g, dim3(256), 0, st, c, n, out);
    else
        hipLaunchKernelGGL(decode_kernel<RENG_HIP_E5M2>, g, dim3(256), 0, st, c, n, out);
    return check_launch("decode");
}

int launch_dequantize(const uint8_t *c, const float *scales, uint64_t rows, uint64_t cols,
                      int format, bool bf16, void *out, hipStream_t st) {
    const dim3 g = stride_grid(rows * cols, 256);
    if (format == RENG_HIP_E4M3) {
        if (bf16) hipLaunchKernelGGL((dequant_kernel<RENG_HIP_E4M3, true>), g, dim3(256), 0, st, c, scales, rows, cols, out);
        else hipLaunchKernelGGL((dequant_kernel<RENG_HIP_E4M3, false>), g, dim3(256), 0, st, c, scales, rows, cols, out);
    } else {
        if (bf16) hipLaunchKernelGGL((dequant_kernel<RENG_HIP_E5M2, true>), g, dim3(256), 0, st, c, scales, rows, cols, out);
        else hipLaunchKernelGGL((dequant_kernel<RENG_HIP_E5M2, false>), g, dim3(256), 0, st, c, scales, rows, cols, out);
    }
    return check_launch("dequantize");
}

int launch_row_errors(const uint16_t *w, const uint8_t *c, const float *scales, uint64_t cols,
                      uint64_t step, uint64_t nsampled, int format, float *mean_rel,
                      float *max_rel, hipStream_t st) {
    uint64_t blocks = nsampled;
    const uint64_t cap = (uint64_t)device_props().cus * 8;
    if (blocks > cap) blocks = cap;
    if (format == RENG_HIP_E4M3)
        hipLaunchKernelGGL(row_errors_kernel<RENG_HIP_E4M3>, dim3((unsigned)blocks), dim3(256), 0, st, w, c, scales, cols, step, nsampled, mean_rel, max_rel);
    else
        hipLaunchKernelGGL(row_errors_kernel<RENG_HIP_E5M2>, dim3((unsigned)blocks), dim3(256), 0, st, w, c, scales, cols, step, nsampled, mean_rel, max_rel);
    return check_launch("row_errors");
}

int run_verify_hw(int format, unsigned long long *d_count, uint32_t *d_first, hipStream_t st) {
    const dim3 g((unsigned)device_props().cus * 8);
    if (format == RENG_HIP_E4M3)
        hipLaunchKernelGGL(verify_hw_kernel<RENG_HIP_E4M3>, g, dim3(256), 0, st, d_count, d_first);
    else
        hipLaunchKernelGGL(verify_hw_kernel<RENG_HIP_E5M2>, g, dim3(256), 0, st, d_count, d_first);
    return check_launch("verify_hw_convert");
}

}  // namespace reng
