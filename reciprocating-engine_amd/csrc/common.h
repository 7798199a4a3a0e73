// common.h - shared pieces of libreng_hip: error state, format traits and the
// exact fp8 encode / decode used on the device.
//
// The exact encoder is an integer formulation of reng-fp8's `encode`
// (crates/reng-fp8/src/lib.rs:154-201): round to nearest even at the format's
// mantissa width, carry into the exponent, saturate to the largest finite code,
// fp8-subnormal range by a variable shift. It is checked against the CPU oracle
// on all 2^32 f32 bit patterns (tests/test_gpu_quantize.py).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/reng_hip.h"

namespace reng {

// ---------------------------------------------------------------- errors

void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define RENG_CHECK_HIP(expr)                                                                  \
    do {                                                                                      \
        hipError_t e_ = (expr);                                                               \
        if (e_ != hipSuccess) {                                                               \
            ::reng::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                              __LINE__);                                                      \
            return e_ == hipErrorOutOfMemory ? RENG_HIP_ENOMEM : RENG_HIP_EDEVICE;            \
        }                                                                                     \
    } while (0)

#define RENG_REQUIRE(cond, ...)                 \
    do {                                        \
        if (!(cond)) {                          \
            ::reng::set_error(__VA_ARGS__);     \
            return RENG_HIP_EINVAL;             \
        }                                       \
    } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char *what);

// Device properties of the current device, cached per device.
struct DeviceProps {
    int cus;
    int max_threads_per_cu;
    size_t hbm_bytes;
    int clock_khz;
    char name[256];
    char arch[64];
};
const DeviceProps &device_props();


// ---------------------------------------------------------------- formats

template <int F>
struct Fp8;

// E4M3: Gaudi hf8 (lib.rs:53-58, 63-127): 3 mantissa bits, bias 7, normal
// exponents -6..7, largest finite 0x77 = 240.
template <>
struct Fp8<RENG_HIP_E4M3> {
    static constexpr int MBITS = 3, BIAS = 7, EMIN = -6, EMAX = 7;
    static constexpr uint32_t MAXCODE = 0x77;
    static constexpr float MAXF = 240.0f;
};

// E5M2: f8: 2 mantissa bits, bias 15, normal exponents -14..15, largest
// finite 0x7b = 57344.
template <>
struct Fp8<RENG_HIP_E5M2> {
    static constexpr int MBITS = 2, BIAS = 15, EMIN = -14, EMAX = 15;
    static constexpr uint32_t MAXCODE = 0x7b;
    static constexpr float MAXF = 57344.0f;
};

// The exact encoder, for finite, infinite and NaN input alike.
template <int F>
__device__ __forceinline__ uint32_t encode_exact(float x) {
    using T = Fp8<F>;
    const uint32_t u = __float_as_uint(x);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return sign | 0x7fu;        // NaN keeps its sign
    const uint32_t e = a >> 23;                      // biased f32 exponent
    constexpr uint32_t SH = 23 - T::MBITS;           // f32 mantissa bits below the fp8 quantum
    constexpr uint32_t ENORM = 127 + T::EMIN;        // f32 exponent of the smallest fp8 normal
    if (e >= ENORM) {
        // Round the whole pattern at bit SH (ties to even); a mantissa carry moves
        // into the exponent field, infinity lands above the largest code.
        const uint32_t t = (a + ((1u << (SH - 1)) - 1u) + ((a >> SH) & 1u)) >> SH;
        const uint32_t c = t - ((127u - T::BIAS) << T::MBITS);
        return sign | (c > T::MAXCODE ? T::MAXCODE : c);
    }
    if (e == 0) return sign;                         // zero and f32 subnormals
    // fp8 subnormal range: n = RNE(|x| / 2^(EMIN - MBITS)), |x| = m24 * 2^(e - 150).
    const uint32_t m24 = (a & 0x7fffffu) | 0x800000u;
    const uint32_t sh = (uint32_t)(150 + T::EMIN - T::MBITS) - e;   // >= 21
    if (sh >= 25) return sign;                       // below half the smallest subnormal
    const uint32_t n = (m24 + ((1u << (sh - 1)) - 1u) + ((m24 >> sh) & 1u)) >> sh;
    return sign | n;                                 // n == 1 << MBITS spells the smallest normal
}

// encode(x / s) with the x86 host's IEEE semantics: the division is correctly
// rounded; a NaN dividend propagates with its sign; an invalid quotient
// (0/0, inf/inf) is x86's default NaN, whose sign bit is set.
template <int F>
__device__ __forceinline__ uint32_t encode_div(float x, float s) {
    if (__builtin_isnan(x)) return ((__float_as_uint(x) >> 24) & 0x80u) | 0x7fu;
    const float q = x / s;
    if (__builtin_isnan(q)) return 0xffu;
    return encode_exact<F>(q);
}

// The exact decoder (lib.rs:206-225): finite codes exactly, the top exponent
// field as +-inf (mantissa 0) or a positive quiet NaN.
template <int F>
__device__ __forceinline__ float decode_exact(uint32_t code) {
    using T = Fp8<F>;
    constexpr uint32_t EF_MAX = (1u << (7 - T::MBITS)) - 1u;
    const uint32_t sign = (code & 0x80u) << 24;
    const uint32_t mant = code & ((1u << T::MBITS) - 1u);
    const uint32_t ef = (code & 0x7fu) >> T::MBITS;
    if (ef == EF_MAX) return mant == 0 ? __uint_as_float(sign | 0x7f800000u) : __uint_as_float(0x7fc00000u);
    if (ef == 0) {
        // mant * 2^(EMIN - MBITS), exact.
        const float v = (float)mant * __uint_as_float((uint32_t)(127 + T::EMIN - T::MBITS) << 23);
        return __uint_as_float(__float_as_uint(v) | sign);
    }
    return __uint_as_float(sign | ((ef + (127u - T::BIAS)) << 23) | (mant << (23 - T::MBITS)));
}

// 2^e for -126 <= e <= 127.
__host__ __device__ __forceinline__ float pow2f(int e) {
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)(e + 127) << 23;
    return v.f;
}

// Largest hardware exponent bias whose range max_finite * 2^(bias - b) covers
// absmax, else the widest (lib.rs:466-475). E4M3 offers {15, 11, 7, 3}
// (ranges 0.9375, 15, 240, 3840), E5M2 only its own 15.
template <int F>
__host__ __device__ __forceinline__ uint32_t choose_exp_bias_t(float absmax) {
    using T = Fp8<F>;
    if (F == RENG_HIP_E4M3) {
        const uint32_t b[4] = {15, 11, 7, 3};
        for (int i = 0; i < 4; ++i)
            if (absmax <= T::MAXF * pow2f(T::BIAS - (int)b[i])) return b[i];
        return 3;
    }
    return 15;
}

// ---------------------------------------------------------------- hardware conversion
// v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32: two f32 -> two OCP e4m3 / e5m2 codes,
// round to nearest even, written into the low or high half of `old`. Exact
// against encode_exact for |x| <= max finite (reng_hip_verify_hw_convert);
// prep() clamps into that range where a caller's quotients could leave it.

template <int F>
__device__ __forceinline__ uint32_t cvt_pk_lo(float a, float b, uint32_t old) {
    if constexpr (F == RENG_HIP_E4M3)
        return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, false);
    else
        return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int)old, false);
}

template <int F>
__device__ __forceinline__ uint32_t cvt_pk_hi(float a, float b, uint32_t old) {
    if constexpr (F == RENG_HIP_E4M3)
        return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, (int)old, true);
    else
        return (uint32_t)__builtin_amdgcn_cvt_pk_bf8_f32(a, b, (int)old, true);
}

template <int F, bool CLAMP>
__device__ __forceinline__ float prep(float q) {
    if constexpr (CLAMP) return __builtin_amdgcn_fmed3f(q, -Fp8<F>::MAXF, Fp8<F>::MAXF);
    return q;
}

// Four codes of four quotients q0..q3 packed into one dword (byte i = code of qi).
template <int F, bool CLAMP>
__device__ __forceinline__ uint32_t cvt4(float q0, float q1, float q2, float q3) {
    uint32_t p = cvt_pk_lo<F>(prep<F, CLAMP>(q0), prep<F, CLAMP>(q1), 0u);
    return cvt_pk_hi<F>(prep<F, CLAMP>(q2), prep<F, CLAMP>(q3), p);
}

// ---------------------------------------------------------------- wave helpers

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint32_t w = (uint32_t)__shfl_xor((int)v, o, 64);
        v = v > w ? v : w;
    }
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the 64 lanes with DPP moves (no LDS round trip): row_shr 1, 2, 4, 8
// leave each 16-lane row's sum in its lane 15; row_bcast 15 and 31 carry the
// rows into lane 63, which is read back as a scalar for every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, true));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_mov<0x111, 0xf>(v);   // row_shr:1
    v += dpp_mov<0x112, 0xf>(v);   // row_shr:2
    v += dpp_mov<0x114, 0xf>(v);   // row_shr:4
    v += dpp_mov<0x118, 0xf>(v);   // row_shr:8
    v += dpp_mov<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_mov<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ---------------------------------------------------------------- RoPE

// Rotate-half RoPE of one dimension pair (d, d + half) (rope_cpu,
// crates/reng-synapse/src/ops.rs:118-135): o0 = x0 cos[d] - x1 sin[d],
// o1 = x1 cos[d + half] + x0 sin[d + half], with the fused multiply-adds
// spelled out so that every kernel that rotates rounds the same way.
__device__ __forceinline__ void rope_rotate(float x0, float x1, float c0, float s0, float c1, float s1, float &o0,
                                            float &o1) {
    o0 = fmaf(x0, c0, -(x1 * s0));
    o1 = fmaf(x1, c1, x0 * s1);
}

// ---------------------------------------------------------------- RMSNorm

// 1 / sqrt(mean(h^2) + eps) of a row h[0, cols) (rms_norm_cpu,
// crates/reng-synapse/src/ops.rs:49-72), summed the way a 1024-thread
// workgroup sums it: thread t takes columns 4t, 4t + 4096, ... (VEC: float4
// loads; cols % 4 == 0, xr 16-byte aligned) or t, t + 1024, ...; each wave's
// partial sums meet in wave_sum_dpp; the 16 wave sums are added in order. A
// workgroup of 1024 / NV threads gets the same bits, each thread standing for
// NV of those 1024. With ADD the row is h = x + bf16 d, written to hr as it is
// formed; otherwise h = x. Every thread gets the result. red: 16 floats of LDS.
constexpr int NORM_VT = 1024;

// A float4's share of the sum of squares, added the way row_inv_rms adds it.
__device__ __forceinline__ float sum_sq4(float ss, const float4 &v) {
    return ss + (v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w);
}

// The end of row_inv_rms: the 16 wave sums in red added in order.
__device__ __forceinline__ float inv_rms_from(const float *red, uint32_t cols, float eps) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < NORM_VT / 64; ++w) s += red[w];
    const float ms = s / (float)cols;
    return 1.0f / sqrtf(ms + eps);
}

template <bool VEC, bool ADD, int NV>
__device__ __forceinline__ float row_inv_rms(const float *__restrict__ xr, const uint16_t *__restrict__ dr,
                                             float *__restrict__ hr, uint32_t cols, float eps, float *red) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const uint32_t vt = threadIdx.x + i * (NORM_VT / NV);
        float ss = 0.0f;
        if constexpr (VEC) {
            for (uint32_t c = vt * 4; c < cols; c += NORM_VT * 4) {
                float4 v = *reinterpret_cast<const float4 *>(xr + c);
                if constexpr (ADD) {
                    const uint32_t w0 = *reinterpret_cast<const uint32_t *>(dr + c);
                    const uint32_t w1 = *reinterpret_cast<const uint32_t *>(dr + c + 2);
                    v.x += __uint_as_float(w0 << 16);
                    v.y += __uint_as_float(w0 & 0xffff0000u);
                    v.z += __uint_as_float(w1 << 16);
                    v.w += __uint_as_float(w1 & 0xffff0000u);
                    *reinterpret_cast<float4 *>(hr + c) = v;
                }
                ss = sum_sq4(ss, v);
            }
        } else {
            for (uint32_t c = vt; c < cols; c += NORM_VT) {
                float v = xr[c];
                if constexpr (ADD) {
                    v += __uint_as_float((uint32_t)dr[c] << 16);
                    hr[c] = v;
                }
                ss += v * v;
            }
        }
        ss = wave_sum_dpp(ss);
        if (lane == 0) red[vt >> 6] = ss;
    }
    __syncthreads();
    return inv_rms_from(red, cols, eps);
}

// bf16 bits (RNE, NaN -> 0x7fc0) of an f32 (lib.rs:41-48).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
    const uint32_t bits = __float_as_uint(x);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    return (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
}

}  // namespace reng
