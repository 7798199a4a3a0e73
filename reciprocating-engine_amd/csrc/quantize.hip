// quantize.hip - the fp8 weight quantizer on CDNA4 (gfx950).
//
// Semantics: reng_fp8::quantize_with (crates/reng-fp8/src/lib.rs:519-563),
// bit-exact on codes and scales. The reference makes two passes over the
// weights (row absmax, then encode with an IEEE divide per element); here one
// workgroup owns a row at a time, holds it in registers between the two
// phases and so reads HBM once: rows*cols*(in_bytes + 1) + 4*rows bytes.
//
// Fast path (a row whose scale s and 1/s are normal f32 and that holds no NaN):
//   r = RN(1/s); if r*s == 1 exactly, x*r IS RN(x/s) and one conversion suffices.
//   Otherwise r_lo = r - 1ulp <= 1/s <= r_hi = r + 1ulp, so by monotonicity of
//   rounding RN(x*r_lo) <= RN(x/s) <= RN(x*r_hi) in magnitude; the fp8 code is
//   monotone in magnitude, so when both ends give the same code it is the code
//   of RN(x/s). The two ends go through v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32
//   (OCP e4m3 / e5m2, round to nearest even), which agree with reng-fp8's
//   encoder on every input of magnitude <= max finite (240 / 57344): checked
//   on all 2^32 patterns by reng_hip_verify_hw_convert. Inputs that could
//   exceed that range are clamped first with v_med3 (saturation is monotone).
//   A lane whose ends disagree (an fp8 midpoint within ~2 ulps; a few in a
//   million) recomputes its vector with the IEEE divide and the exact encoder.
// Slow rows (NaN present, s = inf / 0 / subnormal) use the IEEE divide and the
// exact encoder for every element, with x86's NaN semantics.
#include "common.h"
#include "quantize.h"

namespace reng {

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int F>
__device__ __forceinline__ uint32_t exact4(float x0, float x1, float x2, float x3, float s) {
    return encode_div<F>(x0, s) | (encode_div<F>(x1, s) << 8) | (encode_div<F>(x2, s) << 16) |
           (encode_div<F>(x3, s) << 24);
}

// Block-wide max of a u32; every thread gets the result. red has one slot per wave.
template <int WAVES>
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t *red) {
    v = wave_max_u32(v);
    if constexpr (WAVES == 1) {
        return v;
    } else {
        const int w = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) red[w] = v;
        __syncthreads();
        uint32_t m = red[0];
#pragma unroll
        for (int i = 1; i < WAVES; ++i) m = m > red[i] ? m : red[i];
        __syncthreads();
        return m;
    }
}

template <typename InT>
struct InTraits;
template <>
struct InTraits<uint16_t> {   // bf16 bits
    static constexpr int EPV = 8;
    static constexpr uint32_t INF = 0x7f80u;
    __device__ static float f(uint32_t b) { return __uint_as_float(b << 16); }
};
template <>
struct InTraits<float> {
    static constexpr int EPV = 4;
    static constexpr uint32_t INF = 0x7f800000u;
    __device__ static float f(uint32_t b) { return __uint_as_float(b); }
};

// Scale of one row from its absmax bits, per scheme (lib.rs:537-551); the
// hardware-bias and unit scales arrive precomputed per matrix.
template <typename InT>
__device__ __forceinline__ float row_scale(uint32_t mbits, int scheme, float full,
                                           const float *fixed_scale, int mi) {
    if (scheme == RENG_HIP_PCS) {
        const float m = sizeof(InT) == 2 ? __uint_as_float(mbits << 16) : __uint_as_float(mbits);
        return m > 0.0f ? m / full : 1.0f;
    }
    return fixed_scale ? fixed_scale[mi] : 1.0f;
}

// One workgroup (WAVES waves) per row at a time, VPT 16-byte vectors per thread
// held in registers. Requires: 16-byte aligned rows, cols a multiple of EPV,
// codes rows aligned to the store width.
template <typename InT, int F, int VPT, int WAVES, bool CLAMP>
__global__ __launch_bounds__(64 * WAVES) void quantize_rows_fast(QBatch B, int scheme, float full,
                                                                  const float *__restrict__ fixed_scale,
                                                                  const uint32_t *__restrict__ fixed_bias) {
    using IT = InTraits<InT>;
    constexpr int EPV = IT::EPV;
    constexpr int T = 64 * WAVES;
    __shared__ uint32_t red[WAVES];
    const int tid = threadIdx.x;
    for (uint64_t g = blockIdx.x; g < B.total_rows; g += gridDim.x) {
        int mi = 0;
        while (mi + 1 < B.n && g >= B.m[mi + 1].row_begin) ++mi;
        const QMat &M = B.m[mi];
        const uint64_t row = g - M.row_begin;
        const u32x4 *src = reinterpret_cast<const u32x4 *>(static_cast<const InT *>(M.w) + row * M.ld);
        const int nvec = (int)(M.cols / EPV);

        u32x4 v[VPT];
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = j * T + tid;
            v[j] = i < nvec ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
        }

        // Phase 1: row absmax on the magnitude bits (NaN patterns sort above inf).
        uint32_t mx = 0;
        if constexpr (sizeof(InT) == 2) {
            u16x2 m2 = {0, 0};
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    m2 = __builtin_elementwise_max(m2, __builtin_bit_cast(u16x2, d[k] & 0x7fff7fffu));
            }
            mx = m2.x > m2.y ? m2.x : m2.y;
        } else {
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t a = d[k] & 0x7fffffffu;
                    mx = mx > a ? mx : a;
                }
            }
        }
        mx = block_max<WAVES>(mx, red);
        const bool has_nan = mx > IT::INF;
        if (has_nan) {   // uniform: recompute ignoring NaN (lib.rs:451-454, `v > m`)
            mx = 0;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (sizeof(InT) == 2) {
                        const uint32_t lo = d[k] & 0x7fffu, hi = (d[k] >> 16) & 0x7fffu;
                        if (lo <= IT::INF && lo > mx) mx = lo;
                        if (hi <= IT::INF && hi > mx) mx = hi;
                    } else {
                        const uint32_t a = d[k] & 0x7fffffffu;
                        if (a <= IT::INF && a > mx) mx = a;
                    }
                }
            }
            mx = block_max<WAVES>(mx, red);
        }
        const float s = row_scale<InT>(mx, scheme, full, fixed_scale, mi);
        if (tid == 0) {
            M.scales[row] = s;
            if (row == 0 && M.exp_bias)
                *M.exp_bias = fixed_bias ? fixed_bias[mi] : (uint32_t)Fp8<F>::BIAS;
        }

        // Phase 2: encode from registers.
        uint8_t *dst = M.codes + row * M.cols;
        const bool fast = !has_nan && s >= 0x1p-125f && s <= 0x1p125f;
        if (fast) {
            const float r = 1.0f / s;
            const bool exact = __builtin_fmaf(r, s, -1.0f) == 0.0f;
            const float r_hi = exact ? r : __uint_as_float(__float_as_uint(r) + 1u);
            const float r_lo = exact ? r : __uint_as_float(__float_as_uint(r) - 1u);
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const int i = j * T + tid;
                if (i >= nvec) continue;
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
                if constexpr (sizeof(InT) == 2) {
                    float x[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        x[2 * k] = __uint_as_float(d[k] << 16);
                        x[2 * k + 1] = __uint_as_float(d[k] & 0xffff0000u);
                    }
                    uint32_t h0 = cvt4<F, CLAMP>(x[0] * r_hi, x[1] * r_hi, x[2] * r_hi, x[3] * r_hi);
                    uint32_t h1 = cvt4<F, CLAMP>(x[4] * r_hi, x[5] * r_hi, x[6] * r_hi, x[7] * r_hi);
                    if (!exact) {
                        const uint32_t l0 = cvt4<F, CLAMP>(x[0] * r_lo, x[1] * r_lo, x[2] * r_lo, x[3] * r_lo);
                        const uint32_t l1 = cvt4<F, CLAMP>(x[4] * r_lo, x[5] * r_lo, x[6] * r_lo, x[7] * r_lo);
                        if ((h0 ^ l0) | (h1 ^ l1)) {
                            h0 = exact4<F>(x[0], x[1], x[2], x[3], s);
                            h1 = exact4<F>(x[4], x[5], x[6], x[7], s);
                        }
                    }
                    __builtin_nontemporal_store(u32x2{h0, h1}, reinterpret_cast<u32x2 *>(dst) + i);
                } else {
                    const float x0 = __uint_as_float(d[0]), x1 = __uint_as_float(d[1]);
                    const float x2 = __uint_as_float(d[2]), x3 = __uint_as_float(d[3]);
                    uint32_t h = cvt4<F, CLAMP>(x0 * r_hi, x1 * r_hi, x2 * r_hi, x3 * r_hi);
                    if (!exact) {
                        const uint32_t l = cvt4<F, CLAMP>(x0 * r_lo, x1 * r_lo, x2 * r_lo, x3 * r_lo);
                        if (h ^ l) h = exact4<F>(x0, x1, x2, x3, s);
                    }
                    __builtin_nontemporal_store(h, reinterpret_cast<uint32_t *>(dst) + i);
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const int i = j * T + tid;
                if (i >= nvec) continue;
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
                if constexpr (sizeof(InT) == 2) {
                    const uint32_t h0 = exact4<F>(IT::f(d[0] & 0xffffu), IT::f(d[0] >> 16),
                                                  IT::f(d[1] & 0xffffu), IT::f(d[1] >> 16), s);
                    const uint32_t h1 = exact4<F>(IT::f(d[2] & 0xffffu), IT::f(d[2] >> 16),
                                                  IT::f(d[3] & 0xffffu), IT::f(d[3] >> 16), s);
                    reinterpret_cast<u32x2 *>(dst)[i] = u32x2{h0, h1};
                } else {
                    reinterpret_cast<uint32_t *>(dst)[i] =
                        exact4<F>(IT::f(d[0]), IT::f(d[1]), IT::f(d[2]), IT::f(d[3]), s);
                }
            }
        }
    }
}

// Any shape, pitch and alignment: 256 threads per row, absmax then the exact
// divide-and-encode for every element (the row is read twice, from L2).
template <typename InT, int F>
__global__ __launch_bounds__(256) void quantize_rows_generic(QBatch B, int scheme, float full,
                                                             const float *__restrict__ fixed_scale,
                                                             const uint32_t *__restrict__ fixed_bias) {
    using IT = InTraits<InT>;
    __shared__ uint32_t red[4];
    const int tid = threadIdx.x;
    for (uint64_t g = blockIdx.x; g < B.total_rows; g += gridDim.x) {
        int mi = 0;
        while (mi + 1 < B.n && g >= B.m[mi + 1].row_begin) ++mi;
        const QMat &M = B.m[mi];
        const uint64_t row = g - M.row_begin;
        const InT *src = static_cast<const InT *>(M.w) + row * M.ld;
        uint32_t mx = 0;
        for (uint64_t c = tid; c < M.cols; c += 256) {
            uint32_t b;
            if constexpr (sizeof(InT) == 2) b = src[c] & 0x7fffu;
            else b = __float_as_uint(src[c]) & 0x7fffffffu;
            if (b <= IT::INF && b > mx) mx = b;
        }
        mx = block_max<4>(mx, red);
        const float s = row_scale<InT>(mx, scheme, full, fixed_scale, mi);
        if (tid == 0) {
            M.scales[row] = s;
            if (row == 0 && M.exp_bias)
                *M.exp_bias = fixed_bias ? fixed_bias[mi] : (uint32_t)Fp8<F>::BIAS;
        }
        uint8_t *dst = M.codes + row * M.cols;
        for (uint64_t c = tid; c < M.cols; c += 256) {
            float x;
            if constexpr (sizeof(InT) == 2) x = IT::f(src[c]);
            else x = src[c];
            dst[c] = (uint8_t)encode_div<F>(x, s);
        }
    }
}

// Row absmax (NaN ignored, inf counted) for reng_hip_row_absmax, and the
// per-matrix tensor absmax (as magnitude bits, atomic max) for the
// hardware-bias scheme. out may be NULL; tmax may be NULL.
template <typename InT>
__global__ __launch_bounds__(256) void row_absmax_kernel(QBatch B, float *__restrict__ out,
                                                         uint32_t *__restrict__ tmax) {
    using IT = InTraits<InT>;
    __shared__ uint32_t red[4];
    const int tid = threadIdx.x;
    for (uint64_t g = blockIdx.x; g < B.total_rows; g += gridDim.x) {
        int mi = 0;
        while (mi + 1 < B.n && g >= B.m[mi + 1].row_begin) ++mi;
        const QMat &M = B.m[mi];
        const uint64_t row = g - M.row_begin;
        const InT *src = static_cast<const InT *>(M.w) + row * M.ld;
        uint32_t mx = 0;
        const bool vec = ((reinterpret_cast<uintptr_t>(src) & 15) == 0) && (M.cols % IT::EPV == 0);
        if (vec) {
            const uint4 *s4 = reinterpret_cast<const uint4 *>(src);
            for (uint64_t i = tid; i < M.cols / IT::EPV; i += 256) {
                const uint4 q = s4[i];
                const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (sizeof(InT) == 2) {
                        const uint32_t lo = d[k] & 0x7fffu, hi = (d[k] >> 16) & 0x7fffu;
                        if (lo <= IT::INF && lo > mx) mx = lo;
                        if (hi <= IT::INF && hi > mx) mx = hi;
                    } else {
                        const uint32_t a = d[k] & 0x7fffffffu;
                        if (a <= IT::INF && a > mx) mx = a;
                    }
                }
            }
        } else {
            for (uint64_t c = tid; c < M.cols; c += 256) {
                uint32_t b;
                if constexpr (sizeof(InT) == 2) b = src[c] & 0x7fffu;
                else b = __float_as_uint(src[c]) & 0x7fffffffu;
                if (b <= IT::INF && b > mx) mx = b;
            }
        }
        mx = block_max<4>(mx, red);
        if (tid == 0) {
            if (out) out[g] = sizeof(InT) == 2 ? __uint_as_float(mx << 16) : __uint_as_float(mx);
            if (tmax) atomicMax(tmax + mi, mx);
        }
    }
}

__global__ void zero_u32_kernel(uint32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Per matrix: b = choose_exp_bias(tensor_absmax / backoff), s = 2^(bias - b)
// (lib.rs:545-549).
template <typename InT, int F>
__global__ void hw_bias_kernel(QBatch B, const uint32_t *__restrict__ tmax, float backoff,
                               float *__restrict__ scale_out, uint32_t *__restrict__ bias_out) {
    const int mi = threadIdx.x;
    if (mi >= B.n) return;
    const uint32_t mb = tmax[mi];
    const float tm = sizeof(InT) == 2 ? __uint_as_float(mb << 16) : __uint_as_float(mb);
    const uint32_t b = choose_exp_bias_t<F>(tm / backoff);
    scale_out[mi] = pow2f(Fp8<F>::BIAS - (int)b);
    bias_out[mi] = b;
}

// ------------------------------------------------------------ host launchers

namespace {

struct FastCfg {
    int vpt, waves;
};

// Vectors per thread and waves per row for a row of nvec 16-byte vectors:
// the least padding, then the fewest waves (a single wave needs no LDS).
FastCfg pick_cfg(uint64_t nvec) {
    static const int VPTS[] = {1, 2, 4, 5, 6, 7, 8};
    FastCfg best{0, 0};
    uint64_t best_waste = ~0ull;
    for (int vpt : VPTS) {
        uint64_t waves = (nvec + 64ull * vpt - 1) / (64ull * vpt);
        if (waves < 1) waves = 1;
        if (waves > 16) continue;
        if (waves == 3 || waves == 5 || waves == 6 || waves == 7 || (waves > 8 && waves != 16)) {
            // keep the instantiated set small: 1, 2, 4, 8, 16 waves
            uint64_t w2 = 1;
            while (w2 < waves) w2 <<= 1;
            waves = w2;
        }
        const uint64_t waste = waves * 64ull * vpt - nvec;
        if (waste < best_waste || (waste == best_waste && (int)waves < best.waves)) {
            best_waste = waste;
            best = FastCfg{vpt, (int)waves};
        }
    }
    return best;
}

template <typename InT, int F, int VPT, int WAVES, bool CLAMP>
int launch_fast_t(const QBatch &b, int scheme, float full, const float *fs, const uint32_t *fb,
                  hipStream_t st) {
    auto kern = quantize_rows_fast<InT, F, VPT, WAVES, CLAMP>;
    int per_cu = 0;
    RENG_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 64 * WAVES, 0));
    if (per_cu < 1) per_cu = 1;
    uint64_t grid = (uint64_t)device_props().cus * per_cu;
    if (grid > b.total_rows) grid = b.total_rows;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * WAVES), 0, st, b, scheme, full, fs, fb);
    return check_launch("quantize_rows_fast");
}

template <typename InT, int F, int VPT, bool CLAMP>
int launch_fast_w(int waves, const QBatch &b, int scheme, float full, const float *fs,
                  const uint32_t *fb, hipStream_t st) {
    switch (waves) {
        case 1: return launch_fast_t<InT, F, VPT, 1, CLAMP>(b, scheme, full, fs, fb, st);
        case 2: return launch_fast_t<InT, F, VPT, 2, CLAMP>(b, scheme, full, fs, fb, st);
        case 4: return launch_fast_t<InT, F, VPT, 4, CLAMP>(b, scheme, full, fs, fb, st);
        case 8: return launch_fast_t<InT, F, VPT, 8, CLAMP>(b, scheme, full, fs, fb, st);
        case 16: return launch_fast_t<InT, F, VPT, 16, CLAMP>(b, scheme, full, fs, fb, st);
    }
    set_error("internal: no kernel for %d waves", waves);
    return RENG_HIP_EUNSUPPORTED;
}

template <typename InT, int F, bool CLAMP>
int launch_fast_v(FastCfg c, const QBatch &b, int scheme, float full, const float *fs,
                  const uint32_t *fb, hipStream_t st) {
    switch (c.vpt) {
        case 1: return launch_fast_w<InT, F, 1, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 2: return launch_fast_w<InT, F, 2, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 4: return launch_fast_w<InT, F, 4, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 5: return launch_fast_w<InT, F, 5, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 6: return launch_fast_w<InT, F, 6, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 7: return launch_fast_w<InT, F, 7, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
        case 8: return launch_fast_w<InT, F, 8, CLAMP>(c.waves, b, scheme, full, fs, fb, st);
    }
    set_error("internal: no kernel for %d vectors per thread", c.vpt);
    return RENG_HIP_EUNSUPPORTED;
}

template <typename InT, int F>
int launch_group(const QBatch &b, int key, int scheme, float full, bool clamp, const float *fs,
                 const uint32_t *fb, hipStream_t st) {
    if (key >= 0) {
        const FastCfg c{key / 100, key % 100};
        return clamp ? launch_fast_v<InT, F, true>(c, b, scheme, full, fs, fb, st)
                     : launch_fast_v<InT, F, false>(c, b, scheme, full, fs, fb, st);
    }
    uint64_t grid = (uint64_t)device_props().cus * 8;
    if (grid > b.total_rows) grid = b.total_rows;
    hipLaunchKernelGGL((quantize_rows_generic<InT, F>), dim3((unsigned)grid), dim3(256), 0, st, b,
                       scheme, full, fs, fb);
    return check_launch("quantize_rows_generic");
}

template <typename InT>
int launch_absmax(const QBatch &b, float *out, uint32_t *tmax, hipStream_t st) {
    uint64_t grid = (uint64_t)device_props().cus * 8;
    if (grid > b.total_rows) grid = b.total_rows;
    hipLaunchKernelGGL(row_absmax_kernel<InT>, dim3((unsigned)grid), dim3(256), 0, st, b, out, tmax);
    return check_launch("row_absmax");
}

}  // namespace

// The register-resident kernel configuration of a matrix (vpt * 100 + waves),
// or -1 when it must take the generic kernel (misaligned rows or codes, cols
// not a multiple of the vector width, rows wider than 16 waves x 8 vectors).
int fast_key(const QMat &m, int dtype) {
    const size_t eb = dtype == RENG_HIP_BF16 ? 2 : 4;
    const size_t epv = 16 / eb;
    const size_t store = dtype == RENG_HIP_BF16 ? 8 : 4;
    if (m.cols == 0 || m.cols % epv != 0) return -1;
    if ((reinterpret_cast<uintptr_t>(m.w) & 15) != 0) return -1;
    if ((m.ld * eb) % 16 != 0) return -1;
    if ((reinterpret_cast<uintptr_t>(m.codes) & (store - 1)) != 0) return -1;
    const uint64_t nvec = m.cols / epv;
    if (nvec > 16ull * 64 * 8) return -1;
    const FastCfg c = pick_cfg(nvec);
    return c.vpt > 0 ? c.vpt * 100 + c.waves : -1;
}

int launch_quantize_group(const QBatch &b, int dtype, int format, int scheme, float backoff,
                          int key, hipStream_t st) {
    // Scale inputs: PCS needs full = max_finite * backoff (lib.rs:535); HW needs
    // the per-matrix tensor absmax first (lib.rs:536, 545-549); UNIT is s = 1.
    const float maxf = format == RENG_HIP_E4M3 ? 240.0f : 57344.0f;
    const float full = maxf * backoff;
    const float *fs = nullptr;
    const uint32_t *fb = nullptr;
    if (scheme == RENG_HIP_HW) {
        uint32_t *ws = nullptr;
        RENG_CHECK_HIP(hipMallocAsync(reinterpret_cast<void **>(&ws), 3 * QBATCH * sizeof(uint32_t), st));
        uint32_t *tmax = ws;
        float *scl = reinterpret_cast<float *>(ws + QBATCH);
        uint32_t *bias = ws + 2 * QBATCH;
        hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(QBATCH), 0, st, tmax, QBATCH);
        int rc = check_launch("zero");
        if (rc) return rc;
        rc = dtype == RENG_HIP_BF16 ? launch_absmax<uint16_t>(b, nullptr, tmax, st)
                                    : launch_absmax<float>(b, nullptr, tmax, st);
        if (rc) return rc;
        if (dtype == RENG_HIP_BF16) {
            if (format == RENG_HIP_E4M3)
                hipLaunchKernelGGL((hw_bias_kernel<uint16_t, RENG_HIP_E4M3>), dim3(1), dim3(QBATCH), 0, st, b, tmax, backoff, scl, bias);
            else
                hipLaunchKernelGGL((hw_bias_kernel<uint16_t, RENG_HIP_E5M2>), dim3(1), dim3(QBATCH), 0, st, b, tmax, backoff, scl, bias);
        } else {
            if (format == RENG_HIP_E4M3)
                hipLaunchKernelGGL((hw_bias_kernel<float, RENG_HIP_E4M3>), dim3(1), dim3(QBATCH), 0, st, b, tmax, backoff, scl, bias);
            else
                hipLaunchKernelGGL((hw_bias_kernel<float, RENG_HIP_E5M2>), dim3(1), dim3(QBATCH), 0, st, b, tmax, backoff, scl, bias);
        }
        rc = check_launch("hw_bias");
        if (rc) return rc;
        fs = scl;
        fb = bias;
    }
    // The conversions are only exact up to the format's largest finite value;
    // per-channel scales with backoff <= 1 keep |x / s| <= max_finite * (1 + 2^-22),
    // which rounds to the largest code without a clamp.
    const bool clamp = !(scheme == RENG_HIP_PCS && backoff <= 1.0f);
    int rc;
    if (dtype == RENG_HIP_BF16) {
        rc = format == RENG_HIP_E4M3
                 ? launch_group<uint16_t, RENG_HIP_E4M3>(b, key, scheme, full, clamp, fs, fb, st)
                 : launch_group<uint16_t, RENG_HIP_E5M2>(b, key, scheme, full, clamp, fs, fb, st);
    } else {
        rc = format == RENG_HIP_E4M3
                 ? launch_group<float, RENG_HIP_E4M3>(b, key, scheme, full, clamp, fs, fb, st)
                 : launch_group<float, RENG_HIP_E5M2>(b, key, scheme, full, clamp, fs, fb, st);
    }
    if (fs) {
        // The partials were allocated on this stream; the free is ordered after the encode.
        const hipError_t e = hipFreeAsync(const_cast<float *>(fs) - QBATCH, st);
        if (rc == RENG_HIP_OK && e != hipSuccess) {
            set_error("hipFreeAsync: %s", hipGetErrorString(e));
            rc = RENG_HIP_EDEVICE;
        }
    }
    return rc;
}

int launch_row_absmax(const QBatch &b, int dtype, float *out, hipStream_t st) {
    return dtype == RENG_HIP_BF16 ? launch_absmax<uint16_t>(b, out, nullptr, st)
                                  : launch_absmax<float>(b, out, nullptr, st);
}

}  // namespace reng
