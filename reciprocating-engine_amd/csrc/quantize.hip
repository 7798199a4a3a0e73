// quantize.hip - the fp8 weight quantizer on CDNA4 (gfx950).
//
// Semantics: reng_fp8::quantize_with (crates/reng-fp8/src/lib.rs:519-563),
// bit-exact on codes and scales. The reference makes two passes over the
// weights (row absmax, then encode with an IEEE divide per element); here one
// workgroup owns a row at a time, holds it in registers between the two
// phases and so reads HBM once: rows*cols*(in_bytes + 1) + 4*rows bytes.
//
// Fast path (a row with no NaN and a finite normal scale s): q = RN32(x * RN64(1/s))
// computed in f64 IS the IEEE f32 quotient
// RN32(x / s) that the reference encodes, for every finite x:
//   * x * RN64(1/s) is within |z| * 2^-52 of z = x / s (two f64 roundings);
//   * the quotient of two 24-bit floats is never an f32 midpoint, and when it
//     is not one it lies more than ulp(z) * 2^-25 >= |z| * 2^-49 away from
//     every midpoint (z - t = (X * 2^a - T * S * 2^b) / (S * 2^c) with integer
//     significands X, S < 2^24 and a 25-bit midpoint significand T), so the f64
//     value rounds to the same f32 as z does.
// The f32 quotient then goes through v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 (OCP
// e4m3 / e5m2, round to nearest even), which agree with reng-fp8's encoder on
// every input of magnitude below the first out-of-range midpoint (248 /
// 61440): checked on all 2^32 patterns by reng_hip_verify_hw_convert. Inputs
// that could reach that range (HW and UNIT scales, or a backoff above 1) are
// clamped first with v_med3 (saturation is monotone). A per-channel scale
// s = RN32(m / (max * backoff)) that is normal is within 2^-24 of the exact
// ratio, so with backoff <= 1 no |x / s| passes max * (1 + 2^-23) and no clamp
// is needed; a subnormal s carries fewer significant bits (s = 4 * 2^-149 for
// m = 1000 * 2^-149, E4M3: x / s = 250), so those rows take the slow path.
// Slow rows (a NaN present, s = inf, 0 or subnormal) use the IEEE divide and
// the exact integer encoder for every element, with x86's NaN semantics.
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

// RN32(x * R) through f64: R = RN64(1/s), the product and the narrowing are
// each rounded to nearest even.
__device__ __forceinline__ float quot(float x, double R) { return (float)((double)x * R); }

__device__ __forceinline__ float bf_lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf_hi(uint32_t d) { return __uint_as_float(d & 0xffff0000u); }

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

// One row per workgroup (WAVES waves) at a time, VPT 16-byte vectors per thread
// held in registers between the absmax and the encode. Requires 16-byte
// aligned rows, cols a multiple of EPV and codes rows aligned to the store
// width. FULL: every row fills exactly VPT * 64 * WAVES vectors (no tail
// predication).
template <typename InT, int F, int VPT, int WAVES, bool CLAMP, bool FULL>
__global__ __launch_bounds__(64 * WAVES) void quantize_rows_fast(QBatch B, int scheme, float full,
                                                                  const float *__restrict__ fixed_scale,
                                                                  const uint32_t *__restrict__ fixed_bias) {
    using IT = InTraits<InT>;
    constexpr int EPV = IT::EPV;
    constexpr int CPV = EPV / 4;                 // code dwords per vector: 2 (bf16), 1 (f32)
    constexpr int T = 64 * WAVES;
    __shared__ uint32_t red[WAVES];
    const int tid = threadIdx.x;
    const uint64_t G = gridDim.x;
    uint64_t g = blockIdx.x;
    if (g >= B.total_rows) return;

    // Row g lives in matrix mi; rows only grow, so the lookup only moves forward.
    auto locate = [&](uint64_t gg, int &mi) {
        while (mi + 1 < B.n && gg >= B.m[mi + 1].row_begin) ++mi;
    };
    auto row_src = [&](uint64_t gg, int mi) {
        const QMat &M = B.m[mi];
        return reinterpret_cast<const u32x4 *>(static_cast<const InT *>(M.w) + (gg - M.row_begin) * M.ld);
    };
    auto load = [&](const u32x4 *src, int nvec, u32x4 (&v)[VPT]) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = j * T + tid;
            if (FULL || i < nvec) v[j] = __builtin_nontemporal_load(src + i);
            else v[j] = u32x4{0u, 0u, 0u, 0u};
        }
    };

    int mi = 0;
    locate(g, mi);
    u32x4 v[VPT];
    load(row_src(g, mi), (int)(B.m[mi].cols / EPV), v);
    for (; g < B.total_rows; g += G) {
        const QMat &M = B.m[mi];
        const uint64_t row = g - M.row_begin;
        const int nvec = (int)(M.cols / EPV);

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
                const uint32_t a0 = v[j].x & 0x7fffffffu, a1 = v[j].y & 0x7fffffffu;
                const uint32_t a2 = v[j].z & 0x7fffffffu, a3 = v[j].w & 0x7fffffffu;
                mx = max(max(mx, max(a0, a1)), max(a2, a3));
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
        // The next row's loads go out before this row's encode and stores.
        u32x4 vn[VPT];
        const bool more = g + G < B.total_rows;
        if (more) {
            locate(g + G, mi);
            load(row_src(g + G, mi), (int)(B.m[mi].cols / EPV), vn);
        }

        // Phase 2: codes from registers. q = RN32(x * RN64(1/s)) equals the
        // IEEE f32 quotient RN32(x / s) for every finite x and every finite
        // non-zero s (see the top of this file), so each code is one f64
        // multiply and one hardware conversion; rows whose s is subnormal
        // (fewer significant bits: |x / s| may pass the clamp-free range) or
        // not finite and positive take the exact path.
        uint32_t c[VPT][CPV];
        const bool fast = !has_nan && s >= 1.17549435e-38f && s < __builtin_inff();
        if (fast) {
            const double R = 1.0 / (double)s;
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
                if constexpr (sizeof(InT) == 2) {
                    c[j][0] = cvt4<F, CLAMP>(quot(bf_lo(d[0]), R), quot(bf_hi(d[0]), R),
                                             quot(bf_lo(d[1]), R), quot(bf_hi(d[1]), R));
                    c[j][1] = cvt4<F, CLAMP>(quot(bf_lo(d[2]), R), quot(bf_hi(d[2]), R),
                                             quot(bf_lo(d[3]), R), quot(bf_hi(d[3]), R));
                } else {
                    c[j][0] = cvt4<F, CLAMP>(quot(__uint_as_float(d[0]), R), quot(__uint_as_float(d[1]), R),
                                             quot(__uint_as_float(d[2]), R), quot(__uint_as_float(d[3]), R));
                }
            }
        } else {
            // Slow row: a NaN is present, or s is infinite or zero; the IEEE
            // divide with x86's NaN semantics for every element.
#pragma unroll
            for (int j = 0; j < VPT; ++j) {
                const uint32_t d[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
                if constexpr (sizeof(InT) == 2) {
                    c[j][0] = exact4<F>(bf_lo(d[0]), bf_hi(d[0]), bf_lo(d[1]), bf_hi(d[1]), s);
                    c[j][1] = exact4<F>(bf_lo(d[2]), bf_hi(d[2]), bf_lo(d[3]), bf_hi(d[3]), s);
                } else {
                    c[j][0] = exact4<F>(__uint_as_float(d[0]), __uint_as_float(d[1]),
                                        __uint_as_float(d[2]), __uint_as_float(d[3]), s);
                }
            }
        }
        uint8_t *dst = M.codes + row * M.cols;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int i = j * T + tid;
            if (FULL || i < nvec) {
                if constexpr (CPV == 2)
                    __builtin_nontemporal_store(u32x2{c[j][0], c[j][1]}, reinterpret_cast<u32x2 *>(dst) + i);
                else
                    __builtin_nontemporal_store(c[j][0], reinterpret_cast<uint32_t *>(dst) + i);
            }
        }

        if (more) {
#pragma unroll
            for (int j = 0; j < VPT; ++j) v[j] = vn[j];
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
    bool full;
};

// Exact fits (no tail predication) for the row widths of the Llama / Qwen
// shapes: bf16 1024, 2048, 3584, 4096, 5120, 8192, 14336, 16384, 27648 and
// f32 2048, 8192 columns. Rows of 14336 run as 4 waves of 7 vectors (5.86
// TB/s on the Llama-3.1-8B set against 5.66-5.68 for 7 waves of 4), rows of
// 27648 as 9 waves of 6 (5.74-5.76 TB/s on the Qwen2.5-32B set against 5.69
// for 6 waves of 9).
constexpr FastCfg FULL_CFGS[] = {{8, 1, true}, {7, 1, true}, {7, 4, true}, {5, 2, true}, {8, 2, true},
                                 {8, 4, true}, {6, 9, true}, {2, 1, true}, {4, 1, true}};

FastCfg pick_cfg(uint64_t nvec) {
    for (const FastCfg &c : FULL_CFGS)
        if ((uint64_t)c.vpt * 64 * c.waves == nvec) return c;
    if (nvec <= 512) {
        int vpt = 1;
        while ((uint64_t)vpt * 64 < nvec) vpt <<= 1;
        return FastCfg{vpt, 1, false};
    }
    int waves = 1;
    while ((uint64_t)waves * 512 < nvec) waves <<= 1;
    if (waves > 16) return FastCfg{0, 0, false};
    return FastCfg{8, waves, false};
}

int encode_key(const FastCfg &c) { return c.vpt * 1000 + c.waves * 10 + (c.full ? 1 : 0); }

// Waves per CU for the register-resident kernel: enough rows in flight to keep
// HBM busy, few enough that the rows being read and written at one time stay
// close together (measured on MI355X: 8 waves per CU beat full occupancy; 6
// for one-wave rows of 8 vectors per lane, i.e. 4096 bf16 or 2048 f32 values:
// rows of 4096 on the Llama-3.1-8B set 5.74-5.75 -> 5.97-5.98 TB/s; 10 for
// two-wave rows of 5 vectors, i.e. 5120 bf16: 5.43-5.59 -> 5.79 TB/s on the
// Qwen2.5-32B shapes).
constexpr int QUANT_WAVES_PER_CU = 8;
template <int VPT, int WAVES>
constexpr int quant_waves_per_cu() {
    if constexpr (WAVES == 1 && VPT == 8) return 6;
    else if constexpr (WAVES == 2 && VPT == 5) return 10;
    else return QUANT_WAVES_PER_CU;
}

template <typename InT, int F, int VPT, int WAVES, bool CLAMP, bool FULL>
int launch_fast_t(const QBatch &b, int scheme, float full, const float *fs, const uint32_t *fb,
                  hipStream_t st) {
    auto kern = quantize_rows_fast<InT, F, VPT, WAVES, CLAMP, FULL>;
    const uint64_t cus = (uint64_t)device_props().cus;
    constexpr int WPC = quant_waves_per_cu<VPT, WAVES>();
    uint64_t grid = cus * ((WPC + WAVES - 1) / WAVES);
    // A launch of at most 8 waves' worth of rows per CU (the f32 [2048, 2048]
    // matrix) is latency-bound: every row in flight at once.
    if (b.total_rows <= cus * ((QUANT_WAVES_PER_CU + WAVES - 1) / WAVES) || grid > b.total_rows) grid = b.total_rows;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(64 * WAVES), 0, st, b, scheme, full, fs, fb);
    return check_launch("quantize_rows_fast");
}

template <typename InT, int F, bool CLAMP>
int launch_fast(int key, const QBatch &b, int scheme, float full, const float *fs,
                const uint32_t *fb, hipStream_t st) {
#define RENG_Q(V, W, FU)                                                                       \
    case V * 1000 + W * 10 + FU:                                                                \
        return launch_fast_t<InT, F, V, W, CLAMP, FU>(b, scheme, full, fs, fb, st);
    switch (key) {
        RENG_Q(8, 1, 1) RENG_Q(7, 1, 1) RENG_Q(7, 4, 1) RENG_Q(5, 2, 1) RENG_Q(8, 2, 1)
        RENG_Q(8, 4, 1) RENG_Q(6, 9, 1) RENG_Q(2, 1, 1) RENG_Q(4, 1, 1)
        RENG_Q(1, 1, 0) RENG_Q(2, 1, 0) RENG_Q(4, 1, 0) RENG_Q(8, 1, 0) RENG_Q(8, 2, 0)
        RENG_Q(8, 4, 0) RENG_Q(8, 8, 0) RENG_Q(8, 16, 0)
    }
#undef RENG_Q
    set_error("internal: no quantize kernel for configuration %d", key);
    return RENG_HIP_EUNSUPPORTED;
}

template <typename InT, int F>
int launch_group(const QBatch &b, int key, int scheme, float full, bool clamp, const float *fs,
                 const uint32_t *fb, hipStream_t st) {
    if (key >= 0) {
        return clamp ? launch_fast<InT, F, true>(key, b, scheme, full, fs, fb, st)
                     : launch_fast<InT, F, false>(key, b, scheme, full, fs, fb, st);
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

// The register-resident kernel configuration of a matrix (encode_key),
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
    const FastCfg c = pick_cfg(m.cols / epv);
    return c.vpt > 0 ? encode_key(c) : -1;
}

int launch_quantize_group(const QBatch &b, int dtype, int format, int scheme, float backoff,
                          int key, hipStream_t st) {
    // Scale inputs: PCS needs full = max_finite * backoff (lib.rs:535); HW needs
    // the per-matrix tensor absmax first (lib.rs:536, 545-549); UNIT is s = 1.
    const float maxf = format == RENG_HIP_E4M3 ? 240.0f : 57344.0f;
    const float full = maxf * backoff;
    const float *fs = nullptr;
    const uint32_t *fb = nullptr;
    uint32_t *ws = nullptr;   // the HW scheme's tensor maxima, scales and biases
    if (scheme == RENG_HIP_HW) {
        RENG_CHECK_HIP(hipMallocAsync(reinterpret_cast<void **>(&ws), 3 * QBATCH * sizeof(uint32_t), st));
        uint32_t *tmax = ws;
        float *scl = reinterpret_cast<float *>(ws + QBATCH);
        uint32_t *bias = ws + 2 * QBATCH;
        hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(QBATCH), 0, st, tmax, QBATCH);
        int rc = check_launch("zero");
        if (rc == RENG_HIP_OK)
            rc = dtype == RENG_HIP_BF16 ? launch_absmax<uint16_t>(b, nullptr, tmax, st)
                                        : launch_absmax<float>(b, nullptr, tmax, st);
        if (rc == RENG_HIP_OK) {
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
        }
        if (rc != RENG_HIP_OK) {
            // Ordered after whatever of the above was enqueued; the launch error is the one reported.
            (void)hipFreeAsync(ws, st);
            return rc;
        }
        fs = scl;
        fb = bias;
    }
    // The conversions are only exact up to the format's largest finite value;
    // per-channel scales with backoff <= 1 keep |x / s| <= max_finite * (1 + 2^-23)
    // for a normal s, which rounds to the largest code without a clamp (the
    // kernel sends rows with a subnormal s to its exact path).
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
    if (ws) {
        // Allocated on this stream: the free is ordered after the encode.
        const hipError_t e = hipFreeAsync(ws, st);
        if (rc == RENG_HIP_OK && e != hipSuccess) {
            set_error("hipFreeAsync: %s", hipGetErrorString(e));
            rc = RENG_HIP_EDEVICE;
        }
    }
    return rc;
}

// ------------------------------------------------------------------ stream yardstick

// The quantizer's memory stream with no arithmetic: elems bf16 values in (2
// bytes each), one byte out per value (its high byte). The pattern of the
// quantizer without its arithmetic, the fastest of those measured for this
// stream: a wave takes 8 KB chunks of input (lane l: 16-byte vectors
// 64 j + l, j < 8) grid-strided over 8 waves per CU, requests the next chunk
// before it stores this one (8-byte non-temporal stores); block 0 takes the
// vectors past the last whole chunk.
__device__ __forceinline__ u32x2 high_bytes(const u32x4 &v) {
    // bytes 1 and 3 of x, y and of z, w: the high bytes of eight bf16 values
    return u32x2{__builtin_amdgcn_perm(v.y, v.x, 0x07050301u), __builtin_amdgcn_perm(v.w, v.z, 0x07050301u)};
}

__global__ __launch_bounds__(64) void stream_narrow_kernel(const u32x4 *__restrict__ src, uint64_t vecs,
                                                           u32x2 *__restrict__ dst) {
    constexpr int V = 8;
    constexpr uint64_t C = 64 * V;   // vectors per chunk
    const uint64_t chunks = vecs / C, G = gridDim.x;
    const uint32_t l = threadIdx.x;
    if (blockIdx.x == 0)
        for (uint64_t i = chunks * C + l; i < vecs; i += 64)
            __builtin_nontemporal_store(high_bytes(__builtin_nontemporal_load(src + i)), dst + i);
    uint64_t c = blockIdx.x;
    if (c >= chunks) return;
    u32x4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) v[j] = __builtin_nontemporal_load(src + c * C + j * 64 + l);
    for (; c < chunks; c += G) {
        const bool more = c + G < chunks;
        u32x4 n[V];
        if (more) {
#pragma unroll
            for (int j = 0; j < V; ++j) n[j] = __builtin_nontemporal_load(src + (c + G) * C + j * 64 + l);
        }
#pragma unroll
        for (int j = 0; j < V; ++j) __builtin_nontemporal_store(high_bytes(v[j]), dst + c * C + j * 64 + l);
        if (more) {
#pragma unroll
            for (int j = 0; j < V; ++j) v[j] = n[j];
        }
    }
}

int launch_stream_narrow(const void *src, uint64_t elems, void *dst, hipStream_t st) {
    const uint32_t blocks = (uint32_t)device_props().cus * 8;   // 8 waves per CU
    hipLaunchKernelGGL(stream_narrow_kernel, dim3(blocks), dim3(64), 0, st, static_cast<const u32x4 *>(src),
                       elems / 8, static_cast<u32x2 *>(dst));
    return check_launch("stream_narrow");
}

int launch_row_absmax(const QBatch &b, int dtype, float *out, hipStream_t st) {
    return dtype == RENG_HIP_BF16 ? launch_absmax<uint16_t>(b, out, nullptr, st)
                                  : launch_absmax<float>(b, out, nullptr, st);
}

}  // namespace reng
