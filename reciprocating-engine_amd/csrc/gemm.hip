// gemm.hip - consumers of the quantizer's codes on CDNA4 (gfx950).
//
// 1. gemv_w8a16     (M <= 4): y[m, n] = s[n] * sum_k x[m, k] * decode(c[n, k]).
//    Streams the codes once with 16-byte loads, decodes in registers
//    (v_cvt_pk_f32_fp8 / _bf8), f32 FMA, one wave per output row.
// 2. skinny_w8a16   (4 < M <= 64): the same product on bf16 MFMA
//    (v_mfma_f32_16x16x32_bf16): codes decoded to bf16 in registers
//    (v_cvt_scalef32_pk_bf16_fp8, exact: bf16 holds every e4m3 / e5m2 value),
//    activations as the B operand; the four waves of a block split K and meet
//    in LDS.
// 3. gemm_fp8_scaled: fp8 x fp8 on v_mfma_scale_f32_32x32x64_f8f6f4 (the OCP
//    fp8 formats, whose finite codes 0x00-0x77 / 0x00-0x7b mean what reng-fp8's
//    mean), 128x128 block tiles staged through LDS, epilogue
//    out = acc * sa[m] * sb[n] rounded to bf16.
//
// The reference semantics are gemm_cpu over Quantized::dequantize
// (crates/reng-model/src/bin/fp8_probe.rs:55-67) and the per-channel scaleB of
// fp8_gemm_bf16 (crates/reng-synapse/src/fp8.rs:295-331).
#include "common.h"
#include "gemm.h"

namespace reng {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

template <int F>
__device__ __forceinline__ f32x2 dec2(uint32_t w, bool hi);

template <>
__device__ __forceinline__ f32x2 dec2<RENG_HIP_E4M3>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
}
template <>
__device__ __forceinline__ f32x2 dec2<RENG_HIP_E5M2>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_f32_bf8(w, true) : __builtin_amdgcn_cvt_pk_f32_bf8(w, false);
}

// Two codes (a word of w) -> two bf16, exactly.
template <int F>
__device__ __forceinline__ bf16x2 dec2_bf16(uint32_t w, bool hi);
template <>
__device__ __forceinline__ bf16x2 dec2_bf16<RENG_HIP_E4M3>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
              : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
}
template <>
__device__ __forceinline__ bf16x2 dec2_bf16<RENG_HIP_E5M2>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true)
              : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false);
}

__device__ __forceinline__ float bf_lo(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float bf_hi(uint32_t d) { return __uint_as_float(d & 0xffff0000u); }

// ------------------------------------------------------------------ GEMV

// v_dot2_f32_bf16: acc + a.lo * b.lo + a.hi * b.hi, f32 accumulation.
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b),
                                           acc, false);
}

// 16 codes (a 16-byte load) -> 8 bf16 pairs, exactly.
template <int F>
__device__ __forceinline__ void decode16(const u32x4 &q, uint32_t (&w)[8]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[2 * i] = __builtin_bit_cast(uint32_t, dec2_bf16<F>(d[i], false));
        w[2 * i + 1] = __builtin_bit_cast(uint32_t, dec2_bf16<F>(d[i], true));
    }
}

// One wave per output row (rows strided over all waves of the grid), 16 codes
// per lane per chunk, CPL chunks per lane per group. The wave walks its
// (row, group) pairs as one stream and loads the next pair before consuming
// the current one, so CPL * 1 KB of codes per wave stay in flight through the
// decode, the dot products and the end-of-row reduction. The activation rows
// are staged once per block in LDS as bf16 (XLDS) or read through the caches.
// Codes decode to bf16 pairs in registers and meet the activation in
// v_dot2_f32_bf16 (f32 accumulation).
template <int F, int M, int CPL, bool XLDS>
__global__ __launch_bounds__(512) void gemv_w8a16(const uint16_t *__restrict__ x,
                                                  const uint8_t *__restrict__ codes,
                                                  const float *__restrict__ scales, uint32_t N,
                                                  uint32_t K, uint16_t *__restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint32_t xs[];
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t nch = K / 16;   // 16-code chunks per row
    const uint32_t waves = gridDim.x * (blockDim.x >> 6);
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (tid >> 6);
    const uint32_t gpr = (nch + 64 * CPL - 1) / (64 * CPL);   // groups per row
    const bool ragged = nch % (64 * CPL) != 0;

    auto load = [&](uint32_t r, uint32_t gi, u32x4 (&q)[CPL]) {
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(codes + (size_t)r * K);
        const uint32_t c0 = gi * 64 * CPL + lane;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const uint32_t ch = c0 + u * 64;
            q[u] = (!ragged || ch < nch) ? __builtin_nontemporal_load(wr + ch) : u32x4{0u, 0u, 0u, 0u};
        }
    };

    // The first group's codes are requested before the activation is staged.
    uint32_t r = wave, gi = 0;
    u32x4 qn[CPL];
    if (wave < N) load(r, gi, qn);
    if constexpr (XLDS) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(x);
        u32x4 *dst = reinterpret_cast<u32x4 *>(xs);
        for (uint32_t i = tid; i < M * nch * 2; i += blockDim.x) dst[i] = src[i];
        __syncthreads();
    }
    if (wave >= N) return;
    float acc[M][2];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m][0] = acc[m][1] = 0.0f;
    while (true) {
        u32x4 q[CPL];
#pragma unroll
        for (int u = 0; u < CPL; ++u) q[u] = qn[u];
        // The pair after (r, gi), loaded now.
        uint32_t rn = r, gn = gi + 1;
        if (gn == gpr) {
            gn = 0;
            rn = r + waves;
        }
        if (rn < N) load(rn, gn, qn);

        const uint32_t c0 = gi * 64 * CPL + lane;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const uint32_t ch = c0 + u * 64;
            if (ragged && ch >= nch) continue;
            uint32_t w[8];
            decode16<F>(q[u], w);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                u32x4 xa, xb;
                if constexpr (XLDS) {
                    const u32x4 *xp = reinterpret_cast<const u32x4 *>(xs) + (m * nch + ch) * 2;
                    xa = xp[0];
                    xb = xp[1];
                } else {
                    const u32x4 *xp = reinterpret_cast<const u32x4 *>(x + (size_t)m * K) + ch * 2;
                    xa = xp[0];
                    xb = xp[1];
                }
                acc[m][0] = dot2(w[0], xa.x, acc[m][0]);
                acc[m][1] = dot2(w[1], xa.y, acc[m][1]);
                acc[m][0] = dot2(w[2], xa.z, acc[m][0]);
                acc[m][1] = dot2(w[3], xa.w, acc[m][1]);
                acc[m][0] = dot2(w[4], xb.x, acc[m][0]);
                acc[m][1] = dot2(w[5], xb.y, acc[m][1]);
                acc[m][0] = dot2(w[6], xb.z, acc[m][0]);
                acc[m][1] = dot2(w[7], xb.w, acc[m][1]);
            }
        }
        if (gi + 1 == gpr) {   // end of row r: reduce across the wave and store
            const float s = scales ? scales[r] : 1.0f;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float t = wave_sum_f32(acc[m][0] + acc[m][1]);
                if (lane == m) y[(size_t)m * N + r] = (uint16_t)f32_to_bf16_bits(t * s);
                acc[m][0] = acc[m][1] = 0.0f;
            }
        }
        if (rn >= N) break;
        r = rn;
        gi = gn;
    }
}

// ------------------------------------------------------------------ skinny GEMM

// Block = 4 waves on one 16-row tile of W; wave w takes the K chunks
// c = w, w + 4, ... of 128 codes. Lane l owns row n0 + l % 16 and, within a
// chunk, codes [32 * (l / 16), +32): four MFMA k-slices of 8. The activation
// fragment uses the same k assignment, so the k order inside an MFMA is a
// permutation shared by both operands and the sum is unchanged.
template <int F, int MT>
__global__ __launch_bounds__(256) void skinny_w8a16(const uint16_t *__restrict__ x,
                                                    const uint8_t *__restrict__ codes,
                                                    const float *__restrict__ scales, uint32_t M,
                                                    uint32_t N, uint32_t K, uint16_t *__restrict__ y) {
    __shared__ float red[4][MT][64][4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t n0 = blockIdx.x * 16;
    const int r = lane & 15, g = lane >> 4;
    const uint32_t nrow = n0 + r < N ? n0 + r : N - 1;   // clamp reads; stores are masked
    const uint8_t *wr = codes + (size_t)nrow * K;
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint32_t nchunks = K / 128;
    for (uint32_t c = wave; c < nchunks; c += 4) {
        const uint32_t k0 = c * 128 + 32 * g;
        const u32x4 *wp = reinterpret_cast<const u32x4 *>(wr + k0);
        const u32x4 q0 = __builtin_nontemporal_load(wp), q1 = __builtin_nontemporal_load(wp + 1);
        const uint32_t d[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        bf16x8 a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x2 p0 = dec2_bf16<F>(d[2 * s], false), p1 = dec2_bf16<F>(d[2 * s], true);
            const bf16x2 p2 = dec2_bf16<F>(d[2 * s + 1], false), p3 = dec2_bf16<F>(d[2 * s + 1], true);
            a[s] = bf16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint32_t m = t * 16 + r;
            const uint32_t mm = m < M ? m : M - 1;
            const u32x4 *xp = reinterpret_cast<const u32x4 *>(x + (size_t)mm * K + k0);
            u32x4 xv[4] = {xp[0], xp[1], xp[2], xp[3]};
            if (m >= M) {
#pragma unroll
                for (int s = 0; s < 4; ++s) xv[s] = u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], __builtin_bit_cast(bf16x8, xv[s]),
                                                                 acc[t], 0, 0, 0);
        }
    }
    // D[i][j] of a 16x16 tile: lane l holds column j = l % 16 (m), rows i = 4 * (l / 16) + e (n).
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][t][lane][e] = acc[t][e];
    __syncthreads();
    // 256 threads finish 16 x (16 * MT) outputs.
    for (int o = threadIdx.x; o < 16 * 16 * MT; o += 256) {
        const int t = o / 256, rem = o % 256, ln = rem / 4, e = rem % 4;
        const float v = red[0][t][ln][e] + red[1][t][ln][e] + red[2][t][ln][e] + red[3][t][ln][e];
        const uint32_t m = t * 16 + (ln & 15);
        const uint32_t n = n0 + 4 * (ln >> 4) + e;
        if (m < M && n < N) {
            const float s = scales ? scales[n] : 1.0f;
            y[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(v * s);
        }
    }
}

// ------------------------------------------------------------------ fp8 x fp8 GEMM

// Block tile 128 (m) x 128 (n), K step 128, 4 waves in a 2 x 2 grid, each wave
// 64 x 64 = 2 x 2 MFMA tiles of 32 x 32. Operand layout of the 32x32x64 fp8
// MFMA: lane l holds row (l % 32) and the 32 consecutive k of half l / 32.
// LDS rows are padded to 144 bytes against bank conflicts.
constexpr int GB_M = 128, GB_N = 128, GB_K = 128, G_LDS = GB_K + 16;

template <int FA, int FB>
__global__ __launch_bounds__(256) void gemm_fp8_kernel(const uint8_t *__restrict__ a,
                                                       const float *__restrict__ sa, uint32_t nsa,
                                                       const uint8_t *__restrict__ b,
                                                       const float *__restrict__ sb, uint32_t nsb,
                                                       uint32_t M, uint32_t N, uint32_t K,
                                                       uint16_t *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[GB_M * G_LDS];
    __shared__ __attribute__((aligned(16))) uint8_t lds_b[GB_N * G_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t m0 = blockIdx.y * GB_M, n0 = blockIdx.x * GB_N;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    for (uint32_t k0 = 0; k0 < K; k0 += GB_K) {
        // Global -> LDS: 128 rows x 128 bytes per operand = 1024 16-byte vectors; 4 per thread.
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const int v = it * 256 + tid;
            const int row = v >> 3, col = (v & 7) * 16;
            const uint32_t ga = m0 + row < M ? m0 + row : M - 1;
            const uint32_t gb = n0 + row < N ? n0 + row : N - 1;
            const u32x4 va = *reinterpret_cast<const u32x4 *>(a + (size_t)ga * K + k0 + col);
            const u32x4 vb = *reinterpret_cast<const u32x4 *>(b + (size_t)gb * K + k0 + col);
            *reinterpret_cast<u32x4 *>(lds_a + row * G_LDS + col) = va;
            *reinterpret_cast<u32x4 *>(lds_b + row * G_LDS + col) = vb;
        }
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < GB_K; ks += 64) {
            i32x8 fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint8_t *pa = lds_a + (wm * 64 + i * 32 + (lane & 31)) * G_LDS + ks + 32 * (lane >> 5);
                const u32x4 a0 = *reinterpret_cast<const u32x4 *>(pa);
                const u32x4 a1 = *reinterpret_cast<const u32x4 *>(pa + 16);
                fa[i] = i32x8{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
                const uint8_t *pb = lds_b + (wn * 64 + i * 32 + (lane & 31)) * G_LDS + ks + 32 * (lane >> 5);
                const u32x4 b0 = *reinterpret_cast<const u32x4 *>(pb);
                const u32x4 b1 = *reinterpret_cast<const u32x4 *>(pb + 16);
                fb[i] = i32x8{(int)b0.x, (int)b0.y, (int)b0.z, (int)b0.w, (int)b1.x, (int)b1.y, (int)b1.z, (int)b1.w};
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                        fa[i], fb[j], acc[i][j], FA, FB, 0, 0, 0, 0);
        }
        __syncthreads();
    }
    // D of a 32x32 tile: lane l holds column j = l % 32 (n), rows
    // i = 8 * (e / 4) + 4 * (l / 32) + e % 4 (m) for e = 0..15.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t n = n0 + wn * 64 + j * 32 + (lane & 31);
            if (n >= N) continue;
            const float sbn = nsb == 0 ? 1.0f : (nsb == 1 ? sb[0] : sb[n]);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t m = m0 + wm * 64 + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                if (m >= M) continue;
                const float sam = nsa == 0 ? 1.0f : (nsa == 1 ? sa[0] : sa[m]);
                out[(size_t)m * N + n] = (uint16_t)f32_to_bf16_bits(acc[i][j][e] * sam * sbn);
            }
        }
}

// ------------------------------------------------------------------ launchers

template <int F>
int launch_w8a16_t(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                   uint32_t N, uint32_t K, uint16_t *y, hipStream_t st) {
    if (M > 4 && K % 128 != 0) {
        // The MFMA kernel walks K in 128-code chunks; other widths take the
        // GEMV kernel four activation rows at a time.
        for (uint32_t mb = 0; mb < M; mb += 4) {
            const uint32_t mt = M - mb < 4 ? M - mb : 4;
            const int rc = launch_w8a16_t<F>(x + (size_t)mb * K, codes, scales, mt, N, K,
                                             y + (size_t)mb * N, st);
            if (rc) return rc;
        }
        return RENG_HIP_OK;
    }
    if (M <= 4) {
        // Rows divide evenly over the waves: at most 16 waves per CU, each
        // taking rows_per_wave rows.
        const uint32_t cap = (uint32_t)device_props().cus * 16;
        const uint32_t rpw = (N + cap - 1) / cap;
        const uint32_t waves = (N + rpw - 1) / rpw;
        const size_t xbytes = (size_t)M * K * 2;
        const bool xlds = xbytes <= 64 * 1024;
        const int threads = 512;
        const uint32_t blocks = (waves + threads / 64 - 1) / (threads / 64);
        const size_t lds = xlds ? xbytes : 0;
        // 7 chunks per lane when a row splits into whole groups of 7 (K a multiple
        // of 7168, e.g. 14336), else 4.
        const bool cpl7 = (K / 16) % (64 * 7) == 0;
#define RENG_GEMV(MM, C, XL)                                                                  \
    hipLaunchKernelGGL((gemv_w8a16<F, MM, C, XL>), dim3(blocks), dim3(threads), lds, st, x, codes, \
                       scales, N, K, y)
#define RENG_GEMV_M(MM)                                                   \
    if (cpl7) { if (xlds) RENG_GEMV(MM, 7, true); else RENG_GEMV(MM, 7, false); } \
    else { if (xlds) RENG_GEMV(MM, 4, true); else RENG_GEMV(MM, 4, false); }
        switch (M) {
            case 1: RENG_GEMV_M(1); break;
            case 2: RENG_GEMV_M(2); break;
            case 3: RENG_GEMV_M(3); break;
            default: RENG_GEMV_M(4); break;
        }
#undef RENG_GEMV_M
#undef RENG_GEMV
        return check_launch("gemv_w8a16");
    }
    // Larger M: tiles of 64 activation rows.
    for (uint32_t mb = 0; mb < M; mb += 64) {
        const uint32_t mt = M - mb < 64 ? M - mb : 64;
        const dim3 grid((N + 15) / 16);
        const uint16_t *xb = x + (size_t)mb * K;
        uint16_t *yb = y + (size_t)mb * N;
        switch ((mt + 15) / 16) {
            case 1: hipLaunchKernelGGL((skinny_w8a16<F, 1>), grid, dim3(256), 0, st, xb, codes, scales, mt, N, K, yb); break;
            case 2: hipLaunchKernelGGL((skinny_w8a16<F, 2>), grid, dim3(256), 0, st, xb, codes, scales, mt, N, K, yb); break;
            case 3: hipLaunchKernelGGL((skinny_w8a16<F, 3>), grid, dim3(256), 0, st, xb, codes, scales, mt, N, K, yb); break;
            default: hipLaunchKernelGGL((skinny_w8a16<F, 4>), grid, dim3(256), 0, st, xb, codes, scales, mt, N, K, yb); break;
        }
        const int rc = check_launch("skinny_w8a16");
        if (rc) return rc;
    }
    return RENG_HIP_OK;
}

int launch_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                 uint32_t N, uint32_t K, int format, uint16_t *y, hipStream_t st) {
    return format == RENG_HIP_E4M3 ? launch_w8a16_t<RENG_HIP_E4M3>(x, codes, scales, M, N, K, y, st)
                                   : launch_w8a16_t<RENG_HIP_E5M2>(x, codes, scales, M, N, K, y, st);
}

int launch_fp8_gemm(const uint8_t *a, int fa, const float *sa, uint32_t nsa, const uint8_t *b,
                    int fb, const float *sb, uint32_t nsb, uint32_t M, uint32_t N, uint32_t K,
                    uint16_t *out, hipStream_t st) {
    const dim3 grid((N + GB_N - 1) / GB_N, (M + GB_M - 1) / GB_M);
#define RENG_FP8_GEMM(A, B)                                                                     \
    hipLaunchKernelGGL((gemm_fp8_kernel<A, B>), grid, dim3(256), 0, st, a, sa, nsa, b, sb, nsb, \
                       M, N, K, out)
    if (fa == RENG_HIP_E4M3 && fb == RENG_HIP_E4M3) RENG_FP8_GEMM(0, 0);
    else if (fa == RENG_HIP_E4M3) RENG_FP8_GEMM(0, 1);
    else if (fb == RENG_HIP_E4M3) RENG_FP8_GEMM(1, 0);
    else RENG_FP8_GEMM(1, 1);
#undef RENG_FP8_GEMM
    return check_launch("gemm_fp8");
}

}  // namespace reng
