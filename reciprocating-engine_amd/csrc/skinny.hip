// skinny.hip - y[m, n] = bf16(s[n] * sum_k x[m, k] * decode(c[n, k])) for
// 4 < M <= 16 activation rows (bf16) on bf16 MFMA (gfx950).
//
// The reference semantics are gemm_cpu over Quantized::dequantize
// (crates/reng-model/src/bin/fp8_probe.rs:55-67) with the per-channel scaleB
// of fp8_gemm_bf16 (crates/reng-synapse/src/fp8.rs:295-331).
//
// A block owns 16 NT weight rows; its WPB waves split K between them, so the
// whole product of the block's rows is one block's work: no partial sums
// leave the block and there is one launch. Each wave streams its rows' codes
// and the activation fragments straight into registers (no LDS, no barrier
// until the end), prefetching P 128-code chunks ahead with unconditional,
// clamped loads. v_mfma_f32_16x16x32_bf16: the A operand is 16 weight rows
// x 32 k (codes decoded to bf16 in registers, exact: bf16 holds every e4m3 /
// e5m2 value), the B operand 32 k x 16 activation rows. Within a 128-code
// chunk lane l (row l % 16, group g = l / 16) holds the 32 consecutive codes
// [16 g, 16 g + 16) and [64 + 16 g, 64 + 16 g + 16) of its row (each load
// instruction reads contiguous 64-byte runs), k-steps 0, 1 take the first
// piece's halves and 2, 3 the second's; the activation fragment uses the same
// k assignment (a permutation of k shared by both operands). At the end the waves' accumulators meet in LDS
// and are added in wave order (deterministic), scaled per row and stored as
// four consecutive bf16 per lane.
#include <type_traits>

#include "common.h"
#include "gemm.h"

namespace reng {

namespace skinny {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int CHUNK = 128;   // codes of k per chunk

template <int F>
__device__ __forceinline__ bf16x2 dec2(uint32_t w, bool hi);
template <>
__device__ __forceinline__ bf16x2 dec2<RENG_HIP_E4M3>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
              : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
}
template <>
__device__ __forceinline__ bf16x2 dec2<RENG_HIP_E5M2>(uint32_t w, bool hi) {
    return hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true)
              : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false);
}

// 8 codes (two words) -> 8 bf16.
template <int F>
__device__ __forceinline__ bf16x8 dec8(uint32_t w0, uint32_t w1) {
    const bf16x2 p0 = dec2<F>(w0, false), p1 = dec2<F>(w0, true);
    const bf16x2 p2 = dec2<F>(w1, false), p3 = dec2<F>(w1, true);
    return bf16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// fn(integral_constant<I>) for I = B .. E-1, unrolled at compile time.
template <int B, int E, typename Fn>
__device__ __forceinline__ void static_for(Fn &&fn) {
    if constexpr (B < E) {
        fn(std::integral_constant<int, B>{});
        static_for<B + 1, E>(fn);
    }
}

// One chunk of a wave's operands: NT weight tiles (2 x 16 bytes per lane) and
// MT activation tiles (4 x 16 bytes per lane).
template <int NT, int MT>
struct Chunk {
    u32x4 w[NT][2];
    u32x4 a[MT][4];
};

template <int F, int MT, int NT, int KW, int NW, int P>
__global__ __launch_bounds__(64 * KW * NW) void skinny_mfma(const uint16_t *__restrict__ x,
                                                        const uint8_t *__restrict__ codes,
                                                        const float *__restrict__ scales, uint32_t M, uint32_t N,
                                                        uint32_t K, uint16_t *__restrict__ y) {
    constexpr int TILES = NT * MT;
    __shared__ __attribute__((aligned(16))) f32x4 red[KW > 1 ? KW : 1][KW > 1 ? NW : 1][KW > 1 ? TILES : 1][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave / NW, nw = wave % NW;
    const uint32_t r16 = lane & 15, g = lane >> 4;
    const uint32_t n0 = (blockIdx.x * NW + nw) * (16 * NT);

    // This wave's chunks of K: [c0, c1), possibly empty. Waves with the same
    // kw read the same activation bytes (through L1); waves with the same nw
    // share rows and are added up at the end.
    const uint32_t chunks = K / CHUNK;
    const uint32_t c0 = kw * chunks / KW, c1 = (kw + 1) * chunks / KW;

    // Row pointers (clamped: rows past N / M are read but never stored).
    const uint8_t *wp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        uint32_t n = n0 + t * 16 + r16;
        n = n < N ? n : N - 1;
        wp[t] = codes + (size_t)n * K + 16 * g;
    }
    const uint16_t *ap[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        uint32_t m = mt * 16 + r16;
        m = m < M ? m : M - 1;
        ap[mt] = x + (size_t)m * K + 16 * g;
    }
    auto load = [&](uint32_t c, Chunk<NT, MT> &ch) {
        const size_t ko = (size_t)c * CHUNK;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const u32x4 *p = reinterpret_cast<const u32x4 *>(wp[t] + ko);
            ch.w[t][0] = __builtin_nontemporal_load(p);
            ch.w[t][1] = __builtin_nontemporal_load(p + 4);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const u32x4 *p = reinterpret_cast<const u32x4 *>(ap[mt] + ko);
            ch.a[mt][0] = p[0];
            ch.a[mt][1] = p[1];
            ch.a[mt][2] = p[8];
            ch.a[mt][3] = p[9];
        }
    };

    f32x4 acc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (c0 < c1) {
        // Ring of P chunks in registers; the chunk P - 1 ahead is requested
        // before the current one is consumed (indices clamped to c1 - 1, so
        // every load is unconditional and each use waits only for its own).
        Chunk<NT, MT> ring[P];
#pragma unroll
        for (int p = 0; p < P - 1; ++p) load(c0 + p < c1 ? c0 + p : c1 - 1, ring[p]);
        uint32_t c = c0;
        auto step = [&](auto slot_c) {
            constexpr int SL = decltype(slot_c)::value;
            const uint32_t ahead = c + P - 1;
            load(ahead < c1 ? ahead : c1 - 1, ring[(SL + P - 1) % P]);
            const Chunk<NT, MT> &ch = ring[SL];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                bf16x8 wa[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const u32x4 &q = ch.w[t][j >> 1];
                    wa[t] = (j & 1) ? dec8<F>(q.z, q.w) : dec8<F>(q.x, q.y);
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const bf16x8 b = __builtin_bit_cast(bf16x8, ch.a[mt][j]);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[t], b, acc[t][mt], 0, 0, 0);
                }
            }
            ++c;
        };
        // Unrolled by P so the ring slots are compile-time indices.
        while (c + P <= c1) static_for<0, P>(step);
        // Tail (fewer than P chunks left): the slots continue in order.
        static_for<0, P>([&](auto ic) {
            if (c < c1) step(ic);
        });
    }

    // Waves of the same rows meet in LDS and are added in kw order; tile i of
    // the row group is stored by the wave with kw == i % KW.
    if constexpr (KW > 1) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red[kw][nw][t * MT + mt][lane] = acc[t][mt];
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TILES; ++i) {
        f32x4 s;
        if constexpr (KW > 1) {
            if (i % KW != kw) continue;
            s = red[0][nw][i][lane];
#pragma unroll
            for (int w = 1; w < KW; ++w) s += red[w][nw][i][lane];
        } else {
            s = acc[i / MT][i % MT];
        }
        // D of a 16x16 tile: lane l holds column m = l % 16 and rows
        // n = 4 (l / 16) + e: four consecutive outputs of row m.
        const int t = i / MT, mt = i % MT;
        const uint32_t m = mt * 16 + r16;
        const uint32_t nb = n0 + t * 16 + 4 * g;
        if (m >= M) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t n = nb + e < N ? nb + e : N - 1;
            o[e] = s[e] * (scales ? scales[n] : 1.0f);
        }
        uint16_t *yr = y + (size_t)m * N;
        if (nb + 3 < N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
            *reinterpret_cast<u32x2 *>(yr + nb) =
                u32x2{f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16),
                      f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16)};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (nb + e < N) yr[nb + e] = (uint16_t)f32_to_bf16_bits(o[e]);
        }
    }
}

template <int F, int MT, int NT, int KW, int NW, int P>
int launch_cfg(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N, uint32_t K,
               uint16_t *y, hipStream_t st) {
    const uint32_t rows = 16 * NT * NW;
    const uint32_t blocks = (N + rows - 1) / rows;
    hipLaunchKernelGGL((skinny_mfma<F, MT, NT, KW, NW, P>), dim3(blocks), dim3(64 * KW * NW), 0, st, x, codes,
                       scales, M, N, K, y);
    return check_launch("skinny_mfma");
}

template <int F, int MT>
int launch_mt(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N, uint32_t K,
              uint16_t *y, hipStream_t st) {
    // Enough waves for the chip (about 8 per CU): 32-row blocks of 4 waves on
    // wide matrices, 16-row blocks of 8 waves (K split 8 ways) otherwise.
    constexpr int P = 4;   // prefetch depth in 128-code chunks
    const uint32_t want = 8u * (uint32_t)device_props().cus;
    if ((N + 31) / 32 * 4 >= want) return launch_cfg<F, MT, 2, 4, 1, P>(x, codes, scales, M, N, K, y, st);
    return launch_cfg<F, MT, 1, 8, 1, P>(x, codes, scales, M, N, K, y, st);
}

}  // namespace skinny

// 4 < M <= 16, K % 128 == 0.
int launch_skinny_mfma(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st) {
    using namespace skinny;
    if (format == RENG_HIP_E4M3) return launch_mt<RENG_HIP_E4M3, 1>(x, codes, scales, M, N, K, y, st);
    return launch_mt<RENG_HIP_E5M2, 1>(x, codes, scales, M, N, K, y, st);
}

}  // namespace reng
