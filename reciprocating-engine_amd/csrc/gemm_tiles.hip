// gemm_tiles.hip - the w8a16 product for more than 64 activation rows:
//   y[m, n] = bf16(scales[n] * sum_k x[m, k] * dec(codes[n, k]))
// with x bf16 [M, K] and the quantizer's codes [N, K] (the consumer contract
// of crates/reng-synapse/src/fp8.rs:295-331 at prefill sizes, and the m = 256
// rows crates/reng-model/src/bin/fp8_probe.rs:359-431 times).
//
// Output tiles of BM x BN on v_mfma_f32_32x32x16_bf16: a block of WGM x WGN
// waves, each owning WM x WN tiles of 32 x 32. Per 64-k stage the activation
// rows (128 bytes each) and the code rows (64 bytes each) go global -> LDS
// through global_load_lds_dwordx4 into an S-slot ring with the XOR-swizzled
// 16-byte chunks of mfma_pipe.h. A wave reads its activation fragments as
// bf16 (one ds_read_b128 per 32-row tile and 16-k step) and its code
// fragments as 8 fp8 bytes (one ds_read_b64), decodes the codes to bf16 in
// registers with v_cvt_scalef32_pk_bf16_fp8/bf8 (exact), and feeds both to the
// MFMA with f32 accumulation; the per-channel scale is applied once per output
// in the epilogue. The codes cross HBM once per tile row of the grid; tiles
// run in XCD-major order with m fastest, so the blocks on one XCD that share
// a code tile read it through that XCD's L2.
#include <type_traits>

#include "common.h"
#include "gemm.h"
#include "mfma_pipe.h"

namespace reng {

namespace tiles {

using namespace pipe;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BK = 64;                        // k per pipeline stage
constexpr int A_ROW = 2 * BK, B_ROW = BK;     // bytes of one activation / code row per stage
constexpr int KSTEPS = BK / 16;               // MFMA k-steps per stage

template <int WGM, int WGN, int WM, int WN>
struct Tile {
    static constexpr int W = WGM * WGN;
    static constexpr int BM = 32 * WM * WGM, BN = 32 * WN * WGN;
    static constexpr int A_BYTES = BM * A_ROW, B_BYTES = BN * B_ROW, STAGE = A_BYTES + B_BYTES;
    // 1 KB copies: 8 activation rows or 16 code rows each.
    static constexpr int LA = BM / 8 / W, LB = BN / 16 / W;
    static constexpr int LOADS = LA + LB;
    static_assert(LA * 8 * W == BM && LB * 16 * W == BN, "copies split evenly over the waves");
};

// Two fp8 codes of each 16-bit half of w -> bf16 pairs (exact).
template <int F>
__device__ __forceinline__ uint32_t dec_pair(uint32_t w, bool hi);
template <>
__device__ __forceinline__ uint32_t dec_pair<RENG_HIP_E4M3>(uint32_t w, bool hi) {
    return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                                           : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <>
__device__ __forceinline__ uint32_t dec_pair<RENG_HIP_E5M2>(uint32_t w, bool hi) {
    return __builtin_bit_cast(uint32_t, hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, true)
                                           : __builtin_amdgcn_cvt_scalef32_pk_bf16_bf8(w, 1.0f, false));
}

template <int F, int WGM, int WGN, int WM, int WN, int S>
__global__ __launch_bounds__(64 * WGM * WGN) void w8a16_tiles(const uint16_t *__restrict__ x,
                                                              const uint8_t *__restrict__ codes,
                                                              const float *__restrict__ scales, uint32_t M,
                                                              uint32_t N, uint32_t K, uint32_t tiles_m,
                                                              uint32_t tiles, uint16_t *__restrict__ y,
                                                              uint32_t vec_out) {
    using T = Tile<WGM, WGN, WM, WN>;
    constexpr int BM = T::BM, BN = T::BN, NQ = WM * WN, HALF = NQ / 2;
    static_assert(S >= 2, "at least double-buffered");
    static_assert((S - 1) * T::LOADS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * T::STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;

    // XCD-major tile order, m fastest.
    const uint32_t xcd = blockIdx.x % XCDS, l = blockIdx.x / XCDS;
    const uint32_t per = tiles / XCDS, rem = tiles % XCDS;
    const uint32_t tile = xcd * per + (xcd < rem ? xcd : rem) + l;
    const uint32_t m0 = (tile % tiles_m) * BM, n0 = (tile / tiles_m) * BN;
    const uint32_t n = K / BK;   // stages

    // Copy sources: lane l of an activation copy brings tile row 8 c + l / 8
    // and the chunk stored in slot l % 8 of it; of a code copy, row
    // 16 c + l / 4, slot l % 4. Rows past M / N are clamped (never stored).
    const uint8_t *ga[T::LA];
    const uint8_t *gb[T::LB];
#pragma unroll
    for (int q = 0; q < T::LA; ++q) {
        const uint32_t tr = (wave * T::LA + q) * 8 + lane / 8;
        const uint32_t r = m0 + tr < M ? m0 + tr : M - 1;
        ga[q] = reinterpret_cast<const uint8_t *>(x) + (size_t)r * K * 2 + (((lane % 8) ^ swz<8>(tr)) * 16);
    }
#pragma unroll
    for (int q = 0; q < T::LB; ++q) {
        const uint32_t tr = (wave * T::LB + q) * 16 + lane / 4;
        const uint32_t r = n0 + tr < N ? n0 + tr : N - 1;
        gb[q] = codes + (size_t)r * K + (((lane % 4) ^ swz<4>(tr)) * 16);
    }
    auto issue = [&](uint32_t step, int slot) {
        uint8_t *base = lds + slot * T::STAGE;
#pragma unroll
        for (int q = 0; q < T::LA; ++q)
            copy16_to_lds(ga[q] + (size_t)step * A_ROW, base + (wave * T::LA + q) * 1024);
#pragma unroll
        for (int q = 0; q < T::LB; ++q)
            copy16_to_lds(gb[q] + (size_t)step * B_ROW, base + T::A_BYTES + (wave * T::LB + q) * 1024);
    };
    auto clampi = [&](uint32_t i) { return i < n ? i : n - 1; };

    // Fragments at k-step ks of a stage, lane l: row l % 32 of the 32-row tile
    // and the 8 k of half h = l / 32: activation bytes 32 ks + 16 h (chunk
    // 2 ks + h), codes bytes 16 ks + 8 h (chunk ks, second half for h = 1).
    const uint32_t rl = lane & 31, h = lane >> 5, swa = swz<8>(rl), swb = swz<4>(rl);
    auto read_frags = [&](int slot, int ks, u32x4 (&fa)[WM], u32x2 (&fb)[WN]) {
        const uint8_t *base = lds + slot * T::STAGE;
        const uint32_t oa = ((2 * ks + h) ^ swa) * 16, ob = ((uint32_t)ks ^ swb) * 16 + 8 * h;
#pragma unroll
        for (int i = 0; i < WM; ++i)
            fa[i] = *reinterpret_cast<const u32x4 *>(base + (wm * (32 * WM) + i * 32 + rl) * A_ROW + oa);
#pragma unroll
        for (int j = 0; j < WN; ++j)
            fb[j] = *reinterpret_cast<const u32x2 *>(base + T::A_BYTES + (wn * (32 * WN) + j * 32 + rl) * B_ROW + ob);
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // MFMAs q0 <= q < q1 of the wave's WM x WN tiles (q = i WN + j); the code
    // fragments are decoded once per k-step. D = codes x^T: rows n, columns m.
    auto mfma_part = [&](int q0, int q1, const u32x4 (&fa)[WM], const u32x4 (&wb)[WN]) {
#pragma unroll
        for (int q = q0; q < q1; ++q) {
            const int i = q / WN, j = q % WN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wb[j]),
                                                                __builtin_bit_cast(bf16x8, fa[i]), acc[i][j], 0, 0,
                                                                0);
        }
    };
    auto decode = [&](const u32x2 (&fb)[WN], u32x4 (&wb)[WN]) {
#pragma unroll
        for (int j = 0; j < WN; ++j)
            wb[j] = u32x4{dec_pair<F>(fb[j].x, false), dec_pair<F>(fb[j].x, true), dec_pair<F>(fb[j].y, false),
                          dec_pair<F>(fb[j].y, true)};
    };

    // The pipeline of gemm_fp8_mfma: S stages in flight from the prologue;
    // per stage one barrier once each wave's own copies of the next stage
    // have landed, then the copy of stage t + S into the slot stage t used.
#pragma unroll
    for (int s = 0; s < S; ++s) issue(clampi(s), s);
    wait_vmcnt<(S - 1) * T::LOADS>();
    lds_barrier();
    u32x4 fa[2][WM];
    u32x2 fb[2][WN];
    read_frags(0, 0, fa[0], fb[0]);
    auto kstep = [&](auto cur_c, auto ks_c, uint32_t t) {
        constexpr int CUR = decltype(cur_c)::value, NXT = CUR ^ 1, KSI = decltype(ks_c)::value;
        u32x4 wb[WN];
        decode(fb[CUR], wb);
        if constexpr (KSI + 1 < KSTEPS) {
            read_frags((int)(t % S), KSI + 1, fa[NXT], fb[NXT]);
            mfma_part(0, NQ, fa[CUR], wb);
            interleave<NQ, WM + WN, 0>();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            mfma_part(0, HALF, fa[CUR], wb);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<(S - 2) * T::LOADS>();
            lds_barrier();
            issue(clampi(t + S), (int)(t % S));
            read_frags((int)((t + 1) % S), 0, fa[NXT], fb[NXT]);
            mfma_part(HALF, NQ, fa[CUR], wb);
            interleave<NQ - HALF, WM + WN, T::LOADS>();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    static_assert(KSTEPS == 4, "four k-steps per stage: the fragment sets alternate 0, 1, 0, 1");
    for (uint32_t t = 0; t < n; ++t) {
        kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t);
        kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, t);
        kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 2>{}, t);
        kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 3>{}, t);
    }
    wait_vmcnt<0>();   // the clamped surplus copies land before LDS is released

    // Lane l holds output row m = ... + l % 32 and, per group g of four
    // accumulators, the four consecutive columns n = ... + 8 g + 4 h + e.
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const uint32_t m = m0 + wm * (32 * WM) + i * 32 + rl;
        if (m >= M) continue;
        uint16_t *orow = y + (size_t)m * N;
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t nb = n0 + wn * (32 * WN) + j * 32 + 8 * g + 4 * h;
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t nn = nb + e < N ? nb + e : N - 1;
                    o[e] = acc[i][j][4 * g + e] * (scales ? scales[nn] : 1.0f);
                }
                if (vec_out && nb + 3 < N) {
                    const uint32_t lo = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
                    const uint32_t hi = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
                    *reinterpret_cast<u32x2 *>(orow + nb) = u32x2{lo, hi};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (nb + e < N) orow[nb + e] = (uint16_t)f32_to_bf16_bits(o[e]);
                }
            }
    }
}

template <int F, int WGM, int WGN, int WM, int WN, int S>
int launch_tiles_cfg(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                     uint32_t K, uint16_t *y, hipStream_t st) {
    using T = Tile<WGM, WGN, WM, WN>;
    const uint32_t tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t vec_out = N % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0;
    hipLaunchKernelGGL((w8a16_tiles<F, WGM, WGN, WM, WN, S>), dim3(tiles), dim3(64 * T::W), 0, st, x, codes, scales,
                       M, N, K, tiles_m, tiles, y, vec_out);
    return check_launch("w8a16_tiles");
}

inline uint64_t tile_count(uint32_t M, uint32_t N, uint32_t bm, uint32_t bn) {
    return (uint64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

// Tile choice (measured on MI355X over M = 128-1024 and the Llama-3.1-8B /
// Qwen2.5-32B shapes): the largest tile whose count still covers the chip -
// 256 x 256 (8 waves of 128 x 64) with a tile per CU; 128 x 256 (8 waves of
// 64 x 64) with half the CUs or more, which beats 128 x 128 at twice the
// count (M = 1024 [5120, 5120]: 72 against 93 us); 128 x 128 (8 waves of
// 64 x 32, six stages) from three quarters of the CUs; else 64 x 128.
template <int F>
int launch_tiles_f(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                   uint32_t K, uint16_t *y, hipStream_t st) {
    const uint64_t cus = (uint64_t)device_props().cus;
    if (tile_count(M, N, 256, 256) >= cus) return launch_tiles_cfg<F, 2, 4, 4, 2, 3>(x, codes, scales, M, N, K, y, st);
    if (2 * tile_count(M, N, 128, 256) >= cus)
        return launch_tiles_cfg<F, 2, 4, 2, 2, 3>(x, codes, scales, M, N, K, y, st);
    if (4 * tile_count(M, N, 128, 128) >= 3 * cus)
        return launch_tiles_cfg<F, 2, 4, 2, 1, 6>(x, codes, scales, M, N, K, y, st);
    return launch_tiles_cfg<F, 2, 4, 1, 1, 6>(x, codes, scales, M, N, K, y, st);
}

}  // namespace tiles

// Below half the CUs in 64 x 128 tiles the 64-row kernels, which split K,
// are faster (M = 100 [3000, 4096]: 22.2 against 28.1 us).
bool w8a16_tiles_take(uint32_t M, uint32_t N, uint32_t K) {
    return M > 64 && K % tiles::BK == 0 && 2 * tiles::tile_count(M, N, 64, 128) >= (uint64_t)device_props().cus;
}

int launch_w8a16_tiles(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st) {
    if (format == RENG_HIP_E4M3) return tiles::launch_tiles_f<RENG_HIP_E4M3>(x, codes, scales, M, N, K, y, st);
    return tiles::launch_tiles_f<RENG_HIP_E5M2>(x, codes, scales, M, N, K, y, st);
}

}  // namespace reng
