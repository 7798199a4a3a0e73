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

constexpr int K_ALIGN = 64;   // K granularity the kernels take

// BK codes of k per pipeline stage (64, 128 or 256).
template <int WGM, int WGN, int WM, int WN, int BK>
struct Tile {
    static_assert(BK == 64 || BK == 128 || BK == 256, "stage widths");
    static constexpr int W = WGM * WGN;
    static constexpr int BM = 32 * WM * WGM, BN = 32 * WN * WGN;
    static constexpr int A_ROW = 2 * BK, B_ROW = BK;            // bytes of one activation / code row per stage
    static constexpr int CHA = A_ROW / 16, CHB = B_ROW / 16;    // 16-byte chunks of a row
    static constexpr int RA = 1024 / A_ROW, RB = 1024 / B_ROW;  // rows of a 1 KB copy
    static constexpr int KSTEPS = BK / 16;                      // MFMA k-steps per stage
    static constexpr int A_BYTES = BM * A_ROW, B_BYTES = BN * B_ROW, STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = BM / RA / W, LB = BN / RB / W;    // copies per wave per stage
    static constexpr int LOADS = LA + LB;
    static_assert(LA * RA * W == BM && LB * RB * W == BN, "copies split evenly over the waves");
};

// Chunk slots: chunk c of tile row r sits in slot c ^ swz(r). Activation rows
// (8-32 chunks) XOR the low three bits of c; code rows use the 4-chunk
// permutation of mfma_pipe.h for 4 chunks, else the 8-chunk one.
__device__ __forceinline__ uint32_t swz_a(uint32_t r) { return swz<8>(r); }
template <int CHB>
__device__ __forceinline__ uint32_t swz_b(uint32_t r) { return swz<CHB == 4 ? 4 : 8>(r); }

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

// Work units are (tile, stage) pairs, unit u = tile * n + stage with n = K / BK
// stages per tile. Without SK a block takes one tile's n units, tiles in
// XCD-major order with m fastest. With SK (stream-K) the grid is persistent
// and block b takes units [b U / G, (b + 1) U / G) of all U = tiles * n, so
// every CU gets the same number of stages whatever the tile count; the copy
// pipeline runs straight across tile boundaries. A tile whose units span
// several blocks is finished by the last of them to arrive: each writes its
// partial sums to part (slot b + tile), releases them and increments
// cnt[tile]; the block that sees the
// count reach the segment count adds the partials in block order (the same
// order whichever block arrives last, so the sum is deterministic), writes the
// tile and resets the counter to zero for the next launch. No block waits for
// another.
template <int F, int WGM, int WGN, int WM, int WN, int BK, int S, bool SK>
__global__ __launch_bounds__(64 * WGM * WGN) void w8a16_tiles(const uint16_t *__restrict__ x,
                                                              const uint8_t *__restrict__ codes,
                                                              const float *__restrict__ scales, uint32_t M,
                                                              uint32_t N, uint32_t K, uint32_t tiles_m,
                                                              uint32_t tiles, uint16_t *__restrict__ y,
                                                              uint32_t vec_out, float *__restrict__ part,
                                                              uint32_t *__restrict__ cnt) {
    using T = Tile<WGM, WGN, WM, WN, BK>;
    constexpr int BM = T::BM, BN = T::BN, NQ = WM * WN, HALF = NQ / 2;
    constexpr int A_ROW = T::A_ROW, B_ROW = T::B_ROW, CHA = T::CHA, CHB = T::CHB, KSTEPS = T::KSTEPS;
    static_assert(S >= 2, "at least double-buffered");
    static_assert((S - 1) * T::LOADS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * T::STAGE];
    __shared__ uint32_t last_flag;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WGN, wn = wave % WGN;
    const uint32_t n = K / BK;   // stages per tile
    const uint64_t U = (uint64_t)tiles * n, G = gridDim.x;

    uint64_t ub, ue;   // this block's units
    if constexpr (SK) {
        ub = (uint64_t)blockIdx.x * U / G;
        ue = (uint64_t)(blockIdx.x + 1) * U / G;
    } else {
        const uint32_t xcd = blockIdx.x % XCDS, l = blockIdx.x / XCDS;
        const uint32_t per = tiles / XCDS, rem = tiles % XCDS;
        ub = (uint64_t)(xcd * per + (xcd < rem ? xcd : rem) + l) * n;
        ue = ub + n;
    }
    if (ub >= ue) return;   // (SK) more blocks than units: nothing for this one
    const uint32_t L = (uint32_t)(ue - ub);
    // Under SK: the block holding unit u.
    auto block_of = [&](uint64_t u) { return (uint32_t)(((u + 1) * G - 1) / U); };

    // Copy sources: lane l of activation copy c brings tile row RA c + l / CHA
    // and the chunk stored in slot l % CHA of it; of code copy c, row
    // RB c + l / CHB, slot l % CHB. Rows past M / N are clamped (never stored).
    uint32_t tra[T::LA], ofa[T::LA], trb[T::LB], ofb[T::LB];
#pragma unroll
    for (int q = 0; q < T::LA; ++q) {
        tra[q] = (wave * T::LA + q) * T::RA + lane / CHA;
        ofa[q] = ((lane % CHA) ^ swz_a(tra[q])) * 16;
    }
#pragma unroll
    for (int q = 0; q < T::LB; ++q) {
        trb[q] = (wave * T::LB + q) * T::RB + lane / CHB;
        ofb[q] = ((lane % CHB) ^ swz_b<CHB>(trb[q])) * 16;
    }
    // Copies come in unit order; past the block's last unit they repeat it
    // (surplus copies, never read). Without SK the block's rows are fixed:
    // per-lane pointers plus a stage offset. Under SK a cursor (tile row-block
    // tm, column-block tn, stage ks) follows the copies across tiles.
    const uint32_t t_first = (uint32_t)(ub / n), s_first = (uint32_t)(ub % n);
    uint32_t c_tm = t_first % tiles_m, c_tn = t_first / tiles_m, c_ks = s_first, issued = 0;
    const uint8_t *ga[T::LA];
    const uint8_t *gb[T::LB];
    if constexpr (!SK) {
#pragma unroll
        for (int q = 0; q < T::LA; ++q) {
            const uint32_t r = c_tm * BM + tra[q] < M ? c_tm * BM + tra[q] : M - 1;
            ga[q] = reinterpret_cast<const uint8_t *>(x) + (size_t)r * K * 2 + ofa[q];
        }
#pragma unroll
        for (int q = 0; q < T::LB; ++q) {
            const uint32_t r = c_tn * BN + trb[q] < N ? c_tn * BN + trb[q] : N - 1;
            gb[q] = codes + (size_t)r * K + ofb[q];
        }
    }
    auto issue = [&](int slot) __attribute__((always_inline)) {
        uint8_t *base = lds + slot * T::STAGE;
        if constexpr (!SK) {
            const uint32_t st = issued < L ? issued : L - 1;
            ++issued;
#pragma unroll
            for (int q = 0; q < T::LA; ++q) copy16_to_lds(ga[q] + (size_t)st * A_ROW, base + (wave * T::LA + q) * 1024);
#pragma unroll
            for (int q = 0; q < T::LB; ++q)
                copy16_to_lds(gb[q] + (size_t)st * B_ROW, base + T::A_BYTES + (wave * T::LB + q) * 1024);
            return;
        }
        const uint32_t m0 = c_tm * BM, n0 = c_tn * BN, st = c_ks;
        // Advance without branches (selects on wave-uniform values), so the
        // copies stay in the scheduling region of the MFMAs around them.
        const uint32_t adv = ++issued < L ? 1u : 0u;
        const uint32_t ks1 = c_ks + adv, wrap = ks1 == n ? 1u : 0u;
        const uint32_t tm1 = c_tm + wrap, wrap2 = tm1 == tiles_m ? 1u : 0u;
        c_ks = wrap ? 0u : ks1;
        c_tm = wrap2 ? 0u : tm1;
        c_tn += wrap2;
#pragma unroll
        for (int q = 0; q < T::LA; ++q) {
            const uint32_t r = m0 + tra[q] < M ? m0 + tra[q] : M - 1;
            copy16_to_lds(reinterpret_cast<const uint8_t *>(x) + (size_t)r * K * 2 + (size_t)st * A_ROW + ofa[q],
                          base + (wave * T::LA + q) * 1024);
        }
#pragma unroll
        for (int q = 0; q < T::LB; ++q) {
            const uint32_t r = n0 + trb[q] < N ? n0 + trb[q] : N - 1;
            copy16_to_lds(codes + (size_t)r * K + (size_t)st * B_ROW + ofb[q],
                          base + T::A_BYTES + (wave * T::LB + q) * 1024);
        }
    };

    // Fragments at k-step ks of a stage, lane l: row l % 32 of the 32-row tile
    // and the 8 k of half h = l / 32: activation bytes 32 ks + 16 h (chunk
    // 2 ks + h), codes bytes 16 ks + 8 h (chunk ks, second half for h = 1).
    const uint32_t rl = lane & 31, h = lane >> 5, swa = swz_a(rl), swb = swz_b<CHB>(rl);
    auto read_frags = [&](int slot, int ks, u32x4 (&fa)[WM], u32x2 (&fb)[WN]) __attribute__((always_inline)) {
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
    auto zero_acc = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    };
    zero_acc();

    // MFMAs q0 <= q < q1 of the wave's WM x WN tiles (q = i WN + j); the code
    // fragments are decoded once per k-step. D = codes x^T: rows n, columns m.
    auto mfma_part = [&](int q0, int q1, const u32x4 (&fa)[WM], const u32x4 (&wb)[WN]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = q0; q < q1; ++q) {
            const int i = q / WN, j = q % WN;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, wb[j]),
                                                                __builtin_bit_cast(bf16x8, fa[i]), acc[i][j], 0, 0,
                                                                0);
        }
    };
    auto decode = [&](const u32x2 (&fb)[WN], u32x4 (&wb)[WN]) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < WN; ++j)
            wb[j] = u32x4{dec_pair<F>(fb[j].x, false), dec_pair<F>(fb[j].x, true), dec_pair<F>(fb[j].y, false),
                          dec_pair<F>(fb[j].y, true)};
    };

    // Lane l holds output row m = ... + l % 32 and, per group g of four
    // accumulators, the four consecutive columns n = ... + 8 g + 4 h + e.
    const float *sp = scales ? scales : &one_f32;   // (pointer, stride): no branch per scale
    const uint32_t ss = scales != nullptr;
    auto store_tile = [&](uint32_t t) __attribute__((always_inline)) {
        const uint32_t m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
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
                        o[e] = acc[i][j][4 * g + e] * sp[nn * ss];
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
    };
    // The block's only tile (without SK), once no copy into the ring is in
    // flight: the scaled bf16 values go to a row-major BM x BN tile in LDS
    // (16-byte chunk c of row r in slot slot(r, c): c ^ (r % CC) for a
    // power-of-two CC, else (c + r) % CC), then the block stores whole tile
    // rows, 16 bytes per lane, rather than 8 bytes of each of 32 rows per
    // store instruction.
    auto store_tile_lds = [&](uint32_t t) __attribute__((always_inline)) {
        constexpr int CC = BN / 8, RB = BN * 2, NT = 64 * T::W;   // chunks, bytes of a tile row; threads
        static_assert(S * T::STAGE >= BM * RB, "the output tile fits the operand ring");
        static_assert((BM * CC) % NT == 0, "whole passes");
        auto slot = [](uint32_t r, uint32_t c) -> uint32_t {
            if constexpr ((CC & (CC - 1)) == 0) return c ^ (r % CC);
            else return (c + r) % CC;
        };
        const uint32_t m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;
        wait_vmcnt<0>();
        __syncthreads();
        // The lane index through an empty asm: the epilogue's addresses are
        // computed here rather than hoisted before the main loop (where they
        // would hold registers through it).
        uint32_t te = tid;
        asm volatile("" : "+v"(te));
        const uint32_t rle = te & 31, he = (te >> 5) & 1;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const uint32_t r = wm * (32 * WM) + i * 32 + rle;
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t c = wn * (4 * WN) + 4 * j + g;   // columns 8 c .. 8 c + 7 of the tile
                    const uint32_t nb = n0 + 8 * c + 4 * he;
                    float o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t nn = nb + e < N ? nb + e : N - 1;
                        o[e] = acc[i][j][4 * g + e] * sp[nn * ss];
                    }
                    const uint32_t lo = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
                    const uint32_t hi = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
                    *reinterpret_cast<u32x2 *>(lds + r * RB + slot(r, c) * 16 + 8 * he) = u32x2{lo, hi};
                }
        }
        __syncthreads();
#pragma unroll
        for (int p = 0; p < BM * CC / NT; ++p) {
            const uint32_t ix = p * NT + te, r = ix / CC, c = ix % CC, m = m0 + r, nc = n0 + 8 * c;
            if (m >= M || nc >= N) continue;
            const u32x4 v = *reinterpret_cast<const u32x4 *>(lds + r * RB + slot(r, c) * 16);
            uint16_t *dst = y + (size_t)m * N + nc;
            if (vec_out && nc + 8 <= N) {
                // Non-temporal, as the fp8 GEMM's epilogue (same-box A/B: equal or
                // 0.5-2.5% faster on every tile form's product, M = 256 [14336,
                // 4096] 39.5 -> 38.9 us).
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(dst));
            } else {
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (nc + e < N) dst[e] = (uint16_t)(w[e / 2] >> (16 * (e % 2)));
            }
        }
    };
    // A partial slot holds BM x BN floats: wave w's WM WN 16 accumulators,
    // each as 64 consecutive floats (one per lane). Block b's segment of tile
    // t uses slot b + t: distinct for every (block, tile) pair that meets,
    // since a block only moves to later tiles than the block before it.
    constexpr uint32_t SLOT = BM * BN, WAVE_PART = NQ * 16 * 64;
    auto slot_ptr = [&](uint32_t b, uint32_t t) __attribute__((always_inline)) -> float * {
        return part + ((size_t)b + t) * SLOT + (size_t)wave * WAVE_PART + lane;
    };
    // The end of the block's run on tile t (its last unit u).
    auto finish = [&](uint32_t t) __attribute__((always_inline)) {
        if constexpr (SK) {
            const uint64_t t0 = (uint64_t)t * n;
            if (!(ub <= t0 && ue >= t0 + n)) {
                const uint32_t b0 = block_of(t0), b1 = block_of(t0 + n - 1);
                // Partials and counter go through agent-scope (device-coherent)
                // accesses, which bypass the per-XCD L2s' non-coherent copies;
                // the stores have completed (vmcnt 0) before the count moves.
                // The count is an acquire-release: the block's stores (ordered
                // before it by the barrier) happen before the last block's
                // reads (ordered after its own count by the next barrier).
                float *mine = slot_ptr(blockIdx.x, t);
#pragma unroll
                for (int q = 0; q < NQ; ++q)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        __hip_atomic_store(mine + (q * 16 + e) * 64, acc[q / WN][q % WN][e], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                wait_vmcnt<0>();
                __syncthreads();
                if (tid == 0) {
                    const uint32_t seen = __hip_atomic_fetch_add(cnt + t, 1u, __ATOMIC_ACQ_REL,
                                                                 __HIP_MEMORY_SCOPE_AGENT);
                    last_flag = seen + 1 == b1 - b0 + 1;
                }
                __syncthreads();
                const bool last = last_flag != 0;
                if (last) {
                    zero_acc();
                    for (uint32_t b = b0; b <= b1; ++b) {
                        float *p = slot_ptr(b, t);
#pragma unroll
                        for (int q = 0; q < NQ; ++q)
#pragma unroll
                            for (int e = 0; e < 16; ++e)
                                acc[q / WN][q % WN][e] += __hip_atomic_load(p + (q * 16 + e) * 64, __ATOMIC_RELAXED,
                                                                            __HIP_MEMORY_SCOPE_AGENT);
                    }
                    store_tile(t);
                    if (tid == 0) __hip_atomic_store(cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __syncthreads();   // last_flag is rewritten at the next tile's end
                zero_acc();
                return;
            }
        }
        if constexpr (SK) store_tile(t);
        else store_tile_lds(t);
        zero_acc();
    };

    // The pipeline of gemm_fp8_mfma: S stages in flight from the prologue;
    // per stage one barrier once each wave's own copies of the next stage
    // have landed, then the copy of stage i + S into the slot stage i used.
#pragma unroll
    for (int s = 0; s < S; ++s) issue(s);
    wait_vmcnt<(S - 1) * T::LOADS>();
    lds_barrier();
    u32x4 fa[2][WM];
    u32x2 fb[2][WN];
    read_frags(0, 0, fa[0], fb[0]);
    auto kstep = [&](auto cur_c, auto ks_c, uint32_t i) __attribute__((always_inline)) {
        constexpr int CUR = decltype(cur_c)::value, NXT = CUR ^ 1, KSI = decltype(ks_c)::value;
        u32x4 wb[WN];
        decode(fb[CUR], wb);
        if constexpr (KSI + 1 < KSTEPS) {
            read_frags((int)(i % S), KSI + 1, fa[NXT], fb[NXT]);
            mfma_part(0, NQ, fa[CUR], wb);
            interleave<NQ, WM + WN, 0>();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            mfma_part(0, HALF, fa[CUR], wb);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<(S - 2) * T::LOADS>();
            lds_barrier();
            issue((int)(i % S));
            read_frags((int)((i + 1) % S), 0, fa[NXT], fb[NXT]);
            mfma_part(HALF, NQ, fa[CUR], wb);
            interleave<NQ - HALF, WM + WN, T::LOADS>();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // k-step ks of every stage uses fragment set ks & 1 (KSTEPS is even).
    static_assert(KSTEPS % 2 == 0, "the fragment sets alternate within a stage");
    auto stage = [&](auto self, auto ks_c, uint32_t i) __attribute__((always_inline)) {
        constexpr int KSI = decltype(ks_c)::value;
        kstep(std::integral_constant<int, KSI & 1>{}, ks_c, i);
        if constexpr (KSI + 1 < KSTEPS) self(self, std::integral_constant<int, KSI + 1>{}, i);
    };
    // The block's units tile by tile: a run of stages, then the tile's end.
    uint32_t i = 0, f_t = t_first, f_ks = s_first;
    while (i < L) {
        const uint32_t run = n - f_ks < L - i ? n - f_ks : L - i;
        for (uint32_t r = 0; r < run; ++r, ++i) stage(stage, std::integral_constant<int, 0>{}, i);
        finish(f_t);
        f_ks = 0;
        ++f_t;
    }
    wait_vmcnt<0>();   // the clamped surplus copies land before LDS is released
}

// One launch; under SK, `part` holds (G + tiles - 1) BM BN floats and `cnt`
// one zeroed counter per tile (left zeroed by the launch) for a grid of G
// blocks.
template <int F, int WGM, int WGN, int WM, int WN, int BK, int S, bool SK>
int launch_tiles_cfg(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                     uint32_t K, uint16_t *y, hipStream_t st, uint32_t grid, float *part, uint32_t *cnt) {
    using T = Tile<WGM, WGN, WM, WN, BK>;
    const uint32_t tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
    const uint32_t tiles = tiles_m * tiles_n;
    // Whole 16-byte chunks of output rows (the LDS-staged store; under SK the
    // direct store of 8-byte groups, which this implies).
    const uint32_t vec_out = N % 8 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (!SK) grid = tiles;
    hipLaunchKernelGGL((w8a16_tiles<F, WGM, WGN, WM, WN, BK, S, SK>), dim3(grid), dim3(64 * T::W), 0, st, x, codes,
                       scales, M, N, K, tiles_m, tiles, y, vec_out, part, cnt);
    return check_launch("w8a16_tiles");
}

inline uint64_t tile_count(uint32_t M, uint32_t N, uint32_t bm, uint32_t bn) {
    return (uint64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
}

// Long K (at least 64 stages of 128 codes) over fewer 128 x 128 tiles than
// half the CUs: one tile per block would leave most of the chip idle.
inline bool streamk_suits(uint32_t M, uint32_t N, uint32_t K) {
    return K % 128 == 0 && K >= 8192 && 2 * tile_count(M, N, 128, 128) < (uint64_t)device_props().cus;
}

// Tile choice. Long K (K >= 8192) over fewer 128 x 128 tiles than half the
// CUs runs stream-K on 128 x 128 tiles of 128-code stages (M = 256
// [4096, 14336]: 92.8 -> 66.5 us). Otherwise each form's time is modelled as
// rounds x (c0 + c1 x K / 64), rounds = ceil(tiles / CUs), with (c0, c1) in
// microseconds fitted to graph-replayed timings of every form on eleven
// products (M 128-1024 over the Llama-3.1-8B and Qwen2.5-32B shapes; most
// within 16% of the fit), and the cheapest form runs; on those products that
// is the fastest one measured (M = 256 [4096, 4096] 26.6 -> 21.8 us with
// 64 x 64 tiles, M = 512 [5120, 5120] 64.4 -> 43.2 us with 128 x 128,
// M = 1024 [5120, 27648] 328 -> 308 us with 128 x 160). Stream-K takes
// (G + tiles - 1) BM BN floats of partials (6.3 Mi floats at most on 256
// CUs) and a counter per tile (fewer than 128).
template <int F>
int launch_tiles_f(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                   uint32_t K, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    const uint64_t cus = (uint64_t)device_props().cus;
    const uint64_t t128 = tile_count(M, N, 128, 128);
    if (streamk_suits(M, N, K)) {
        using T = Tile<2, 4, 2, 1, 128>;
        const uint64_t units = t128 * (K / 128);
        const uint32_t grid = (uint32_t)(units < cus ? units : cus);
        const size_t floats = ((size_t)grid + t128 - 1) * T::BM * T::BN;
        int rc = RENG_HIP_OK;
        float *part = split_partials(floats, st, fixed, &rc);
        if (rc) return rc;
        uint32_t *cnt = fixed ? static_tile_counters(&rc) : tile_counters((uint32_t)t128, st, &rc);
        if (rc) return rc;
        return launch_tiles_cfg<F, 2, 4, 2, 1, 128, 3, true>(x, codes, scales, M, N, K, y, st, grid, part, cnt);
    }
    struct Cand {
        uint32_t bm, bn;
        float c0, c1;
        bool fits;
    };
    const Cand cands[] = {
        {256, 256, 28.6f, 1.130f, true},            // 8 waves of 128 x 64, 64-code stages, 3 slots
        {128, 256, 18.1f, 0.703f, true},            // 8 waves of 64 x 64, 3 slots
        {128, 160, 5.6f, 0.700f, K % 128 == 0},     // 4 waves of 32 x 160, 128-code stages, 2 slots
        {128, 128, 10.2f, 0.465f, true},            // 8 waves of 64 x 32, 6 slots
        {64, 128, 5.0f, 0.348f, true},              // 8 waves of 32 x 32, 6 slots
        {64, 64, 0.0f, 0.251f, true},               // 4 waves of 32 x 32, 6 slots
    };
    int pick = 0;
    float best = 0.0f;
    for (int i = 0; i < 6; ++i) {
        if (!cands[i].fits) continue;
        const uint64_t rounds = (tile_count(M, N, cands[i].bm, cands[i].bn) + cus - 1) / cus;
        const float est = (float)rounds * (cands[i].c0 + cands[i].c1 * (float)(K / 64));
        if (i == 0 || est < best) pick = i, best = est;
    }
    switch (pick) {
    case 0: return launch_tiles_cfg<F, 2, 4, 4, 2, 64, 3, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    case 1: return launch_tiles_cfg<F, 2, 4, 2, 2, 64, 3, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    case 2: return launch_tiles_cfg<F, 4, 1, 1, 5, 128, 2, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    case 3: return launch_tiles_cfg<F, 2, 4, 2, 1, 64, 6, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    case 4: return launch_tiles_cfg<F, 2, 4, 1, 1, 64, 6, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    default: return launch_tiles_cfg<F, 2, 2, 1, 1, 64, 6, false>(x, codes, scales, M, N, K, y, st, 0, nullptr, nullptr);
    }
}

}  // namespace tiles

// Below half the CUs in 64 x 128 tiles the 64-row kernels, which split K,
// are faster (M = 100 [3000, 4096]: 22.2 against 28.1 us) - unless the
// product suits stream-K.
bool w8a16_tiles_take(uint32_t M, uint32_t N, uint32_t K) {
    return M > 64 && K % tiles::K_ALIGN == 0 &&
           (tiles::streamk_suits(M, N, K) || 2 * tiles::tile_count(M, N, 64, 128) >= (uint64_t)device_props().cus);
}

int launch_w8a16_tiles(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    if (format == RENG_HIP_E4M3) return tiles::launch_tiles_f<RENG_HIP_E4M3>(x, codes, scales, M, N, K, y, st, fixed);
    return tiles::launch_tiles_f<RENG_HIP_E5M2>(x, codes, scales, M, N, K, y, st, fixed);
}

}  // namespace reng
