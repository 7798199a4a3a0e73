// skinny.hip - y[m, n] = bf16(s[n] * sum_k x[m, k] * decode(c[n, k])) for
// up to 64 activation rows (bf16) on bf16 MFMA (gfx950); gemm.hip sends a
// product of one row (or two with a short K) to its GEMV instead.
//
// The reference semantics are gemm_cpu over Quantized::dequantize
// (crates/reng-model/src/bin/fp8_probe.rs:55-67) with the per-channel scaleB
// of fp8_gemm_bf16 (crates/reng-synapse/src/fp8.rs:295-331).
//
// The MFMA operand layout wants 16 different weight rows across a wave's
// lanes, which read straight from memory is 16 rows x 64 bytes per load
// instruction: that pattern streams HBM at ~4 TB/s on this device against
// ~5.5 TB/s for 4 rows x 256 bytes. So the codes (and the activation) go
// through LDS: copied in 4 x 256-byte pieces by global_load_lds and read back
// transposed (skinny_rows for M <= 16: whole-K blocks, no partial sums in
// memory; skinny_wide for 16 < M <= 64, where a block must cover many weight
// rows per activation byte it reads, and for the M <= 16 products skinny_rows
// runs on too few blocks: it splits K over blocks and merges the splits'
// partial sums inside the same launch).
#include <map>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.h"
#include "gemm.h"

namespace reng {

namespace skinny {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int CHUNK = 128;     // codes of k per chunk
constexpr int STAGE_K = 256;   // codes of k per pipeline stage (two chunks)

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

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at [15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((N & 0xf) | (7 << 4) | (0xf << 8) | ((N >> 4) << 14));
}

// One global_load_lds_dwordx4: 16 bytes per lane from g into LDS at
// l + 16 * lane (l is wave-uniform). A __device__ function because the
// kernel's lambdas cannot form the LDS address-space cast in their host-side
// instantiation.
__device__ __forceinline__ void copy16(const uint8_t *g, uint8_t *l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 16, 0, 0);
}
// The same for code bytes, which every block reads once: the non-temporal
// policy (nt) keeps them from displacing the activation the blocks share in
// L2 (the copy stream alone on Qwen2.5-7B M = 64: [18944, 3584] 18.2 -> 17.6 us,
// [3584, 18944] 15.4 -> 14.1 us).
__device__ __forceinline__ void copy16_nt(const uint8_t *g, uint8_t *l) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)l, 16, 0, 2);
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads have returned, so copies may
// overwrite the slot they read.
__device__ __forceinline__ void wait_lgkm0() {
    asm volatile("" ::: "memory");   // LDS accesses before the wait stay before it
    __builtin_amdgcn_s_waitcnt(0xf | (7 << 4) | (0 << 8) | (3 << 14));
    asm volatile("" ::: "memory");
}

// A workgroup barrier without the vmcnt(0) of __syncthreads' fence; the memory
// clobbers keep LDS accesses on their side of it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A block of KW x NW waves owns 16 NT NW weight rows; wave (kw, nw) takes the
// rows [16 NT nw, +16 NT) of the block over the kw-th of KW equal runs of
// 128-code chunks of K. A pipeline stage is 256 codes (two chunks; the last
// stage of a run may hold only one). Each wave streams its stages into a
// private S-slot LDS ring with global_load_lds, so its loop has no barrier:
//   weights, per 16-row tile: 4 copies of 4 rows x 256 bytes (contiguous
//     256-byte runs per row), 16-byte piece p of row r stored in slot p ^ (r % 16);
//   activation: MA / 2 copies of 2 rows x 512 bytes (256 bf16), 8-element
//     piece p of row r stored in slot p ^ (r % 16); rows >= M repeat row M - 1.
// The loop issues only these copies (no loads into registers), so the waits
// are explicit s_waitcnt vmcnt: stage st + S - 1 is requested before stage st
// is consumed, and consuming st waits for all but the (S - 1) newer stages.
// MFMA operands are read back with ds_read_b128 in the v_mfma_f32_16x16x32_bf16
// layout (the XOR slots make each 16-lane phase hit 16 distinct 16-byte bank
// groups): lane l takes weight row l % 16, codes [16 g, +16) and [64 + 16 g,
// +16) of a chunk (g = l / 16; k-steps 0, 1 and 2, 3), decoded to bf16 in
// registers (exact), and the activation row l % 16 at the same k. At the end
// the KW partial tiles of a row group meet in LDS and are added in kw order.
template <int F, int MA, int NT, int KW, int NW, int S, int ACTK>
__global__ __launch_bounds__(64 * KW * NW) void skinny_rows(const uint16_t *__restrict__ x,
                                                            const uint8_t *__restrict__ codes,
                                                            const float *__restrict__ scales, uint32_t M,
                                                            uint32_t N, uint32_t K, uint16_t *__restrict__ y) {
    constexpr int TILE = 16 * STAGE_K;               // one 16-row tile of a stage, bytes
    constexpr bool AR = ACTK > 0;                    // activation resident in LDS (K <= ACTK chunks)
    constexpr int WBYTES = NT * TILE, ABYTES = AR ? 0 : MA * STAGE_K * 2;
    constexpr int SLOT = WBYTES + ABYTES, RING = S * SLOT;
    constexpr int CA = AR ? 0 : MA / 2, C = 4 * NT + CA;   // copies per stage
    constexpr int ACT_BYTES = ACTK * MA * CHUNK * 2;       // [chunk][MA rows][256 B]
    static_assert(S >= 2 && (S - 1) * C < 64, "pipeline depth");
    // Every wave must reach the barrier after the activation copies: with one
    // run of K per wave (KW = 1) each wave has at least one chunk.
    static_assert(!AR || KW == 1, "the resident activation needs KW = 1");
    constexpr int W = KW * NW;
    constexpr int RED = KW > 1 ? W * NT * 1024 : 0;
    constexpr int LDS0 = W * RING > RED ? W * RING : RED;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS0 + ACT_BYTES];
    uint8_t *act = lds + LDS0;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave / NW, nw = wave % NW;
    const uint32_t r16 = lane & 15, g = lane >> 4;
    const uint32_t n0 = (blockIdx.x * NW + nw) * (16 * NT);
    const uint32_t chunks = K / CHUNK;
    const uint32_t c0 = kw * chunks / KW, c1 = (kw + 1) * chunks / KW;
    const uint32_t nst = (c1 - c0 + 1) / 2;
    uint8_t *ring = lds + wave * RING;

    // Copy sources. Weight copy (t, i), lane j: row rr = 4 i + j / 16 of tile
    // t, piece p = (j % 16) ^ rr. Activation copy i, lane j: row 2 i + j / 32,
    // piece p = (j % 32) ^ (row % 16). Pieces in a stage's second chunk step
    // back one chunk in a one-chunk stage (copied, never read).
    const uint8_t *wsrc[NT][4];
    uint32_t whi = 0;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t rr = 4 * i + g, p = r16 ^ rr;
            uint32_t n = n0 + 16 * t + rr;
            n = n < N ? n : N - 1;   // rows past N are read but never stored
            wsrc[t][i] = codes + (size_t)n * K + (size_t)c0 * CHUNK + (p >> 3) * CHUNK + (p & 7) * 16;
            whi |= (p >> 3) << (4 * t + i);
        }
    const uint16_t *asrc[CA > 0 ? CA : 1];
    uint32_t ahi = 0;
#pragma unroll
    for (int i = 0; i < CA; ++i) {
        const uint32_t row = 2 * i + (lane >> 5), p = (lane & 31) ^ (row & 15);
        const uint32_t m = row < M ? row : M - 1;
        asrc[i] = x + (size_t)m * K + (size_t)c0 * CHUNK + (p >> 4) * CHUNK + (p & 15) * 8;
        ahi |= (p >> 4) << i;
    }
    auto one_chunk = [&](uint32_t st) { return c0 + 2 * st + 1 >= c1; };
    auto copies = [&](uint32_t st) {
        const bool half = one_chunk(st);
        uint8_t *slot = ring + (st % S) * SLOT;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t back = (half && ((whi >> (4 * t + i)) & 1)) ? CHUNK : 0u;
                copy16_nt(wsrc[t][i] + (size_t)st * STAGE_K - back, slot + t * TILE + i * 1024);
            }
#pragma unroll
        for (int i = 0; i < CA; ++i) {
            const uint32_t back = (half && ((ahi >> i) & 1)) ? CHUNK : 0u;
            copy16(reinterpret_cast<const uint8_t *>(asrc[i] + (size_t)st * STAGE_K - back),
                   slot + WBYTES + i * 1024);
        }
    };

    f32x4 acc[NT][2];   // two accumulators per tile: even and odd k-steps
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Chunk h of a stage: weight pieces 8 h + g, 8 h + 4 + g; activation
    // elements 128 h + 16 g + 8 (j & 1) + 64 (j >> 1) for k-step j, i.e. piece
    // 16 h + 2 g + (j & 1) + 8 (j >> 1).
    const uint32_t am = r16 < M ? r16 : M - 1;
    auto compute = [&](uint32_t st) {
        const bool half = one_chunk(st);
        const uint8_t *slot = ring + (st % S) * SLOT;
        const uint8_t *arow = slot + WBYTES + am * (STAGE_K * 2);
        const uint32_t cc = c0 + 2 * st;   // the stage's first chunk
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            if (h == 1 && half) break;
            u32x4 w[NT][2];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint8_t *tb = slot + t * TILE + r16 * STAGE_K;
                w[t][0] = *reinterpret_cast<const u32x4 *>(tb + (((8 * h + g) ^ r16) * 16));
                w[t][1] = *reinterpret_cast<const u32x4 *>(tb + (((8 * h + 4 + g) ^ r16) * 16));
            }
            u32x4 a[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (AR) {
                    const uint32_t p = 2 * g + (j & 1) + 8 * (j >> 1);   // piece within chunk cc + h
                    a[j] = *reinterpret_cast<const u32x4 *>(act + ((cc + h) * MA + am) * (CHUNK * 2) +
                                                            ((p ^ (am & 15)) * 16));
                } else {
                    const uint32_t p = 16 * h + 2 * g + (j & 1) + 8 * (j >> 1);
                    a[j] = *reinterpret_cast<const u32x4 *>(arow + ((p ^ (am & 15)) * 16));
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x8 b = __builtin_bit_cast(bf16x8, a[j]);
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const u32x4 &q = w[t][j >> 1];
                    const bf16x8 wa = (j & 1) ? dec8<F>(q.z, q.w) : dec8<F>(q.x, q.y);
                    acc[t][j & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa, b, acc[t][j & 1], 0, 0, 0);
                }
            }
        }
    };

    // The scales of this lane's output rows, requested before any copy (older
    // than everything the explicit waits count; used after the loop).
    float sc[NT][4];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t n = n0 + t * 16 + 4 * g + e;
            sc[t][e] = scales ? scales[n < N ? n : N - 1] : 1.0f;
        }

    if constexpr (AR) {
        // The whole activation, once per block: chunk-major, row r's 16-byte
        // piece p of a chunk in slot p ^ (r % 16); copies of 4 rows x 256 B
        // spread over the waves, issued before any weight copy.
        constexpr uint32_t PER = MA / 4;   // copies per chunk
        for (uint32_t q = wave; q < chunks * PER; q += W) {
            const uint32_t ch = q / PER, r0 = 4 * (q % PER), rr = r0 + (lane >> 4);
            const uint32_t p = (lane & 15) ^ (rr & 15);
            const uint32_t m = rr < M ? rr : M - 1;
            copy16(reinterpret_cast<const uint8_t *>(x + (size_t)m * K + (size_t)ch * CHUNK + p * 8),
                   act + (ch * MA + r0) * (CHUNK * 2));
        }
    }
    if (c0 < c1) {
#pragma unroll
        for (int s = 0; s < S - 1; ++s)
            if ((uint32_t)s < nst) copies(s);
        if constexpr (AR) {
            wait_vmcnt<0>();   // this wave's activation copies (and first stages) have landed
            lds_barrier();     // ... and every other wave's
        }
        for (uint32_t st = 0; st < nst; ++st) {
            if (st + S - 1 < nst) {
                wait_lgkm0();                // slot (st - 1) % S has been read
                copies(st + S - 1);
                wait_vmcnt<(S - 1) * C>();   // stage st has landed; S - 1 newer stages in flight
            } else {
                wait_vmcnt<0>();             // the last S - 1 stages: nothing newer to keep
            }
            asm volatile("" ::: "memory");   // no LDS read moves above the wait
            compute(st);
            asm volatile("" ::: "memory");   // ... nor the next copies above these reads
        }
    }
    f32x4 fin[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) fin[t] = acc[t][0] + acc[t][1];

    // Waves of the same rows meet in LDS (every ring is idle: the last stage
    // waited for vmcnt 0) and are added in kw order; tile t of a row group is
    // finished by the wave with kw == t % KW.
    f32x4 *red = reinterpret_cast<f32x4 *>(lds);
    if constexpr (KW > 1) {
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; ++t) red[((kw * NW + nw) * NT + t) * 64 + lane] = fin[t];
        __syncthreads();
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        f32x4 s;
        if constexpr (KW > 1) {
            if (t % KW != kw) continue;
            s = red[(nw * NT + t) * 64 + lane];
#pragma unroll
            for (int w = 1; w < KW; ++w) s += red[((w * NW + nw) * NT + t) * 64 + lane];
        } else {
            s = fin[t];
        }
        // D of a 16x16 tile: lane l holds column m = l % 16 and rows
        // n = 4 (l / 16) + e: four consecutive outputs of row m.
        const uint32_t m = r16;
        const uint32_t nb = n0 + t * 16 + 4 * g;
        if (m >= M) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = s[e] * sc[t][e];
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

template <int F, int MA, int NT, int KW, int NW, int S, int ACTK = 0>
int launch_cfg(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N, uint32_t K,
               uint16_t *y, hipStream_t st) {
    const uint32_t rows = 16 * NT * NW;
    const uint32_t blocks = (N + rows - 1) / rows;
    hipLaunchKernelGGL((skinny_rows<F, MA, NT, KW, NW, S, ACTK>), dim3(blocks), dim3(64 * KW * NW), 0, st, x, codes,
                       scales, M, N, K, y);
    return check_launch("skinny_rows");
}

// One block per CU at these LDS sizes (96-160 KB), so the grid is sized for a
// single round: the fewest rows per block (16, 32, 64, 80 or 128) whose grid
// fits on the CUs; narrow blocks split K over their waves. The 80-row form
// (5 waves of 16 rows, M <= 8, K <= 4096) holds the activation in LDS for the
// whole block instead of copying it per stage; on [18944, 3584] it keeps 237
// CUs busy where 128-row blocks keep 148 (M = 8: 16.7 -> 14.8 us).
template <int F, int MA>
int launch_ma(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N, uint32_t K,
              uint16_t *y, hipStream_t st) {
    const uint32_t cus = (uint32_t)device_props().cus;
    constexpr int S3 = MA == 8 ? 3 : 2;   // ring depth of the 2-tile configurations (LDS)
    if ((N + 15) / 16 <= cus) {
        if constexpr (MA == 8) return launch_cfg<F, MA, 1, 8, 1, 2>(x, codes, scales, M, N, K, y, st);
        else return launch_cfg<F, MA, 1, 4, 1, 3>(x, codes, scales, M, N, K, y, st);
    }
    if ((N + 31) / 32 <= cus) return launch_cfg<F, MA, 2, 4, 1, 2>(x, codes, scales, M, N, K, y, st);
    if ((N + 63) / 64 <= cus) return launch_cfg<F, MA, 2, 2, 2, S3>(x, codes, scales, M, N, K, y, st);
    if constexpr (MA == 8) {
        if ((N + 79) / 80 <= cus && K / CHUNK <= 32)
            return launch_cfg<F, MA, 1, 1, 5, 3, 32>(x, codes, scales, M, N, K, y, st);
    }
    return launch_cfg<F, MA, 2, 1, 4, S3>(x, codes, scales, M, N, K, y, st);
}


// Up to 64 activation rows over many weight rows per activation byte. At
// M = 64 the activation is 128 bytes per k against R bytes of codes for R
// weight rows, so a block covers R = 32 NTW rows (32 to 128) and shares one
// copy of each stage between its 4 waves: stages of BK = 128 codes in an
// S-slot LDS ring (one barrier per stage), filled by global_load_lds
//   codes: R / 8 copies of 8 rows x 128 bytes, piece p of row r in slot p ^ swz8(r);
//   activation: 16 MT rows (>= M repeat row M - 1), 4 rows x 256 bytes per copy,
//     8-element piece p of row r in slot p ^ (r % 16);
// spread over the NWV waves. The waves form a WNC x WMC grid (WMC = 2 for
// MT >= 2, 1 for MT = 1): wave (wn, wm) computes rows [wn R / WNC, +R / WNC)
// against activation tiles wm, wm + WMC, ... (< MT).
//
// Blocks split K until the grid fills the CUs (split s takes chunks
// [s cps, +cps)). The splits of a row tile meet inside the launch: each block
// writes its f32 fragments to the tile's slot for its split, counts itself in
// on cnt[tile], and the last block of the tile to count in reads every split's
// fragments, adds them in split order (the same order whichever block is
// last, so the sums are deterministic), applies the scales, writes the tile
// and resets the counter for the next launch. No block waits for another.
// With splits, the grid is XCD-major: block b runs on XCD b % 8 (workgroups
// are dealt to the 8 XCDs round-robin) and takes tile (b / 8 / splits) * 8 +
// b % 8, so a tile's splits share one XCD's L2, where the partials go with
// plain stores and come back with L1-bypassing (sc0) loads. If the device was
// not seen to place workgroups that way (split_coherence), the partials go
// through agent-coherent (sc1) stores and loads instead.
//
// Why the last block sees every partial: each block's partial stores have
// completed (vmcnt 0: acknowledged by the L2, or with sc1 by memory) before
// its count is issued; the count is one atomic read-modify-write per tile, so
// the block that sees splits - 1 counts before its own comes after every
// other block's count; and it issues its loads only once its own count has
// returned. With COH 0 every block of the tile runs on one XCD and so writes
// and reads the same L2 (the loads skip the L1); with COH 1 the sc1 stores
// and loads are coherent across XCDs. This is gfx950's ordering of these
// accesses, not a release / acquire pair of the HIP memory model: at agent
// scope that pair would write back and invalidate the XCD's whole L2
// (buffer_wbl2 / buffer_inv) in every block. The split tests call each
// product repeatedly and check every output and bit-identical repeats.
__device__ __forceinline__ uint32_t swz8(uint32_t r) { return (r ^ ((r >> 3) & 1)) & 7; }

// The tile's last block learns it here; its frag then hold the sums over the
// splits. Slot (tile, split) holds NWV waves x NF x 64 f32x4, fragment f of
// lane l of wave w at (w NF + f) 64 + l. Every block of the tile calls this
// (it has barriers). part is addressed through a buffer resource of
// part_bytes, so the loads of a group past the last split fetch nothing.
template <int NF, int COH, int NWV>
__device__ __forceinline__ bool merge_splits(f32x4 (&frag)[NF], float *part, uint32_t part_bytes, uint32_t *cnt,
                                             uint32_t tile, uint32_t split, uint32_t splits, uint32_t *flag) {
    constexpr uint32_t WAVES = NWV;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(part, 0, part_bytes, 0x00020000);
    constexpr uint32_t slot = WAVES * NF * 64 * 16;   // bytes per (tile, split)
    const uint32_t lo = (uint32_t)(wave * NF * 64 + lane) * 16;
    const uint32_t mine = (tile * splits + split) * slot + lo;
    constexpr int ST = COH ? 16 : 0, LD = COH ? 16 : 1;   // sc1 both ways, or plain stores and sc0 loads
#pragma unroll
    for (int f = 0; f < NF; ++f)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, frag[f]), rs, mine + f * 1024, 0, ST);
    asm volatile("" ::: "memory");
    wait_vmcnt<0>();   // this wave's fragments are in the cache the last block reads
    __syncthreads();
    if (tid == 0) {
        const uint32_t seen = __hip_atomic_fetch_add(cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = seen + 1 == splits;
    }
    __syncthreads();
    if (!*flag) return false;
    asm volatile("" ::: "memory");
    // GS splits' fragments (32 loads per lane at most) requested together,
    // then added in order.
    constexpr int GS = NF >= 16 ? 2 : NF >= 8 ? 4 : 8;
    const uint32_t base = tile * splits * slot + lo;
    constexpr uint32_t PAST = 0xf8000000u;   // past any part_bytes (<= 0xf0000000): loads nothing
    for (uint32_t s0 = 0; s0 < splits; s0 += GS) {
        u32x4 v[GS][NF];
#pragma unroll
        for (int i = 0; i < GS; ++i) {
            const uint32_t off = s0 + i < splits ? base + (s0 + i) * slot : PAST;
#pragma unroll
            for (int f = 0; f < NF; ++f) v[i][f] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + f * 1024, 0, LD);
        }
        asm volatile("" ::: "memory");   // all of the group's loads before the first add
#pragma unroll
        for (int i = 0; i < GS; ++i) {
            const bool ok = s0 + i < splits, first = s0 + i == 0;
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const f32x4 x = __builtin_bit_cast(f32x4, v[i][f]);
                const f32x4 n = first ? x : frag[f] + x;
                frag[f] = ok ? n : frag[f];
            }
        }
    }
    if (tid == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

template <int F, int MT, int NTW, int S, int COH, int NWV, bool RAG>
__global__ __launch_bounds__(64 * NWV) void skinny_wide(const uint16_t *__restrict__ x, const uint8_t *__restrict__ codes,
                                                   const float *__restrict__ scales, uint32_t M, uint32_t N,
                                                   uint32_t K, uint32_t tiles, uint32_t splits, uint32_t cps,
                                                   uint16_t *__restrict__ y, float *part, uint32_t part_bytes,
                                                   uint32_t *cnt) {
    constexpr int BK = CHUNK, R = 32 * NTW, AR = 16 * MT;
    constexpr int WB = R * BK, AB = AR * BK * 2, SLOT = WB + AB;
    constexpr int WC = R / 8, AC = AR / 4;          // copies per stage (block)
    static_assert(WC % NWV == 0 && AC % NWV == 0, "copies split evenly over the waves");
    constexpr int C = (WC + AC) / NWV;              // copies per stage per wave
    static_assert(S >= 2 && (S - 2) * C < 64, "vmcnt");
    constexpr int WMC = MT >= 2 ? 2 : 1, WNC = NWV / WMC;
    constexpr int TPW = R / (16 * WNC);             // 16-row tiles per wave
    static_assert(TPW >= 1 && TPW * 16 * WNC == R, "rows split evenly over the wave rows");
    constexpr int MTW = (MT + WMC - 1) / WMC;       // activation tiles per wave
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * SLOT];
    __shared__ uint32_t last_flag;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave / WMC, wm = wave % WMC;
    const uint32_t r16 = lane & 15, g = lane >> 4;
    uint32_t tile = blockIdx.x, split = 0;
    if (splits > 1) {
        const uint32_t j = blockIdx.x / 8;
        tile = (j / splits) * 8 + blockIdx.x % 8;
        split = j % splits;
        if (tile >= tiles) return;   // the XCD-major grid's padding
    }
    const uint32_t n0 = tile * R;
    // RAG: K is not a multiple of the 128-code chunk (a multiple of 16), and
    // the last chunk holds kr < 128 codes. Its copies past K read the row's
    // first piece instead (in bounds), and its compute zeroes both operands
    // past K, so the padding adds exact zeros. (A template argument: the
    // checks cost the whole-chunk products 5% on small shapes.)
    const uint32_t chunks = (K + CHUNK - 1) / CHUNK, kr = K - (chunks - 1) * CHUNK;
    const uint32_t kc0 = split * cps, kc1 = kc0 + cps < chunks ? kc0 + cps : chunks;
    const uint32_t nst = kc1 - kc0;
    const uint32_t st_ragged = RAG && kc1 == chunks ? nst - 1 : 0xffffffffu;   // stage of the short chunk

    // This wave's copies q = wave + NWV c: q < WC a code copy, else activation copy q - WC.
    const uint8_t *src[C];
    uint32_t dst[C], unit[C], back[C], past = 0;   // past bit c: copy c's piece lies past K in the short chunk
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int q = wave + NWV * c;
        if (q < WC) {
            const uint32_t rr = q * 8 + lane / 8, p = (lane % 8) ^ swz8(rr);
            uint32_t n = n0 + rr;
            n = n < N ? n : N - 1;   // rows past N are read but never stored
            src[c] = codes + (size_t)n * K + (size_t)kc0 * CHUNK + p * 16;
            dst[c] = q * 1024;
            unit[c] = 1;
            back[c] = kc0 * CHUNK + p * 16;   // src[c] - back[c]: the row's first byte
            past |= (16 * p >= kr ? 1u : 0u) << c;
        } else {
            const int qa = q - WC;
            const uint32_t row = qa * 4 + lane / 16, p = (lane % 16) ^ (row & 15);
            const uint32_t m = row < M ? row : M - 1;
            src[c] = reinterpret_cast<const uint8_t *>(x + (size_t)m * K + (size_t)kc0 * CHUNK + p * 8);
            dst[c] = WB + qa * 1024;
            unit[c] = 2;
            back[c] = (kc0 * CHUNK + p * 8) * 2;
            past |= (8 * p >= kr ? 1u : 0u) << c;
        }
    }
    auto copies = [&](uint32_t st) {
        uint8_t *slot = lds + (st % S) * SLOT;
        if constexpr (RAG) {
            const bool short_chunk = st == st_ragged;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                // A piece past K in the short chunk reads the row's first piece
                // instead (in bounds; zeroed in the compute).
                const uint8_t *from =
                    short_chunk && ((past >> c) & 1) ? src[c] - back[c] : src[c] + (size_t)st * BK * unit[c];
                if (unit[c] == 1) copy16_nt(from, slot + dst[c]);
                else copy16(from, slot + dst[c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < C; ++c) {
                if (unit[c] == 1) copy16_nt(src[c] + (size_t)st * BK, slot + dst[c]);
                else copy16(src[c] + (size_t)st * BK * 2, slot + dst[c]);
            }
        }
    };

    f32x4 acc[TPW * MTW];   // fragment (t, u) at t MTW + u
#pragma unroll
    for (int f = 0; f < TPW * MTW; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Lane l's k-step j of a chunk takes codes and activation [kb, kb + 8),
    // kb = 16 (l / 16) + 8 (j % 2) + 64 (j / 2); in the short chunk those past
    // K are zeroed (kr is a multiple of 16, so a run of 8 is all in or all out).
    auto compute = [&](uint32_t st, auto short_c) {
        constexpr bool SHORT = decltype(short_c)::value;
        const uint8_t *slot = lds + (st % S) * SLOT;
        u32x4 w[TPW][2];
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const uint32_t rr = wn * (R / WNC) + t * 16 + r16;
            const uint8_t *rb = slot + rr * BK;
            w[t][0] = *reinterpret_cast<const u32x4 *>(rb + ((g ^ swz8(rr)) * 16));
            w[t][1] = *reinterpret_cast<const u32x4 *>(rb + (((4 + g) ^ swz8(rr)) * 16));
        }
        u32x4 a[MTW][4];
#pragma unroll
        for (int u = 0; u < MTW; ++u) {
            const int mt = wm + WMC * u;
            uint32_t am = (mt < MT ? mt : MT - 1) * 16 + r16;
            am = am < M ? am : M - 1;
            const uint8_t *arow = slot + WB + am * (BK * 2);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t p = 2 * g + (j & 1) + 8 * (j >> 1);
                a[u][j] = *reinterpret_cast<const u32x4 *>(arow + ((p ^ (am & 15)) * 16));
                if constexpr (SHORT) {
                    if (8 * p >= kr) a[u][j] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                const u32x4 &q = w[t][j >> 1];
                bf16x8 wa = (j & 1) ? dec8<F>(q.z, q.w) : dec8<F>(q.x, q.y);
                if constexpr (SHORT) {
                    if (16 * g + 8 * (j & 1) + 64 * (j >> 1) >= kr) wa = bf16x8{};
                }
#pragma unroll
                for (int u = 0; u < MTW; ++u) {
                    if (wm + WMC * u >= MT) break;
                    acc[t * MTW + u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        wa, __builtin_bit_cast(bf16x8, a[u][j]), acc[t * MTW + u], 0, 0, 0);
                }
            }
        }
    };

    // The scales of this lane's output rows, requested before any copy (older
    // than everything the explicit waits count; used after the loop).
    float sc[TPW][4];
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t n = n0 + wn * (R / WNC) + t * 16 + 4 * g + e;
            sc[t][e] = scales ? scales[n < N ? n : N - 1] : 1.0f;
        }

#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if ((uint32_t)s < nst) copies(s);
    for (uint32_t st = 0; st < nst; ++st) {
        if (st + S - 2 < nst) wait_vmcnt<(S - 2) * C>();   // own copies of stage st landed
        else wait_vmcnt<0>();
        wait_lgkm0();
        lds_barrier();   // everyone's copies of st landed; slot (st - 1) % S has been read
        if (st + S - 1 < nst) copies(st + S - 1);
        if (RAG && st == st_ragged) compute(st, std::integral_constant<bool, RAG>{});
        else compute(st, std::false_type{});
    }

    if (splits > 1 && !merge_splits<TPW * MTW, COH, NWV>(acc, part, part_bytes, cnt, tile, split, splits, &last_flag))
        return;

    // Lane holds column m = 16 mt + l % 16 and rows n = 4 (l / 16) + e.
#pragma unroll
    for (int u = 0; u < MTW; ++u) {
        const int mt = wm + WMC * u;
        if (mt >= MT) break;
        const uint32_t m = mt * 16 + r16;
        if (m >= M) continue;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            const uint32_t nb = n0 + wn * (R / WNC) + t * 16 + 4 * g;
            const f32x4 s = acc[t * MTW + u];
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = s[e] * sc[t][e];
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
}

// The copy stream of skinny_wide and nothing else, a yardstick for bench.py:
// the same grid, block, S-slot LDS ring, copies (codes R / 8 x 1 KB and
// activation 16 MT rows per stage, by global_load_lds), waits and barriers,
// with no fragment reads, decodes, MFMAs or output. Its time is the floor that
// the kernel's data movement alone sets. sink gets one word if a (never
// matching) value turns up, which keeps the copies live.
template <int MT, int NTW, int S, int NWV>
__global__ __launch_bounds__(64 * NWV) void stage_copy_kernel(const uint16_t *__restrict__ x,
                                                              const uint8_t *__restrict__ codes, uint32_t M,
                                                              uint32_t N, uint32_t K, uint32_t cps, uint32_t *sink) {
    constexpr int BK = CHUNK, R = 32 * NTW, AR = 16 * MT;
    constexpr int WB = R * BK, AB = AR * BK * 2, SLOT = WB + AB;
    constexpr int WC = R / 8, AC = AR / 4;
    constexpr int C = (WC + AC) / NWV;
    static_assert(WC % NWV == 0 && AC % NWV == 0 && S >= 2 && (S - 2) * C < 64, "as skinny_wide");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * SLOT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t n0 = blockIdx.x * R;
    const uint32_t chunks = K / CHUNK;
    const uint32_t kc0 = blockIdx.y * cps, kc1 = kc0 + cps < chunks ? kc0 + cps : chunks;
    const uint32_t nst = kc1 - kc0;
    const uint8_t *src[C];
    uint32_t dst[C], unit[C];
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const int q = wave + NWV * c;
        if (q < WC) {
            const uint32_t rr = q * 8 + lane / 8, p = (lane % 8) ^ swz8(rr);
            uint32_t n = n0 + rr;
            n = n < N ? n : N - 1;
            src[c] = codes + (size_t)n * K + (size_t)kc0 * CHUNK + p * 16;
            dst[c] = q * 1024;
            unit[c] = 1;
        } else {
            const int qa = q - WC;
            const uint32_t row = qa * 4 + lane / 16, p = (lane % 16) ^ (row & 15);
            const uint32_t m = row < M ? row : M - 1;
            src[c] = reinterpret_cast<const uint8_t *>(x + (size_t)m * K + (size_t)kc0 * CHUNK + p * 8);
            dst[c] = WB + qa * 1024;
            unit[c] = 2;
        }
    }
    auto copies = [&](uint32_t st) {
        uint8_t *slot = lds + (st % S) * SLOT;
#pragma unroll
        for (int c = 0; c < C; ++c) {
            if (unit[c] == 1) copy16_nt(src[c] + (size_t)st * BK, slot + dst[c]);
            else copy16(src[c] + (size_t)st * BK * 2, slot + dst[c]);
        }
    };
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if ((uint32_t)s < nst) copies(s);
    for (uint32_t st = 0; st < nst; ++st) {
        if (st + S - 2 < nst) wait_vmcnt<(S - 2) * C>();
        else wait_vmcnt<0>();
        wait_lgkm0();
        lds_barrier();
        if (st + S - 1 < nst) copies(st + S - 1);
    }
    wait_vmcnt<0>();
    lds_barrier();
    const uint32_t v = reinterpret_cast<const uint32_t *>(lds)[tid];
    if (v == 0x9e3779b9u) sink[0] = v;
}

// The XCD of each workgroup of a 1-D grid (hardware register XCC_ID).
__global__ __launch_bounds__(64) void xcc_probe(uint32_t *out) {
    if (threadIdx.x == 0) out[blockIdx.x] = __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xfu;
}

// The cache policy of the split merge: 0 (plain stores, sc0 loads) once the
// device has been seen to run workgroup b on the XCD of workgroup b % 8, as
// the XCD-major grid needs; 1 (agent-coherent sc1 stores and loads, right
// wherever blocks run) until then and if it was not. The check runs once per
// device, over 2048 workgroups, on the caller's stream when a call may
// allocate and the stream is not being captured. The policy changes where the
// partials travel, never the sums.
uint32_t split_coherence(hipStream_t st, bool may_check) {
    static std::mutex mu;
    static std::map<int, bool> periodic;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1u;
    std::lock_guard<std::mutex> lk(mu);
    const auto it = periodic.find(dev);
    if (it != periodic.end()) return it->second ? 0u : 1u;
    if (!may_check) return 1u;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return 1u;
    constexpr uint32_t G = 2048;
    uint32_t *d = nullptr;
    if (hipMalloc(&d, G * sizeof(uint32_t)) != hipSuccess) return 1u;
    std::vector<uint32_t> h(G, 0xffffffffu);
    (void)hipGetLastError();   // the launch check below sees this launch's error only
    hipLaunchKernelGGL(xcc_probe, dim3(G), dim3(64), 0, st, d);
    const bool ran = hipGetLastError() == hipSuccess &&
                     hipMemcpyAsync(h.data(), d, G * sizeof(uint32_t), hipMemcpyDeviceToHost, st) == hipSuccess &&
                     hipStreamSynchronize(st) == hipSuccess;
    (void)hipFree(d);
    if (!ran) return 1u;
    bool ok = true;
    for (uint32_t i = 0; i < G; ++i) ok = ok && h[i] < 16 && h[i] == h[i % 8];
    periodic[dev] = ok;
    return ok ? 0u : 1u;
}

// A launch of skinny_wide: R = 32 ntw rows per block, an s-slot ring, the
// product's row tiles and K splits (cps chunks each).
struct WidePlan {
    uint32_t ntw, s, nwv, tiles, splits, cps;
};

// Rows per block first: for 16 < M <= 64 (mt >= 2), 64 on small matrices (the
// partials of more splits cost more than the activation re-reads) or 32 where
// 64-row blocks split as far as they go would keep under half the CUs busy
// (Qwen2.5-7B kv [512, 3584] at M = 64: 8.84 -> 6.94 us), or exactly half
// with 32-row blocks split at most 8 ways (Llama-3.1-8B kv [1024, 4096] at
// M = 64 8.07 -> 7.42 us, M = 32 6.55 -> 6.23 us; [2048, 2048] 7.50 -> 7.11
// us; [512, 8192], 16 ways, stays at 64 rows: 9.10 against 9.37 us); on large ones 128
// (half the activation bytes per code). With an even number of activation
// tiles the 64- and 128-row blocks run 8 waves (two per SIMD, each issuing
// half the copies and computing half the tiles): the copy stream is what
// bounds these products, and 8 waves move it 5-10% faster than 4 (M = 64
// Qwen2.5-7B q/o 10.8 -> 10.0 us, down 25.3 -> 23.4 us; gate/up 23.3 us in
// 96-row 4-wave blocks -> 22.2 us in 128-row 8-wave ones, same-box replays). With 4 waves (mt = 3) 128-row blocks give way
// to 96-row ones where they leave over 30% of the CUs idle and 96-row ones
// cover more. For M <= 16 (mt = 1, one 16-row activation tile) 64, or 128 on
// large matrices, 4 waves. Ring depths from sweeps of 3-6 stages on MI355X.
// Then the splits: as many as keep each XCD's share of the grid (ceil(tiles /
// 8) row tiles times the splits) within its CUs, so the grid runs in one
// round, with at least 4 chunks (512 codes) per split.
WidePlan wide_plan(uint32_t mt, uint32_t N, uint32_t K) {
    const uint32_t cus = (uint32_t)device_props().cus, per_xcd = cus / 8 > 0 ? cus / 8 : 1;
    const uint32_t chunks = (K + CHUNK - 1) / CHUNK, max_splits = chunks / 4 > 1 ? chunks / 4 : 1;
    auto tiles_of = [&](uint32_t R) { return (N + R - 1) / R; };
    auto splits_of = [&](uint32_t R) {
        const uint32_t t = tiles_of(R);
        if (t >= cus) return 1u;
        const uint32_t sp = per_xcd / ((t + 7) / 8);
        return sp < 1 ? 1u : sp > max_splits ? max_splits : sp;
    };
    const bool small = (uint64_t)N * K <= (16ull << 20);
    WidePlan p{2, 4, 4, 0, 1, chunks};
    if (mt >= 2) {
        if (small) {
            const uint32_t half64 = 2 * tiles_of(64) * max_splits;
            if (half64 < cus || (half64 == cus && splits_of(32) <= 8)) p.ntw = 1;
        } else if (mt % 2 == 0) {
            p.ntw = 4;
        } else {
            const uint32_t b128 = tiles_of(128) * splits_of(128), b96 = tiles_of(96) * splits_of(96);
            if (10 * b128 < 7 * cus && b96 > b128) {
                p.ntw = 3;
            } else {
                p.ntw = 4;
                p.s = 3;
            }
        }
        if (mt % 2 == 0 && p.ntw % 2 == 0) p.nwv = 8;
    } else if (!small) {
        p.ntw = 4;
    }
    const uint32_t R = 32 * p.ntw;
    p.tiles = tiles_of(R);
    const uint32_t sp = splits_of(R);
    p.cps = (chunks + sp - 1) / sp;
    p.splits = (chunks + p.cps - 1) / p.cps;
    return p;
}

template <int F, int MT, int NTW, int S, int NWV>
int launch_wide_cfg(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                    uint32_t K, uint16_t *y, hipStream_t st, const SplitScratch *fixed, const WidePlan &p) {
    constexpr uint32_t WMC = MT >= 2 ? 2 : 1, TPW = 32 * NTW / (16 * (NWV / WMC)), MTW = (MT + WMC - 1) / WMC;
    float *part = nullptr;
    uint32_t *cnt = nullptr, coh = 0, grid = p.tiles;
    size_t bytes = 0;
    if (p.splits > 1) {
        bytes = (size_t)p.tiles * p.splits * NWV * TPW * MTW * 64 * 16;
        if (bytes > 0xf0000000ull) {
            set_error("skinny_wide: %zu bytes of split partials exceed the 32-bit offsets", bytes);
            return RENG_HIP_EINVAL;
        }
        int rc = RENG_HIP_OK;
        part = split_partials(bytes / sizeof(float), st, fixed, &rc);
        if (rc) return rc;
        if (fixed && p.tiles > STATIC_TILE_COUNTERS) {
            set_error("skinny_wide: %u row tiles exceed the %u static tile counters", p.tiles, STATIC_TILE_COUNTERS);
            return RENG_HIP_EINVAL;
        }
        cnt = fixed ? static_tile_counters(&rc) : tile_counters(p.tiles, st, &rc);
        if (rc) return rc;
        coh = split_coherence(st, fixed == nullptr);
        grid = 8 * ((p.tiles + 7) / 8) * p.splits;
    }
#define RENG_WIDE(C, RG)                                                                                        \
    hipLaunchKernelGGL((skinny_wide<F, MT, NTW, S, C, NWV, RG>), dim3(grid), dim3(64 * NWV), 0, st, x, codes, scales, \
                       M, N, K, p.tiles, p.splits, p.cps, y, part, (uint32_t)bytes, cnt)
    const bool rag = K % CHUNK != 0;
    if (coh) {
        if (rag) RENG_WIDE(1, true); else RENG_WIDE(1, false);
    } else {
        if (rag) RENG_WIDE(0, true); else RENG_WIDE(0, false);
    }
#undef RENG_WIDE
    return check_launch("skinny_wide");
}

template <int F, int MT>
int launch_wide_mt(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                   uint32_t K, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    const WidePlan p = wide_plan(MT, N, K);
    if constexpr (MT == 1) {
        if (p.ntw == 4) return launch_wide_cfg<F, 1, 4, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
        return launch_wide_cfg<F, 1, 2, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
    } else if constexpr (MT % 2 == 0) {
        switch (p.ntw) {
            case 1: return launch_wide_cfg<F, MT, 1, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
            case 4: return launch_wide_cfg<F, MT, 4, 4, 8>(x, codes, scales, M, N, K, y, st, fixed, p);
            default: return launch_wide_cfg<F, MT, 2, 4, 8>(x, codes, scales, M, N, K, y, st, fixed, p);
        }
    } else {
        switch (p.ntw) {
            case 1: return launch_wide_cfg<F, MT, 1, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
            case 3: return launch_wide_cfg<F, MT, 3, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
            case 4: return launch_wide_cfg<F, MT, 4, 3, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
            default: return launch_wide_cfg<F, MT, 2, 4, 4>(x, codes, scales, M, N, K, y, st, fixed, p);
        }
    }
}

// The stage-copy yardstick on the blocks skinny_wide would take for this
// product (its rows per block, ring and splits; a (tiles, splits) grid).
template <int MT, int NTW, int S, int NWV>
int launch_stage_copy_cfg(const uint16_t *x, const uint8_t *codes, uint32_t M, uint32_t N, uint32_t K,
                          uint32_t *sink, hipStream_t st, const WidePlan &p) {
    hipLaunchKernelGGL((stage_copy_kernel<MT, NTW, S, NWV>), dim3(p.tiles, p.splits), dim3(64 * NWV), 0, st, x, codes,
                       M, N, K, p.cps, sink);
    return check_launch("stage_copy");
}

template <int MT>
int launch_stage_copy_mt(const uint16_t *x, const uint8_t *codes, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t *sink, hipStream_t st) {
    const WidePlan p = wide_plan(MT, N, K);
    if constexpr (MT % 2 == 0) {
        switch (p.ntw) {
            case 1: return launch_stage_copy_cfg<MT, 1, 4, 4>(x, codes, M, N, K, sink, st, p);
            case 4: return launch_stage_copy_cfg<MT, 4, 4, 8>(x, codes, M, N, K, sink, st, p);
            default: return launch_stage_copy_cfg<MT, 2, 4, 8>(x, codes, M, N, K, sink, st, p);
        }
    } else {
        switch (p.ntw) {
            case 1: return launch_stage_copy_cfg<MT, 1, 4, 4>(x, codes, M, N, K, sink, st, p);
            case 3: return launch_stage_copy_cfg<MT, 3, 4, 4>(x, codes, M, N, K, sink, st, p);
            case 4: return launch_stage_copy_cfg<MT, 4, 3, 4>(x, codes, M, N, K, sink, st, p);
            default: return launch_stage_copy_cfg<MT, 2, 4, 4>(x, codes, M, N, K, sink, st, p);
        }
    }
}

template <int F>
int launch_wide_f(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                  uint32_t K, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    switch ((M + 15) / 16) {
        case 1: return launch_wide_mt<F, 1>(x, codes, scales, M, N, K, y, st, fixed);
        case 2: return launch_wide_mt<F, 2>(x, codes, scales, M, N, K, y, st, fixed);
        case 3: return launch_wide_mt<F, 3>(x, codes, scales, M, N, K, y, st, fixed);
        default: return launch_wide_mt<F, 4>(x, codes, scales, M, N, K, y, st, fixed);
    }
}

}  // namespace skinny

// 16 < M <= 64, K % 128 == 0: skinny_wide's copy stream alone (a yardstick).
int launch_stage_copy(const uint16_t *x, const uint8_t *codes, uint32_t M, uint32_t N, uint32_t K, uint32_t *sink,
                      hipStream_t st) {
    using namespace skinny;
    switch ((M + 15) / 16) {
        case 2: return launch_stage_copy_mt<2>(x, codes, M, N, K, sink, st);
        case 3: return launch_stage_copy_mt<3>(x, codes, M, N, K, sink, st);
        default: return launch_stage_copy_mt<4>(x, codes, M, N, K, sink, st);
    }
}

// 2 <= M <= 16, K % 128 == 0 (rows past M repeat row M - 1 and are not stored).
// skinny_rows runs a product in one round of whole-K blocks; skinny_wide's
// one-activation-tile form splits K over blocks and merges the splits in the
// launch. The split form takes long rows (K >= 8192: Qwen2.5-7B down
// [3584, 18944] at M = 8 17.9 -> 15.0 us, M = 16 22.3 -> 15.0 us; at M <= 8
// not where 16-row tiles fill the CUs, below), and for
// 8 < M <= 16 every product but those whose 16-row tiles fill between half
// and all of the CUs ([3584, 3584]: 6.5 against 6.9 us; kv [512, 3584]
// 5.6 -> 5.1 us, gate/up [18944, 3584] 21.5 -> 17.5 us).
int launch_skinny_mfma(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    using namespace skinny;
    const uint32_t cus = (uint32_t)device_props().cus, t16 = (N + 15) / 16;
    // Long rows stay whole-K at M <= 8 where skinny_rows' one 16-row tile per
    // workgroup keeps (nearly) every CU busy: Llama-3.1-8B down [4096, 14336]
    // M = 8 13.8 -> 13.0 us, M = 4 13.9 -> 11.9 us, [4096, 8192] M = 8 10.8 ->
    // 8.7 us; not with CUs idle (Qwen2.5-7B down, 224 tiles: 16.0 against 14.9
    // us) nor at M = 16 (15.9 against 13.8 us).
    const bool full16 = M <= 8 && t16 <= cus && 16 * t16 >= 15 * cus;
    const bool split = (K >= 8192 && !full16) || (M > 8 && !(t16 <= cus && 2 * t16 > cus));
    if (split) {
        if (format == RENG_HIP_E4M3) return launch_wide_mt<RENG_HIP_E4M3, 1>(x, codes, scales, M, N, K, y, st, fixed);
        return launch_wide_mt<RENG_HIP_E5M2, 1>(x, codes, scales, M, N, K, y, st, fixed);
    }
    if (M <= 8) {
        if (format == RENG_HIP_E4M3) return launch_ma<RENG_HIP_E4M3, 8>(x, codes, scales, M, N, K, y, st);
        return launch_ma<RENG_HIP_E5M2, 8>(x, codes, scales, M, N, K, y, st);
    }
    if (format == RENG_HIP_E4M3) return launch_ma<RENG_HIP_E4M3, 16>(x, codes, scales, M, N, K, y, st);
    return launch_ma<RENG_HIP_E5M2, 16>(x, codes, scales, M, N, K, y, st);
}

// 1 <= M <= 64 on skinny_wide (16 < M, or any M whose K is not a multiple of
// 128: its last chunk is short), K % 16 == 0.
int launch_skinny_wide(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    using namespace skinny;
    if (format == RENG_HIP_E4M3) return launch_wide_f<RENG_HIP_E4M3>(x, codes, scales, M, N, K, y, st, fixed);
    return launch_wide_f<RENG_HIP_E5M2>(x, codes, scales, M, N, K, y, st, fixed);
}

}  // namespace reng
