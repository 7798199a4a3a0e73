// gemm_fp8.hip - fp8 x fp8 GEMM on CDNA4 MFMA (gfx950):
//   out[m, n] = bf16(sum_k dec(a[m, k]) * dec(b[n, k]) * sa[m] * sb[n])
// with a [M, K] and b [N, K] both K-contiguous (the [K, m] / [K, N] device
// sizes of gemm_fp8_scaled with transpose_b, crates/reng-synapse/src/fp8.rs:295-331).
//
// v_mfma_f32_32x32x64_f8f6f4 on the OCP fp8 formats, whose finite codes
// 0x00-0x77 (e4m3) / 0x00-0x7b (e5m2) mean exactly what reng-fp8's codes mean.
//
// Two kernels: gemm_fp8_wide (further down) for shapes of whole 256 x 256 /
// 256 x 128 tiles, and gemm_fp8_mfma for everything else. gemm_fp8_mfma:
// block = 2 x 2 waves; a wave owns WM x WN tiles of 32 x 32, so the block tile
// is BM = 64 WM by BN = 64 WN. A pipeline stage covers BK = 64 KS codes of k.
// Each stage's operand rows are copied global -> LDS by the waves'
// global_load_lds_dwordx4 (1 KB per instruction, no VGPR staging) into an
// S-slot ring; a row's 16-byte chunks are stored XOR-swizzled (swz) so that
// the 32-byte fragment reads (two ds_read_b128 per operand tile) are free of
// bank conflicts. One barrier per stage: before it a wave waits only for its
// own copies of the next stage (s_waitcnt vmcnt with the later stages still in
// flight); after it the wave issues the copy of stage t + S into the slot
// stage t used and reads the next stage's first fragments, interleaved with
// the second half of the current stage's MFMAs.
//
// Tiles are spread over the 8 XCDs so that the blocks resident on one XCD at a
// time hold consecutive tiles, m fastest: they share the weight rows
// b[n0:n0+BN] through that XCD's L2. The output goes out as 8-byte stores of
// four consecutive n (the MFMA computes D = B A^T, so a lane holds four
// consecutive output columns of one row).
#include <type_traits>

#include "common.h"
#include "gemm.h"
#include "mfma_pipe.h"
#include "tile_order.h"

namespace reng {

namespace fp8gemm {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

using namespace pipe;

constexpr int FK = 64;     // codes of k per MFMA k-step

// Block tile BM x BN (2 x 2 waves of WM x WN MFMA tiles), KS k-steps (64 codes
// each) per pipeline stage.
template <int WM, int WN, int KS>
struct Fp8Tile {
    static constexpr int BM = 64 * WM, BN = 64 * WN, BK = FK * KS;
    static constexpr int CH = BK / 16;                 // 16-byte chunks per LDS row
    static constexpr int ROWS = 1024 / BK;             // rows per 1 KB copy
    static constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK, STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = BM / 4 / ROWS, LB = BN / 4 / ROWS;   // copies per wave per stage
    static constexpr int LOADS = LA + LB;
};

template <int FA, int FB, int WM, int WN, int KS, int S>
__global__ __launch_bounds__(256) void gemm_fp8_mfma(const uint8_t *__restrict__ a,
                                                     const float *__restrict__ sa, uint32_t nsa,
                                                     const uint8_t *__restrict__ b,
                                                     const float *__restrict__ sb, uint32_t nsb,
                                                     uint32_t M, uint32_t N, uint32_t K, uint32_t tiles_m,
                                                     uint32_t tiles, uint16_t *__restrict__ out, uint32_t vec_out) {
    using T = Fp8Tile<WM, WN, KS>;
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, CH = T::CH;
    static_assert(S >= 2, "at least double-buffered");
    static_assert((S - 1) * T::LOADS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * T::STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: keeps LDS bases scalar
    const int wm = wave >> 1, wn = wave & 1;

    // Tile of this block: the XCD (blockIdx % 8) takes a contiguous run.
    const uint32_t x = blockIdx.x % XCDS, l = blockIdx.x / XCDS;
    const uint32_t per = tiles / XCDS, rem = tiles % XCDS;
    const uint32_t tile = x * per + (x < rem ? x : rem) + l;
    const uint32_t m0 = (tile % tiles_m) * BM, n0 = (tile / tiles_m) * BN;
    const uint32_t n = K / BK;   // stages

    // Copy sources: lane l of a copy brings tile row r = base + l / CH and the
    // chunk that lands in slot l % CH of that row, i.e. chunk
    // (l % CH) ^ swz(r). Rows past M / N are clamped (never stored).
    const uint8_t *ga[T::LA];
    const uint8_t *gb[T::LB];
#pragma unroll
    for (int q = 0; q < T::LA; ++q) {
        const uint32_t tr = wave * (BM / 4) + q * T::ROWS + lane / CH;
        uint32_t r = m0 + tr;
        r = r < M ? r : M - 1;
        ga[q] = a + (size_t)r * K + (((lane % CH) ^ swz<CH>(tr)) * 16);
    }
#pragma unroll
    for (int q = 0; q < T::LB; ++q) {
        const uint32_t tr = wave * (BN / 4) + q * T::ROWS + lane / CH;
        uint32_t r = n0 + tr;
        r = r < N ? r : N - 1;
        gb[q] = b + (size_t)r * K + (((lane % CH) ^ swz<CH>(tr)) * 16);
    }
    auto issue = [&](uint32_t step, int slot) {
        uint8_t *base = lds + slot * T::STAGE;
        const size_t ko = (size_t)step * BK;
#pragma unroll
        for (int q = 0; q < T::LA; ++q) copy16_to_lds(ga[q] + ko, base + (wave * (BM / 4) + q * T::ROWS) * BK);
#pragma unroll
        for (int q = 0; q < T::LB; ++q)
            copy16_to_lds(gb[q] + ko, base + T::A_BYTES + (wave * (BN / 4) + q * T::ROWS) * BK);
    };
    auto clampi = [&](uint32_t i) { return i < n ? i : n - 1; };

    // Fragment of a 32-row tile at k-step ks: lane l holds row l % 32 and the
    // 32 codes of k half l / 32, chunks 4 ks + 2h and 4 ks + 2h + 1 of the row.
    const uint32_t rl = lane & 31, h = lane >> 5, sw = swz<CH>(rl);
    auto read_frags = [&](int slot, int ks, i32x8 (&fa)[WM], i32x8 (&fb)[WN]) {
        const uint8_t *base = lds + slot * T::STAGE;
        const uint32_t o0 = ((4 * ks + 2 * h) ^ sw) * 16, o1 = ((4 * ks + 2 * h + 1) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const uint8_t *p = base + (wm * (BM / 2) + i * 32 + rl) * BK;
            const u32x4 x0 = *reinterpret_cast<const u32x4 *>(p + o0);
            const u32x4 x1 = *reinterpret_cast<const u32x4 *>(p + o1);
            fa[i] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const uint8_t *p = base + T::A_BYTES + (wn * (BN / 2) + j * 32 + rl) * BK;
            const u32x4 x0 = *reinterpret_cast<const u32x4 *>(p + o0);
            const u32x4 x1 = *reinterpret_cast<const u32x4 *>(p + o1);
            fb[j] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    auto mfma_rows = [&](int i0, int i1, const i32x8 (&fa)[WM], const i32x8 (&fb)[WN]) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], acc[i][j], FB, FA, 0, 0,
                                                                            0, 0);
    };

    // Prologue: stages 0 .. S-1 in flight (indices clamped to the last step, so
    // every wave issues the same number of copies), then the first fragments.
#pragma unroll
    for (int s = 0; s < S; ++s) issue(clampi(s), s);
    wait_vmcnt<(S - 1) * T::LOADS>();
    lds_barrier();
    i32x8 fa[2][WM], fb[2][WN];
    read_frags(0, 0, fa[0], fb[0]);

    // One k-step on the fragment set CUR while the next k-step's fragments go
    // into the other set; the last k-step of a stage starts with the barrier
    // that publishes stage t + 1 and frees stage t's slot.
    auto kstep = [&](auto cur_c, auto ks_c, uint32_t t) {
        constexpr int CUR = decltype(cur_c)::value, NXT = CUR ^ 1, KSI = decltype(ks_c)::value;
        if constexpr (KSI + 1 < KS) {
            read_frags((int)(t % S), KSI + 1, fa[NXT], fb[NXT]);
            mfma_rows(0, WM, fa[CUR], fb[CUR]);
            interleave<WM * WN, 2 * (WM + WN), 0>();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            // This k-step's fragments (the stage's last) are in registers once
            // the wave's LDS reads are done; after the barrier no wave reads
            // stage t's slot again, so the copy of stage t + S goes there, and
            // stage t + 1 (landed: the vmcnt wait) is read during all of this
            // k-step's MFMAs. The copies go out first, back to back: the
            // compiler keeps LDS reads behind LDS-bound copies issued before
            // them, and reads placed ahead of the copies in program order get
            // a vmcnt wait on those copies.
            wait_lgkm0();
            wait_vmcnt<(S - 2) * T::LOADS>();
            lds_barrier();
            issue(clampi(t + S), (int)(t % S));
            read_frags((int)((t + 1) % S), 0, fa[NXT], fb[NXT]);
            mfma_rows(0, WM, fa[CUR], fb[CUR]);
            __builtin_amdgcn_sched_group_barrier(0x060, T::LOADS, 0);
            interleave<WM * WN, 2 * (WM + WN), 0>();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Stage t's k-steps use fragment sets (t * KS + ks) & 1.
    auto stage = [&](auto par_c, uint32_t t) {
        constexpr int P = decltype(par_c)::value;
        kstep(std::integral_constant<int, (P * KS) & 1>{}, std::integral_constant<int, 0>{}, t);
        if constexpr (KS > 1)
            kstep(std::integral_constant<int, (P * KS + 1) & 1>{}, std::integral_constant<int, 1>{}, t);
    };
    static_assert(KS == 1 || KS == 2, "one or two k-steps per stage");
    uint32_t t = 0;
    for (; t + 1 < n; t += 2) {
        stage(std::integral_constant<int, 0>{}, t);
        stage(std::integral_constant<int, 1>{}, t + 1);
    }
    if (t < n) stage(std::integral_constant<int, 0>{}, t);
    wait_vmcnt<0>();   // the clamped surplus copies land before LDS is released
    (void)BK;

    // acc[i][j] is D = B A^T of a 32 x 32 tile: lane l holds column
    // m = l % 32 (activation row) and rows n = 8 (e / 4) + 4 (l / 32) + e % 4,
    // so each group of four e is four consecutive outputs of row m: one 8-byte
    // store.
    // Scales as (pointer, stride), as in gemm_fp8_wide: no branches on the scale form.
    const float *sap = nsa == 0 ? &one_f32 : sa, *sbp = nsb == 0 ? &one_f32 : sb;
    const uint32_t sas = nsa > 1, sbs = nsb > 1;
    auto store = [&](const f32x16 (&v)[WM][WN]) {
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const uint32_t m = m0 + wm * (BM / 2) + i * 32 + rl;
            if (m >= M) continue;
            const float sam = sap[m * sas];
            uint16_t *orow = out + (size_t)m * N;
#pragma unroll
            for (int j = 0; j < WN; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const uint32_t nb = n0 + wn * (BN / 2) + j * 32 + 8 * g + 4 * h;
                    float o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t nn = nb + e < N ? nb + e : N - 1;
                        o[e] = v[i][j][4 * g + e] * sam * sbp[nn * sbs];
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
    store(acc);
}

struct Fp8Args {
    const uint8_t *a;
    int fa;
    const float *sa;
    uint32_t nsa;
    const uint8_t *b;
    int fb;
    const float *sb;
    uint32_t nsb;
    uint32_t M, N, K;
    uint16_t *out;
};

// One launch of the (WM, WN, KS, S) kernel.
template <int WM, int WN, int KS, int S>
int launch_fp8_cfg(const Fp8Args &g, hipStream_t st) {
    using T = Fp8Tile<WM, WN, KS>;
    const uint32_t tiles_m = (g.M + T::BM - 1) / T::BM, tiles_n = (g.N + T::BN - 1) / T::BN;
    const uint32_t tiles = tiles_m * tiles_n;
    // 8-byte output stores need every row start 8-byte aligned.
    const uint32_t vec_out = g.N % 4 == 0 && reinterpret_cast<uintptr_t>(g.out) % 8 == 0;
#define RENG_FP8_LAUNCH(A, B)                                                                                \
    hipLaunchKernelGGL((gemm_fp8_mfma<A, B, WM, WN, KS, S>), dim3(tiles), dim3(256), 0, st, g.a, g.sa, g.nsa, \
                       g.b, g.sb, g.nsb, g.M, g.N, g.K, tiles_m, tiles, g.out, vec_out)
    if (g.fa == RENG_HIP_E4M3 && g.fb == RENG_HIP_E4M3) RENG_FP8_LAUNCH(0, 0);
    else if (g.fa == RENG_HIP_E4M3) RENG_FP8_LAUNCH(0, 1);
    else if (g.fb == RENG_HIP_E4M3) RENG_FP8_LAUNCH(1, 0);
    else RENG_FP8_LAUNCH(1, 1);
#undef RENG_FP8_LAUNCH
    return check_launch("gemm_fp8_mfma");
}

// ------------------------------------------------------------ wide tiles
//
// The large-output form: 8 waves (2 x 4, two per SIMD) over a BM x BN tile of
// 256 x 256 or 256 x 128, K in 128-code stages. A wave owns WM x WN MFMA
// tiles (4 x 2: 128 x 64 outputs, or 4 x 1). The operand copies are
// buffer_load_dwordx4 ... lds through a buffer resource: the per-lane part of
// the address (row within the copy, swizzled chunk) is one VGPR for every
// copy of the wave, and the copy's row base and k offset ride in the scalar
// soffset, so the copy addresses cost no registers. Only shapes that divide
// into whole tiles take this form (every row read exists; no clamping).
// Two waves per SIMD let one wave's MFMAs run while the other waits on its
// fragment reads or the stage barrier; the 256 x 256 tile halves the operand
// bytes each output needs against 128 x 128.

__device__ __forceinline__ void copy16_buf(__amdgpu_buffer_rsrc_t r, uint8_t *l, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)l, 16, voff, soff, 0, 0);
}

// WGM x WGN waves (default 2 x 4), each owning WM x WN MFMA tiles of 32 x 32.
template <int WM, int WN, int BK_ = 128, int WGM_ = 2, int WGN_ = 4>
struct WideTile {
    static constexpr int WGM = WGM_, WGN = WGN_, NW = WGM * WGN;   // wave grid, waves
    static constexpr int BM = 32 * WM * WGM, BN = 32 * WN * WGN, BK = BK_;
    static_assert(BK == 64 || BK == 128, "one or two k-steps per stage");
    static constexpr int CH = BK / 16, ROWS = 1024 / BK;   // chunks per LDS row, rows per 1 KB copy
    static constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK, STAGE = A_BYTES + B_BYTES;
    static constexpr int LA = BM / ROWS / NW, LB = BN / ROWS / NW;   // copies per wave per stage
    static constexpr int LOADS = LA + LB;
    static_assert(LA * ROWS * NW == BM && LB * ROWS * NW == BN, "copies split evenly");
};

template <int FA, int FB, int WM, int WN, int BKW, int S, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_fp8_wide(const uint8_t *__restrict__ a,
                                                                const float *__restrict__ sa, uint32_t nsa,
                                                                const uint8_t *__restrict__ b,
                                                                const float *__restrict__ sb, uint32_t nsb, uint32_t M,
                                                                uint32_t N, uint32_t K, uint32_t tiles_m,
                                                                uint32_t tiles, uint16_t *__restrict__ out,
                                                                uint32_t ldo, uint32_t mapm) {
    using T = WideTile<WM, WN, BKW, WGM, WGN>;
    constexpr int BM = T::BM, BN = T::BN, BK = T::BK, CH = T::CH, ROWS = T::ROWS, KS = BK / FK, NT = 64 * T::NW;
    static_assert(S >= 2, "at least double-buffered");
    static_assert((S - 1) * T::LOADS < 64, "vmcnt range");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * T::STAGE];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / T::WGN, wn = wave % T::WGN;

    // XCD-major tile order (wide_tile_of, tile_order.h): XCD x takes a
    // contiguous run of tiles, m fastest (as gemm_fp8_mfma), or a block of mapm
    // m-tiles by per / mapm n-tiles where the launcher found that to read fewer
    // operand rows per XCD.
    uint32_t mt, nt;
    wide_tile_of(blockIdx.x, tiles_m, tiles, mapm, mt, nt);
    const uint32_t m0 = mt * BM, n0 = nt * BN;
    const uint32_t n = K / BK;

    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)a, 0, M * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *)b, 0, N * K, 0x00020000);
    // Lane part of a copy: tile row (copy base) + lane / CH, the chunk that
    // lands in slot lane % CH. The swizzle reads the row's low five bits and a
    // copy's base is a multiple of ROWS, so there are 32 / ROWS lane parts.
    constexpr int VAR = 32 / ROWS;
    uint32_t voff[VAR];
#pragma unroll
    for (int v = 0; v < VAR; ++v)
        voff[v] = (uint32_t)(lane / CH) * K + (((lane % CH) ^ swz<CH>(v * ROWS + lane / CH)) * 16);
    auto issue = [&](uint32_t step, int slot) {
        uint8_t *base = lds + slot * T::STAGE;
        const uint32_t ko = step * BK;
#pragma unroll
        for (int q = 0; q < T::LA; ++q) {
            const uint32_t c = wave * T::LA + q, tr0 = c * ROWS;
            copy16_buf(ra, base + tr0 * BK, voff[c % VAR], (m0 + tr0) * K + ko);
        }
#pragma unroll
        for (int q = 0; q < T::LB; ++q) {
            const uint32_t c = wave * T::LB + q, tr0 = c * ROWS;
            copy16_buf(rb, base + T::A_BYTES + tr0 * BK, voff[c % VAR], (n0 + tr0) * K + ko);
        }
    };
    auto clampi = [&](uint32_t i) { return i < n ? i : n - 1; };

    const uint32_t rl = lane & 31, h = lane >> 5, sw = swz<CH>(rl);
    auto read_frags = [&](int slot, int ks, i32x8 (&fa)[WM], i32x8 (&fb)[WN]) {
        const uint8_t *base = lds + slot * T::STAGE;
        const uint32_t o0 = ((4 * ks + 2 * h) ^ sw) * 16, o1 = ((4 * ks + 2 * h + 1) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const uint8_t *p = base + (wm * (32 * WM) + i * 32 + rl) * BK;
            const u32x4 x0 = *reinterpret_cast<const u32x4 *>(p + o0);
            const u32x4 x1 = *reinterpret_cast<const u32x4 *>(p + o1);
            fa[i] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const uint8_t *p = base + T::A_BYTES + (wn * (32 * WN) + j * 32 + rl) * BK;
            const u32x4 x0 = *reinterpret_cast<const u32x4 *>(p + o0);
            const u32x4 x1 = *reinterpret_cast<const u32x4 *>(p + o1);
            fb[j] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
        }
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
    auto mfma_rows = [&](int i0, int i1, const i32x8 (&fa)[WM], const i32x8 (&fb)[WN]) {
#pragma unroll
        for (int i = i0; i < i1; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fb[j], fa[i], acc[i][j], FB, FA, 0, 0,
                                                                            0, 0);
    };

    // The pipeline of gemm_fp8_mfma: S stages in flight from the prologue;
    // per stage one barrier after each wave's own copies of the next stage
    // have landed, then the copy of stage t + S into the slot stage t used.
#pragma unroll
    for (int s = 0; s < S; ++s) issue(clampi(s), s);
    wait_vmcnt<(S - 1) * T::LOADS>();
    lds_barrier();
    i32x8 fa[2][WM], fb[2][WN];
    read_frags(0, 0, fa[0], fb[0]);
    auto kstep = [&](auto cur_c, auto ks_c, uint32_t t) {
        constexpr int CUR = decltype(cur_c)::value, NXT = CUR ^ 1, KSI = decltype(ks_c)::value;
        if constexpr (KSI + 1 < KS) {
            read_frags((int)(t % S), KSI + 1, fa[NXT], fb[NXT]);
            mfma_rows(0, WM, fa[CUR], fb[CUR]);
            interleave<WM * WN, 2 * (WM + WN), 0>();
            __builtin_amdgcn_sched_barrier(0);
        } else {
            // This k-step's fragments (the stage's last) are in registers once
            // the wave's LDS reads are done; after the barrier no wave reads
            // stage t's slot again, so the copy of stage t + S goes there, and
            // stage t + 1 (landed: the vmcnt wait) is read during all of this
            // k-step's MFMAs. The copies go out first, back to back: the
            // compiler keeps LDS reads behind LDS-bound copies issued before
            // them, and reads placed ahead of the copies in program order get
            // a vmcnt wait on those copies.
            wait_lgkm0();
            wait_vmcnt<(S - 2) * T::LOADS>();
            lds_barrier();
            issue(clampi(t + S), (int)(t % S));
            read_frags((int)((t + 1) % S), 0, fa[NXT], fb[NXT]);
            mfma_rows(0, WM, fa[CUR], fb[CUR]);
            __builtin_amdgcn_sched_group_barrier(0x060, T::LOADS, 0);
            interleave<WM * WN, 2 * (WM + WN), 0>();
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    uint32_t t = 0;
    if constexpr (KS == 2) {
        for (; t + 1 < n; t += 2) {
            kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t);
            kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, t);
            kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t + 1);
            kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, t + 1);
        }
        if (t < n) {
            kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t);
            kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, t);
        }
    } else {
        for (; t + 1 < n; t += 2) {
            kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t);
            kstep(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{}, t + 1);
        }
        if (t < n) kstep(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, t);
    }
    wait_vmcnt<0>();   // the clamped surplus copies land before LDS is released

    // Epilogue through LDS (the operand ring is free once every wave is past
    // the barrier): lane l holds output row l % 32 of each 32-row tile and,
    // per group g of four accumulators, four consecutive columns; the scaled
    // bf16 values go to a row-major BM x BN tile whose 16-byte chunks are
    // rotated by row (chunk c of row r in slot slot(r, c): c ^ (r % CC) for a
    // power-of-two CC, else (c + r) % CC), then the block stores whole tile
    // rows with 16-byte stores, so every store instruction writes contiguous
    // row segments rather than 16 bytes of each of 32 rows. The stores are
    // non-temporal: the output (a third of the launch's HBM traffic on
    // [1024, 14336, 4096]) goes out in one burst at every tile's end and is not
    // read again here (M = 1024 [14336, 4096] 59.9 -> 57.3 us, [2048, 4096,
    // 4096] 36.7 -> 35.1 us; the Qwen2.5-32B shapes equal or 1-3% faster).
    constexpr int CC = BN / 8, RB = BN * 2;   // 16-byte chunks / bytes of a bf16 tile row
    auto slot = [](uint32_t r, uint32_t c) -> uint32_t {
        if constexpr ((CC & (CC - 1)) == 0) return c ^ (r % CC);
        else return (c + r) % CC;
    };
    static_assert(S * T::STAGE >= BM * RB, "the output tile fits the operand ring");
    // Scales as (pointer, stride): no scale reads 1.0 from one_f32, a single
    // scale has stride 0, so the loads below take no branches.
    const float *sap = nsa == 0 ? &one_f32 : sa, *sbp = nsb == 0 ? &one_f32 : sb;
    const uint32_t sas = nsa > 1, sbs = nsb > 1;
    // The lane index through an empty asm: the epilogue's addresses and scale
    // loads are computed here rather than hoisted before the main loop.
    uint32_t te = tid;
    asm volatile("" : "+v"(te));
    const uint32_t rle = te & 31, he = (te >> 5) & 1;
    float sbv[WN][4][4];
#pragma unroll
    for (int j = 0; j < WN; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                sbv[j][g][e] = sbp[(n0 + wn * (32 * WN) + j * 32 + 8 * g + 4 * he + e) * sbs];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const uint32_t r = wm * (32 * WM) + i * 32 + rle;
        const float sam = sap[(m0 + r) * sas];
        uint8_t *lrow = lds + r * RB;
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t c = wn * (4 * WN) + 4 * j + g;   // columns 8 c .. 8 c + 7 of the tile
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = acc[i][j][4 * g + e] * sam * sbv[j][g][e];
                const uint32_t lo = f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16);
                const uint32_t hi = f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16);
                *reinterpret_cast<u32x2 *>(lrow + slot(r, c) * 16 + 8 * he) = u32x2{lo, hi};
            }
    }
    __syncthreads();
    static_assert((BM * CC) % NT == 0, "whole passes");
#pragma unroll
    for (int p = 0; p < BM * CC / NT; ++p) {
        const uint32_t i = p * NT + te, r = i / CC, c = i % CC;
        const u32x4 v = *reinterpret_cast<const u32x4 *>(lds + r * RB + slot(r, c) * 16);
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4 *>(out + (size_t)(m0 + r) * ldo + n0 + 8 * c));
    }
}

// Whether the wide (WM, WN) form takes this product: whole tiles, K in whole
// stages, byte offsets in 31 bits, 16-byte aligned output rows.
template <int WM, int WN, int BK = 128, int WGM = 2, int WGN = 4>
bool wide_fits(const Fp8Args &g) {
    using T = WideTile<WM, WN, BK, WGM, WGN>;
    return g.M % T::BM == 0 && g.N % T::BN == 0 && g.K % T::BK == 0 && (uint64_t)g.M * g.K < (1ull << 31) &&
           (uint64_t)g.N * g.K < (1ull << 31) && reinterpret_cast<uintptr_t>(g.out) % 16 == 0;
}

// A wide form as a dispatch candidate: whether it takes the product, its
// tile, and its fitted time model (c0, c1).
struct WideCand {
    bool fits;
    uint32_t bm, bn;
    float c0, c1;
};

template <int WM, int WN, int WGM, int WGN>
WideCand wide_cand(const Fp8Args &g, float c0, float c1) {
    using T = WideTile<WM, WN, 128, WGM, WGN>;
    return WideCand{wide_fits<WM, WN, 128, WGM, WGN>(g), (uint32_t)T::BM, (uint32_t)T::BN, c0, c1};
}

// 2-D XCD blocks of tiles (wide_mapm, tile_order.h): on the kv projection
// [1024, 1024, 5120] (64 x 64 tiles: 16 m-tiles of which an XCD's run of 32
// covers all, plus 2 n-tiles) blocks of 4 x 8 read 768 operand rows per XCD
// instead of 1152: 15.0 -> 14.3-14.5 us. On the larger Qwen2.5-32B shapes the
// m-fastest runs already read the fewest rows.
//
// ldo is the output's row stride in elements (0: N); a launch over a column
// range of a wider output passes the whole output's N.
template <int WM, int WN, int BK, int S, int WGM = 2, int WGN = 4>
int launch_fp8_wide(const Fp8Args &g, hipStream_t st, uint32_t ldo = 0) {
    using T = WideTile<WM, WN, BK, WGM, WGN>;
    const uint32_t tiles_m = g.M / T::BM, tiles = tiles_m * (g.N / T::BN);
    const uint32_t mapm = wide_mapm(tiles_m, g.N / T::BN, T::BM, T::BN);
    const uint32_t ld = ldo ? ldo : g.N;
#define RENG_FP8_WIDE(A, B)                                                                                      \
    hipLaunchKernelGGL((gemm_fp8_wide<A, B, WM, WN, BK, S, WGM, WGN>), dim3(tiles), dim3(64 * T::NW), 0, st, g.a, g.sa, \
                       g.nsa, g.b, g.sb, g.nsb, g.M, g.N, g.K, tiles_m, tiles, g.out, ld, mapm)
    if (g.fa == RENG_HIP_E4M3 && g.fb == RENG_HIP_E4M3) RENG_FP8_WIDE(0, 0);
    else if (g.fa == RENG_HIP_E4M3) RENG_FP8_WIDE(0, 1);
    else if (g.fb == RENG_HIP_E4M3) RENG_FP8_WIDE(1, 0);
    else RENG_FP8_WIDE(1, 1);
#undef RENG_FP8_WIDE
    return check_launch("gemm_fp8_wide");
}

// The columns [n0, n0 + n) of a product as a product of its own: the codes and
// per-channel scales of those weight rows, the output's columns from n0 (the
// launch writes them with the whole output's row stride).
inline Fp8Args column_range(const Fp8Args &g, uint32_t n0, uint32_t n) {
    Fp8Args r = g;
    r.b = g.b + (size_t)n0 * g.K;
    if (g.nsb > 1) {   // one scale per weight row: those of the range
        r.sb = g.sb + n0;
        r.nsb = n;
    }
    r.N = n;
    r.out = g.out + n0;
    return r;
}

// A grid of 256 x 256 tiles that is not a whole number of rounds pays for its
// last, partial round in full. The mixed plan runs whole rounds of 256 x 256
// tiles over the leading n1 columns, then one round of 256 x 192 tiles over
// the rest (a second launch): on [1024, 27648, 5120] 252 + 240 tiles instead of
// 432 in two rounds. The narrower tile reads 0.875x the operand rows per output
// and its round measured 0.82-0.85x as long, so the plan gains 2-3% there
// (141-146 -> 138-141 us; K = 10240: 260-263 -> 253-254 us), not the 16% of a
// tile-count model: these tiles' rounds take time in proportion to the operand
// bytes they copy. (One launch holding both forms, the second's workgroups
// dispatched as the first's finish, measured the same as two launches.)
// n1 = 0: no plan. est uses the 256 x 192 form's (c0, c1) fitted to its
// timings at K = 2560, 5120 and 10240.
struct MixedPlan {
    uint32_t n1;
    float est;
};

inline MixedPlan mixed_plan(const Fp8Args &g, uint64_t cus, float c0a, float c1a, float c0b, float c1b) {
    using TA = WideTile<4, 2, 128, 2, 4>;
    using TB = WideTile<2, 3, 128, 4, 2>;
    MixedPlan best{0, 0.0f};
    if (g.M % TA::BM != 0 || g.N % 64 != 0 || g.K % TA::BK != 0) return best;
    const uint64_t tiles_m = g.M / TA::BM, stages = g.K / TA::BK;
    const uint64_t rounds_a = tiles_m * (g.N / TA::BN) / cus;   // whole rounds of the 256 x 256 tiles
    for (uint64_t r = 1; r <= rounds_a; ++r) {
        const uint64_t amax = r * cus / tiles_m;
        for (uint64_t a = amax; a + 3 > amax && a > 0; --a) {
            if (a * TA::BN >= g.N) continue;
            const uint64_t rest = g.N - a * TA::BN;
            if (rest % TB::BN != 0 || tiles_m * (rest / TB::BN) > cus) continue;
            if (!wide_fits<4, 2, 128, 2, 4>(column_range(g, 0, (uint32_t)(a * TA::BN))) ||
                !wide_fits<2, 3, 128, 4, 2>(column_range(g, (uint32_t)(a * TA::BN), (uint32_t)rest)))
                continue;
            const float est = (float)((tiles_m * a + cus - 1) / cus) * (c0a + c1a * (float)stages) +
                              (c0b + c1b * (float)stages);
            if (best.n1 == 0 || est < best.est) best = MixedPlan{(uint32_t)(a * TA::BN), est};
        }
    }
    return best;
}

}  // namespace fp8gemm

int launch_fp8_gemm(const uint8_t *a, int fa, const float *sa, uint32_t nsa, const uint8_t *b, int fb,
                    const float *sb, uint32_t nsb, uint32_t M, uint32_t N, uint32_t K, uint16_t *out,
                    hipStream_t st) {
    using namespace fp8gemm;
    const Fp8Args g{a, fa, sa, nsa, b, fb, sb, nsb, M, N, K, out};
    const uint64_t cus = (uint64_t)device_props().cus;
    // Whole tiles: the wide forms. Each candidate's time is modelled as
    // rounds x (c0 + c1 x stages), rounds = ceil(tiles / CUs), stages = K / 128,
    // with (c0, c1) in microseconds fitted to timings of every form on eleven
    // products (M 256-2048, N 1024-27648, K 4096-27648; shorter K is an
    // extrapolation). Most timings lie within 10% of the fit, 64 x 64 and
    // 256 x 128 up to 26% above it when their tiles take a single round. The
    // cheapest form runs; on those products that is the fastest one measured.
    const WideCand cands[] = {
        wide_cand<4, 2, 2, 4>(g, 16.2f, 1.318f),   // 256 x 256, 8 waves, 2 slots
        wide_cand<2, 2, 4, 2>(g, 12.2f, 0.739f),   // 256 x 128, 8 waves, 3 slots
        wide_cand<1, 5, 4, 1>(g, 8.6f, 0.658f),    // 128 x 160, 4 waves, 3 slots
        wide_cand<2, 2, 2, 2>(g, 6.5f, 0.550f),    // 128 x 128, 4 waves, 3 slots
        wide_cand<1, 1, 2, 2>(g, 1.1f, 0.246f),    // 64 x 64, 4 waves, 4 slots
    };
    int pick = -1;
    float best = 0.0f;
    for (int i = 0; i < (int)(sizeof(cands) / sizeof(cands[0])); ++i) {
        if (!cands[i].fits) continue;
        const uint64_t tiles = (uint64_t)(M / cands[i].bm) * (N / cands[i].bn);
        const float est = (float)((tiles + cus - 1) / cus) * (cands[i].c0 + cands[i].c1 * (float)(K / 128));
        if (pick < 0 || est < best) pick = i, best = est;
    }
    const MixedPlan mp = mixed_plan(g, cus, cands[0].c0, cands[0].c1, 8.2f, 1.353f);
    if (mp.n1 != 0 && (pick < 0 || mp.est < best)) {
        const int rc = launch_fp8_wide<4, 2, 128, 2>(column_range(g, 0, mp.n1), st, N);
        if (rc != RENG_HIP_OK) return rc;
        return launch_fp8_wide<2, 3, 128, 2, 4, 2>(column_range(g, mp.n1, N - mp.n1), st, N);
    }
    switch (pick) {
    case 0: return launch_fp8_wide<4, 2, 128, 2>(g, st);
    case 1: return launch_fp8_wide<2, 2, 128, 3, 4, 2>(g, st);
    case 2: return launch_fp8_wide<1, 5, 128, 3, 4, 1>(g, st);
    case 3: return launch_fp8_wide<2, 2, 128, 3, 2, 2>(g, st);
    case 4: return launch_fp8_wide<1, 1, 128, 4, 2, 2>(g, st);
    default: break;
    }
    // Ragged shapes: by how many tiles each size gives for the chip (measured
    // on the M = 1024 prefill shapes): the largest tile that still fills every
    // CU; 256 x 128 for long K; 64 x 64 for small outputs.
    const uint64_t t256 = (uint64_t)((M + 255) / 256) * ((N + 255) / 256);
    const uint64_t t128 = (uint64_t)((M + 127) / 128) * ((N + 127) / 128);
    if (t256 >= cus) return launch_fp8_cfg<4, 4, 2, 2>(g, st);
    if (t128 >= cus) return K > 8192 ? launch_fp8_cfg<4, 2, 2, 3>(g, st) : launch_fp8_cfg<2, 2, 2, 2>(g, st);
    if (K > 8192 && 2 * t128 >= cus) return launch_fp8_cfg<4, 2, 2, 3>(g, st);
    return launch_fp8_cfg<1, 1, 2, 4>(g, st);
}

}  // namespace reng
