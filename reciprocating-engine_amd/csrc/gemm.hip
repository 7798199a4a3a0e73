// gemm.hip - consumers of the quantizer's codes on CDNA4 (gfx950).
//
// 1. gemv_rows      (M = 1, 1024 < K <= 32768; M = 2, 1024 < K <= 8192) and
//    gemv_w8a16     (the other M = 1, M = 2 with K <= 1024 or 8192 < K <=
//                    16384, M <= 4 when K % 128 != 0):
//                    y[m, n] = s[n] * sum_k x[m, k] * decode(c[n, k]); with
//                    M = 1 gemv_w8a16 also has residual-add, SwiGLU-pair and
//                    RoPE-pair epilogues and an RMSNorm prologue.
//    Both stream the codes once with 16-byte loads, decode in registers to
//    bf16 (v_cvt_scalef32_pk_bf16_fp8 / _bf8) and accumulate with
//    v_dot2_f32_bf16, one wave per output row, in the same order.
// 2. The other M <= 64: the same product on bf16 MFMA with the codes and the
//    activation staged through LDS (skinny.hip); larger M in tiles of 64.
// (The fp8 x fp8 product of gemm_fp8_scaled is in gemm_fp8.hip.)
//
// The reference semantics are gemm_cpu over Quantized::dequantize
// (crates/reng-model/src/bin/fp8_probe.rs:55-67) and the per-channel scaleB of
// fp8_gemm_bf16 (crates/reng-synapse/src/fp8.rs:295-331).
#include <map>
#include <mutex>
#include <utility>

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

// A workgroup barrier that waits for this wave's LDS accesses only (no
// vmcnt(0) as __syncthreads' fence has), so global loads stay in flight
// across it; the memory clobbers keep LDS accesses on their side of it.
__device__ __forceinline__ void lds_sync() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xf | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

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
//
// Epilogues (M = 1): EPI_RESID writes f32 yres[n] = res[n] + bf16(y[n]) (a
// projection and its residual add); EPI_SWIGLU takes rows in (gate, up) pairs
// (row 2i of the matrix is gate row i, row 2i + 1 up row i), a wave computes
// both rows of a pair, and y[i] = bf16(silu(bf16 gate) * bf16 up). Each is the
// arithmetic of add_bf16_f32 / silu_mul_bf16 (layer.hip) after the plain
// GEMV: a row's sum does not depend on which wave computes it.
//
// EPI_ROPE takes the rows of a stacked [q; k; v] projection in rotation pairs
// (row 2p, 2p + 1 = dimensions d, d + half of one q or k head, then v rows two
// by two; RopeOut gives the order) and writes the pair rotated into q and the
// key cache row, or copied into the value cache row: rope_append (layer.hip)
// after the plain GEMV, through the same rope_rotate.
enum { EPI_PLAIN = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_ROPE = 3 };

struct RopeOut {
    uint16_t *q, *k_row, *v_row;   // [nh * hd], [nkv * hd], [nkv * hd] bf16
    const float *sn, *cs;          // this position's rows of the tables, [hd]
    uint32_t half, q_pairs, qk_pairs;   // hd / 2, nh * half, (nh + nkv) * half
};

__device__ __forceinline__ void rope_store(const RopeOut &ro, uint32_t p, uint32_t b0, uint32_t b1) {
    if (p < ro.qk_pairs) {
        const bool isq = p < ro.q_pairs;
        const uint32_t pp = isq ? p : p - ro.q_pairs, head = pp / ro.half, d = pp % ro.half;
        float o0, o1;
        rope_rotate(__uint_as_float(b0 << 16), __uint_as_float(b1 << 16), ro.cs[d], ro.sn[d], ro.cs[d + ro.half],
                    ro.sn[d + ro.half], o0, o1);
        uint16_t *dst = (isq ? ro.q : ro.k_row) + (size_t)head * 2 * ro.half + d;
        dst[0] = (uint16_t)f32_to_bf16_bits(o0);
        dst[ro.half] = (uint16_t)f32_to_bf16_bits(o1);
    } else {
        const uint32_t i = p - ro.qk_pairs;
        ro.v_row[2 * i] = (uint16_t)b0;
        ro.v_row[2 * i + 1] = (uint16_t)b1;
    }
}

__device__ __forceinline__ uint16_t silu_mul_bits(uint32_t g, uint32_t u) {
    const float gv = __uint_as_float(g << 16), uv = __uint_as_float(u << 16);
    return (uint16_t)f32_to_bf16_bits(gv / (1.0f + expf(-gv)) * uv);
}

//
// Prologue PRO_NORM (M = 1, XLDS): x is an f32 row h [K] and the row staged is
// bf16(h * inv * gamma), its RMSNorm, inv formed as row_inv_rms forms it in a
// 1024-thread workgroup (so the staged row is rms_norm_rows' output, bit for
// bit); PRO_NORM_VEC takes h four columns at a time (K % 4 == 0, h and gamma
// 16-byte aligned), as rms_norm_rows' VEC form does.
enum { PRO_NONE = 0, PRO_NORM = 1, PRO_NORM_VEC = 2 };

template <int F, int M, int CPL, bool XLDS, bool RAGGED, int EPI = EPI_PLAIN, int PRO = PRO_NONE>
__global__ __launch_bounds__(512) void gemv_w8a16(const uint16_t *__restrict__ x,
                                                  const uint8_t *__restrict__ codes,
                                                  const float *__restrict__ scales, uint32_t N,
                                                  uint32_t K, uint16_t *__restrict__ y, const float *res,
                                                  float *yres, const float *__restrict__ gamma, float eps,
                                                  RopeOut ro) {
    static_assert(EPI == EPI_PLAIN || M == 1, "the fused epilogues take one activation row");
    static_assert(PRO == PRO_NONE || (M == 1 && XLDS), "the RMSNorm prologue stages one row in LDS");
    constexpr bool PAIRS = EPI == EPI_SWIGLU || EPI == EPI_ROPE;
    extern __shared__ __attribute__((aligned(16))) uint32_t xs[];
    __shared__ float red[PRO == PRO_NONE ? 1 : NORM_VT / 64];
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t nch = K / 16;   // 16-code chunks per row
    const uint32_t waves = gridDim.x * (blockDim.x >> 6);
    const uint32_t wave = blockIdx.x * (blockDim.x >> 6) + (tid >> 6);
    const uint32_t gpr = (nch + 64 * CPL - 1) / (64 * CPL);   // groups per row
    // The wave's i-th row: wave + i * waves, or with PAIRS row 2p + (i & 1) of
    // pair p = wave + (i / 2) * waves.
    auto row_at = [&](uint32_t i) -> uint32_t {
        return PAIRS ? 2 * (wave + (i >> 1) * waves) + (i & 1) : wave + i * waves;
    };

    // Loads are unconditional (indices clamped into the matrix) so the wait
    // before each use covers exactly the loads issued before it; a ragged
    // tail's surplus chunks are zeroed after the load.
    auto load = [&](uint32_t r, uint32_t gi, u32x4 (&q)[CPL]) {
        r = r < N ? r : N - 1;
        const u32x4 *wr = reinterpret_cast<const u32x4 *>(codes + (size_t)r * K);
        const uint32_t c0 = gi * 64 * CPL + lane;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            const uint32_t ch = c0 + u * 64;
            q[u] = __builtin_nontemporal_load(wr + (RAGGED && ch >= nch ? nch - 1 : ch));
        }
    };

    // The first group's codes and the scales are requested before the
    // activation is staged.
    uint32_t r = row_at(0), gi = 0;
    u32x4 qn[CPL];
    // Lane j holds the scale of this wave's row ri + j (ri = rows done,
    // refilled every 64 rows), so an end-of-row multiply reads it with
    // readlane instead of waiting a memory round trip.
    uint32_t ri = 0;
    float sv = 1.0f;
    auto scales_from = [&](uint32_t first) {   // lanes past the last row repeat it (never read)
        const uint32_t rr = row_at(first + lane);
        sv = scales[rr < N ? rr : N - 1];
    };
    // The four-column RMSNorm prologue on rows of up to 8192 columns holds its
    // share of h and gamma in registers (columns 4 tid + 2048 m, m < 4). In
    // issue order: the scales, h and gamma, then the wave's first two code
    // groups, every load unconditional (indices clamped; a wave past the last
    // row reads row N - 1 and stores nothing). Loads leave the vmcnt count in
    // order, so the prologue waits for h and gamma alone, its barriers wait on
    // LDS only, and the codes stay in flight through it.
    constexpr bool REGP = PRO == PRO_NORM_VEC;
    const bool regp = REGP && K <= 4 * 2048;
    float4 hreg[4], greg[4];
    u32x4 q2[CPL];
    uint32_t r2 = r, g2 = gi + 1;
    if (g2 == gpr) {
        g2 = 0;
        r2 = PAIRS ? ((r & 1) ? r - 1 + 2 * waves : r + 1) : r + waves;
    }
    bool second = false;
    if (regp) {
        if (scales) scales_from(0);
        const float *xf = reinterpret_cast<const float *>(x);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t c = tid * 4 + 2048 * m < K ? tid * 4 + 2048 * m : K - 4;
            hreg[m] = *reinterpret_cast<const float4 *>(xf + c);
            greg[m] = *reinterpret_cast<const float4 *>(gamma + c);
        }
        load(r, gi, qn);
        // A wave with a single group asks for it again (an L2 hit), not for
        // another row's bytes.
        second = r2 < N;
        load(second ? r2 : r, second ? g2 : gi, q2);
    } else if (r < N) {
        load(r, gi, qn);
        if (scales) scales_from(0);
    }
    if constexpr (REGP) {
        if (regp) {
            // row_inv_rms's sum: virtual thread vt = tid + 512 i takes columns
            // 4 vt + 4096 u, i.e. m = i + 2 u.
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                float ss = 0.0f;
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    if (tid * 4 + 2048 * (i + 2 * u) < K) ss = sum_sq4(ss, hreg[i + 2 * u]);
                ss = wave_sum_dpp(ss);
                if (lane == 0) red[(tid + 512 * i) >> 6] = ss;
            }
            lds_sync();
            const float inv = inv_rms_from(red, K, eps);
            uint16_t *dst = reinterpret_cast<uint16_t *>(xs);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t c = tid * 4 + 2048 * m;
                if (c >= K) continue;
                const float4 v = hreg[m], g = greg[m];
                const uint32_t lo = f32_to_bf16_bits(v.x * inv * g.x) | (f32_to_bf16_bits(v.y * inv * g.y) << 16);
                const uint32_t hi = f32_to_bf16_bits(v.z * inv * g.z) | (f32_to_bf16_bits(v.w * inv * g.w) << 16);
                *reinterpret_cast<u32x2 *>(dst + c) = u32x2{lo, hi};
            }
            lds_sync();
        }
    }
    if constexpr (PRO != PRO_NONE) {
        if (!regp) {
            const float *xf = reinterpret_cast<const float *>(x);
            const float inv = row_inv_rms<PRO == PRO_NORM_VEC, false, NORM_VT / 512>(xf, nullptr, nullptr, K, eps, red);
            uint16_t *dst = reinterpret_cast<uint16_t *>(xs);
            if constexpr (PRO == PRO_NORM_VEC) {
                for (uint32_t c = tid * 4; c < K; c += 512 * 4) {
                    const float4 v = *reinterpret_cast<const float4 *>(xf + c);
                    const float4 gv = *reinterpret_cast<const float4 *>(gamma + c);
                    const uint32_t lo = f32_to_bf16_bits(v.x * inv * gv.x) | (f32_to_bf16_bits(v.y * inv * gv.y) << 16);
                    const uint32_t hi = f32_to_bf16_bits(v.z * inv * gv.z) | (f32_to_bf16_bits(v.w * inv * gv.w) << 16);
                    *reinterpret_cast<u32x2 *>(dst + c) = u32x2{lo, hi};
                }
            } else {
                for (uint32_t c = tid; c < K; c += 512) dst[c] = (uint16_t)f32_to_bf16_bits(xf[c] * inv * gamma[c]);
            }
            __syncthreads();
        }
    } else if constexpr (XLDS) {
        const u32x4 *src = reinterpret_cast<const u32x4 *>(x);
        u32x4 *dst = reinterpret_cast<u32x4 *>(xs);
        for (uint32_t i = tid; i < M * nch * 2; i += blockDim.x) dst[i] = src[i];
        __syncthreads();
    }
    if (r >= N) return;
    uint32_t gate_bits = 0;   // PAIRS: the pair's first row, held until its second row ends
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
            rn = PAIRS ? ((r & 1) ? r - 1 + 2 * waves : r + 1) : r + waves;
        }
        if (second) {   // (rn, gn) is (r2, g2), requested before the prologue
#pragma unroll
            for (int u = 0; u < CPL; ++u) qn[u] = q2[u];
            second = false;
        } else if (rn < N) {
            load(rn, gn, qn);   // none past the wave's last row
        }

        const uint32_t c0 = gi * 64 * CPL + lane;
#pragma unroll
        for (int u = 0; u < CPL; ++u) {
            uint32_t ch = c0 + u * 64;
            uint32_t w[8];
            decode16<F>(q[u], w);
            if (RAGGED && ch >= nch) {
#pragma unroll
                for (int i = 0; i < 8; ++i) w[i] = 0u;
                ch = nch - 1;
            }
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
            const float s = scales ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv), ri & 63)) : 1.0f;
            if (scales && (++ri & 63) == 0) scales_from(ri);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float t = wave_sum_dpp(acc[m][0] + acc[m][1]);
                if constexpr (EPI == EPI_RESID) {
                    if (lane == 0) yres[r] = res[r] + __uint_as_float(f32_to_bf16_bits(t * s) << 16);
                } else if constexpr (EPI == EPI_SWIGLU) {
                    const uint32_t b = f32_to_bf16_bits(t * s);
                    if (r & 1) {
                        if (lane == 0) y[r >> 1] = silu_mul_bits(gate_bits, b);
                    } else {
                        gate_bits = b;
                    }
                } else if constexpr (EPI == EPI_ROPE) {
                    const uint32_t b = f32_to_bf16_bits(t * s);
                    if (r & 1) {
                        if (lane == 0) rope_store(ro, r >> 1, gate_bits, b);
                    } else {
                        gate_bits = b;
                    }
                } else {
                    if (lane == m) y[(size_t)m * N + r] = (uint16_t)f32_to_bf16_bits(t * s);
                }
                acc[m][0] = acc[m][1] = 0.0f;
            }
        }
        if (rn >= N) break;
        r = rn;
        gi = gn;
    }
}

// ------------------------------------------------------------------ GEMV, M = 1

// One wave per output row; the row's CPR 1 KB chunks (K <= 32768) stream
// through a window of GEMV_WINDOW chunks: the first min(CPR, GEMV_WINDOW) are
// requested at the start, and chunk c + GEMV_WINDOW is requested just before
// chunk c is consumed. In issue order: the row's scale, this thread's share of
// the activation (into registers, then LDS), the row's first chunks; the
// activation is written to LDS and the block barrier waits on LDS only, so the
// codes stay in flight through it. Every load is an ordinary (compiler-tracked)
// load, issued unconditionally (indices clamped), so the compiler waits for
// chunk c alone before consuming it while the later chunks are still in
// flight. Measured on MI355X against the former walk (R rows per wave in
// U-chunk steps, untracked loads): [14336, 4096] 10.64 -> 10.12 us, [4096,
// 4096] 4.92 -> 4.46 us, with a plain one-launch read of the same codes at
// 9.5-9.6 us. On 14 KB rows ([4096, 14336]) the whole row in flight served the
// rows in no useful order (block end times spread over 4 us) and took 10.6-11.3
// us; a window of 10 chunks takes 10.3 (7: 10.45, 12: 10.33, 14: 10.65).
// What is left over the plain read on both shapes is the stores of y: the
// same kernel with them taken out takes 9.87 / 10.04 us, as does a load-only
// variant that stores y (9.94 / 10.18), against 9.65 / 9.95 without them.
//
// A lane takes the same 16 codes of every 1 KB chunk (k = 1024 c + 16 lane ..
// + 16) and adds the products in gemv_w8a16's order (chunks in order, even and
// odd words into two accumulators, then wave_sum_dpp), so the two kernels give
// the same bits and the fused forms of gemv_w8a16 equal this GEMV followed by
// their epilogue. A ragged last chunk (K % 1024 != 0) masks the lanes past K.
constexpr int GEMV_WINDOW = 10;

//
// EPI_RESID (the decode step's projections that feed the residual stream)
// writes f32 yres[n] = res[n] + bf16(y[n]) instead of y: gemv_w8a16's residual
// epilogue on the same row sums, so the same bits.
//
// MR activation rows (1 or 2; x [MR, K], y [MR, N]): each wave still streams
// one weight row, its chunks met by every activation row in LDS (MR x CPR x
// 2 KB at most 64 KB), with the same lanes, order and accumulators per
// activation row as for one, so an MR = 2 product equals two MR = 1 products
// bit for bit.
template <int F, int CPR, int WPB, int EPI = EPI_PLAIN, int MR = 1>
// (No __restrict__ on the inputs: loads through a restrict pointer to const may
// be treated as invariant and moved across the compiler barriers that fix the
// issue order.)
__global__ __launch_bounds__(64 * WPB) void gemv_rows(const uint16_t *x, const uint8_t *codes,
                                                      const float *scales, uint32_t N, uint32_t K,
                                                      uint16_t *__restrict__ y, const float *res,
                                                      float *__restrict__ yres) {
    static_assert(EPI == EPI_PLAIN || EPI == EPI_RESID, "plain or residual rows");
    static_assert(MR == 1 || (MR == 2 && EPI == EPI_PLAIN), "two activation rows: plain output only");
    static_assert(MR * CPR <= 32, "the activation's LDS copy is at most 64 KB");
    constexpr uint32_t XMAX = CPR * 128;                             // 16-byte activation pieces at most
    constexpr uint32_t XPT = (XMAX + 64 * WPB - 1) / (64 * WPB);     // pieces per thread
    __shared__ __attribute__((aligned(16))) u32x4 xs[MR * XMAX];
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t n = blockIdx.x * WPB + __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t nr = n < N ? n : N - 1;   // a wave past the last row reads row N - 1, stores nothing
    const uint32_t xp = K / 8;               // 16-byte activation pieces per row
    const uint32_t live = (K & 1023) ? (K & 1023) >> 4 : 64;   // lanes of the last chunk inside the row
    const float sv = scales ? scales[nr] : 1.0f;
    const u32x4 *x16 = reinterpret_cast<const u32x4 *>(x);
    u32x4 xt[MR][XPT];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (uint32_t j = 0; j < XPT; ++j) {
            const uint32_t i = tid + j * 64 * WPB;
            xt[r][j] = x16[r * xp + (i < xp ? i : xp - 1)];
        }
    // The codes are requested after the scale and the activation.
    asm volatile("" ::: "memory");
    const u32x4 *wr = reinterpret_cast<const u32x4 *>(codes + (size_t)nr * K);
    u32x4 q[CPR];
    auto request = [&](int c) {
        const uint32_t lc = c == CPR - 1 && lane >= live ? live - 1 : lane;
        q[c] = __builtin_nontemporal_load(wr + 64 * c + lc);
        asm volatile("" ::: "memory");   // issued in chunk order, the order they are consumed in
    };
#pragma unroll
    for (int c = 0; c < CPR && c < GEMV_WINDOW; ++c) request(c);
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (uint32_t j = 0; j < XPT; ++j) {
            const uint32_t i = tid + j * 64 * WPB;
            if (i < xp) xs[r * XMAX + i] = xt[r][j];
        }
    lds_sync();
    // Past K in a ragged last chunk: no codes, and no activation past the LDS
    // copy either (a mask, not a branch, so the waits stay per chunk).
    const uint32_t keep_last = lane < live ? ~0u : 0u;
    float a0[MR], a1[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) a0[r] = a1[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < CPR; ++c) {
        if (c + GEMV_WINDOW < CPR) request(c + GEMV_WINDOW);
        uint32_t wv[8];
        decode16<F>(q[c], wv);
        if (c == CPR - 1) {
#pragma unroll
            for (int i = 0; i < 8; ++i) wv[i] &= keep_last;
        }
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            u32x4 xa = xs[r * XMAX + 128 * c + 2 * lane], xb = xs[r * XMAX + 128 * c + 2 * lane + 1];
            if (c == CPR - 1) {
                xa &= keep_last;
                xb &= keep_last;
            }
            a0[r] = dot2(wv[0], xa.x, a0[r]);
            a1[r] = dot2(wv[1], xa.y, a1[r]);
            a0[r] = dot2(wv[2], xa.z, a0[r]);
            a1[r] = dot2(wv[3], xa.w, a1[r]);
            a0[r] = dot2(wv[4], xb.x, a0[r]);
            a1[r] = dot2(wv[5], xb.y, a1[r]);
            a0[r] = dot2(wv[6], xb.z, a0[r]);
            a1[r] = dot2(wv[7], xb.w, a1[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const float t = wave_sum_dpp(a0[r] + a1[r]);
        if (lane == 0 && n < N) {
            const uint32_t b = f32_to_bf16_bits(t * sv);
            if constexpr (EPI == EPI_RESID) yres[n] = res[n] + __uint_as_float(b << 16);
            else y[(size_t)r * N + n] = (uint16_t)b;
        }
    }
}

// ------------------------------------------------------------------ read yardstick

// Reads `chunks` 1 KB chunks: wave w takes chunks w, w + W, ... one at a time
// (16-byte non-temporal loads, one 1 KB chunk per wave in flight), the pattern
// that read a GEMV-sized buffer fastest on this device (measured over 1-8
// chunks in flight per wave and 8-32 waves per CU). The XOR of the data keeps
// the loads live; sink is written only if the XOR hits a fixed value, so the
// launch writes (almost) nothing.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *__restrict__ p, uint64_t chunks,
                                                          uint32_t *sink) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t W = (uint64_t)gridDim.x * 4, w = blockIdx.x * 4 + (threadIdx.x >> 6);
    uint32_t acc = 0;
    for (uint64_t c = w; c < chunks; c += W) {
        const u32x4 v = __builtin_nontemporal_load(p + c * 64 + lane);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;
}

int launch_stream_read(const void *p, size_t bytes, uint32_t *sink, hipStream_t st) {
    const uint32_t blocks = (uint32_t)device_props().cus * 8;   // 32 waves per CU
    hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, st, static_cast<const u32x4 *>(p),
                       (uint64_t)(bytes / 1024), sink);
    return check_launch("stream_read");
}

uint32_t stream_read_sink_words() { return (uint32_t)device_props().cus * 8; }

// ------------------------------------------------------------------ launchers

// Split-K partials live in a grow-only f32 buffer per (device, stream): calls on
// one stream are ordered, so they can share it; calls on different streams get
// different buffers. No allocation once a stream has seen its largest product.
// The buffers live until the process ends (keyed by the stream handle: a
// stream destroyed while its work is still queued must not have its handle
// reused by another before that work ends). Growing it synchronizes the stream
// and calls hipMalloc, which a stream under graph capture cannot do: that case
// is refused (warm the stream up with the largest product first, or use the
// allocation-free entry point).
float *split_workspace(size_t floats, hipStream_t st, int *rc) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<float *, size_t>> bufs;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(mu);
    auto &e = bufs[{dev, st}];
    if (e.second < floats) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
            set_error("the split-K workspace would grow to %zu bytes while the stream is captured: run the "
                      "product once on this stream before capturing, or call reng_hip_gemm_w8a16_noalloc",
                      floats * sizeof(float));
            *rc = RENG_HIP_EINVAL;
            return nullptr;
        }
        if (e.first) {
            // The old buffer may still be read by work queued on this stream.
            const hipError_t se = hipStreamSynchronize(st);
            if (se != hipSuccess) {
                set_error("hipStreamSynchronize: %s", hipGetErrorString(se));
                *rc = RENG_HIP_EDEVICE;
                return nullptr;
            }
            (void)hipFree(e.first);
            e.first = nullptr;
            e.second = 0;
        }
        void *p = nullptr;
        const hipError_t ae = hipMalloc(&p, floats * sizeof(float));
        if (ae != hipSuccess) {
            set_error("hipMalloc(split workspace, %zu bytes): %s", floats * sizeof(float), hipGetErrorString(ae));
            *rc = RENG_HIP_ENOMEM;
            return nullptr;
        }
        e.first = static_cast<float *>(p);
        e.second = floats;
    }
    *rc = RENG_HIP_OK;
    return e.first;
}

// The allocation-free entry point's partials: a static array in device memory,
// one copy per device (the code object's), whose address each device resolves
// once with hipGetSymbolAddress. In host code `scratch` names a host-side
// stand-in, never the device memory: only the looked-up address is passed on.
static __device__ __align__(256) float scratch[STATIC_SCRATCH_FLOATS];

float *static_split_scratch(int *rc) {
    static std::mutex mu;
    static std::map<int, float *> addr;
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) {
        set_error("hipGetDevice: %s", hipGetErrorString(ge));
        *rc = RENG_HIP_EDEVICE;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu);
    auto it = addr.find(dev);
    if (it == addr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_error("hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
            *rc = RENG_HIP_EDEVICE;
            return nullptr;
        }
        it = addr.emplace(dev, static_cast<float *>(p)).first;
    }
    *rc = RENG_HIP_OK;
    return it->second;
}

// Stream-K tile counters: zeroed when allocated, and every launch that uses
// them leaves them zeroed (the last block of each split tile resets its
// counter). One grow-only buffer per (device, stream), as split_workspace.
uint32_t *tile_counters(uint32_t count, hipStream_t st, int *rc) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, std::pair<uint32_t *, uint32_t>> bufs;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lk(mu);
    auto &e = bufs[{dev, st}];
    if (e.second < count) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
            set_error("the stream-K tile counters would grow to %u while the stream is captured: run the product "
                      "once on this stream before capturing",
                      count);
            *rc = RENG_HIP_EINVAL;
            return nullptr;
        }
        if (e.first) {
            const hipError_t se = hipStreamSynchronize(st);
            if (se != hipSuccess) {
                set_error("hipStreamSynchronize: %s", hipGetErrorString(se));
                *rc = RENG_HIP_EDEVICE;
                return nullptr;
            }
            (void)hipFree(e.first);
            e.first = nullptr;
            e.second = 0;
        }
        void *p = nullptr;
        hipError_t ae = hipMalloc(&p, (size_t)count * sizeof(uint32_t));
        if (ae == hipSuccess) ae = hipMemset(p, 0, (size_t)count * sizeof(uint32_t));
        if (ae != hipSuccess) {
            if (p) (void)hipFree(p);
            set_error("tile counters (%u): %s", count, hipGetErrorString(ae));
            *rc = RENG_HIP_ENOMEM;
            return nullptr;
        }
        e.first = static_cast<uint32_t *>(p);
        e.second = count;
    }
    *rc = RENG_HIP_OK;
    return e.first;
}

// The allocation-free entry point's tile counters: zero from load, left zeroed
// by every launch, one copy per device (resolved as `scratch` is).
static __device__ __align__(256) uint32_t counters[STATIC_TILE_COUNTERS];

uint32_t *static_tile_counters(int *rc) {
    static std::mutex mu;
    static std::map<int, uint32_t *> addr;
    int dev = 0;
    const hipError_t ge = hipGetDevice(&dev);
    if (ge != hipSuccess) {
        set_error("hipGetDevice: %s", hipGetErrorString(ge));
        *rc = RENG_HIP_EDEVICE;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(mu);
    auto it = addr.find(dev);
    if (it == addr.end()) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(counters));
        if (e != hipSuccess || !p) {
            set_error("hipGetSymbolAddress(counters) on device %d: %s", dev, hipGetErrorString(e));
            *rc = RENG_HIP_EDEVICE;
            return nullptr;
        }
        it = addr.emplace(dev, static_cast<uint32_t *>(p)).first;
    }
    *rc = RENG_HIP_OK;
    return it->second;
}

float *split_partials(size_t floats, hipStream_t st, const SplitScratch *fixed, int *rc) {
    if (!fixed) return split_workspace(floats, st, rc);
    if (floats > fixed->floats) {
        set_error("this product's split-K plan needs %zu bytes of scratch; the static scratch holds %zu "
                  "(reng_hip_gemm_w8a16 allocates what it needs)",
                  floats * sizeof(float), fixed->floats * sizeof(float));
        *rc = RENG_HIP_EINVAL;
        return nullptr;
    }
    *rc = RENG_HIP_OK;
    return fixed->ptr;
}

// The GEMV's launch for M <= 4 rows: rows (or row groups of `unit`, which a
// wave takes together) divide evenly over the waves, at most 16 waves per CU;
// the activation is staged in LDS when it fits in 64 KB; 7 chunks per lane
// when a row splits into whole groups of 7 (K a multiple of 7168, e.g.
// 14336), else 4.
struct GemvPlan {
    static constexpr int threads = 512;
    uint32_t blocks;
    size_t lds;
    bool xlds, cpl7, ragged;
};

GemvPlan gemv_plan(uint32_t M, uint32_t N, uint32_t K, uint32_t unit) {
    GemvPlan p;
    const uint32_t units = N / unit;
    const uint32_t cap = (uint32_t)device_props().cus * 16;
    const uint32_t rpw = (units + cap - 1) / cap;
    const uint32_t waves = (units + rpw - 1) / rpw;
    const size_t xbytes = (size_t)M * K * 2;
    p.xlds = xbytes <= 64 * 1024;
    p.blocks = (waves + GemvPlan::threads / 64 - 1) / (GemvPlan::threads / 64);
    p.lds = p.xlds ? xbytes : 0;
    p.cpl7 = (K / 16) % (64 * 7) == 0;
    p.ragged = (K / 16) % (64 * (p.cpl7 ? 7 : 4)) != 0;
    return p;
}

template <int F, int EPI, int PRO = PRO_NONE>
int launch_gemv_epi_t(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                      uint16_t *y, const float *res, float *yres, const float *gamma, float eps, hipStream_t st,
                      const RopeOut &ro = RopeOut{}) {
    const GemvPlan p = gemv_plan(1, N, K, EPI == EPI_SWIGLU || EPI == EPI_ROPE ? 2 : 1);
    if (PRO != PRO_NONE && !p.xlds) {
        set_error("K = %u: the RMSNorm prologue stages the row in 64 KB of LDS (K <= 32768)", K);
        return RENG_HIP_EINVAL;
    }
#define RENG_GEMV_E(C, XL, RG)                                                                                  \
    hipLaunchKernelGGL((gemv_w8a16<F, 1, C, XL, RG, EPI, PRO>), dim3(p.blocks), dim3(GemvPlan::threads), p.lds, \
                       st, x, codes, scales, N, K, y, res, yres, gamma, eps, ro)
    if constexpr (PRO != PRO_NONE) {
        if (p.cpl7) RENG_GEMV_E(7, true, false);
        else if (p.ragged) RENG_GEMV_E(4, true, true);
        else RENG_GEMV_E(4, true, false);
    } else {
#define RENG_GEMV_EX(C, RG) \
    if (p.xlds) RENG_GEMV_E(C, true, RG); else RENG_GEMV_E(C, false, RG);
        if (p.cpl7) { RENG_GEMV_EX(7, false) }
        else if (p.ragged) { RENG_GEMV_EX(4, true) }
        else { RENG_GEMV_EX(4, false) }
#undef RENG_GEMV_EX
    }
#undef RENG_GEMV_E
    return check_launch(EPI == EPI_SWIGLU ? "gemv_w8a16 (SwiGLU pairs)"
                        : EPI == EPI_ROPE  ? "gemv_w8a16 (RoPE pairs)"
                        : EPI == EPI_RESID ? "gemv_w8a16 (residual)"
                                           : "gemv_w8a16 (RMSNorm)");
}

template <int F, int EPI>
int launch_gemv_norm_t(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                       uint32_t N, uint32_t K, uint16_t *y, hipStream_t st) {
    const uint16_t *xa = reinterpret_cast<const uint16_t *>(x);
    const bool vec =
        K % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 15) == 0;
    return vec ? launch_gemv_epi_t<F, EPI, PRO_NORM_VEC>(xa, codes, scales, N, K, y, nullptr, nullptr, gamma, eps, st)
               : launch_gemv_epi_t<F, EPI, PRO_NORM>(xa, codes, scales, N, K, y, nullptr, nullptr, gamma, eps, st);
}

template <int F>
int launch_gemv_norm_rope_t(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                            uint32_t N, uint32_t K, const RopeOut &ro, hipStream_t st) {
    const uint16_t *xa = reinterpret_cast<const uint16_t *>(x);
    const bool vec =
        K % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 15) == 0;
    return vec ? launch_gemv_epi_t<F, EPI_ROPE, PRO_NORM_VEC>(xa, codes, scales, N, K, nullptr, nullptr, nullptr,
                                                               gamma, eps, st, ro)
               : launch_gemv_epi_t<F, EPI_ROPE, PRO_NORM>(xa, codes, scales, N, K, nullptr, nullptr, nullptr, gamma,
                                                           eps, st, ro);
}

int launch_gemv_norm_rope(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                          uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t K, int format, const float *sin_row,
                          const float *cos_row, uint16_t *q, uint16_t *k_row, uint16_t *v_row, hipStream_t st) {
    RopeOut ro;
    ro.q = q;
    ro.k_row = k_row;
    ro.v_row = v_row;
    ro.sn = sin_row;
    ro.cs = cos_row;
    ro.half = hd / 2;
    ro.q_pairs = nh * ro.half;
    ro.qk_pairs = (nh + nkv) * ro.half;
    const uint32_t N = (nh + 2 * nkv) * hd;
    return format == RENG_HIP_E4M3 ? launch_gemv_norm_rope_t<RENG_HIP_E4M3>(x, gamma, eps, codes, scales, N, K, ro, st)
                                   : launch_gemv_norm_rope_t<RENG_HIP_E5M2>(x, gamma, eps, codes, scales, N, K, ro, st);
}

int launch_gemv_norm(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                     uint32_t N, uint32_t K, int format, bool swiglu, uint16_t *y, hipStream_t st) {
    if (format == RENG_HIP_E4M3)
        return swiglu ? launch_gemv_norm_t<RENG_HIP_E4M3, EPI_SWIGLU>(x, gamma, eps, codes, scales, N, K, y, st)
                      : launch_gemv_norm_t<RENG_HIP_E4M3, EPI_PLAIN>(x, gamma, eps, codes, scales, N, K, y, st);
    return swiglu ? launch_gemv_norm_t<RENG_HIP_E5M2, EPI_SWIGLU>(x, gamma, eps, codes, scales, N, K, y, st)
                  : launch_gemv_norm_t<RENG_HIP_E5M2, EPI_PLAIN>(x, gamma, eps, codes, scales, N, K, y, st);
}


int launch_gemv_swiglu(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                       int format, uint16_t *y, hipStream_t st) {
    return format == RENG_HIP_E4M3
               ? launch_gemv_epi_t<RENG_HIP_E4M3, EPI_SWIGLU>(x, codes, scales, N, K, y, nullptr, nullptr, nullptr,
                                                              0.0f, st)
               : launch_gemv_epi_t<RENG_HIP_E5M2, EPI_SWIGLU>(x, codes, scales, N, K, y, nullptr, nullptr, nullptr,
                                                              0.0f, st);
}

// gemv_rows' launch: one wave per row, 4-wave blocks for rows of up to 8 KB
// when there are more than 16 rows per CU, else 8-wave blocks (fewer copies
// of a long activation per CU): [14336, 4096] 10.12 us with 4-wave blocks
// against 10.25 with 8, [4096, 4096] 4.54 against 4.46.
template <int F, int CPR, int EPI, int MR>
int launch_gemv_rows_c(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                       uint16_t *y, const float *res, float *yres, hipStream_t st) {
    if constexpr (CPR <= 8) {
        if (N > (uint32_t)device_props().cus * 16) {
            hipLaunchKernelGGL((gemv_rows<F, CPR, 4, EPI, MR>), dim3((N + 3) / 4), dim3(256), 0, st, x, codes, scales,
                               N, K, y, res, yres);
            return check_launch(EPI == EPI_RESID ? "gemv_rows (residual)" : "gemv_rows");
        }
    }
    hipLaunchKernelGGL((gemv_rows<F, CPR, 8, EPI, MR>), dim3((N + 7) / 8), dim3(512), 0, st, x, codes, scales, N, K,
                       y, res, yres);
    return check_launch(EPI == EPI_RESID ? "gemv_rows (residual)" : "gemv_rows");
}

// Rows of 2..32 KB (1024 < K <= 32768: the activation's LDS copy is at most
// 64 KB); the caller sends the rest to gemv_w8a16. Past 16 chunks the load
// window is what keeps the rows in order: M = 1 [5120, 27648] 27.9 -> 23.1-23.3
// us, [3584, 18944] 13.6 -> 12.0 us against the strided walk (a plain read of
// the codes 20.7 / 10.8 us).
template <int F, int EPI = EPI_PLAIN, int MR = 1>
int launch_gemv_rows(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                     uint16_t *y, hipStream_t st, const float *res = nullptr, float *yres = nullptr) {
    switch ((K + 1023) / 1024) {
#define RENG_ROWS(C)                                                                          \
    case C:                                                                                   \
        if constexpr (MR * C <= 32) return launch_gemv_rows_c<F, C, EPI, MR>(x, codes, scales, N, K, y, res, yres, st); \
        break;
        RENG_ROWS(2) RENG_ROWS(3) RENG_ROWS(4) RENG_ROWS(5) RENG_ROWS(6) RENG_ROWS(7) RENG_ROWS(8) RENG_ROWS(9)
        RENG_ROWS(10) RENG_ROWS(11) RENG_ROWS(12) RENG_ROWS(13) RENG_ROWS(14) RENG_ROWS(15) RENG_ROWS(16)
        RENG_ROWS(17) RENG_ROWS(18) RENG_ROWS(19) RENG_ROWS(20) RENG_ROWS(21) RENG_ROWS(22) RENG_ROWS(23)
        RENG_ROWS(24) RENG_ROWS(25) RENG_ROWS(26) RENG_ROWS(27) RENG_ROWS(28) RENG_ROWS(29) RENG_ROWS(30)
        RENG_ROWS(31) RENG_ROWS(32)
#undef RENG_ROWS
        default:
            break;
    }
    set_error("gemv_rows: K = %u outside 1025..%u for %d activation rows", K, 32768u / MR, MR);
    return RENG_HIP_EINVAL;
}

int launch_gemv_residual(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                         int format, const float *res, float *y, hipStream_t st) {
    // Rows of 2..32 KB on gemv_rows (the decode step's o and down projections:
    // [4096, 4096] 5.07 -> 4.5 us, [4096, 14336] 11.6 -> 10.4 us on the same
    // row sums), the rest on the strided walk.
    if (K > 1024 && K <= 32768)
        return format == RENG_HIP_E4M3
                   ? launch_gemv_rows<RENG_HIP_E4M3, EPI_RESID>(x, codes, scales, N, K, nullptr, st, res, y)
                   : launch_gemv_rows<RENG_HIP_E5M2, EPI_RESID>(x, codes, scales, N, K, nullptr, st, res, y);
    return format == RENG_HIP_E4M3
               ? launch_gemv_epi_t<RENG_HIP_E4M3, EPI_RESID>(x, codes, scales, N, K, nullptr, res, y, nullptr, 0.0f, st)
               : launch_gemv_epi_t<RENG_HIP_E5M2, EPI_RESID>(x, codes, scales, N, K, nullptr, res, y, nullptr, 0.0f, st);
}

template <int F>
int launch_w8a16_t(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                   uint32_t N, uint32_t K, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    // One activation row of 1 to 32 KB: a wave per row, its chunks through a
    // load window; x and codes are 16-byte aligned (checked by the entry point).
    if (M == 1 && K > 1024 && K <= 32768)
        return launch_gemv_rows<F>(x, codes, scales, N, K, y, st);
    // Two rows of 1 to 8 KB: the same kernel with both rows in LDS (Llama
    // [14336, 4096] 12.99 -> 11.56 us, Qwen2.5-7B [18944, 3584] 15.53 -> 12.9 us
    // against the strided walk). Longer rows stay there: at [4096, 14336] the
    // two 28 KB copies hold a CU to two blocks (13.65 against 13.02 us).
    if (M == 2 && K > 1024 && K <= 8192)
        return launch_gemv_rows<F, EPI_PLAIN, 2>(x, codes, scales, N, K, y, st);
    // More than 64 rows: output tiles on the bf16 MFMA, each code tile read
    // once per 64-256 activation rows (the 64-row loop below re-reads every
    // code once per 64 rows: M = 256 [14336, 4096] 86.8 -> 41.6 us).
    if (M > 64 && K % 64 == 0 && w8a16_tiles_take(M, N, K))
        return launch_w8a16_tiles(x, codes, scales, M, N, K, F, y, st, fixed);
    if (M > 4 && K % 128 != 0) {
        // K not a multiple of the 128-code chunk: skinny_wide (its last chunk
        // short, zero-padded in registers) on up to 64 activation rows at a
        // time, each code read once per 64 rows (the GEMV would read it once
        // per 4).
        for (uint32_t mb = 0; mb < M; mb += 64) {
            const uint32_t mt = M - mb < 64 ? M - mb : 64;
            const int rc = launch_skinny_wide(x + (size_t)mb * K, codes, scales, mt, N, K, F, y + (size_t)mb * N, st,
                                              fixed);
            if (rc) return rc;
        }
        return RENG_HIP_OK;
    }
    // Three or four rows, or two once the activation outgrows the GEMV's LDS
    // copy: the MFMA kernel (activation rows padded to 8) is faster than the
    // GEMV's per-row dot products (Qwen2.5-7B [3584, 18944]: M = 3 26.3 ->
    // 16.6 us, M = 2 22.5 -> 16.6 us; M = 2 with K <= 8192 takes gemv_rows
    // above, and up to 16384 the strided GEMV below).
    if (M >= 2 && M <= 4 && K % 128 == 0 && (M >= 3 || (size_t)M * K * 2 > 64 * 1024))
        return launch_skinny_mfma(x, codes, scales, M, N, K, F, y, st, fixed);
    if (M <= 4) {
        const GemvPlan p = gemv_plan(M, N, K, 1);
        const uint32_t blocks = p.blocks;
        const int threads = GemvPlan::threads;
        const size_t lds = p.lds;
        const bool xlds = p.xlds, cpl7 = p.cpl7, ragged = p.ragged;
#define RENG_GEMV(MM, C, XL, RG)                                                                   \
    hipLaunchKernelGGL((gemv_w8a16<F, MM, C, XL, RG>), dim3(blocks), dim3(threads), lds, st, x, codes, \
                       scales, N, K, y, nullptr, nullptr, nullptr, 0.0f, RopeOut{})
#define RENG_GEMV_X(MM, C, RG) \
    if (xlds) RENG_GEMV(MM, C, true, RG); else RENG_GEMV(MM, C, false, RG);
#define RENG_GEMV_M(MM)                                  \
    if (cpl7) { RENG_GEMV_X(MM, 7, false) }              \
    else if (ragged) { RENG_GEMV_X(MM, 4, true) }        \
    else { RENG_GEMV_X(MM, 4, false) }
        switch (M) {
            case 1: RENG_GEMV_M(1); break;
            case 2: RENG_GEMV_M(2); break;
            case 3: RENG_GEMV_M(3); break;
            default: RENG_GEMV_M(4); break;
        }
#undef RENG_GEMV_M
#undef RENG_GEMV_X
#undef RENG_GEMV
        return check_launch("gemv_w8a16");
    }
    // Larger M: tiles of up to 64 activation rows on the MFMA kernels.
    for (uint32_t mb = 0; mb < M; mb += 64) {
        const uint32_t mt = M - mb < 64 ? M - mb : 64;
        const int rc = mt <= 16 ? launch_skinny_mfma(x + (size_t)mb * K, codes, scales, mt, N, K, F, y + (size_t)mb * N, st,
                                                     fixed)
                                : launch_skinny_wide(x + (size_t)mb * K, codes, scales, mt, N, K, F, y + (size_t)mb * N, st,
                                                     fixed);
        if (rc) return rc;
    }
    return RENG_HIP_OK;
}

int launch_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                 uint32_t N, uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed) {
    return format == RENG_HIP_E4M3 ? launch_w8a16_t<RENG_HIP_E4M3>(x, codes, scales, M, N, K, y, st, fixed)
                                   : launch_w8a16_t<RENG_HIP_E5M2>(x, codes, scales, M, N, K, y, st, fixed);
}

}  // namespace reng
