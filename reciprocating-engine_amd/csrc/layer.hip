// layer.hip - the steps of one Llama decoder layer at decode time (one token
// per call) around its seven fp8 GEMVs (csrc/gemm.hip), on device buffers:
//
//   n  = bf16(rms_norm(x, g1))                       reng_hip_rms_norm_bf16
//   q, k, v = n W{q,k,v}^T                           (fp8 GEMV)
//   rotate-half RoPE of q and k at position p; k, v
//   appended to the layer's bf16 cache as row p      reng_hip_rope_append
//   a  = softmax(scale q K^T) V over rows 0..p       reng_hip_attention_decode(_split)
//   h  = x + a Wo^T; n2 = bf16(rms_norm(h, g2))     (fp8 GEMV), reng_hip_add_rms_norm_bf16
//   g, u = n2 W{g,u}^T                               (fp8 GEMV)
//   y  = h + (silu(g) * u) Wd^T                      reng_hip_silu_mul_bf16, (fp8 GEMV), add
//
// The semantics are the reference's CPU decoder layer, causal, in its Llama
// form (pre-norm, SiLU gate, GQA, rotate-half RoPE): layer_cpu,
// crates/reng-synapse/src/model.rs:2903-3100, with rms_norm_cpu
// (crates/reng-synapse/src/ops.rs:49-72) and rope_cpu (ops.rs:118-135). The
// residual stream is f32; what feeds a GEMV is bf16 (the w8a16 contract).
// These are latency-bound per token (a few KB each); only the GEMVs stream
// HBM.
#include "common.h"

namespace reng {

namespace layer {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_bf16(float v) { return (uint16_t)f32_to_bf16_bits(v); }

// Sum over the block (blockDim.x a multiple of 64, at most 1024), returned to
// every thread.
__device__ __forceinline__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_sum_dpp(v);
    __syncthreads();   // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int w = 0; w < waves; ++w) s += red[w];
    return s;
}

__device__ __forceinline__ float block_max(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
    for (int w = 1; w < waves; ++w) m = fmaxf(m, red[w]);
    return m;
}

// out[r, c] = bf16(h[r, c] * inv_r * g[c]), inv_r = 1 / sqrt(mean_c h[r, c]^2 +
// eps) (rms_norm_cpu, ops.rs:49-72), h = x, or with ADD h = x + d (d a bf16
// branch output), which is also written out. One 1024-thread workgroup per
// row (row_inv_rms); VEC moves four columns per thread and access (cols % 4
// == 0, aligned rows), so a row of up to 4096 columns is one load per thread.
template <bool VEC, bool ADD>
__global__ __launch_bounds__(NORM_VT) void rms_norm_rows(const float *__restrict__ x,
                                                         const uint16_t *__restrict__ d,
                                                         const float *__restrict__ g, uint32_t cols, float eps,
                                                         float *__restrict__ h, uint16_t *__restrict__ out) {
    __shared__ float red[NORM_VT / 64];
    const size_t base = (size_t)blockIdx.x * cols;
    const float *xr = x + base;
    float *hr = ADD ? h + base : nullptr;
    uint16_t *orow = out + base;
    const float inv = row_inv_rms<VEC, ADD, 1>(xr, ADD ? d + base : nullptr, hr, cols, eps, red);
    // The second pass reads back what this thread read (or wrote) in the first.
    const float *src = ADD ? hr : xr;
    if constexpr (VEC) {
        for (uint32_t c = threadIdx.x * 4; c < cols; c += NORM_VT * 4) {
            const float4 v = *reinterpret_cast<const float4 *>(src + c);
            const float4 gv = *reinterpret_cast<const float4 *>(g + c);
            const uint32_t lo = f32_bf16(v.x * inv * gv.x) | ((uint32_t)f32_bf16(v.y * inv * gv.y) << 16);
            const uint32_t hi = f32_bf16(v.z * inv * gv.z) | ((uint32_t)f32_bf16(v.w * inv * gv.w) << 16);
            *reinterpret_cast<u32x2 *>(orow + c) = u32x2{lo, hi};
        }
    } else {
        for (uint32_t c = threadIdx.x; c < cols; c += NORM_VT) orow[c] = f32_bf16(src[c] * inv * g[c]);
    }
}

// Rotate-half RoPE of one position (rope_cpu, ops.rs:118-135): for d < half,
// o[d] = x[d] cos[d] - x[d + half] sin[d] and o[d + half] = x[d + half]
// cos[d + half] + x[d] sin[d + half]. Blocks 0 .. nh - 1 rotate the q heads
// in place; blocks nh .. nh + nkv - 1 rotate k head g into k_row and copy v
// head g into v_row (the cache rows of this position).
__global__ __launch_bounds__(64) void rope_append(uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
                                                  const uint16_t *__restrict__ v, uint32_t nh, uint32_t hd,
                                                  const float *__restrict__ sn, const float *__restrict__ cs,
                                                  uint16_t *__restrict__ k_row, uint16_t *__restrict__ v_row) {
    const uint32_t b = blockIdx.x, half = hd / 2;
    const uint16_t *src;
    uint16_t *dst;
    if (b < nh) {
        src = q + (size_t)b * hd;
        dst = q + (size_t)b * hd;
    } else {
        const uint32_t g = b - nh;
        src = k + (size_t)g * hd;
        dst = k_row + (size_t)g * hd;
        for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) v_row[(size_t)g * hd + d] = v[(size_t)g * hd + d];
    }
    for (uint32_t d = threadIdx.x; d < half; d += blockDim.x) {
        const float x0 = bf16_f32(src[d]), x1 = bf16_f32(src[d + half]);
        float o0, o1;
        rope_rotate(x0, x1, cs[d], sn[d], cs[d + half], sn[d + half], o0, o1);
        dst[d] = f32_bf16(o0);
        dst[d + half] = f32_bf16(o1);
    }
}

// ---------------------------------------------------------------- attention
//
// One query row per head against cache rows 0 .. len - 1 (the causal row of
// layer_cpu's attention, model.rs:3010-3050): s_j = scale * q_h . k_j[g],
// p = softmax(s), out_h = sum_j p_j v_j[g], with g = h / (nh / nkv).
//
// The cache is cut into S splits of `chunk` rows; workgroup (s, y) reads the
// key and value rows of split s once for gb query heads that share
// key/value head g (gb divides nh / nkv, at most ATT_GMAX), 256 rows at a time
// with an online softmax. Per tile: the first ATT_VPF value rows of each
// thread, the keys and the thread's slice of q are requested together (one
// memory round trip); phase 1 forms the scores (16 lanes per key row, bf16
// pairs into v_dot2_f32_bf16, 16-byte loads when head_dim % 8 == 0) into LDS;
// the tile's max and sum update the running (m, l) per head; phase 2
// accumulates exp(s_j - m) v_j in registers (a thread per value dimension pair
// and row phase, so a wave's load is whole rows). With S = 1 the workgroup
// writes bf16(o / l); otherwise the unnormalised o and (m, l) of its split go
// to the workspace and attention_combine merges the splits.
constexpr int ATT_NW = 16, ATT_THREADS = 64 * ATT_NW, ATT_TILE = 16 * ATT_NW, ATT_GMAX = 4;
constexpr int ATT_SPLIT_MAX = 64, ATT_SPLIT_ROWS = 256, ATT_ONE_PASS_MAX = 512;
constexpr int ATT_VPF = 16;   // value rows per thread requested with the tile's keys

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), acc,
                                           false);
}

struct AttnPlan {
    uint32_t splits, chunk;
};

// One pass (S = 1) for caches of up to 512 rows or without a workspace; else
// S = min(64, ceil(len / 256)) splits of equal length (the last one shorter),
// none empty.
inline AttnPlan attn_plan(size_t len, bool split) {
    if (!split || len <= (size_t)ATT_ONE_PASS_MAX) return {1u, (uint32_t)len};
    size_t s = (len + ATT_SPLIT_ROWS - 1) / ATT_SPLIT_ROWS;
    if (s > (size_t)ATT_SPLIT_MAX) s = ATT_SPLIT_MAX;
    const size_t chunk = (len + s - 1) / s;
    return {(uint32_t)((len + chunk - 1) / chunk), (uint32_t)chunk};
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Sum over each 16-lane row, left in the row's lane 15.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_mov<0x111, 0xf>(v);   // row_shr:1
    v += dpp_mov<0x112, 0xf>(v);   // row_shr:2
    v += dpp_mov<0x114, 0xf>(v);   // row_shr:4
    v += dpp_mov<0x118, 0xf>(v);   // row_shr:8
    return v;
}

template <bool V8>
__global__ __launch_bounds__(ATT_THREADS) void attention_split(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, uint32_t nh,
    uint32_t nkv, uint32_t hd, uint32_t len, uint32_t chunk, uint32_t gb, float scale, float *__restrict__ part,
    uint16_t *__restrict__ out) {
    extern __shared__ float op[];   // [nph][gb][hd]: the row phases' o, summed at the end
    __shared__ float sc[ATT_GMAX][ATT_TILE];
    __shared__ float mrun[ATT_GMAX], lrun[ATT_GMAX], corr[ATT_GMAX];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t per_kv = nh / nkv, s = blockIdx.x;
    // One head per workgroup: y walks the key/value heads fastest, so the query
    // heads of one key/value head sit gridDim.x * nkv blocks apart (on one XCD
    // when that is a multiple of 8) and share its rows in L2.
    const uint32_t h0 = gb == 1 ? (blockIdx.y % nkv) * per_kv + blockIdx.y / nkv : blockIdx.y * gb;
    const uint32_t g = h0 / per_kv;
    const size_t pitch = (size_t)nkv * hd;
    const uint32_t j0 = s * chunk, j1 = min(len, j0 + chunk);
    const uint16_t *kbase = kc + (size_t)g * hd, *vbase = vc + (size_t)g * hd, *qbase = q + (size_t)h0 * hd;
    if (tid < ATT_GMAX) {
        mrun[tid] = -INFINITY;
        lrun[tid] = 0.0f;
    }
    // Phase 2: dimension pair dp of the tile rows ph, ph + nph, ...
    const uint32_t npairs = hd / 2, dpb = npairs < ATT_THREADS ? npairs : ATT_THREADS, nph = ATT_THREADS / dpb;
    const uint32_t ph = tid / dpb, dp = tid % dpb;
    const bool active = ph < nph;
    float o[ATT_GMAX][2];
#pragma unroll
    for (int h = 0; h < ATT_GMAX; ++h) o[h][0] = o[h][1] = 0.0f;
    __syncthreads();

    const uint32_t l16 = lane & 15, rg = lane >> 4;
    for (uint32_t t0 = j0; t0 < j1; t0 += ATT_TILE) {
        const uint32_t n = min((uint32_t)ATT_TILE, j1 - t0);
        uint32_t vpf[ATT_VPF];
#pragma unroll
        for (int i = 0; i < ATT_VPF; ++i) {
            const uint32_t jj = ph + i * nph;
            vpf[i] = active && jj < n
                         ? *reinterpret_cast<const uint32_t *>(vbase + (size_t)(t0 + jj) * pitch + 2 * dp)
                         : 0u;
        }
        // Phase 1: rows wave * 16 + it * 4 + rg of the tile.
        float acc[4][ATT_GMAX];
#pragma unroll
        for (int it = 0; it < 4; ++it)
#pragma unroll
            for (int h = 0; h < ATT_GMAX; ++h) acc[it][h] = 0.0f;
        if constexpr (V8) {
            const uint32_t npc = hd / 8;
            for (uint32_t pc = l16; pc < npc; pc += 16) {
                uint4 kv[4], qv[ATT_GMAX];
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const uint32_t jj = wave * 16 + it * 4 + rg;
                    kv[it] = jj < n ? *reinterpret_cast<const uint4 *>(kbase + (size_t)(t0 + jj) * pitch + 8 * pc)
                                    : uint4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int h = 0; h < ATT_GMAX; ++h)
                    qv[h] = h < (int)gb ? *reinterpret_cast<const uint4 *>(qbase + (size_t)h * hd + 8 * pc)
                                        : uint4{0u, 0u, 0u, 0u};
#pragma unroll
                for (int h = 0; h < ATT_GMAX; ++h) {
                    if (h >= (int)gb) break;
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        float a = acc[it][h];
                        a = dot2_bf16(qv[h].x, kv[it].x, a);
                        a = dot2_bf16(qv[h].y, kv[it].y, a);
                        a = dot2_bf16(qv[h].z, kv[it].z, a);
                        a = dot2_bf16(qv[h].w, kv[it].w, a);
                        acc[it][h] = a;
                    }
                }
            }
        } else {
            const uint32_t npc = hd / 2;
            for (uint32_t pc = l16; pc < npc; pc += 16) {
                uint32_t kv[4], qv[ATT_GMAX];
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const uint32_t jj = wave * 16 + it * 4 + rg;
                    kv[it] = jj < n ? *reinterpret_cast<const uint32_t *>(kbase + (size_t)(t0 + jj) * pitch + 2 * pc)
                                    : 0u;
                }
#pragma unroll
                for (int h = 0; h < ATT_GMAX; ++h)
                    qv[h] = h < (int)gb ? *reinterpret_cast<const uint32_t *>(qbase + (size_t)h * hd + 2 * pc) : 0u;
#pragma unroll
                for (int h = 0; h < ATT_GMAX; ++h) {
                    if (h >= (int)gb) break;
#pragma unroll
                    for (int it = 0; it < 4; ++it) acc[it][h] = dot2_bf16(qv[h], kv[it], acc[it][h]);
                }
            }
        }
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint32_t jj = wave * 16 + it * 4 + rg;
#pragma unroll
            for (int h = 0; h < ATT_GMAX; ++h) {
                if (h >= (int)gb) break;
                const float v = row16_sum(acc[it][h]);
                if (l16 == 15) sc[h][jj] = jj < n ? v * scale : -INFINITY;
            }
        }
        __syncthreads();
        // Running max and sum: wave h owns head h.
        if (wave < gb) {
            const uint32_t h = wave;
            float v[ATT_TILE / 64];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < ATT_TILE / 64; ++i) {
                v[i] = sc[h][lane + 64 * i];
                mx = fmaxf(mx, v[i]);
            }
            const float mo = mrun[h], mn = fmaxf(mo, wave_max_f32(mx));
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < ATT_TILE / 64; ++i) {
                const float p = lane + 64 * i < n ? expf(v[i] - mn) : 0.0f;
                sc[h][lane + 64 * i] = p;
                ps += p;
            }
            ps = wave_sum_dpp(ps);
            if (lane == 0) {
                const float c = expf(mo - mn);   // 0 on the first tile (mo = -inf)
                corr[h] = c;
                lrun[h] = lrun[h] * c + ps;
                mrun[h] = mn;
            }
        }
        __syncthreads();
        // Phase 2.
        if (active) {
#pragma unroll
            for (int h = 0; h < ATT_GMAX; ++h) {
                if (h >= (int)gb) break;
                const float c = corr[h];
                o[h][0] *= c;
                o[h][1] *= c;
            }
            auto accumulate = [&](uint32_t jj, uint32_t w) {
                const float a0 = __uint_as_float(w << 16), a1 = __uint_as_float(w & 0xffff0000u);
#pragma unroll
                for (int h = 0; h < ATT_GMAX; ++h) {
                    if (h >= (int)gb) break;
                    const float p = sc[h][jj];
                    o[h][0] += p * a0;
                    o[h][1] += p * a1;
                }
            };
#pragma unroll
            for (int i = 0; i < ATT_VPF; ++i) {
                const uint32_t jj = ph + i * nph;
                if (jj < n) accumulate(jj, vpf[i]);
            }
            for (uint32_t jj = ph + ATT_VPF * nph; jj < n; jj += nph)
                accumulate(jj, *reinterpret_cast<const uint32_t *>(vbase + (size_t)(t0 + jj) * pitch + 2 * dp));
        }
        __syncthreads();
    }
    // Sum the row phases' o.
    if (active) {
#pragma unroll
        for (int h = 0; h < ATT_GMAX; ++h) {
            if (h >= (int)gb) break;
            op[((size_t)ph * gb + h) * hd + 2 * dp] = o[h][0];
            op[((size_t)ph * gb + h) * hd + 2 * dp + 1] = o[h][1];
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < gb * hd; i += ATT_THREADS) {
        const uint32_t h = i / hd;
        float v = 0.0f;
        for (uint32_t r = 0; r < nph; ++r) v += op[(size_t)r * gb * hd + i];
        if (part == nullptr) {
            out[(size_t)h0 * hd + i] = f32_bf16(v / lrun[h]);
        } else {
            part[((size_t)s * nh + h0) * hd + i] = v;
        }
    }
    if (part != nullptr && tid < gb) {
        float *ml = part + (size_t)gridDim.x * nh * hd;
        ml[((size_t)s * nh + h0 + tid) * 2] = mrun[tid];
        ml[((size_t)s * nh + h0 + tid) * 2 + 1] = lrun[tid];
    }
}

// attention_split for head_dim % 8 == 0, head_dim <= 128 and 16-byte aligned
// q, caches: a lane holds eight dimensions (one 16-byte piece) of a key row
// and of the same value row, 16 lanes a row, so phase 2 accumulates the rows
// phase 1 scored, from registers, eight dimensions per lane; the lanes of one
// piece are summed across the wave (xor 16, 32) and across the waves in LDS.
__global__ __launch_bounds__(ATT_THREADS) void attention_split16(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ kc, const uint16_t *__restrict__ vc, uint32_t nh,
    uint32_t nkv, uint32_t hd, uint32_t len, uint32_t chunk, uint32_t gb, float scale, float *__restrict__ part,
    uint16_t *__restrict__ out) {
    __shared__ float op[ATT_NW][ATT_GMAX][128];
    __shared__ float sc[ATT_GMAX][ATT_TILE];
    __shared__ float mrun[ATT_GMAX], lrun[ATT_GMAX], corr[ATT_GMAX];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t per_kv = nh / nkv, s = blockIdx.x;
    const uint32_t h0 = gb == 1 ? (blockIdx.y % nkv) * per_kv + blockIdx.y / nkv : blockIdx.y * gb;
    const uint32_t g = h0 / per_kv;
    const size_t pitch = (size_t)nkv * hd;
    const uint32_t j0 = s * chunk, j1 = min(len, j0 + chunk);
    const uint32_t l16 = lane & 15, rg = lane >> 4, npc = hd / 8;
    const bool piece = l16 < npc;   // lanes past the row's pieces load nothing
    const uint16_t *kbase = kc + (size_t)g * hd + 8 * l16, *vbase = vc + (size_t)g * hd + 8 * l16;
    uint4 qv[ATT_GMAX];
#pragma unroll
    for (int h = 0; h < ATT_GMAX; ++h)
        qv[h] = piece && h < (int)gb ? *reinterpret_cast<const uint4 *>(q + (size_t)(h0 + h) * hd + 8 * l16)
                                     : uint4{0u, 0u, 0u, 0u};
    if (tid < ATT_GMAX) {
        mrun[tid] = -INFINITY;
        lrun[tid] = 0.0f;
    }
    float o[ATT_GMAX][8];
#pragma unroll
    for (int h = 0; h < ATT_GMAX; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.0f;
    __syncthreads();

    for (uint32_t t0 = j0; t0 < j1; t0 += ATT_TILE) {
        const uint32_t n = min((uint32_t)ATT_TILE, j1 - t0);
        uint4 kv[4], vv[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint32_t jj = wave * 16 + it * 4 + rg;
            const bool ok = piece && jj < n;
            const size_t off = (size_t)(t0 + jj) * pitch;
            kv[it] = ok ? *reinterpret_cast<const uint4 *>(kbase + off) : uint4{0u, 0u, 0u, 0u};
            vv[it] = ok ? *reinterpret_cast<const uint4 *>(vbase + off) : uint4{0u, 0u, 0u, 0u};
        }
        // Phase 1: scores of rows wave * 16 + it * 4 + rg.
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint32_t jj = wave * 16 + it * 4 + rg;
#pragma unroll
            for (int h = 0; h < ATT_GMAX; ++h) {
                if (h >= (int)gb) break;
                float a = dot2_bf16(qv[h].x, kv[it].x, 0.0f);
                a = dot2_bf16(qv[h].y, kv[it].y, a);
                a = dot2_bf16(qv[h].z, kv[it].z, a);
                a = dot2_bf16(qv[h].w, kv[it].w, a);
                a = row16_sum(a);
                if (l16 == 15) sc[h][jj] = jj < n ? a * scale : -INFINITY;
            }
        }
        __syncthreads();
        if (wave < gb) {
            const uint32_t h = wave;
            float v[ATT_TILE / 64];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < ATT_TILE / 64; ++i) {
                v[i] = sc[h][lane + 64 * i];
                mx = fmaxf(mx, v[i]);
            }
            const float mo = mrun[h], mn = fmaxf(mo, wave_max_f32(mx));
            float ps = 0.0f;
#pragma unroll
            for (int i = 0; i < ATT_TILE / 64; ++i) {
                const float p = lane + 64 * i < n ? expf(v[i] - mn) : 0.0f;
                sc[h][lane + 64 * i] = p;
                ps += p;
            }
            ps = wave_sum_dpp(ps);
            if (lane == 0) {
                const float c = expf(mo - mn);   // 0 on the first tile (mo = -inf)
                corr[h] = c;
                lrun[h] = lrun[h] * c + ps;
                mrun[h] = mn;
            }
        }
        __syncthreads();
        // Phase 2: the same rows' values, eight dimensions per lane.
#pragma unroll
        for (int h = 0; h < ATT_GMAX; ++h) {
            if (h >= (int)gb) break;
            const float c = corr[h];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[h][e] *= c;
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const float p = sc[h][wave * 16 + it * 4 + rg];   // 0 past n
                const uint4 w = vv[it];
                o[h][0] += p * __uint_as_float(w.x << 16);
                o[h][1] += p * __uint_as_float(w.x & 0xffff0000u);
                o[h][2] += p * __uint_as_float(w.y << 16);
                o[h][3] += p * __uint_as_float(w.y & 0xffff0000u);
                o[h][4] += p * __uint_as_float(w.z << 16);
                o[h][5] += p * __uint_as_float(w.z & 0xffff0000u);
                o[h][6] += p * __uint_as_float(w.w << 16);
                o[h][7] += p * __uint_as_float(w.w & 0xffff0000u);
            }
        }
        __syncthreads();
    }
    // The four row groups of a wave, then the waves.
#pragma unroll
    for (int h = 0; h < ATT_GMAX; ++h) {
        if (h >= (int)gb) break;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = o[h][e];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (rg == 0 && piece) op[wave][h][8 * l16 + e] = v;
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < gb * hd; i += ATT_THREADS) {
        const uint32_t h = i / hd, d = i % hd;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < ATT_NW; ++w) v += op[w][h][d];
        if (part == nullptr) {
            out[(size_t)h0 * hd + i] = f32_bf16(v / lrun[h]);
        } else {
            part[((size_t)s * nh + h0) * hd + i] = v;
        }
    }
    if (part != nullptr && tid < gb) {
        float *ml = part + (size_t)gridDim.x * nh * hd;
        ml[((size_t)s * nh + h0 + tid) * 2] = mrun[tid];
        ml[((size_t)s * nh + h0 + tid) * 2 + 1] = lrun[tid];
    }
}

// out_h = sum_s w_s o_s / sum_s w_s l_s with w_s = exp(m_s - max_s m_s): the
// splits of attention_split merged. One 256-thread workgroup per head. Thread
// t requests split t's (m, l) and dimension t of every split's o together,
// before the first barrier, so the merge costs one memory round trip (the o
// values do not depend on the weights); dimensions past 256 are read after.
constexpr int COMBINE_THREADS = 256;
__global__ __launch_bounds__(COMBINE_THREADS) void attention_combine(const float *__restrict__ part, uint32_t nh,
                                                                     uint32_t hd, uint32_t splits,
                                                                     uint16_t *__restrict__ out) {
    __shared__ float wsp[ATT_SPLIT_MAX];
    __shared__ float red[COMBINE_THREADS / 64];
    const uint32_t h = blockIdx.x, tid = threadIdx.x;
    const float *ml = part + (size_t)splits * nh * hd;
    const float m = tid < splits ? ml[((size_t)tid * nh + h) * 2] : -INFINITY;
    const float l = tid < splits ? ml[((size_t)tid * nh + h) * 2 + 1] : 0.0f;
    const bool first = tid < hd;
    float pv[ATT_SPLIT_MAX];
#pragma unroll
    for (int i = 0; i < ATT_SPLIT_MAX; ++i)
        pv[i] = first && (uint32_t)i < splits ? part[((size_t)i * nh + h) * hd + tid] : 0.0f;
    const float mx = block_max(m, red);
    const float w = tid < splits ? expf(m - mx) : 0.0f;
    const float den = block_sum(tid < splits ? w * l : 0.0f, red);
    if (tid < splits) wsp[tid] = w / den;
    __syncthreads();
    if (first) {
        float v = 0.0f;
#pragma unroll
        for (int i = 0; i < ATT_SPLIT_MAX; ++i)
            if ((uint32_t)i < splits) v += wsp[i] * pv[i];
        out[(size_t)h * hd + tid] = f32_bf16(v);
    }
    for (uint32_t d = tid + COMBINE_THREADS; d < hd; d += COMBINE_THREADS) {
        float v = 0.0f;
#pragma unroll 16
        for (uint32_t i = 0; i < splits; ++i) v += wsp[i] * part[((size_t)i * nh + h) * hd + d];
        out[(size_t)h * hd + d] = f32_bf16(v);
    }
}

// out = bf16(silu(g) * u), silu(g) = g / (1 + exp(-g)) (layer_cpu's act,
// model.rs:3070-3080).
__global__ void silu_mul_bf16(const uint16_t *__restrict__ gate, const uint16_t *__restrict__ up, size_t n,
                              uint16_t *__restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        const float gv = bf16_f32(gate[i]);
        out[i] = f32_bf16(gv / (1.0f + expf(-gv)) * bf16_f32(up[i]));
    }
}

// out = x + d (f32 residual stream plus a bf16 branch output).
__global__ void add_bf16_f32(const float *__restrict__ x, const uint16_t *__restrict__ d, size_t n,
                             float *__restrict__ out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = x[i] + bf16_f32(d[i]);
}

unsigned grid_for(size_t n, unsigned threads) {
    const size_t cap = (size_t)device_props().cus * 4;
    const size_t b = (n + threads - 1) / threads;
    return (unsigned)(b < 1 ? 1 : b > cap ? cap : b);
}

}  // namespace layer

}  // namespace reng

using namespace reng;
using namespace reng::layer;

namespace {
hipStream_t stream_of(void *s) { return static_cast<hipStream_t>(s); }
}

namespace {

template <bool ADD>
int launch_norm(const float *x, const uint16_t *d, const float *gamma, size_t rows, size_t cols, float eps, float *h,
                uint16_t *out, hipStream_t st) {
    const uintptr_t a16 = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma) |
                          reinterpret_cast<uintptr_t>(h);
    const uintptr_t a8 = reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(out);
    const bool vec = cols % 4 == 0 && (a16 & 15) == 0 && (a8 & 7) == 0;
    if (vec)
        hipLaunchKernelGGL((rms_norm_rows<true, ADD>), dim3((unsigned)rows), dim3(NORM_VT), 0, st, x, d, gamma,
                           (uint32_t)cols, eps, h, out);
    else
        hipLaunchKernelGGL((rms_norm_rows<false, ADD>), dim3((unsigned)rows), dim3(NORM_VT), 0, st, x, d, gamma,
                           (uint32_t)cols, eps, h, out);
    return check_launch("rms_norm_rows");
}

}  // namespace

RENG_HIP_API int reng_hip_rms_norm_bf16(const float *x, const float *gamma, size_t rows, size_t cols, float eps,
                                        uint16_t *out, void *stream) {
    clear_error();
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(rows <= 0x7fffffff && cols <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(x && gamma && out, "null pointer");
    RENG_REQUIRE(eps >= 0.0f, "eps %g is negative", (double)eps);
    return launch_norm<false>(x, nullptr, gamma, rows, cols, eps, nullptr, out, stream_of(stream));
}

RENG_HIP_API int reng_hip_add_rms_norm_bf16(const float *x, const uint16_t *d, const float *gamma, size_t rows,
                                            size_t cols, float eps, float *h, uint16_t *out, void *stream) {
    clear_error();
    RENG_REQUIRE(rows > 0 && cols > 0, "empty shape %zu x %zu", rows, cols);
    RENG_REQUIRE(rows <= 0x7fffffff && cols <= 0x7fffffff, "dimension too large");
    RENG_REQUIRE(x && d && gamma && h && out, "null pointer");
    RENG_REQUIRE(eps >= 0.0f, "eps %g is negative", (double)eps);
    return launch_norm<true>(x, d, gamma, rows, cols, eps, h, out, stream_of(stream));
}

RENG_HIP_API int reng_hip_rope_append(uint16_t *q, const uint16_t *k, const uint16_t *v, size_t n_heads,
                                      size_t n_kv_heads, size_t head_dim, const float *sin_row, const float *cos_row,
                                      uint16_t *k_row, uint16_t *v_row, void *stream) {
    clear_error();
    RENG_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%zu query heads are not a multiple of %zu key/value heads", n_heads, n_kv_heads);
    RENG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim %zu is not even in [2, 1024]",
                 head_dim);
    RENG_REQUIRE(n_heads + n_kv_heads <= 0x7fffffff, "too many heads");
    RENG_REQUIRE(q && k && v && sin_row && cos_row && k_row && v_row, "null pointer");
    hipLaunchKernelGGL(rope_append, dim3((unsigned)(n_heads + n_kv_heads)), dim3(64), 0, stream_of(stream), q, k, v,
                       (uint32_t)n_heads, (uint32_t)head_dim, sin_row, cos_row, k_row, v_row);
    return check_launch("rope_append");
}

namespace {

// The largest divisor of the query heads per key/value head that is at most
// ATT_GMAX: the heads one workgroup serves from one read of the cache; smaller
// while that leaves fewer workgroups than CUs.
uint32_t head_group(size_t per_kv, size_t splits, size_t n_heads) {
    const size_t cus = (size_t)device_props().cus;
    for (size_t g = per_kv < (size_t)ATT_GMAX ? per_kv : (size_t)ATT_GMAX; g > 1; --g)
        if (per_kv % g == 0 && splits * (n_heads / g) >= cus) return (uint32_t)g;
    return 1;
}

size_t split_part_bytes(size_t splits, size_t n_heads, size_t head_dim) {
    return splits < 2 ? 0 : splits * n_heads * (head_dim + 2) * sizeof(float);
}

int attention_args(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache, size_t n_heads,
                   size_t n_kv_heads, size_t head_dim, size_t len, const uint16_t *out) {
    RENG_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                 "%zu query heads are not a multiple of %zu key/value heads", n_heads, n_kv_heads);
    RENG_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 1024, "head_dim %zu is not even in [2, 1024]",
                 head_dim);
    RENG_REQUIRE(len >= 1 && len <= RENG_HIP_ATTENTION_MAX_LEN, "cache length %zu is not in [1, %d]", len,
                 RENG_HIP_ATTENTION_MAX_LEN);
    RENG_REQUIRE(n_heads <= 0x7fffffff, "too many heads");
    RENG_REQUIRE(q && k_cache && v_cache && out, "null pointer");
    RENG_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
                   reinterpret_cast<uintptr_t>(v_cache)) & 3) == 0,
                 "q, k_cache and v_cache must be 4-byte aligned");
    return RENG_HIP_OK;
}

int launch_attention(const uint16_t *q, const uint16_t *kc, const uint16_t *vc, size_t nh, size_t nkv, size_t hd,
                     size_t len, float scale, float *part, uint16_t *out, hipStream_t st) {
    const AttnPlan p = attn_plan(len, part != nullptr);
    const uint32_t gb = p.splits > 1 ? head_group(nh / nkv, p.splits, nh) : 1u;
    const size_t npairs = hd / 2, dpb = npairs < (size_t)ATT_THREADS ? npairs : (size_t)ATT_THREADS;
    const size_t lds = (ATT_THREADS / dpb) * gb * hd * sizeof(float);
    const bool v8 = hd % 8 == 0 && ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(q)) & 15) == 0;
    const bool v16 = v8 && hd <= 128 && (reinterpret_cast<uintptr_t>(vc) & 15) == 0;
    float *wp = p.splits > 1 ? part : nullptr;
    const dim3 grid(p.splits, (unsigned)(nh / gb));
    if (v16)
        hipLaunchKernelGGL(attention_split16, grid, dim3(ATT_THREADS), 0, st, q, kc, vc, (uint32_t)nh, (uint32_t)nkv,
                           (uint32_t)hd, (uint32_t)len, p.chunk, gb, scale, wp, out);
    else if (v8)
        hipLaunchKernelGGL(attention_split<true>, grid, dim3(ATT_THREADS), lds, st, q, kc, vc, (uint32_t)nh,
                           (uint32_t)nkv, (uint32_t)hd, (uint32_t)len, p.chunk, gb, scale, wp, out);
    else
        hipLaunchKernelGGL(attention_split<false>, grid, dim3(ATT_THREADS), lds, st, q, kc, vc, (uint32_t)nh,
                           (uint32_t)nkv, (uint32_t)hd, (uint32_t)len, p.chunk, gb, scale, wp, out);
    if (int rc = check_launch("attention_split")) return rc;
    if (p.splits < 2) return RENG_HIP_OK;
    hipLaunchKernelGGL(attention_combine, dim3((unsigned)nh), dim3(COMBINE_THREADS), 0, st, wp, (uint32_t)nh,
                       (uint32_t)hd, p.splits, out);
    return check_launch("attention_combine");
}

}  // namespace

RENG_HIP_API int reng_hip_attention_decode(const uint16_t *q, const uint16_t *k_cache, const uint16_t *v_cache,
                                           size_t n_heads, size_t n_kv_heads, size_t head_dim, size_t len,
                                           float scale, uint16_t *out, void *stream) {
    clear_error();
    if (int rc = attention_args(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, len, out)) return rc;
    return launch_attention(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, len, scale, nullptr, out,
                            stream_of(stream));
}

RENG_HIP_API size_t reng_hip_attention_workspace_bytes(size_t n_heads, size_t head_dim, size_t len) {
    if (len > RENG_HIP_ATTENTION_MAX_LEN) len = RENG_HIP_ATTENTION_MAX_LEN;
    if (len <= (size_t)ATT_ONE_PASS_MAX || n_heads > 0x7fffffff || head_dim > 1024) return 0;
    size_t s = (len + ATT_SPLIT_ROWS - 1) / ATT_SPLIT_ROWS;
    if (s > (size_t)ATT_SPLIT_MAX) s = ATT_SPLIT_MAX;
    return split_part_bytes(s, n_heads, head_dim);
}

RENG_HIP_API int reng_hip_attention_decode_split(const uint16_t *q, const uint16_t *k_cache,
                                                 const uint16_t *v_cache, size_t n_heads, size_t n_kv_heads,
                                                 size_t head_dim, size_t len, float scale, void *workspace,
                                                 size_t workspace_bytes, uint16_t *out, void *stream) {
    clear_error();
    if (int rc = attention_args(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, len, out)) return rc;
    const size_t need = split_part_bytes(attn_plan(len, true).splits, n_heads, head_dim);
    RENG_REQUIRE(workspace_bytes >= need, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
    RENG_REQUIRE(need == 0 || workspace, "null workspace");
    RENG_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 3) == 0, "workspace must be 4-byte aligned");
    // A cache short enough for one split takes the one-pass form and leaves the workspace alone.
    float *part = need ? static_cast<float *>(workspace) : nullptr;
    return launch_attention(q, k_cache, v_cache, n_heads, n_kv_heads, head_dim, len, scale, part, out,
                            stream_of(stream));
}

RENG_HIP_API int reng_hip_silu_mul_bf16(const uint16_t *gate, const uint16_t *up, size_t n, uint16_t *out,
                                        void *stream) {
    clear_error();
    RENG_REQUIRE(n > 0, "empty vector");
    RENG_REQUIRE(gate && up && out, "null pointer");
    hipLaunchKernelGGL(silu_mul_bf16, dim3(grid_for(n, 256)), dim3(256), 0, stream_of(stream), gate, up, n, out);
    return check_launch("silu_mul_bf16");
}

RENG_HIP_API int reng_hip_add_bf16_f32(const float *x, const uint16_t *d, size_t n, float *out, void *stream) {
    clear_error();
    RENG_REQUIRE(n > 0, "empty vector");
    RENG_REQUIRE(x && d && out, "null pointer");
    hipLaunchKernelGGL(add_bf16_f32, dim3(grid_for(n, 256)), dim3(256), 0, stream_of(stream), x, d, n, out);
    return check_launch("add_bf16_f32");
}
