// gemm.h - internal interface to the GEMV / GEMM kernels (the public contract
// is include/reng_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reng {

// Where a launch keeps its split-K partials: fixed == nullptr takes the
// library's grow-only per-stream buffer (split_workspace, which may allocate);
// otherwise the `floats` floats at ptr, and a plan that needs more is refused.
struct SplitScratch {
    float *ptr;
    size_t floats;
};

int launch_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                 uint32_t N, uint32_t K, int format, uint16_t *y, hipStream_t st,
                 const SplitScratch *fixed = nullptr);
// The per-device address of the library's static split-K scratch array
// (STATIC_SCRATCH_FLOATS floats), looked up once per device; sets *rc.
constexpr size_t STATIC_SCRATCH_FLOATS = (size_t)8 << 20;   // 32 MiB
float *static_split_scratch(int *rc);
// M = 1 with a fused epilogue: f32 y[n] = res[n] + bf16((W x)[n]) (residual), or
// over rows in (gate, up) pairs, y[i] = bf16(silu(bf16 (W x)[2i]) * bf16 (W x)[2i + 1]) (N even).
int launch_gemv_residual(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                         int format, const float *res, float *y, hipStream_t st);
int launch_gemv_swiglu(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t N, uint32_t K,
                       int format, uint16_t *y, hipStream_t st);
// M = 1 with an RMSNorm prologue: the activation is bf16(rms_norm(x) * gamma), x f32 [K], K <= 32768; the
// plain or the SwiGLU-pair epilogue.
int launch_gemv_norm(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                     uint32_t N, uint32_t K, int format, bool swiglu, uint16_t *y, hipStream_t st);
// The RMSNorm prologue over a [q; k; v] projection whose rows come in rotation pairs, with RoPE and the
// cache-row writes as the epilogue (N = (nh + 2 nkv) hd).
int launch_gemv_norm_rope(const float *x, const float *gamma, float eps, const uint8_t *codes, const float *scales,
                          uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t K, int format, const float *sin_row,
                          const float *cos_row, uint16_t *q, uint16_t *k_row, uint16_t *v_row, hipStream_t st);
// 2 <= M <= 16 bf16 activation rows, K % 128 == 0 (csrc/skinny.hip).
int launch_skinny_mfma(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed);
// Up to 64 bf16 activation rows on skinny_wide (16 < M, or K % 128 != 0), K % 16 == 0 (csrc/skinny.hip).
int launch_skinny_wide(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed);
// More than 64 activation rows, K % 64 == 0, on whole output tiles
// (csrc/gemm_tiles.hip). w8a16_tiles_take says whether the tiled kernel takes
// the product (enough tiles for the chip; otherwise the 64-row kernels loop).
bool w8a16_tiles_take(uint32_t M, uint32_t N, uint32_t K);
int launch_w8a16_tiles(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M, uint32_t N,
                       uint32_t K, int format, uint16_t *y, hipStream_t st, const SplitScratch *fixed);
// Zeroed stream-K tile counters (every launch leaves them zeroed): a grow-only
// buffer per (device, stream), or the library's static array
// (STATIC_TILE_COUNTERS of them per device) for callers that cannot allocate.
constexpr uint32_t STATIC_TILE_COUNTERS = 4096;
uint32_t *tile_counters(uint32_t count, hipStream_t st, int *rc);
uint32_t *static_tile_counters(int *rc);
// A grow-only f32 workspace of at least `floats` for split-K partials, one per
// (device, stream) (csrc/gemm.hip); sets *rc. It refuses to grow while the
// stream is being captured into a graph.
float *split_workspace(size_t floats, hipStream_t st, int *rc);
// The partials of a launch: from `fixed` when given (refusing a plan that
// needs more than it holds), else from split_workspace.
float *split_partials(size_t floats, hipStream_t st, const SplitScratch *fixed, int *rc);
// The read yardstick: bytes / 1024 whole 1 KB chunks of p read once; sink
// holds stream_read_sink_words() words (written only by chance).
int launch_stream_read(const void *p, size_t bytes, uint32_t *sink, hipStream_t st);
uint32_t stream_read_sink_words();
// The stage-copy yardstick: skinny_wide's copy stream (16 < M <= 64,
// K % 128 == 0) on its own grid with no arithmetic; sink holds one word.
int launch_stage_copy(const uint16_t *x, const uint8_t *codes, uint32_t M, uint32_t N, uint32_t K, uint32_t *sink,
                      hipStream_t st);
int launch_fp8_gemm(const uint8_t *a, int fa, const float *sa, uint32_t nsa, const uint8_t *b,
                    int fb, const float *sb, uint32_t nsb, uint32_t M, uint32_t N, uint32_t K,
                    uint16_t *out, hipStream_t st);

}  // namespace reng
