// gemm.h - internal interface to the GEMV / GEMM kernels (the public contract
// is include/reng_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reng {

int launch_w8a16(const uint16_t *x, const uint8_t *codes, const float *scales, uint32_t M,
                 uint32_t N, uint32_t K, int format, uint16_t *y, hipStream_t st);
int launch_fp8_gemm(const uint8_t *a, int fa, const float *sa, uint32_t nsa, const uint8_t *b,
                    int fb, const float *sb, uint32_t nsb, uint32_t M, uint32_t N, uint32_t K,
                    uint16_t *out, hipStream_t st);

// Grow-only f32 scratch for k-split partial sums, one per (device, stream):
// calls on one stream are ordered and share it. Sets *rc and returns null on
// failure.
float *split_workspace(size_t floats, hipStream_t st, int *rc);

}  // namespace reng
