// codec.h - internal interface to the elementwise fp8 kernels (the public
// contract is include/reng_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reng {

int launch_encode(const float *x, uint64_t n, int format, uint8_t *out, hipStream_t st);
int launch_decode(const uint8_t *c, uint64_t n, int format, float *out, hipStream_t st);
int launch_dequantize(const uint8_t *c, const float *scales, uint64_t rows, uint64_t cols,
                      int format, bool bf16, void *out, hipStream_t st);
int launch_row_errors(const uint16_t *w, const uint8_t *c, const float *scales, uint64_t cols,
                      uint64_t step, uint64_t nsampled, int format, float *mean_rel,
                      float *max_rel, hipStream_t st);
int run_verify_hw(int format, unsigned long long *d_count, uint32_t *d_first, hipStream_t st);

}  // namespace reng
