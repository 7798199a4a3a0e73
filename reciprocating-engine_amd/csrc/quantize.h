// quantize.h - internal interface between the C-ABI layer and the quantizer
// kernels (not installed; the public contract is include/reng_hip.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reng {

// Matrices per launch: their descriptors travel by value in the kernel
// arguments, so a batch needs no device-side table and no allocation.
constexpr int QBATCH = 32;

struct QMat {
    const void *w;
    uint8_t *codes;
    float *scales;
    uint32_t *exp_bias;
    uint64_t cols, ld;
    uint64_t row_begin;   // first row of this matrix in the batch's row space
};

struct QBatch {
    QMat m[QBATCH];
    int n;
    uint64_t total_rows;
};

int fast_key(const QMat &m, int dtype);
int launch_quantize_group(const QBatch &b, int dtype, int format, int scheme, float backoff,
                          int key, hipStream_t st);
int launch_row_absmax(const QBatch &b, int dtype, float *out, hipStream_t st);
// The stream yardstick: elems bf16 in, their high bytes out (elems % 8 == 0).
int launch_stream_narrow(const void *src, uint64_t elems, void *dst, hipStream_t st);

}  // namespace reng
