// staging.h - reng_hip_quantize_host's host -> device -> host pipeline (staging.hip).
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace reng {

// Quantizes a host matrix through pinned staging slots; the arguments are
// already checked. Returns a RENG_HIP_* code (the error text set on failure).
int quantize_host_staged(const void *w, int dtype, size_t rows, size_t cols, int format, int scaling, float backoff,
                         uint8_t *codes, float *scales, uint32_t *exp_bias);

}  // namespace reng
