// reng_fp8.hpp - the reng-fp8 crate's API (crates/reng-fp8/src/lib.rs) in C++,
// over the reng_hip C ABI (include/reng_hip.h): the same names, the same
// argument meaning, the same refusals. Where the Rust crate panics on an
// assert, these functions throw std::invalid_argument with the same message;
// a device failure throws std::runtime_error carrying the library's message.
// Every numeric result comes from the GPU (libreng_hip.so); the host only
// stages buffers.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace reng_fp8 {

// ------------------------------------------------------------ Fp8Format (lib.rs:53-147)

enum class Fp8Format : int { E4M3 = 0, E5M2 = 1 };

uint32_t mantissa_bits(Fp8Format f);     // 3 | 2
uint32_t exponent_bits(Fp8Format f);     // 4 | 5
uint32_t exponent_bias(Fp8Format f);     // 7 | 15
uint8_t max_finite_code(Fp8Format f);    // 0x77 | 0x7b
float max_finite(Fp8Format f);           // 240 | 57344
uint8_t nan_code(Fp8Format f);           // 0x7f
int32_t syn_data_type(Fp8Format f);      // 8192 | 16384
std::vector<uint32_t> hw_exponent_biases(Fp8Format f);   // {15, 11, 7, 3} | {15}
const char *name(Fp8Format f);           // "e4m3" | "e5m2"
std::optional<Fp8Format> format_from_name(std::string_view s);

// ------------------------------------------------------------ Scaling (lib.rs:240-279)

enum class Scaling : int { PerChannel = 0, HwExpBias = 1, Unit = 2 };

std::optional<Scaling> scaling_from_name(std::string_view s);
const char *name(Scaling s);   // "pcs" | "hw" | "unit"

// ------------------------------------------------------------ scalars (lib.rs:33-48, 154-236)

float bf16_to_f32(uint16_t x);
uint16_t f32_to_bf16(float x);

// encode / decode run on the GPU; the vector forms are the ones to use in bulk.
uint8_t encode(float x, Fp8Format fmt);
float decode(uint8_t code, Fp8Format fmt);
std::vector<uint8_t> encode(const std::vector<float> &x, Fp8Format fmt);
std::vector<float> decode(const std::vector<uint8_t> &codes, Fp8Format fmt);

// ------------------------------------------------------------ Quantized (lib.rs:281-345)

struct Quantized {
    Fp8Format format;
    Scaling scaling;
    size_t rows = 0;
    size_t cols = 0;
    std::vector<uint8_t> codes;   // rows * cols, row-major
    std::vector<float> scales;    // rows
    uint32_t exp_bias = 0;

    size_t code_bytes() const { return codes.size(); }
    // The [rows] scale vector for the scaleB operand; nullptr for HwExpBias / Unit.
    const std::vector<float> *scale_operand() const;
    std::vector<float> dequantize() const;
    std::vector<uint16_t> dequantize_bf16() const;
};

// ------------------------------------------------------------ errors (lib.rs:347-431)

struct RowError {
    float mean_rel;
    float max_rel;
    bool operator==(const RowError &o) const { return mean_rel == o.mean_rel && max_rel == o.max_rel; }
};

std::vector<RowError> row_errors(const std::vector<uint16_t> &w, const Quantized &q);
std::vector<RowError> sample_row_errors(const std::vector<uint16_t> &w, const Quantized &q,
                                        size_t max_rows);
// The same over a borrowed span (an mmap'd checkpoint view).
std::vector<RowError> row_errors(const uint16_t *w, size_t len, const Quantized &q);
std::vector<RowError> sample_row_errors(const uint16_t *w, size_t len, const Quantized &q,
                                        size_t max_rows);

// ------------------------------------------------------------ quantize (lib.rs:433-563)

std::vector<float> row_absmax(const std::vector<uint16_t> &w, size_t rows, size_t cols);
std::vector<float> row_absmax(const uint16_t *w, size_t len, size_t rows, size_t cols);
uint32_t choose_exp_bias(float absmax, Fp8Format fmt);

constexpr float DEFAULT_BACKOFF = 1.0f;

Quantized quantize(const std::vector<uint16_t> &w, size_t rows, size_t cols, Fp8Format fmt,
                   Scaling scaling);
Quantized quantize_with(const std::vector<uint16_t> &w, size_t rows, size_t cols, Fp8Format fmt,
                        Scaling scaling, float backoff);
// The same over a borrowed span (an mmap'd checkpoint view).
Quantized quantize_with(const uint16_t *w, size_t len, size_t rows, size_t cols, Fp8Format fmt,
                        Scaling scaling, float backoff);

// ------------------------------------------------------------ consumer (crates/reng-synapse/src/fp8.rs)

// One fp8 operand (fp8.rs:85-109): device sizes fastest first, the codes, and
// the exponent bias its metadata carries (the values read are
// decode(code) * 2^(exponent_bias(format) - exp_bias), fp8_probe.rs:187-215).
struct Fp8Operand {
    std::string name;
    std::vector<uint64_t> sizes;
    const std::vector<uint8_t> *codes;
    Fp8Format format;
    uint32_t exp_bias;
};

// gemm_fp8_scaled (fp8.rs:295-331): A [K, m], B [K, N] with transpose_b, out
// [N, m] (fastest first), optional scale operands (`[1]` or `[m]` for A,
// `[1]` or `[N]` for B; a missing side is a unit scale, fp8.rs:123-131). The
// bf16 result is returned as f32, as the reference reads its output back.
std::vector<float> gemm_fp8_scaled(const Fp8Operand &a, const Fp8Operand &b,
                                   const std::vector<float> *scale_a,
                                   const std::vector<float> *scale_b,
                                   const std::vector<uint64_t> &out_sizes, bool transpose_b);

// The mixed pair the engine wants (bf16 activation, fp8 weight, fp8.rs:244-276),
// with the per-output-channel scales of a PerChannel weight (or none):
// y[m, n] = x[m, :] . dequantize(q)[n, :], bf16 out returned as f32.
std::vector<float> gemm_w8a16(const std::vector<uint16_t> &x, size_t m, const Quantized &q);

}  // namespace reng_fp8
