// fp8_probe.hpp - the device acceptance probes of crates/reng-model/src/bin/
// fp8_probe.rs (lines 35-431), retargeted to this library: each probe runs a
// device path of libreng_hip.so and reads it against a host reference, and
// prints one line ending in PASS or FAIL.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "reng_fp8.hpp"

namespace reng_probe {

using reng_fp8::Fp8Format;
using reng_fp8::Quantized;

// The reference probe's deterministic inputs (fp8_probe.rs:35-53): a
// Llama-like bf16 weight with a large channel every 977 elements, and
// activations in the post-norm range.
std::vector<uint16_t> weights(size_t rows, size_t cols);
std::vector<float> activations(size_t n);

// c[m, n] = sum_t a[m, t] * b[n, t] in f32, t sequential (fp8_probe.rs:55-67).
std::vector<float> gemm_cpu(const std::vector<float> &a, const std::vector<float> &b, size_t m, size_t k,
                            size_t n);
// |got - want|_2 / max(|want|_2, 1e-12) (fp8_probe.rs:69-78).
float rel_l2(const std::vector<float> &got, const std::vector<float> &want);

// The probe's host reference for a code's value: the closed form of
// reng_fp8::decode (lib.rs:206-225).
float host_decode(uint8_t code, Fp8Format fmt);
// The probe's host reference for the clipping cast: the code of the nearest
// finite value (ties to the even code), saturating at the largest finite
// magnitude, sign | 0x7f for NaN - a search over the decoded table, not the
// encoder's arithmetic.
uint8_t host_encode(float x, Fp8Format fmt);

// What the fp8 x fp8 product reads from an operand whose scale is its
// exponent bias: decode(code) * 2^(exponent_bias(format) - exp_bias)
// (fp8_probe.rs:187-215). Throws std::logic_error for a PerChannel matrix,
// whose scales only the scaled form carries.
std::vector<float> device_values(const Quantized &q);

struct Checks {
    int ran = 0, failed = 0;
    void line(const std::string &name, const std::string &detail, bool ok);
};

void check_decode(Checks &c, Fp8Format fmt);
void check_cast(Checks &c, Fp8Format fmt);
// The mixed pair (bf16 activation, fp8 weight with per-channel scales): the
// reference's stack refuses it; here it is the decode path (gemm_w8a16).
void check_mixed(Checks &c, const Quantized &q, size_t m, size_t k, size_t n);
// fp8 x fp8 with the weight's scale as its exponent bias.
void check_gemm(Checks &c, const Quantized &q_hw, size_t m, size_t k, size_t n, Fp8Format fmt);
// fp8 x fp8 in both operand forms: no scales, and [1] x per-channel scaleB.
void check_gemm_scaled(Checks &c, const Quantized &q, size_t m, size_t k, size_t n, Fp8Format fmt);

}  // namespace reng_probe
