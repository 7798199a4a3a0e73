// fp8_probe.cpp - see fp8_probe.hpp.
#include "fp8_probe.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <stdexcept>

namespace reng_probe {

using reng_fp8::Fp8Operand;
using reng_fp8::Scaling;

std::vector<uint16_t> weights(size_t rows, size_t cols) {
    std::vector<uint16_t> out(rows * cols);
    for (size_t i = 0; i < out.size(); ++i) {
        const float x = ((float)((i * 2654435761ull) % 65536) / 65536.0f - 0.5f) * 0.08f;
        const float outlier = i % 977 == 0 ? 12.0f : 1.0f;
        out[i] = reng_fp8::f32_to_bf16(x * outlier);
    }
    return out;
}

std::vector<float> activations(size_t n) {
    std::vector<float> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = ((float)((i * 7919) % 2003) - 1000.0f) / 700.0f;
    return out;
}

std::vector<float> gemm_cpu(const std::vector<float> &a, const std::vector<float> &b, size_t m, size_t k,
                            size_t n) {
    std::vector<float> c(n * m, 0.0f);
    for (size_t row = 0; row < m; ++row)
        for (size_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (size_t t = 0; t < k; ++t) acc += a[row * k + t] * b[j * k + t];
            c[row * n + j] = acc;
        }
    return c;
}

float rel_l2(const std::vector<float> &got, const std::vector<float> &want) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < got.size() && i < want.size(); ++i) {
        const double d = (double)(got[i] - want[i]);
        num += d * d;
        den += (double)want[i] * (double)want[i];
    }
    return (float)(std::sqrt(num) / std::max(std::sqrt(den), 1e-12));
}

float host_decode(uint8_t code, Fp8Format fmt) {
    const uint32_t mb = reng_fp8::mantissa_bits(fmt);
    const int bias = (int)reng_fp8::exponent_bias(fmt);
    const float sign = (code & 0x80) ? -1.0f : 1.0f;
    const uint32_t mant = code & ((1u << mb) - 1), ef = (code & 0x7fu) >> mb;
    if (ef == (1u << reng_fp8::exponent_bits(fmt)) - 1) return mant == 0 ? sign * INFINITY : NAN;
    const float frac = (float)mant / (float)(1u << mb);
    return ef == 0 ? sign * std::ldexp(frac, 1 - bias) : sign * std::ldexp(1.0f + frac, (int)ef - bias);
}

uint8_t host_encode(float x, Fp8Format fmt) {
    const uint8_t sign = std::signbit(x) ? 0x80 : 0x00;
    if (std::isnan(x)) return sign | reng_fp8::nan_code(fmt);
    const float a = std::fabs(x);
    const uint8_t maxc = reng_fp8::max_finite_code(fmt);
    if (a >= host_decode(maxc, fmt)) return sign | maxc;
    // The positive finite values increase with the code: the largest code
    // at or below a, then the nearer of it and the next one (ties to the
    // even code, whose mantissa is even).
    uint8_t lo = 0;
    for (uint8_t c = 0; c <= maxc; ++c)
        if (host_decode(c, fmt) <= a) lo = c;
    const uint8_t hi = lo + 1;
    const float dl = a - host_decode(lo, fmt), dh = host_decode(hi, fmt) - a;
    const uint8_t c = dl < dh ? lo : dh < dl ? hi : (lo % 2 == 0 ? lo : hi);
    return sign | c;
}

std::vector<float> device_values(const Quantized &q) {
    if (q.scaling == Scaling::PerChannel)
        throw std::logic_error(
            "the fp8 x fp8 product without scale operands does not see per-channel scales; use the scaleB "
            "operand for those");
    const float factor = std::ldexp(1.0f, (int)reng_fp8::exponent_bias(q.format) - (int)q.exp_bias);
    std::vector<float> out(q.codes.size());
    for (size_t i = 0; i < out.size(); ++i) out[i] = host_decode(q.codes[i], q.format) * factor;
    return out;
}

void Checks::line(const std::string &name, const std::string &detail, bool ok) {
    ++ran;
    if (!ok) ++failed;
    std::printf("%-28s %s %s\n", name.c_str(), detail.c_str(), ok ? "PASS" : "FAIL");
    std::fflush(stdout);
}

namespace {

std::string fmt_f(const char *f, double v) {
    char b[64];
    std::snprintf(b, sizeof b, f, v);
    return b;
}

std::vector<uint16_t> bf16(const std::vector<float> &x) {
    std::vector<uint16_t> out(x.size());
    for (size_t i = 0; i < x.size(); ++i) out[i] = reng_fp8::f32_to_bf16(x[i]);
    return out;
}

std::vector<float> host_dequantize(const Quantized &q) {
    std::vector<float> out(q.codes.size());
    for (size_t r = 0; r < q.rows; ++r)
        for (size_t c = 0; c < q.cols; ++c)
            out[r * q.cols + c] = host_decode(q.codes[r * q.cols + c], q.format) * q.scales[r];
    return out;
}

}  // namespace

void check_decode(Checks &c, Fp8Format fmt) {
    const std::string name = std::string("decode-") + reng_fp8::name(fmt);
    try {
        std::vector<uint8_t> codes(256);
        for (int i = 0; i < 256; ++i) codes[i] = (uint8_t)i;
        const std::vector<float> got = reng_fp8::decode(codes, fmt);
        int bad = 0;
        for (int i = 0; i < 256; ++i) {
            const float w = host_decode((uint8_t)i, fmt);
            if (std::isfinite(w) && std::fabs(got[i] - w) > 0.0f) {
                if (bad++ == 0) std::printf("  first mismatch at code %#04x: device %g, host %g\n", i, got[i], w);
            }
        }
        c.line(name, std::to_string(bad) + " of 256 codes differ:", bad == 0);
    } catch (const std::exception &e) {
        c.line(name, std::string(e.what()) + ":", false);
    }
}

void check_cast(Checks &c, Fp8Format fmt) {
    const std::string name = std::string("cast-clip-") + reng_fp8::name(fmt);
    try {
        std::vector<float> x = activations(256);
        x[0] = 250.0f;
        x[1] = -300.0f;
        x[2] = 0.001f;
        x[3] = 1.375f;
        x[4] = -3.3f;
        // Rounded to bf16 on the way in, as the engine's uploads are.
        std::vector<float> xb(x.size());
        for (size_t i = 0; i < x.size(); ++i) xb[i] = reng_fp8::bf16_to_f32(reng_fp8::f32_to_bf16(x[i]));
        const std::vector<float> got = reng_fp8::decode(reng_fp8::encode(xb, fmt), fmt);
        int bad = 0;
        for (size_t i = 0; i < x.size(); ++i)
            if (std::fabs(got[i] - host_decode(host_encode(xb[i], fmt), fmt)) > 0.0f) ++bad;
        c.line(name, std::to_string(bad) + " of " + std::to_string(x.size()) + " values differ:", bad == 0);
    } catch (const std::exception &e) {
        c.line(name, std::string(e.what()) + ":", false);
    }
}

void check_mixed(Checks &c, const Quantized &q, size_t m, size_t k, size_t n) {
    const std::string name = "gemm-mixed-bf16-fp8-m" + std::to_string(m);
    try {
        const std::vector<uint16_t> a = bf16(activations(m * k));
        std::vector<float> af(a.size());
        for (size_t i = 0; i < a.size(); ++i) af[i] = reng_fp8::bf16_to_f32(a[i]);
        const std::vector<float> got = reng_fp8::gemm_w8a16(a, m, q);
        const float rel = rel_l2(got, gemm_cpu(af, host_dequantize(q), m, k, n));
        c.line(name, "accepted (the decode path here), rel_L2 " + fmt_f("%.4f", rel) + " against the dequantized product:",
               rel < 0.02f);
    } catch (const std::exception &e) {
        c.line(name, std::string(e.what()) + ":", false);
    }
}

void check_gemm(Checks &c, const Quantized &q_hw, size_t m, size_t k, size_t n, Fp8Format fmt) {
    const std::string name = "gemm-fp8-m" + std::to_string(m);
    try {
        if (q_hw.scaling != Scaling::HwExpBias) throw std::logic_error("the plain form carries its scale as the exponent bias");
        const std::vector<uint16_t> a_bf16 = bf16(activations(m * k));
        const Quantized a_q = reng_fp8::quantize(a_bf16, m, k, fmt, Scaling::Unit);
        const std::vector<float> want = gemm_cpu(device_values(a_q), device_values(q_hw), m, k, n);
        const Fp8Operand a{"A", {k, m}, &a_q.codes, fmt, a_q.exp_bias};
        const Fp8Operand b{"W", {k, n}, &q_hw.codes, fmt, q_hw.exp_bias};
        const float rel = rel_l2(reng_fp8::gemm_fp8_scaled(a, b, nullptr, nullptr, {n, m}, true), want);
        c.line(name,
               "rel_L2 " + fmt_f("%.4f", rel) + " at weight exp_bias " + std::to_string(q_hw.exp_bias) +
                   " against the dequantized product:",
               rel < 0.02f);
    } catch (const std::exception &e) {
        c.line(name, std::string(e.what()) + ":", false);
    }
}

void check_gemm_scaled(Checks &c, const Quantized &q, size_t m, size_t k, size_t n, Fp8Format fmt) {
    const std::string m_s = std::to_string(m);
    try {
        if (q.scaling != Scaling::PerChannel) throw std::logic_error("the scaled form carries its scale as scaleB");
        const std::vector<uint16_t> a_bf16 = bf16(activations(m * k));
        const Quantized a_q = reng_fp8::quantize(a_bf16, m, k, fmt, Scaling::Unit);
        const std::vector<float> a_deq = device_values(a_q);
        const Fp8Operand a{"A", {k, m}, &a_q.codes, fmt, a_q.exp_bias};
        const Fp8Operand b{"W", {k, n}, &q.codes, fmt, reng_fp8::exponent_bias(fmt)};
        // Two inputs: the product over the codes as read, scales left out.
        std::vector<float> raw(q.codes.size());
        for (size_t i = 0; i < raw.size(); ++i) raw[i] = host_decode(q.codes[i], fmt);
        const float rel2 = rel_l2(reng_fp8::gemm_fp8_scaled(a, b, nullptr, nullptr, {n, m}, true),
                                  gemm_cpu(a_deq, raw, m, k, n));
        c.line("fp8_gemm_bf16-2in-m" + m_s, "rel_L2 " + fmt_f("%.4f", rel2) + " against the unscaled product:",
               rel2 < 0.02f);
        // Four inputs: a unit scaleA and the per-channel scaleB.
        const std::vector<float> one{1.0f};
        const float rel4 = rel_l2(reng_fp8::gemm_fp8_scaled(a, b, &one, q.scale_operand(), {n, m}, true),
                                  gemm_cpu(a_deq, host_dequantize(q), m, k, n));
        c.line("fp8_gemm_bf16-pcs-m" + m_s, "rel_L2 " + fmt_f("%.4f", rel4) + " against the dequantized product:",
               rel4 < 0.02f);
    } catch (const std::exception &e) {
        c.line("fp8_gemm_bf16-m" + m_s, std::string(e.what()) + ":", false);
    }
}

}  // namespace reng_probe
