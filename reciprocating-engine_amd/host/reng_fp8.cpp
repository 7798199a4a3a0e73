// reng_fp8.cpp - the reng-fp8 API over libreng_hip (see reng_fp8.hpp).
#include "reng_fp8.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>

#include "../../include/reng_hip.h"

namespace reng_fp8 {

namespace {

std::string lower_trim(std::string_view s) {
    size_t a = 0, b = s.size();
    while (a < b && std::isspace((unsigned char)s[a])) ++a;
    while (b > a && std::isspace((unsigned char)s[b - 1])) --b;
    std::string out(s.substr(a, b - a));
    for (char &c : out) c = (char)std::tolower((unsigned char)c);
    return out;
}

// A status from the C ABI as the Rust crate would report it: argument errors
// are the panics of the reference's asserts, anything else a device failure.
void check(int rc) {
    if (rc == RENG_HIP_OK) return;
    const std::string msg = reng_hip_last_error();
    if (rc == RENG_HIP_EINVAL) throw std::invalid_argument(msg);
    throw std::runtime_error("reng-hip: " + msg);
}

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw std::runtime_error(std::string("reng-hip: ") + what + ": " + hipGetErrorString(e));
}

// Device staging buffer.
class DevBuf {
public:
    explicit DevBuf(size_t bytes) {
        if (bytes) check_hip(hipMalloc(&p_, bytes), "hipMalloc");
    }
    DevBuf(const void *host, size_t bytes) : DevBuf(bytes) {
        if (bytes) check_hip(hipMemcpy(p_, host, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    ~DevBuf() {
        if (p_) (void)hipFree(p_);
    }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    template <typename T>
    T *as() const { return static_cast<T *>(p_); }
    void to_host(void *host, size_t bytes) const {
        if (bytes) check_hip(hipMemcpy(host, p_, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }

private:
    void *p_ = nullptr;
};

void synchronize() { check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

}  // namespace

// ------------------------------------------------------------ formats

uint32_t mantissa_bits(Fp8Format f) { return f == Fp8Format::E4M3 ? 3u : 2u; }
uint32_t exponent_bits(Fp8Format f) { return 8u - 1u - mantissa_bits(f); }
uint32_t exponent_bias(Fp8Format f) { return f == Fp8Format::E4M3 ? 7u : 15u; }
uint8_t max_finite_code(Fp8Format f) {
    const uint32_t m = mantissa_bits(f);
    return (uint8_t)((((1u << exponent_bits(f)) - 2u) << m) | ((1u << m) - 1u));
}
float max_finite(Fp8Format f) {
    // (2 - 2^-m) * 2^emax, emax = 2^e - 2 - bias: 240 and 57344.
    const int m = (int)mantissa_bits(f);
    const int emax = (int)((1u << exponent_bits(f)) - 2u) - (int)exponent_bias(f);
    return std::ldexp(2.0f - std::ldexp(1.0f, -m), emax);
}
uint8_t nan_code(Fp8Format) { return 0x7f; }
int32_t syn_data_type(Fp8Format f) { return f == Fp8Format::E4M3 ? 1 << 13 : 1 << 14; }
std::vector<uint32_t> hw_exponent_biases(Fp8Format f) {
    return f == Fp8Format::E4M3 ? std::vector<uint32_t>{15, 11, 7, 3} : std::vector<uint32_t>{15};
}
const char *name(Fp8Format f) { return f == Fp8Format::E4M3 ? "e4m3" : "e5m2"; }
std::optional<Fp8Format> format_from_name(std::string_view s) {
    const std::string t = lower_trim(s);
    if (t == "e4m3" || t == "fp8_143" || t == "hf8") return Fp8Format::E4M3;
    if (t == "e5m2" || t == "fp8_152" || t == "f8") return Fp8Format::E5M2;
    return std::nullopt;
}

std::optional<Scaling> scaling_from_name(std::string_view s) {
    const std::string t = lower_trim(s);
    if (t == "pcs" || t == "per-channel" || t == "perchannel") return Scaling::PerChannel;
    if (t == "hw" || t == "hw-exp-bias" || t == "expbias") return Scaling::HwExpBias;
    if (t == "unit" || t == "none") return Scaling::Unit;
    return std::nullopt;
}
const char *name(Scaling s) {
    return s == Scaling::PerChannel ? "pcs" : s == Scaling::HwExpBias ? "hw" : "unit";
}

// ------------------------------------------------------------ scalars

float bf16_to_f32(uint16_t x) {
    const uint32_t u = (uint32_t)x << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t f32_to_bf16(float x) {
    uint32_t bits;
    std::memcpy(&bits, &x, 4);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

std::vector<uint8_t> encode(const std::vector<float> &x, Fp8Format fmt) {
    std::vector<uint8_t> out(x.size());
    if (x.empty()) return out;
    DevBuf dx(x.data(), x.size() * 4), dc(x.size());
    check(reng_hip_encode(dx.as<float>(), x.size(), (int)fmt, dc.as<uint8_t>(), nullptr));
    dc.to_host(out.data(), out.size());
    return out;
}

std::vector<float> decode(const std::vector<uint8_t> &codes, Fp8Format fmt) {
    std::vector<float> out(codes.size());
    if (codes.empty()) return out;
    DevBuf dc(codes.data(), codes.size()), dx(codes.size() * 4);
    check(reng_hip_decode(dc.as<uint8_t>(), codes.size(), (int)fmt, dx.as<float>(), nullptr));
    dx.to_host(out.data(), out.size() * 4);
    return out;
}

uint8_t encode(float x, Fp8Format fmt) { return encode(std::vector<float>{x}, fmt)[0]; }
float decode(uint8_t code, Fp8Format fmt) { return decode(std::vector<uint8_t>{code}, fmt)[0]; }

// ------------------------------------------------------------ Quantized

const std::vector<float> *Quantized::scale_operand() const {
    return scaling == Scaling::PerChannel ? &scales : nullptr;
}

std::vector<float> Quantized::dequantize() const {
    std::vector<float> out(rows * cols);
    DevBuf dc(codes.data(), codes.size()), ds(scales.data(), scales.size() * 4), dout(out.size() * 4);
    check(reng_hip_dequantize(dc.as<uint8_t>(), ds.as<float>(), rows, cols, (int)format, RENG_HIP_F32,
                              dout.as<void>(), nullptr));
    dout.to_host(out.data(), out.size() * 4);
    return out;
}

std::vector<uint16_t> Quantized::dequantize_bf16() const {
    std::vector<uint16_t> out(rows * cols);
    DevBuf dc(codes.data(), codes.size()), ds(scales.data(), scales.size() * 4), dout(out.size() * 2);
    check(reng_hip_dequantize(dc.as<uint8_t>(), ds.as<float>(), rows, cols, (int)format, RENG_HIP_BF16,
                              dout.as<void>(), nullptr));
    dout.to_host(out.data(), out.size() * 2);
    return out;
}

// ------------------------------------------------------------ errors

static std::vector<RowError> errors_impl(const uint16_t *w, size_t len, const Quantized &q, size_t max_rows) {
    if (len != q.rows * q.cols) throw std::invalid_argument("weight length against the shape");
    if (q.rows == 0) return {};
    const size_t n = max_rows == 0 ? q.rows : std::min(max_rows, q.rows);
    const size_t step = (q.rows + n - 1) / n;
    const size_t k = (q.rows + step - 1) / step;
    DevBuf dw(w, len * 2), dc(q.codes.data(), q.codes.size()), ds(q.scales.data(), q.scales.size() * 4);
    DevBuf dmean(k * 4), dmax(k * 4);
    check(reng_hip_row_errors(dw.as<uint16_t>(), dc.as<uint8_t>(), ds.as<float>(), q.rows, q.cols, (int)q.format,
                              max_rows, dmean.as<float>(), dmax.as<float>(), nullptr));
    std::vector<float> mean(k), mx(k);
    dmean.to_host(mean.data(), k * 4);
    dmax.to_host(mx.data(), k * 4);
    std::vector<RowError> out(k);
    for (size_t i = 0; i < k; ++i) out[i] = RowError{mean[i], mx[i]};
    return out;
}

std::vector<RowError> row_errors(const uint16_t *w, size_t len, const Quantized &q) {
    return errors_impl(w, len, q, 0);
}

std::vector<RowError> sample_row_errors(const uint16_t *w, size_t len, const Quantized &q, size_t max_rows) {
    if (len != q.rows * q.cols) throw std::invalid_argument("weight length against the shape");
    if (max_rows == 0) throw std::invalid_argument("max_rows must be positive");
    return errors_impl(w, len, q, max_rows);
}

std::vector<RowError> row_errors(const std::vector<uint16_t> &w, const Quantized &q) {
    return row_errors(w.data(), w.size(), q);
}

std::vector<RowError> sample_row_errors(const std::vector<uint16_t> &w, const Quantized &q, size_t max_rows) {
    return sample_row_errors(w.data(), w.size(), q, max_rows);
}

// ------------------------------------------------------------ quantize

std::vector<float> row_absmax(const uint16_t *w, size_t len, size_t rows, size_t cols) {
    if (len != rows * cols) throw std::invalid_argument("weight length against the shape");
    std::vector<float> out(rows);
    if (rows == 0 || cols == 0) return out;
    DevBuf dw(w, len * 2), dout(rows * 4);
    check(reng_hip_row_absmax(dw.as<void>(), RENG_HIP_BF16, rows, cols, cols, dout.as<float>(), nullptr));
    dout.to_host(out.data(), rows * 4);
    return out;
}

std::vector<float> row_absmax(const std::vector<uint16_t> &w, size_t rows, size_t cols) {
    return row_absmax(w.data(), w.size(), rows, cols);
}

uint32_t choose_exp_bias(float absmax, Fp8Format fmt) { return reng_hip_choose_exp_bias(absmax, (int)fmt); }

Quantized quantize_with(const uint16_t *w, size_t len, size_t rows, size_t cols, Fp8Format fmt, Scaling scaling,
                        float backoff) {
    // The asserts of lib.rs:527-532, with their messages.
    if (!(rows > 0 && cols > 0))
        throw std::invalid_argument("empty shape " + std::to_string(rows) + " x " + std::to_string(cols));
    if (len != rows * cols) throw std::invalid_argument("weight length against the shape");
    if (!(backoff > 0.0f && std::isfinite(backoff))) {
        char b[64];
        std::snprintf(b, sizeof b, "%g", (double)backoff);
        throw std::invalid_argument(std::string("backoff ") + b + " is not positive and finite");
    }
    Quantized q;
    q.format = fmt;
    q.scaling = scaling;
    q.rows = rows;
    q.cols = cols;
    q.codes.resize(rows * cols);
    q.scales.resize(rows);
    check(reng_hip_quantize_host(w, RENG_HIP_BF16, rows, cols, (int)fmt, (int)scaling, backoff, q.codes.data(),
                                 q.scales.data(), &q.exp_bias));
    return q;
}

Quantized quantize_with(const std::vector<uint16_t> &w, size_t rows, size_t cols, Fp8Format fmt, Scaling scaling,
                        float backoff) {
    return quantize_with(w.data(), w.size(), rows, cols, fmt, scaling, backoff);
}

Quantized quantize(const std::vector<uint16_t> &w, size_t rows, size_t cols, Fp8Format fmt, Scaling scaling) {
    return quantize_with(w, rows, cols, fmt, scaling, DEFAULT_BACKOFF);
}

// ------------------------------------------------------------ consumer

std::vector<float> gemm_fp8_scaled(const Fp8Operand &a, const Fp8Operand &b, const std::vector<float> *scale_a,
                                   const std::vector<float> *scale_b, const std::vector<uint64_t> &out_sizes,
                                   bool transpose_b) {
    if (!transpose_b) throw std::invalid_argument(b.name + ": only the transpose_b form ([K, N] read as [N, K]) is wired");
    if (a.sizes.size() != 2 || b.sizes.size() != 2 || out_sizes.size() != 2)
        throw std::invalid_argument("gemm_fp8_scaled: operands and output are 2-D");
    const size_t K = a.sizes[0], M = a.sizes[1], N = b.sizes[1];
    if (b.sizes[0] != K) throw std::invalid_argument(a.name + " / " + b.name + ": contraction sizes differ");
    if (out_sizes[0] != N || out_sizes[1] != M) throw std::invalid_argument("gemm_fp8_scaled: output must be [N, m]");
    if (!a.codes || a.codes->size() != K * M) throw std::invalid_argument(a.name + ": codes against the sizes");
    if (!b.codes || b.codes->size() != K * N) throw std::invalid_argument(b.name + ": codes against the sizes");
    for (const auto *s : {scale_a, scale_b})
        if (s && s->empty()) throw std::invalid_argument("an empty scale vector");
    // The exponent bias of an operand's metadata scales what the device reads
    // by 2^(default - bias) (fp8_probe.rs:187-215): fold it into the scales.
    auto fold = [](const Fp8Operand &o, const std::vector<float> *s) {
        const float f = std::ldexp(1.0f, (int)exponent_bias(o.format) - (int)o.exp_bias);
        std::vector<float> out = s ? *s : std::vector<float>{};
        if (f != 1.0f) {
            if (out.empty()) out.push_back(1.0f);
            for (float &v : out) v *= f;
        }
        return out;
    };
    const std::vector<float> sa = fold(a, scale_a), sb = fold(b, scale_b);
    DevBuf da(a.codes->data(), a.codes->size()), db(b.codes->data(), b.codes->size());
    DevBuf dsa(sa.data(), sa.size() * 4), dsb(sb.data(), sb.size() * 4), dout(M * N * 2);
    check(reng_hip_gemm_fp8_scaled(da.as<uint8_t>(), (int)a.format, sa.empty() ? nullptr : dsa.as<float>(), sa.size(),
                                   db.as<uint8_t>(), (int)b.format, sb.empty() ? nullptr : dsb.as<float>(), sb.size(),
                                   M, N, K, dout.as<uint16_t>(), nullptr));
    std::vector<uint16_t> y(M * N);
    dout.to_host(y.data(), y.size() * 2);
    std::vector<float> out(y.size());
    for (size_t i = 0; i < y.size(); ++i) out[i] = bf16_to_f32(y[i]);
    return out;
}

std::vector<float> gemm_w8a16(const std::vector<uint16_t> &x, size_t m, const Quantized &q) {
    if (x.size() != m * q.cols) throw std::invalid_argument("activation length against the shape");
    DevBuf dx(x.data(), x.size() * 2), dc(q.codes.data(), q.codes.size()), ds(q.scales.data(), q.scales.size() * 4);
    DevBuf dy(m * q.rows * 2);
    check(reng_hip_gemm_w8a16(dx.as<uint16_t>(), dc.as<uint8_t>(), ds.as<float>(), m, q.rows, q.cols, (int)q.format,
                              dy.as<uint16_t>(), nullptr));
    std::vector<uint16_t> y(m * q.rows);
    dy.to_host(y.data(), y.size() * 2);
    synchronize();
    std::vector<float> out(y.size());
    for (size_t i = 0; i < y.size(); ++i) out[i] = bf16_to_f32(y[i]);
    return out;
}

}  // namespace reng_fp8
