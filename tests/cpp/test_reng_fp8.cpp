// test_reng_fp8.cpp - the reng-fp8 crate's own tests (crates/reng-fp8/src/lib.rs:633-926
// and crates/reng-fp8/tests/fixtures.rs:113-292) run against the C++ API of
// reciprocating-engine_amd/host, whose numerics all come from libreng_hip.so
// on the GPU. The serial reference path those tests compare the parallel one
// with (absmax_range / encode_range) is the CPU oracle here (oracle/fp8_oracle.h),
// used only as the checker.
//
//   test_reng_fp8 [--cpu-only] [--fixture PATH] [NAME_SUBSTRING]
//
// --cpu-only runs the tests that touch no device (constants, names, bf16
// helpers, the exponent-bias choice, argument refusals, the fixture file).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

#include "../../oracle/fp8_oracle.h"
#include "../../reciprocating-engine_amd/host/json.hpp"
#include "../../reciprocating-engine_amd/host/reng_fp8.hpp"

using namespace reng_fp8;

namespace {

struct Failure {
    std::string msg;
};

void expect(bool ok, const std::string &msg) {
    if (!ok) throw Failure{msg};
}

std::string hex(unsigned v) {
    char b[16];
    std::snprintf(b, sizeof b, "%#04x", v);
    return b;
}

std::string num(double v) {
    char b[40];
    std::snprintf(b, sizeof b, "%.9g", v);
    return b;
}

uint16_t b(float x) { return f32_to_bf16(x); }

template <typename E>
void expect_throws(const std::function<void()> &f, const std::string &needle, const std::string &what) {
    try {
        f();
    } catch (const E &e) {
        expect(std::string(e.what()).find(needle) != std::string::npos,
               what + ": message '" + e.what() + "' lacks '" + needle + "'");
        return;
    }
    throw Failure{what + ": no exception"};
}

uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

float from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

std::string g_fixture = "tests/golden/fp8_cast.json";

// ------------------------------------------------------------------ host-only tests

void format_constants_host() {
    expect(max_finite(Fp8Format::E4M3) == 240.0f, "E4M3 max_finite");
    expect(max_finite_code(Fp8Format::E4M3) == 0x77, "E4M3 max_finite_code");
    expect(syn_data_type(Fp8Format::E4M3) == 8192, "E4M3 syn_data_type");
    expect(max_finite(Fp8Format::E5M2) == 57344.0f, "E5M2 max_finite");
    expect(max_finite_code(Fp8Format::E5M2) == 0x7b, "E5M2 max_finite_code");
    expect(syn_data_type(Fp8Format::E5M2) == 16384, "E5M2 syn_data_type");
    expect(format_from_name("E4M3") == Fp8Format::E4M3, "from_name E4M3");
    expect(format_from_name("f8") == Fp8Format::E5M2, "from_name f8");
    expect(format_from_name(" hf8 ") == Fp8Format::E4M3, "from_name hf8 (trimmed)");
    expect(!format_from_name("fp4").has_value(), "from_name fp4");
    expect(scaling_from_name("hw") == Scaling::HwExpBias, "scaling hw");
    expect(scaling_from_name("pcs") == Scaling::PerChannel, "scaling pcs");
    expect(scaling_from_name("unit") == Scaling::Unit, "scaling unit");
    expect(!scaling_from_name("bogus").has_value(), "scaling bogus");
    expect(std::string(name(Fp8Format::E5M2)) == "e5m2" && std::string(name(Scaling::HwExpBias)) == "hw", "names");
    expect(hw_exponent_biases(Fp8Format::E4M3) == std::vector<uint32_t>{15, 11, 7, 3}, "E4M3 biases");
    expect(hw_exponent_biases(Fp8Format::E5M2) == std::vector<uint32_t>{15}, "E5M2 biases");
    for (Fp8Format f : {Fp8Format::E4M3, Fp8Format::E5M2}) {
        expect(mantissa_bits(f) == orc_mantissa_bits((int)f), "mantissa bits");
        expect(exponent_bits(f) + mantissa_bits(f) == 7, "exponent bits");
        expect(exponent_bias(f) == orc_exponent_bias((int)f), "exponent bias");
        expect(max_finite(f) == orc_max_finite((int)f), "max_finite against the oracle");
        expect(nan_code(f) == 0x7f, "nan code");
    }
}

void bf16_helpers_agree_with_the_oracle() {
    // Every 65537th f32 pattern (all exponents, signs and rounding cases),
    // plus the specials.
    for (uint64_t u = 0; u <= 0xffffffffull; u += 65537) {
        const float x = from_bits((uint32_t)u);
        expect(f32_to_bf16(x) == orc_f32_to_bf16(x), "f32_to_bf16 " + hex((unsigned)u));
    }
    for (uint32_t u : {0x00000000u, 0x80000000u, 0x7f800000u, 0xff800000u, 0x7fc00000u, 0xffc00001u,
                       0x3f808000u, 0x3f818000u, 0x7f7fffffu}) {
        expect(f32_to_bf16(from_bits(u)) == orc_f32_to_bf16(from_bits(u)), "f32_to_bf16 special " + hex(u));
    }
    for (uint32_t h = 0; h < 65536; ++h) {
        const float x = bf16_to_f32((uint16_t)h);
        expect(bits(x) == bits(orc_bf16_to_f32((uint16_t)h)), "bf16_to_f32 " + hex(h));
    }
}

void hw_exp_bias_picks_the_finest_range_that_fits_host() {
    const Fp8Format f = Fp8Format::E4M3;
    expect(choose_exp_bias(0.5f, f) == 15, "0.5");
    expect(choose_exp_bias(0.9375f, f) == 15, "0.9375");
    expect(choose_exp_bias(1.0f, f) == 11, "1.0");
    expect(choose_exp_bias(15.0f, f) == 11, "15");
    expect(choose_exp_bias(16.0f, f) == 7, "16");
    expect(choose_exp_bias(1000.0f, f) == 3, "1000");
    expect(choose_exp_bias(1e9f, f) == 3, "1e9");
    expect(choose_exp_bias(1e9f, Fp8Format::E5M2) == 15, "E5M2");
    // Against the oracle over a sweep of magnitudes, both formats.
    for (Fp8Format g : {Fp8Format::E4M3, Fp8Format::E5M2})
        for (int e = -30; e <= 30; ++e)
            for (float m : {1.0f, 0.9375f, 0.96875f, 1.5f}) {
                const float a = std::ldexp(m, e);
                expect(choose_exp_bias(a, g) == orc_choose_exp_bias(a, (int)g), "choose_exp_bias " + num(a));
            }
}

void asserts_keep_their_messages() {
    const std::vector<uint16_t> w(8, b(1.0f));
    expect_throws<std::invalid_argument>([&] { (void)quantize_with(w, 0, 8, Fp8Format::E4M3, Scaling::PerChannel, 1.0f); },
                                         "empty shape 0 x 8", "zero rows");
    expect_throws<std::invalid_argument>([&] { (void)quantize_with(w, 2, 0, Fp8Format::E4M3, Scaling::PerChannel, 1.0f); },
                                         "empty shape 2 x 0", "zero cols");
    expect_throws<std::invalid_argument>([&] { (void)quantize(w, 3, 4, Fp8Format::E4M3, Scaling::PerChannel); },
                                         "weight length against the shape", "length");
    for (float bo : {0.0f, -1.0f, INFINITY, NAN})
        expect_throws<std::invalid_argument>(
            [&] { (void)quantize_with(w, 2, 4, Fp8Format::E4M3, Scaling::PerChannel, bo); },
            "is not positive and finite", "backoff " + num(bo));
    Quantized q;
    q.format = Fp8Format::E4M3;
    q.scaling = Scaling::PerChannel;
    q.rows = 2;
    q.cols = 4;
    q.codes.assign(8, 0);
    q.scales.assign(2, 1.0f);
    expect_throws<std::invalid_argument>([&] { (void)row_errors(std::vector<uint16_t>(7), q); },
                                         "weight length against the shape", "row_errors length");
    expect_throws<std::invalid_argument>([&] { (void)sample_row_errors(w, q, 0); }, "max_rows must be positive",
                                         "sample_row_errors zero");
    expect_throws<std::invalid_argument>([&] { (void)row_absmax(w, 3, 3); }, "weight length against the shape",
                                         "row_absmax length");
}

// ------------------------------------------------------------------ fixture

std::vector<uint16_t> hex_u16(const std::string &s) {
    std::vector<uint16_t> out(s.size() / 4);
    for (size_t i = 0; i < out.size(); ++i) out[i] = (uint16_t)std::stoul(s.substr(i * 4, 4), nullptr, 16);
    return out;
}

std::vector<uint8_t> hex_u8(const std::string &s) {
    std::vector<uint8_t> out(s.size() / 2);
    for (size_t i = 0; i < out.size(); ++i) out[i] = (uint8_t)std::stoul(s.substr(i * 2, 2), nullptr, 16);
    return out;
}

reng_json::Value doc() {
    std::ifstream f(g_fixture);
    if (!f) throw Failure{"cannot open the fixture " + g_fixture};
    std::stringstream ss;
    ss << f.rdbuf();
    return reng_json::parse(ss.str());
}

struct Case {
    std::string name;
    Fp8Format fmt;
    Scaling scaling;
    size_t rows, cols;
    uint32_t exp_bias;
    std::vector<uint16_t> w;
    std::vector<float> scales;
    std::vector<uint8_t> codes;
    bool has_torch_raw = false;
    std::vector<uint8_t> torch_raw;
    std::vector<double> mean_rel, max_rel;
};

std::vector<Case> cases() {
    const reng_json::Value d = doc();
    const auto &raw = d["cases"];
    std::vector<Case> out;
    for (size_t k = 0; k < raw.size(); ++k) {
        const auto &c = raw[k];
        Case cs;
        cs.name = c["name"].as_str();
        const std::string from =
            c.has("bf16_from") && c["bf16_from"].kind == reng_json::Value::String ? c["bf16_from"].as_str() : "";
        if (from.empty()) {
            cs.w = hex_u16(c["bf16_hex"].as_str());
        } else {
            bool found = false;
            for (const auto &o : out)
                if (o.name == from) {
                    cs.w = o.w;
                    found = true;
                }
            expect(found, cs.name + ": shares weights with unknown case " + from);
        }
        cs.fmt = format_from_name(c["format"].as_str()).value();
        cs.scaling = scaling_from_name(c["scaling"].as_str()).value();
        cs.rows = c["rows"].as_u64();
        cs.cols = c["cols"].as_u64();
        cs.exp_bias = (uint32_t)c["exp_bias"].as_u64();
        for (const auto &s : c["scale_bits"].arr) cs.scales.push_back(from_bits((uint32_t)s.as_u64()));
        cs.codes = hex_u8(c["codes_hex"].as_str());
        if (c.has("torch_raw_hex") && c["torch_raw_hex"].kind == reng_json::Value::String) {
            cs.has_torch_raw = true;
            cs.torch_raw = hex_u8(c["torch_raw_hex"].as_str());
        }
        for (const auto &v : c["mean_rel"].arr) cs.mean_rel.push_back(v.as_f64());
        for (const auto &v : c["max_rel"].arr) cs.max_rel.push_back(v.as_f64());
        out.push_back(std::move(cs));
    }
    return out;
}

Quantized quantized(const Case &c) { return quantize(c.w, c.rows, c.cols, c.fmt, c.scaling); }

void the_fixture_is_the_one_the_generator_writes() {
    const auto d = doc();
    expect(d["generator"].as_str() == "tools/fp8_fixtures.py", "generator");
    const size_t n = d["cases"].size();
    expect(n >= 12, std::to_string(n) + " cases");
    size_t ckpt = 0;
    for (const auto &c : d["cases"].arr)
        if (c["name"].as_str().rfind("ckpt_", 0) == 0) ++ckpt;
    expect(ckpt >= 6, "no checkpoint cases");
    // Every case resolves (shared weights, hex lengths against the shape).
    for (const Case &c : cases()) {
        expect(c.w.size() == c.rows * c.cols, c.name + ": weights against the shape");
        expect(c.codes.size() == c.rows * c.cols, c.name + ": codes against the shape");
        expect(c.scales.size() == c.rows && c.mean_rel.size() == c.rows, c.name + ": per-row vectors");
    }
}

// ------------------------------------------------------------------ device tests (lib.rs)

void e4m3_codes_match_the_device_cast() {
    const std::vector<std::pair<float, uint8_t>> cs = {
        {0.0f, 0x00},  {1.0f, 0x38},   {1.375f, 0x3b}, {-3.3f, 0xc5},  {100.0f, 0x6c},     {0.01f, 0x05},
        {0.0625f, 0x18}, {17.0f, 0x58}, {240.0f, 0x77}, {-240.0f, 0xf7}, {250.0f, 0x77},    {300.0f, 0x77},
        {0.001f, 0x01}, {1e-9f, 0x00},  {INFINITY, 0x77}, {-INFINITY, 0xf7}};
    std::vector<float> x;
    for (auto &p : cs) x.push_back(p.first);
    x.push_back(NAN);
    const auto got = encode(x, Fp8Format::E4M3);
    for (size_t i = 0; i < cs.size(); ++i)
        expect(got[i] == cs[i].second, "encode(" + num(cs[i].first) + ") = " + hex(got[i]));
    expect((got.back() & 0x7f) == 0x7f, "encode(NaN)");
    expect(encode(1.375f, Fp8Format::E4M3) == 0x3b, "scalar encode");
}

void e5m2_codes_match_the_device_cast() {
    const std::vector<std::pair<float, uint8_t>> cs = {
        {1.375f, 0x3e}, {250.0f, 0x5c}, {300.0f, 0x5d}, {-240.0f, 0xdc}, {1.0f, 0x3c}};
    for (auto &p : cs) expect(encode(p.first, Fp8Format::E5M2) == p.second, "encode(" + num(p.first) + ")");
    const auto d = decode(std::vector<uint8_t>{0x3e, 0x5c, 0x5d, 0xdc}, Fp8Format::E5M2);
    expect(d[0] == 1.5f && d[1] == 256.0f && d[2] == 320.0f && d[3] == -256.0f, "decode");
}

void format_constants_device() {
    expect(std::isinf(decode(0x78, Fp8Format::E4M3)), "0x78 is infinite");
    expect(std::isnan(decode(0x7f, Fp8Format::E4M3)), "0x7f is NaN");
}

void every_code_round_trips_through_the_encoder() {
    for (Fp8Format f : {Fp8Format::E4M3, Fp8Format::E5M2}) {
        std::vector<uint8_t> codes(256);
        for (int c = 0; c < 256; ++c) codes[c] = (uint8_t)c;
        const auto v = decode(codes, f);
        for (int c = 0; c < 256; ++c) {
            const float want = orc_decode((uint8_t)c, (int)f);
            expect(bits(v[c]) == bits(want) || (std::isnan(v[c]) && std::isnan(want)),
                   std::string(name(f)) + " decode " + hex(c));
        }
        std::vector<float> finite;
        std::vector<uint8_t> want;
        for (int c = 0; c < 256; ++c)
            if (std::isfinite(v[c])) {
                finite.push_back(v[c]);
                want.push_back((uint8_t)c);
            }
        const auto back = encode(finite, f);
        for (size_t i = 0; i < back.size(); ++i)
            expect(back[i] == want[i], std::string(name(f)) + " code " + hex(want[i]) + " value " + num(finite[i]));
    }
}

void rounding_is_to_nearest_even() {
    const auto c = encode(std::vector<float>{1.0625f, 1.1875f, 1.0626f}, Fp8Format::E4M3);
    expect(c[0] == 0x38, "1.0625 ties to even");
    expect(c[1] == 0x3a, "1.1875 ties to even");
    expect(c[2] == 0x39, "above the tie rounds up");
}

void per_channel_scales_stretch_each_row_to_full_scale() {
    std::vector<uint16_t> w;
    for (float x : {0.5f, -1.0f, 0.25f, 0.0f, 100.0f, -50.0f, 12.5f, 0.0f}) w.push_back(b(x));
    const auto q = quantize(w, 2, 4, Fp8Format::E4M3, Scaling::PerChannel);
    expect(q.scales.size() == 2, "two scales");
    expect(q.scales[0] == 1.0f / 240.0f, "scale 0");
    expect(q.scales[1] == 100.0f / 240.0f, "scale 1");
    expect(q.exp_bias == 7, "exp bias");
    expect((q.codes[1] & 0x7f) == 0x77 && (q.codes[4] & 0x7f) == 0x77, "absmax on the top code");
    expect(q.scale_operand() && q.scale_operand()->size() == 2, "scale operand");
    const auto d = q.dequantize();
    expect(std::fabs(d[0] - 0.5f) < 0.5f * 0.07f && std::fabs(d[4] - 100.0f) < 100.0f * 0.07f, "round trip");
}

void hw_exp_bias_picks_the_finest_range_that_fits() {
    std::vector<uint16_t> w;
    for (int i = 0; i < 64; ++i) w.push_back(b(((float)i - 32.0f) / 64.0f));
    const auto q = quantize(w, 4, 16, Fp8Format::E4M3, Scaling::HwExpBias);
    expect(q.exp_bias == 15, "exp bias " + std::to_string(q.exp_bias));
    for (float s : q.scales) expect(s == 1.0f / 256.0f, "scale " + num(s));
    expect(q.scale_operand() == nullptr, "no scale operand");
}

void unit_scaling_leaves_the_codes_alone() {
    std::vector<uint16_t> w;
    for (float x : {1.0f, 2.0f, 0.5f, 100.0f}) w.push_back(b(x));
    const auto q = quantize(w, 1, 4, Fp8Format::E4M3, Scaling::Unit);
    expect(q.scales == std::vector<float>{1.0f}, "unit scale");
    expect(q.codes[0] == encode(1.0f, Fp8Format::E4M3) && q.codes[3] == encode(100.0f, Fp8Format::E4M3), "codes");
    expect(q.scale_operand() == nullptr, "no scale operand");
}

void dequantize_of_quantize_is_within_the_format_resolution() {
    const size_t rows = 32, cols = 128;
    std::vector<uint16_t> w(rows * cols);
    for (size_t i = 0; i < w.size(); ++i) {
        const float x = (float)((i * 2654435761ull) % 65536) / 65536.0f - 0.5f;
        w[i] = b(x * (1.0f + (float)(i / cols)));
    }
    const auto q = quantize(w, rows, cols, Fp8Format::E4M3, Scaling::PerChannel);
    const auto errs = row_errors(w, q);
    expect(errs.size() == rows, "one error per row");
    for (size_t r = 0; r < rows; ++r) {
        expect(errs[r].max_rel <= 0.0626f, "row " + std::to_string(r) + " max_rel " + num(errs[r].max_rel));
        expect(errs[r].mean_rel < 0.03f, "row " + std::to_string(r) + " mean_rel " + num(errs[r].mean_rel));
    }
    const auto bf = q.dequantize_bf16();
    const auto f = q.dequantize();
    expect(bf.size() == f.size(), "sizes");
    for (size_t i = 0; i < f.size(); ++i) expect(bf[i] == f32_to_bf16(f[i]), "bf16 round trip at " + std::to_string(i));
    // dequantize against the oracle, bit for bit.
    std::vector<float> want(rows * cols);
    orc_dequantize(q.codes.data(), q.scales.data(), rows, cols, (int)q.format, want.data());
    for (size_t i = 0; i < f.size(); ++i) expect(bits(f[i]) == bits(want[i]), "dequantize at " + std::to_string(i));
}

// The serial reference of the two tests below: the oracle run on one thread.
void check_against_serial(const std::vector<uint16_t> &w, size_t rows, size_t cols, Scaling scaling,
                          const Quantized &par) {
    std::vector<float> absmax(rows);
    orc_row_absmax(w.data(), rows, cols, absmax.data());
    expect(absmax == row_absmax(w, rows, cols), std::string(name(scaling)) + ": row_absmax");
    std::vector<uint8_t> codes(rows * cols);
    std::vector<float> scales(rows);
    const uint32_t eb = orc_quantize_with(w.data(), rows, cols, (int)par.format, (int)scaling, 1.0f, codes.data(),
                                          scales.data(), 1);
    expect(par.exp_bias == eb, std::string(name(scaling)) + ": exp bias");
    expect(par.scales == scales, std::string(name(scaling)) + ": scales");
    expect(par.codes == codes, std::string(name(scaling)) + ": codes");
}

void the_parallel_path_agrees_with_the_serial_one() {
    const size_t rows = 512, cols = 4096;
    std::vector<uint16_t> w(rows * cols);
    for (size_t i = 0; i < w.size(); ++i) w[i] = b((float)((int)((i * 7919) % 2003) - 1000) / 977.0f);
    expect(orc_split(rows, cols) > 1, "the parallel path was not taken");
    const auto par = quantize(w, rows, cols, Fp8Format::E4M3, Scaling::PerChannel);
    std::vector<float> absmax(rows);
    orc_row_absmax(w.data(), rows, cols, absmax.data());
    for (size_t r = 0; r < rows; ++r) expect(par.scales[r] == absmax[r] / 240.0f, "scale " + std::to_string(r));
    check_against_serial(w, rows, cols, Scaling::PerChannel, par);
}

void the_parallel_path_carries_a_ragged_last_chunk() {
    const size_t rows = 67, cols = 16 * 1024;
    std::vector<uint16_t> w(rows * cols);
    for (size_t i = 0; i < w.size(); ++i) w[i] = b((float)((int)((i * 7919) % 2003) - 1000) / 977.0f);
    const int threads = orc_split(rows, cols);
    expect(threads > 1, "the parallel path was not taken");
    expect(rows % (size_t)threads != 0, "the last chunk is not ragged");
    for (Scaling s : {Scaling::PerChannel, Scaling::HwExpBias, Scaling::Unit}) {
        const auto par = quantize(w, rows, cols, Fp8Format::E4M3, s);
        check_against_serial(w, rows, cols, s, par);
        bool any = false;
        for (size_t i = (rows - 1) * cols; i < rows * cols; ++i) any |= par.codes[i] != 0;
        expect(any, std::string(name(s)) + ": the last row was never encoded");
    }
}

void the_hardware_bias_scheme_is_the_identity_for_e5m2() {
    const size_t rows = 4, cols = 32;
    std::vector<uint16_t> w(rows * cols);
    for (size_t i = 0; i < w.size(); ++i) w[i] = b((float)((int)((i * 37) % 101) - 50) / 13.0f);
    const auto hw = quantize(w, rows, cols, Fp8Format::E5M2, Scaling::HwExpBias);
    const auto unit = quantize(w, rows, cols, Fp8Format::E5M2, Scaling::Unit);
    expect(hw.exp_bias == exponent_bias(Fp8Format::E5M2), "exp bias");
    expect(hw.scales == std::vector<float>(rows, 1.0f), "scales");
    expect(hw.codes == unit.codes, "codes");
}

void sampling_agrees_with_the_full_error_pass() {
    const size_t rows = 16, cols = 64;
    std::vector<uint16_t> w(rows * cols);
    for (size_t i = 0; i < w.size(); ++i) w[i] = b((float)((int)((i * 37) % 101) - 50) / 50.0f);
    const auto q = quantize(w, rows, cols, Fp8Format::E4M3, Scaling::PerChannel);
    const auto all = row_errors(w, q);
    expect(sample_row_errors(w, q, rows) == all, "every row");
    const auto s = sample_row_errors(w, q, 4);
    expect(s.size() == 4, "four rows");
    for (size_t k = 0; k < s.size(); ++k) expect(s[k] == all[k * 4], "sample " + std::to_string(k));
    expect(sample_row_errors(w, q, 1000).size() == rows, "more rows than there are");
    // Against the oracle.
    std::vector<float> mean(rows), mx(rows);
    orc_row_errors(w.data(), q.codes.data(), q.scales.data(), rows, cols, (int)q.format, mean.data(), mx.data());
    for (size_t r = 0; r < rows; ++r)
        expect(all[r].max_rel == mx[r] && std::fabs(all[r].mean_rel - mean[r]) <= 3e-7f * mean[r],
               "row " + std::to_string(r) + " against the oracle");
}

void zero_rows_keep_a_unit_scale() {
    const std::vector<uint16_t> w(8, 0);
    const auto q = quantize(w, 2, 4, Fp8Format::E4M3, Scaling::PerChannel);
    expect(q.scales == std::vector<float>{1.0f, 1.0f}, "unit scales");
    expect(q.codes == std::vector<uint8_t>(8, 0), "zero codes");
    const auto e = row_errors(w, q);
    expect(e[0] == RowError{0.0f, 0.0f}, "zero error");
}

void a_backoff_leaves_headroom() {
    std::vector<uint16_t> w;
    for (float x : {1.0f, -0.5f, 0.25f, 0.125f}) w.push_back(b(x));
    const auto q = quantize_with(w, 1, 4, Fp8Format::E4M3, Scaling::PerChannel, 0.5f);
    expect(q.scales[0] == 1.0f / 120.0f, "scale");
    expect(q.codes[0] == 0x6f, "code " + hex(q.codes[0]));
    expect(decode(q.codes[0], Fp8Format::E4M3) == 120.0f, "value");
}

// ------------------------------------------------------------------ device tests (fixtures.rs)

void scales_match_torchs_input_bit_for_bit() {
    for (const Case &c : cases()) {
        const auto q = quantized(c);
        expect(q.rows == c.rows, c.name);
        expect(q.exp_bias == c.exp_bias, c.name + " exponent bias");
        for (size_t r = 0; r < c.rows; ++r)
            expect(bits(q.scales[r]) == bits(c.scales[r]), c.name + " scale " + std::to_string(r));
    }
}

void codes_match_the_torch_cast() {
    for (const Case &c : cases()) {
        const auto q = quantized(c);
        expect(q.codes.size() == c.codes.size(), c.name);
        size_t bad = 0, first = 0;
        for (size_t i = 0; i < q.codes.size(); ++i)
            if (q.codes[i] != c.codes[i] && bad++ == 0) first = i;
        expect(bad == 0, c.name + ": " + std::to_string(bad) + " of " + std::to_string(q.codes.size()) +
                             " codes differ, first at " + std::to_string(first));
    }
}

void the_only_divergence_from_torch_is_the_saturation() {
    int checked = 0;
    for (const Case &c : cases()) {
        if (!c.has_torch_raw) continue;
        ++checked;
        const auto q = quantized(c);
        const uint8_t reserved = c.fmt == Fp8Format::E4M3 ? 0x78 : 0x7c;
        int saturated = 0;
        for (size_t i = 0; i < q.codes.size(); ++i) {
            const uint8_t ours = q.codes[i], theirs = c.torch_raw[i];
            if ((theirs & reserved) == reserved) {
                ++saturated;
                expect(ours == ((theirs & 0x80) | max_finite_code(c.fmt)), c.name + " index " + std::to_string(i));
            } else {
                expect(ours == theirs, c.name + " index " + std::to_string(i));
            }
        }
        expect(saturated > 0, c.name + ": nothing saturated");
    }
    expect(checked >= 2, "no saturation cases in the fixture");
}

void row_error_statistics_match_numpy() {
    for (const Case &c : cases()) {
        const auto q = quantized(c);
        const auto errs = row_errors(c.w, q);
        expect(errs.size() == c.mean_rel.size(), c.name);
        for (size_t r = 0; r < errs.size(); ++r) {
            const double wm = c.mean_rel[r], wx = c.max_rel[r];
            expect(std::fabs((double)errs[r].mean_rel - wm) <= 1e-6 + 1e-5 * wm,
                   c.name + " row " + std::to_string(r) + ": mean_rel " + num(errs[r].mean_rel) + " against " + num(wm));
            expect(std::fabs((double)errs[r].max_rel - wx) <= 1e-6 + 1e-5 * wx,
                   c.name + " row " + std::to_string(r) + ": max_rel " + num(errs[r].max_rel) + " against " + num(wx));
        }
    }
}

void checkpoint_rows_quantize_within_the_formats_resolution() {
    int seen = 0;
    for (const Case &c : cases()) {
        if (c.name.rfind("ckpt_", 0) != 0 || c.scaling != Scaling::PerChannel) continue;
        ++seen;
        const auto q = quantized(c);
        const auto errs = row_errors(c.w, q);
        for (size_t r = 0; r < errs.size(); ++r) {
            expect(errs[r].mean_rel < 0.03f, c.name + " row " + std::to_string(r) + ": mean " + num(errs[r].mean_rel));
            expect(errs[r].max_rel <= 0.25f, c.name + " row " + std::to_string(r) + ": max " + num(errs[r].max_rel));
        }
        const auto back = q.dequantize();
        for (size_t r = 0; r < q.rows; ++r) {
            const size_t base = r * q.cols;
            float am = 0.0f;
            size_t ai = 0;
            for (size_t i = 0; i < q.cols; ++i) {
                const float v = std::fabs(bf16_to_f32(c.w[base + i]));
                if (v > am) {
                    am = v;
                    ai = i;
                }
            }
            const float want = bf16_to_f32(c.w[base + ai]), got = back[base + ai];
            expect(std::fabs(got - want) <= std::fabs(want) * 1e-6f,
                   c.name + " row " + std::to_string(r) + ": absmax weight " + num(want) + " came back as " + num(got));
        }
    }
    expect(seen >= 3, "no per-channel checkpoint cases");
}

// ------------------------------------------------------------------ the consumer side

std::vector<uint16_t> pseudo_bf16(size_t n, uint64_t seed, float amp) {
    std::vector<uint16_t> out(n);
    uint64_t s = seed * 0x9e3779b97f4a7c15ull + 1;
    for (size_t i = 0; i < n; ++i) {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        const float u = (float)((s >> 11) & 0xffffff) / 16777216.0f - 0.5f;
        out[i] = b(u * amp);
    }
    return out;
}

std::vector<float> to_f32(const std::vector<uint16_t> &v) {
    std::vector<float> out(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = bf16_to_f32(v[i]);
    return out;
}

void gemm_w8a16_matches_the_host_matmul() {
    const size_t N = 384, K = 1024;
    for (Fp8Format f : {Fp8Format::E4M3, Fp8Format::E5M2})
        for (Scaling s : {Scaling::PerChannel, Scaling::HwExpBias})
            for (size_t m : {1, 3, 8, 40}) {
                const auto w = pseudo_bf16(N * K, 7 + m, 0.08f);
                const auto x = pseudo_bf16(m * K, 100 + m, 2.0f);
                const auto q = quantize(w, N, K, f, s);
                const auto y = gemm_w8a16(x, m, q);
                const auto deq = q.dequantize();
                const auto xf = to_f32(x);
                std::vector<float> want(m * N);
                orc_gemm(xf.data(), deq.data(), m, K, N, want.data(), 8);
                const float rel = orc_rel_l2(y.data(), want.data(), m * N);
                expect(rel < 1e-2f, std::string(name(f)) + ":" + name(s) + " m=" + std::to_string(m) +
                                        " rel-L2 " + num(rel));
            }
}

void gemm_fp8_scaled_matches_the_host_matmul() {
    // A: pcs-quantized activations [K, m]; B: an hw-biased weight [K, N]
    // with transpose_b, its exponent bias carried as metadata.
    const size_t m = 256, N = 384, K = 512;
    const auto x = pseudo_bf16(m * K, 3, 4.0f);
    const auto w = pseudo_bf16(N * K, 5, 0.05f);
    const auto qa = quantize(x, m, K, Fp8Format::E4M3, Scaling::PerChannel);
    const auto qb = quantize(w, N, K, Fp8Format::E4M3, Scaling::HwExpBias);
    expect(qb.exp_bias != exponent_bias(Fp8Format::E4M3), "the weight did not take a non-default bias");
    const Fp8Operand a{"x", {K, m}, &qa.codes, qa.format, qa.exp_bias};
    const Fp8Operand bo{"w", {K, N}, &qb.codes, qb.format, qb.exp_bias};
    const auto y = gemm_fp8_scaled(a, bo, qa.scale_operand(), qb.scale_operand(), {N, m}, true);
    const auto da = qa.dequantize(), db = qb.dequantize();
    std::vector<float> want(m * N);
    orc_gemm(da.data(), db.data(), m, K, N, want.data(), 8);
    const float rel = orc_rel_l2(y.data(), want.data(), m * N);
    expect(rel < 1e-2f, "rel-L2 " + num(rel));
    expect_throws<std::invalid_argument>(
        [&] { (void)gemm_fp8_scaled(a, bo, nullptr, nullptr, {N, m}, false); }, "transpose_b", "no transpose");
    expect_throws<std::invalid_argument>(
        [&] { (void)gemm_fp8_scaled(a, bo, nullptr, nullptr, {m, N}, true); }, "output must be", "output sizes");
}

struct Test {
    const char *name;
    bool device;
    void (*fn)();
};

const Test TESTS[] = {
    {"format_constants_host", false, format_constants_host},
    {"bf16_helpers_agree_with_the_oracle", false, bf16_helpers_agree_with_the_oracle},
    {"hw_exp_bias_picks_the_finest_range_that_fits_host", false, hw_exp_bias_picks_the_finest_range_that_fits_host},
    {"asserts_keep_their_messages", false, asserts_keep_their_messages},
    {"the_fixture_is_the_one_the_generator_writes", false, the_fixture_is_the_one_the_generator_writes},
    {"e4m3_codes_match_the_device_cast", true, e4m3_codes_match_the_device_cast},
    {"e5m2_codes_match_the_device_cast", true, e5m2_codes_match_the_device_cast},
    {"format_constants_device", true, format_constants_device},
    {"every_code_round_trips_through_the_encoder", true, every_code_round_trips_through_the_encoder},
    {"rounding_is_to_nearest_even", true, rounding_is_to_nearest_even},
    {"per_channel_scales_stretch_each_row_to_full_scale", true, per_channel_scales_stretch_each_row_to_full_scale},
    {"hw_exp_bias_picks_the_finest_range_that_fits", true, hw_exp_bias_picks_the_finest_range_that_fits},
    {"unit_scaling_leaves_the_codes_alone", true, unit_scaling_leaves_the_codes_alone},
    {"dequantize_of_quantize_is_within_the_format_resolution", true,
     dequantize_of_quantize_is_within_the_format_resolution},
    {"the_parallel_path_agrees_with_the_serial_one", true, the_parallel_path_agrees_with_the_serial_one},
    {"the_parallel_path_carries_a_ragged_last_chunk", true, the_parallel_path_carries_a_ragged_last_chunk},
    {"the_hardware_bias_scheme_is_the_identity_for_e5m2", true, the_hardware_bias_scheme_is_the_identity_for_e5m2},
    {"sampling_agrees_with_the_full_error_pass", true, sampling_agrees_with_the_full_error_pass},
    {"zero_rows_keep_a_unit_scale", true, zero_rows_keep_a_unit_scale},
    {"a_backoff_leaves_headroom", true, a_backoff_leaves_headroom},
    {"scales_match_torchs_input_bit_for_bit", true, scales_match_torchs_input_bit_for_bit},
    {"codes_match_the_torch_cast", true, codes_match_the_torch_cast},
    {"the_only_divergence_from_torch_is_the_saturation", true, the_only_divergence_from_torch_is_the_saturation},
    {"row_error_statistics_match_numpy", true, row_error_statistics_match_numpy},
    {"checkpoint_rows_quantize_within_the_formats_resolution", true,
     checkpoint_rows_quantize_within_the_formats_resolution},
    {"gemm_w8a16_matches_the_host_matmul", true, gemm_w8a16_matches_the_host_matmul},
    {"gemm_fp8_scaled_matches_the_host_matmul", true, gemm_fp8_scaled_matches_the_host_matmul},
};

}  // namespace

int main(int argc, char **argv) {
    bool cpu_only = false;
    std::string filter;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--cpu-only") {
            cpu_only = true;
        } else if (a == "--fixture" && i + 1 < argc) {
            g_fixture = argv[++i];
        } else {
            filter = a;
        }
    }
    int run = 0, failed = 0;
    for (const Test &t : TESTS) {
        if (cpu_only && t.device) continue;
        if (!filter.empty() && std::string(t.name).find(filter) == std::string::npos) continue;
        ++run;
        std::printf("%s ... ", t.name);
        std::fflush(stdout);
        try {
            t.fn();
            std::printf("ok\n");
        } catch (const Failure &f) {
            ++failed;
            std::printf("FAILED: %s\n", f.msg.c_str());
        } catch (const std::exception &e) {
            ++failed;
            std::printf("FAILED (exception): %s\n", e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d run, %d failed\n", run, failed);
    return failed == 0 && run > 0 ? 0 : 1;
}
