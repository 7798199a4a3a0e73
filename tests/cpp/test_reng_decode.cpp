// test_reng_decode.cpp - drives reng_model::Fp8Decoder (reciprocating-engine_amd/host/
// fp8_decoder.hpp) for tests/test_gpu_decode.py.
//
//   test_reng_decode --refusals <model_dir>
//       (host only) the configurations the decode step refuses, each with its message
//   test_reng_decode <model_dir> <in.f32> <out.f32> <tokens> [--fp8 <spec>] [--cached]
//       loads the checkpoint with the fp8 switch on, runs every layer over
//       positions 0 .. tokens - 1 on the rows of in ([tokens, hidden] f32) and
//       writes out ([layers, tokens, hidden] f32); --cached takes the codes
//       from the model directory's saved codes file and fails if it is not
//       current
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../include/reng_hip.h"
#include "../../reciprocating-engine_amd/host/fp8_decoder.hpp"

using namespace reng_model;

namespace {

int failures = 0;

void expect_error(const std::string &what, const std::function<void()> &f, const std::string &needle) {
    try {
        f();
    } catch (const Error &e) {
        if (std::string(e.what()).find(needle) != std::string::npos) {
            std::printf("%-44s ok: %s\n", what.c_str(), e.what());
            return;
        }
        std::printf("%-44s FAILED: message '%s' lacks '%s'\n", what.c_str(), e.what(), needle.c_str());
        ++failures;
        return;
    }
    std::printf("%-44s FAILED: no error\n", what.c_str());
    ++failures;
}

int refusals(const std::string &dir) {
    const LlamaConfig cfg = LlamaConfig::load(dir);
    // bf16 weights only: no codes to decode from.
    const LlamaWeights plain = load_weights(dir, cfg);
    expect_error("weights without fp8 codes", [&] { Fp8Decoder d(cfg, plain, 8); }, "carry no fp8 codes");
    LlamaWeights w = plain;
    w.fp8.emplace();   // shapes are checked after the config, so an empty set suffices here
    auto with = [&](const std::function<void(LlamaConfig &)> &edit) {
        return [&, edit] {
            LlamaConfig c = cfg;
            edit(c);
            Fp8Decoder d(c, w, 8);
        };
    };
    expect_error("model_type qwen2", with([](LlamaConfig &c) { c.model_type = "qwen2"; }), "model_type qwen2");
    expect_error("rope_scaling", with([](LlamaConfig &c) { c.has_rope_scaling = true; }), "rope_scaling");
    expect_error("sliding_window", with([](LlamaConfig &c) { c.sliding_window = 4096; }), "sliding_window");
    expect_error("query_pre_attn_scalar", with([](LlamaConfig &c) { c.query_pre_attn_scalar = 256.0f; }),
                 "attention scale override");
    expect_error("odd head_dim", with([](LlamaConfig &c) { c.head_dim_ = 15; }), "is not even");
    expect_error("heads not a multiple of kv heads", with([](LlamaConfig &c) { c.num_key_value_heads = 3; }),
                 "not a multiple");
    expect_error("no positions", [&] { Fp8Decoder d(cfg, w, 0); }, "max_positions 0");
    expect_error("too many positions", [&] { Fp8Decoder d(cfg, w, RENG_HIP_ATTENTION_MAX_LEN + 1); },
                 "max_positions");
    expect_error("fp8 layers do not match", [&] { Fp8Decoder d(cfg, w, 8); }, "fp8 layers do not match");
    // A hidden row past the GEMV's LDS stage (checked before any shape or device work).
    LlamaWeights wide = plain;
    wide.fp8.emplace(plain.layers.size());
    expect_error("hidden_size past 32768", [&] {
        LlamaConfig c = cfg;
        c.hidden_size = 40960;
        Fp8Decoder d(c, wide, 8);
    }, "hidden_size 40960");
    std::printf("%d failed\n", failures);
    return failures ? 1 : 0;
}

std::vector<float> read_f32(const std::string &path, size_t n) {
    std::vector<float> v(n);
    FILE *f = std::fopen(path.c_str(), "rb");
    if (!f || std::fread(v.data(), 4, n, f) != n) throw Error("cannot read " + path);
    std::fclose(f);
    return v;
}

}  // namespace

int main(int argc, char **argv) {
    try {
        if (argc == 3 && std::string(argv[1]) == "--refusals") return refusals(argv[2]);
        std::optional<Fp8Config> fp8 = Fp8Config{};
        bool cached = false, usage = argc < 5;
        for (int i = 5; i < argc && !usage; ++i) {
            const std::string a = argv[i];
            if (a == "--fp8" && i + 1 < argc) fp8 = fp8_switch(std::string_view(argv[++i]), true);
            else if (a == "--cached") cached = true;
            else usage = true;
        }
        if (usage) {
            std::fprintf(stderr,
                         "usage: test_reng_decode <model_dir> <in.f32> <out.f32> <tokens> [--fp8 <spec>] [--cached]\n");
            return 2;
        }
        const std::string dir = argv[1];
        const size_t tokens = std::strtoull(argv[4], nullptr, 10);
        const LlamaConfig cfg = LlamaConfig::load(dir);
        Fp8Load loaded;
        if (cached) {
            loaded = load_weights_fp8_cached(dir, cfg, fp8, false);
            if (!loaded.from_file) throw Error(std::string("no current ") + FP8_CODES_FILE + " in " + dir);
            std::printf("codes from %s\n", FP8_CODES_FILE);
        } else {
            auto [fresh, report] = load_weights_fp8(dir, cfg, fp8);
            loaded.weights = std::move(fresh);
            loaded.report = report;
        }
        const LlamaWeights &w = loaded.weights;
        if (loaded.report) std::printf("%s\n", loaded.report->to_string().c_str());
        Fp8Decoder dec(cfg, w, tokens);
        const size_t hidden = cfg.hidden_size;
        const std::vector<float> in = read_f32(argv[2], tokens * hidden);
        std::vector<float> out;
        out.reserve(dec.layers() * tokens * hidden);
        for (size_t li = 0; li < dec.layers(); ++li)
            for (size_t p = 0; p < tokens; ++p) {
                const std::vector<float> x(in.begin() + p * hidden, in.begin() + (p + 1) * hidden);
                const std::vector<float> y = dec.step(li, x, p);
                out.insert(out.end(), y.begin(), y.end());
            }
        // A position out of order is refused.
        try {
            (void)dec.step(0, std::vector<float>(hidden, 0.0f), 0);
            std::fprintf(stderr, "a repeated position was not refused\n");
            return 1;
        } catch (const Error &) {
        }
        FILE *f = std::fopen(argv[3], "wb");
        if (!f || std::fwrite(out.data(), 4, out.size(), f) != out.size()) throw Error("cannot write output");
        std::fclose(f);
        std::printf("decoded %zu layers x %zu positions\n", dec.layers(), tokens);
        return 0;
    } catch (const std::exception &e) {
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
