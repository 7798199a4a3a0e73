// reng-fp8-quantize - quantize a checkpoint's projections to fp8 (on the GPU,
// through libreng_hip.so) and report what it costs: bytes before and after
// and the relative error of the round trip. The same command line, output
// and refusals as crates/reng-model/src/bin/fp8_quantize.rs:1-141.
//
//   reng-fp8-quantize <model_dir> [--fp8 <spec>] [--per-matrix] [--layers <n>] [--save]
//
// <spec> is the value the RENG_FP8 switch takes: a format (e4m3, e5m2), a
// scale scheme (pcs, hw, unit) and backoff=<f32>, colon- or comma-separated;
// the default is e4m3:pcs. --per-matrix prints a line per matrix of the first
// --layers layers (default 1) as well as the totals. --save, which the
// reference does not have, also writes the codes and scales beside the
// checkpoint (model.fp8.safetensors, read back by load_weights_fp8_cached).
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "reng_model.hpp"

using namespace reng_model;

namespace {

const char *USAGE = "usage: reng-fp8-quantize <model_dir> [--fp8 <spec>] [--per-matrix] [--layers <n>] [--save]";

struct Args {
    std::string dir;
    Fp8Config fp8;
    bool per_matrix = false;
    bool save = false;
    size_t layers = 1;
};

Args parse_args(int argc, char **argv) {
    std::vector<std::string> a(argv + 1, argv + argc);
    if (a.empty()) throw Error(USAGE);
    if (a[0][0] == '-') throw Error("the model directory comes first, not \"" + a[0] + "\"\n" + USAGE);
    Args out;
    out.dir = a[0];
    // The environment first, so RENG_FP8=e5m2 works here as everywhere; an
    // off value leaves this binary nothing to do, so it says so.
    const char *env = std::getenv("RENG_FP8");
    auto sw = fp8_switch(env ? std::optional<std::string_view>(env) : std::nullopt, true);
    if (!sw)
        throw Error(std::string("RENG_FP8=") + (env ? env : "") +
                    " turns the fp8 switch off and reng-fp8-quantize does nothing else; unset it or pass "
                    "--fp8 <spec>");
    out.fp8 = *sw;
    for (size_t i = 1; i < a.size();) {
        if (a[i] == "--per-matrix") {
            out.per_matrix = true;
            i += 1;
        } else if (a[i] == "--save") {
            out.save = true;
            i += 1;
        } else if (a[i] == "--fp8") {
            if (i + 1 >= a.size()) throw Error(USAGE);
            auto c = fp8_switch(a[i + 1], true);
            if (!c) throw Error("--fp8 " + a[i + 1] + ": that switch is off");
            out.fp8 = *c;
            i += 2;
        } else if (a[i] == "--layers") {
            if (i + 1 >= a.size()) throw Error(USAGE);
            char *end = nullptr;
            const unsigned long long n = std::strtoull(a[i + 1].c_str(), &end, 10);
            if (a[i + 1].empty() || *end != '\0' || a[i + 1][0] == '-')
                throw Error("--layers: invalid digit found in string");
            out.layers = (size_t)n;
            i += 2;
        } else {
            throw Error("unknown flag " + a[i] + "\n" + USAGE);
        }
    }
    return out;
}

int run(int argc, char **argv) {
    const Args a = parse_args(argc, argv);
    const LlamaConfig cfg = LlamaConfig::load(a.dir);
    const auto t0 = std::chrono::steady_clock::now();
    LlamaWeights w = load_weights(a.dir, cfg);
    std::printf("%s: %zu layers, hidden %zu, intermediate %zu, loaded in %.2f s\n", a.dir.c_str(),
                cfg.num_hidden_layers, cfg.hidden_size, cfg.intermediate_size,
                std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    std::printf("fp8 scheme: %s\n", a.fp8.to_string().c_str());
    const Fp8Report report = w.quantize_fp8(cfg, a.fp8);
    std::printf("fp8: %s\n", report.to_string().c_str());
    const double gib = (double)(1u << 30);
    const double after = (double)(report.fp8_bytes + report.scale_bytes);
    std::printf("projection bytes: %.3f GiB -> %.3f GiB (%.2fx, %.3f GiB saved)\n", report.bf16_bytes / gib,
                after / gib, report.bf16_bytes / after, (report.bf16_bytes - after) / gib);
    if (a.save) {
        save_fp8(a.dir, w, a.fp8, report);
        std::printf("saved %s/%s\n", a.dir.c_str(), FP8_CODES_FILE);
    }
    if (a.per_matrix) {
        const auto &fp8 = *w.fp8;
        for (size_t li = 0; li < fp8.size() && li < a.layers; ++li) {
            const LayerTensors &l = w.layers[li];
            const Bf16Slice *bf16[7] = {&l.wq, &l.wk, &l.wv, &l.wo, &l.wg, &l.wu, &l.wd};
            const auto mats = fp8[li].matrices();
            for (size_t k = 0; k < mats.size(); ++k) {
                const reng_fp8::Quantized &q = *mats[k].second;
                const Bf16Slice &src = *bf16[k];
                const auto errs = reng_fp8::sample_row_errors(src.data(), src.size(), q, FP8_ERROR_ROWS);
                double mean = 0.0;
                float mx = 0.0f;
                for (const auto &e : errs) {
                    mean += (double)e.mean_rel;
                    mx = std::max(mx, e.max_rel);
                }
                mean /= (double)std::max<size_t>(errs.size(), 1);
                float absmax = 0.0f;
                for (float v : reng_fp8::row_absmax(src.data(), src.size(), q.rows, q.cols)) absmax = std::max(absmax, v);
                std::printf("  l%zu %-3s [%zu, %zu] bias %u absmax %.4f mean_rel %.4f max_rel %.4f\n", li, mats[k].first,
                            q.rows, q.cols, q.exp_bias, (double)absmax, mean, (double)mx);
            }
        }
    }
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    try {
        return run(argc, argv);
    } catch (const std::exception &e) {
        std::fprintf(stderr, "Error: %s\n", e.what());
        return 1;
    }
}
