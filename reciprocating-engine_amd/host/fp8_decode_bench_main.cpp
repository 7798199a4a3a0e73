// reng-fp8-decode-bench - times the fp8 decode step (reng_model::Fp8Decoder,
// fp8_decoder.hpp) on one GPU: a stack of Llama-shaped layers with random
// finite E4M3 codes and per-row scales (no checkpoint needed), every layer
// stepped over positions 0 .. P - 1, and prints one JSON line with the mean
// time of one layer-step against the HBM bytes that step must move (the
// layer's codes and scales, and the key / value cache rows it attends over).
//
//   reng-fp8-decode-bench [--layers L] [--positions P] [--hidden H]
//                         [--intermediate I] [--heads Q] [--kv-heads KV]
//
// Defaults: the Llama-3.1-8B layer (hidden 4096, intermediate 14336, 32
// heads, 8 key/value heads, head_dim 128), 4 layers (872 MB of codes, past
// the 256 MB Infinity Cache, so every step reads its layer from HBM), 512
// positions. The layers' RoPE has no scaling (the step refuses Llama 3.1's
// rope_scaling; the kernels' cost does not depend on it).
#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fp8_decoder.hpp"

using namespace reng_model;

namespace {

const char *USAGE =
    "usage: reng-fp8-decode-bench [--layers L] [--positions P] [--hidden H] [--intermediate I] [--heads Q] "
    "[--kv-heads KV]";

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

struct Args {
    size_t layers = 4, positions = 512, hidden = 4096, inter = 14336, heads = 32, kv = 8;
};

Args parse(int argc, char **argv) {
    Args a;
    for (int i = 1; i < argc; i += 2) {
        const std::string k = argv[i];
        if (i + 1 >= argc) throw Error(k + " needs a value\n" + USAGE);
        char *end = nullptr;
        const unsigned long long v = std::strtoull(argv[i + 1], &end, 10);
        if (!*argv[i + 1] || *end != '\0' || argv[i + 1][0] == '-' || v == 0)
            throw Error(k + ": not a positive integer: " + argv[i + 1]);
        if (k == "--layers") a.layers = v;
        else if (k == "--positions") a.positions = v;
        else if (k == "--hidden") a.hidden = v;
        else if (k == "--intermediate") a.inter = v;
        else if (k == "--heads") a.heads = v;
        else if (k == "--kv-heads") a.kv = v;
        else throw Error("unknown flag " + k + "\n" + USAGE);
    }
    return a;
}

// xorshift64*: codes and scales without a library generator.
struct Rng {
    uint64_t s;
    uint64_t next() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 2685821657736338717ull;
    }
};

// A [rows, cols] E4M3 matrix of random finite codes (magnitude field <= 0x77)
// and per-row scales in [1e-3, 2e-3).
reng_fp8::Quantized random_matrix(Rng &rng, size_t rows, size_t cols) {
    reng_fp8::Quantized q;
    q.format = reng_fp8::Fp8Format::E4M3;
    q.scaling = reng_fp8::Scaling::PerChannel;
    q.rows = rows;
    q.cols = cols;
    q.codes.resize(rows * cols);
    for (size_t i = 0; i < q.codes.size(); i += 8) {
        uint64_t r = rng.next();
        for (size_t j = 0; j < 8 && i + j < q.codes.size(); ++j, r >>= 8) {
            const uint8_t b = (uint8_t)r;
            q.codes[i + j] = (uint8_t)((b & 0x80) | ((b & 0x7f) % 0x78));
        }
    }
    q.scales.resize(rows);
    for (float &s : q.scales) s = 1e-3f * (1.0f + (float)(rng.next() >> 40) / 16777216.0f);
    q.exp_bias = 7;
    return q;
}

int run(int argc, char **argv) {
    const Args a = parse(argc, argv);
    if (a.hidden % a.heads != 0 || a.heads % a.kv != 0)
        throw Error("hidden must divide into heads and heads into key/value heads");
    LlamaConfig cfg;
    cfg.model_type = "llama";
    cfg.hidden_size = a.hidden;
    cfg.intermediate_size = a.inter;
    cfg.num_hidden_layers = a.layers;
    cfg.num_attention_heads = a.heads;
    cfg.num_key_value_heads = a.kv;
    cfg.rms_norm_eps = 1e-5f;
    cfg.rope_theta = 500000.0f;
    const size_t hd = cfg.head_dim(), qd = cfg.q_dim(), kvd = a.kv * hd;

    LlamaWeights w;
    w.layers.resize(a.layers);
    for (LayerTensors &t : w.layers) t.g1 = t.g2 = std::vector<float>(a.hidden, 1.0f);
    Rng rng{0x9e3779b97f4a7c15ull};
    std::vector<LayerFp8> fp8(a.layers);
    for (LayerFp8 &l : fp8) {
        l.wq = random_matrix(rng, qd, a.hidden);
        l.wk = random_matrix(rng, kvd, a.hidden);
        l.wv = random_matrix(rng, kvd, a.hidden);
        l.wo = random_matrix(rng, a.hidden, qd);
        l.wg = random_matrix(rng, a.inter, a.hidden);
        l.wu = random_matrix(rng, a.inter, a.hidden);
        l.wd = random_matrix(rng, a.hidden, a.inter);
    }
    size_t code_bytes = 0, scale_bytes = 0;
    for (const auto &m : fp8[0].matrices()) {
        code_bytes += m.second->codes.size();
        scale_bytes += m.second->scales.size() * 4;
    }
    w.fp8 = std::move(fp8);
    Fp8Decoder dec(cfg, w, a.positions);

    // Every token enters the stack as the same row x0 (an embedding), so the
    // residual stream grows through the layers only, not across positions.
    float *x0 = nullptr, *x = nullptr;
    hip_ok(hipMalloc(&x0, a.hidden * sizeof(float)), "hipMalloc");
    hip_ok(hipMalloc(&x, a.hidden * sizeof(float)), "hipMalloc");
    std::vector<float> hx(a.hidden);
    for (float &v : hx) v = (float)((int64_t)(rng.next() >> 40) - (1 << 23)) / (float)(1 << 23);
    hip_ok(hipMemcpy(x0, hx.data(), a.hidden * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy");
    hipStream_t st = nullptr;
    hip_ok(hipStreamCreate(&st), "hipStreamCreate");
    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");

    // One untimed pass over every position, then the timed pass. A token runs
    // through the layers in order, as a decoder does.
    auto pass = [&]() {
        for (size_t p = 0; p < a.positions; ++p)
            for (size_t li = 0; li < a.layers; ++li) dec.step_device(li, li == 0 ? x0 : x, x, p, st);
    };
    pass();
    hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize");
    dec.reset();
    hip_ok(hipEventRecord(e0, st), "hipEventRecord");
    const auto t0 = std::chrono::steady_clock::now();
    pass();
    hip_ok(hipEventRecord(e1, st), "hipEventRecord");
    hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
    const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    float ms = 0.0f;
    hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
    std::vector<float> y(a.hidden);
    hip_ok(hipMemcpy(y.data(), x, a.hidden * sizeof(float), hipMemcpyDeviceToHost), "hipMemcpy");
    bool finite = true;
    for (float v : y) finite = finite && v == v && v - v == 0.0f;

    const double steps = (double)(a.layers * a.positions);
    const double us = ms * 1e3 / steps;
    // Mean cache rows attended per step: positions 0 .. P - 1 attend p + 1 rows.
    const double rows = (double)(a.positions + 1) / 2.0;
    const double bytes = (double)code_bytes + (double)scale_bytes + 2.0 * rows * (double)kvd * 2.0;
    std::printf("{\"workload\": \"fp8 decode step, Llama-shaped layer\", \"hidden\": %zu, \"intermediate\": %zu, "
                "\"heads\": %zu, \"kv_heads\": %zu, \"head_dim\": %zu, \"layers\": %zu, \"positions\": %zu, "
                "\"us_per_layer_step\": %.2f, \"tokens_per_s_per_layer\": %.0f, \"bytes_per_layer_step\": %.0f, "
                "\"GBps\": %.1f, \"hbm_frac\": %.3f, \"host_wall_s\": %.3f, "
                "\"output_finite\": %s}\n",
                a.hidden, a.inter, a.heads, a.kv, hd, a.layers, a.positions, us, 1e6 / us, bytes,
                bytes / (us * 1e-6) / 1e9, bytes / (us * 1e-6) / 8.0e12, wall, finite ? "true" : "false");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipStreamDestroy(st);
    (void)hipFree(x);
    (void)hipFree(x0);
    return finite ? 0 : 1;
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
