// test_reng_model.cpp - the fp8 slice of reng-model in C++ (reciprocating-engine_amd/host/
// reng_model.hpp) against the reference crate's own tests
// (crates/reng-model/src/lib.rs:4437-4606: write_tiny_llama, the switch, the
// switch off, the switch on) plus the safetensors loader's edge cases and a
// bit-for-bit comparison of every quantized projection with the CPU oracle.
//
//   test_reng_model [--cpu-only] [NAME_SUBSTRING]
#include <dirent.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "../../oracle/fp8_oracle.h"
#include "../../reciprocating-engine_amd/host/fp8_probe.hpp"
#include "../../reciprocating-engine_amd/host/reng_model.hpp"

using namespace reng_model;
using reng_fp8::Fp8Format;
using reng_fp8::Scaling;

namespace {

struct Failure {
    std::string msg;
};

void expect(bool ok, const std::string &msg) {
    if (!ok) throw Failure{msg};
}

template <typename E = Error>
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

// A fresh temporary directory, removed (with its files) at scope exit.
struct TempDir {
    std::string path;
    TempDir() {
        char tmpl[] = "/tmp/reng_model_test_XXXXXX";
        const char *p = mkdtemp(tmpl);
        if (!p) throw Failure{"mkdtemp failed"};
        path = p;
    }
    ~TempDir() {
        DIR *d = opendir(path.c_str());
        if (d) {
            while (dirent *e = readdir(d)) {
                const std::string n = e->d_name;
                if (n != "." && n != "..") unlink((path + "/" + n).c_str());
            }
            closedir(d);
        }
        rmdir(path.c_str());
    }
};

void write_file(const std::string &path, const std::string &bytes) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) throw Failure{"cannot write " + path};
    std::fwrite(bytes.data(), 1, bytes.size(), f);
    std::fclose(f);
}

struct T {
    std::string name;
    std::string dtype;               // BF16, F32, F16
    std::vector<size_t> shape;
    std::string data;                // little-endian bytes
};

// A safetensors file of the given tensors, in order; pad_odd puts one byte
// before the data section's first tensor (an odd offset).
std::string safetensors_bytes(const std::vector<T> &ts, bool pad_odd = false) {
    std::string data;
    if (pad_odd) data.push_back('\0');
    std::string header = "{";
    for (size_t i = 0; i < ts.size(); ++i) {
        const size_t start = data.size();
        data += ts[i].data;
        std::string shape = "[";
        for (size_t k = 0; k < ts[i].shape.size(); ++k) shape += (k ? ", " : "") + std::to_string(ts[i].shape[k]);
        shape += "]";
        header += (i ? "," : "") + std::string("\"") + ts[i].name + "\":{\"dtype\":\"" + ts[i].dtype +
                  "\",\"shape\":" + shape + ",\"data_offsets\":[" + std::to_string(start) + "," +
                  std::to_string(data.size()) + "]}";
    }
    header += "}";
    while (header.size() % 8 != 0) header.push_back(' ');
    std::string out(8, '\0');
    uint64_t n = header.size();
    for (int i = 0; i < 8; ++i) out[i] = (char)((n >> (8 * i)) & 0xff);
    return out + header + data;
}

std::string bf16_bytes(const std::vector<uint16_t> &v) {
    std::string s(v.size() * 2, '\0');
    std::memcpy(&s[0], v.data(), s.size());
    return s;
}

// write_tiny_llama (lib.rs:4437-4500): one layer, hidden 8, intermediate 16,
// every tensor bf16 from the same LCG, one large weight per tensor.
LlamaConfig write_tiny_llama(const std::string &dir) {
    const std::string cfg_text =
        "{\"model_type\": \"llama\", \"hidden_size\": 8, \"intermediate_size\": 16,\n"
        " \"num_hidden_layers\": 1, \"num_attention_heads\": 2,\n"
        " \"num_key_value_heads\": 2, \"rms_norm_eps\": 1e-5, \"vocab_size\": 8,\n"
        " \"tie_word_embeddings\": true}";
    write_file(dir + "/config.json", cfg_text);
    const std::vector<std::pair<std::string, std::vector<size_t>>> tensors = {
        {"model.embed_tokens.weight", {8, 8}},
        {"model.layers.0.input_layernorm.weight", {8}},
        {"model.layers.0.post_attention_layernorm.weight", {8}},
        {"model.layers.0.self_attn.q_proj.weight", {8, 8}},
        {"model.layers.0.self_attn.k_proj.weight", {8, 8}},
        {"model.layers.0.self_attn.v_proj.weight", {8, 8}},
        {"model.layers.0.self_attn.o_proj.weight", {8, 8}},
        {"model.layers.0.mlp.gate_proj.weight", {16, 8}},
        {"model.layers.0.mlp.up_proj.weight", {16, 8}},
        {"model.layers.0.mlp.down_proj.weight", {8, 16}},
        {"model.norm.weight", {8}},
    };
    std::vector<T> ts;
    uint32_t seed = 1;
    for (const auto &t : tensors) {
        size_t n = 1;
        for (size_t d : t.second) n *= d;
        std::vector<uint16_t> v(n);
        for (size_t k = 0; k < n; ++k) {
            seed = seed * 1664525u + 1013904223u;
            float x = (float)(seed >> 8) / 65535.0f / 256.0f - 0.5f;
            if (k == 0) x = x * 30.0f;
            v[k] = reng_fp8::f32_to_bf16(x);
        }
        ts.push_back(T{t.first, "BF16", t.second, bf16_bytes(v)});
    }
    write_file(dir + "/model.safetensors", safetensors_bytes(ts));
    return LlamaConfig::load(dir);
}

// w.fp8 as the oracle quantizes w's projections with q (host only), and the
// report of that pass with made-up error figures.
Fp8Report oracle_fp8(const LlamaConfig &cfg, LlamaWeights &w, const Fp8Config &q) {
    (void)cfg;
    Fp8Report r;
    std::vector<LayerFp8> out(w.layers.size());
    for (size_t l = 0; l < w.layers.size(); ++l) {
        const LayerTensors &t = w.layers[l];
        const Bf16Slice *src[7] = {&t.wq, &t.wk, &t.wv, &t.wo, &t.wg, &t.wu, &t.wd};
        reng_fp8::Quantized *dst[7] = {&out[l].wq, &out[l].wk, &out[l].wv, &out[l].wo,
                                       &out[l].wg, &out[l].wu, &out[l].wd};
        const size_t hid = cfg.hidden_size, inter = cfg.intermediate_size, qd = cfg.q_dim();
        const size_t kvd = cfg.n_kv_heads() * cfg.head_dim();
        const size_t rows[7] = {qd, kvd, kvd, hid, inter, inter, hid};
        for (size_t k = 0; k < 7; ++k) {
            reng_fp8::Quantized &x = *dst[k];
            x.format = q.format;
            x.scaling = q.scaling;
            x.rows = rows[k];
            x.cols = src[k]->size() / rows[k];
            x.codes.resize(x.rows * x.cols);
            x.scales.resize(x.rows);
            const std::vector<uint16_t> wv = src[k]->to_vector();
            x.exp_bias = orc_quantize_with(wv.data(), x.rows, x.cols, (int)q.format, (int)q.scaling, q.backoff,
                                           x.codes.data(), x.scales.data(), 8);
            r.matrices += 1;
            r.bf16_bytes += wv.size() * 2;
            r.fp8_bytes += x.codes.size();
            r.scale_bytes += x.scales.size() * 4;
        }
    }
    r.mean_rel = 0.0123f;
    r.max_rel = 0.0456f;
    r.secs = 1.5;
    w.fp8 = std::move(out);
    return r;
}

// ------------------------------------------------------------------ host-only

void the_fp8_switch_reads_the_variable_and_the_flag() {
    expect(!fp8_switch(std::nullopt, false).has_value(), "off by default");
    for (const char *off : {"", "0", "off", "false", "no", " OFF "}) {
        expect(!fp8_switch(std::string_view(off), false).has_value(), std::string("off: ") + off);
        expect(!fp8_switch(std::string_view(off), true).has_value(), std::string("off with flag: ") + off);
    }
    const Fp8Config def;
    expect(fp8_switch(std::nullopt, true) == def, "flag alone");
    for (const char *on : {"1", "on", "true", "YES"}) expect(fp8_switch(std::string_view(on), false) == def, on);
    expect(def.format == Fp8Format::E4M3 && def.scaling == Scaling::PerChannel, "defaults");
    expect(def.to_string() == "e4m3/pcs backoff 1", "display: " + def.to_string());
    auto c = fp8_switch(std::string_view("e5m2:hw"), false).value();
    expect(c.format == Fp8Format::E5M2 && c.scaling == Scaling::HwExpBias, "e5m2:hw");
    c = fp8_switch(std::string_view("unit,backoff=0.5"), false).value();
    expect(c.scaling == Scaling::Unit && c.backoff == 0.5f, "unit,backoff=0.5");
    expect(c.to_string() == "e4m3/unit backoff 0.5", "display: " + c.to_string());
    expect_throws([] { (void)fp8_switch(std::string_view("e4m3:banana"), false); },
                  "RENG_FP8: unknown setting \"banana\" (expected a format, a scale scheme or backoff=<f32>)",
                  "banana");
    expect_throws([] { (void)fp8_switch(std::string_view("backoff=0"), false); }, "RENG_FP8 backoff 0 is not in (0, 1]",
                  "backoff=0");
    expect_throws([] { (void)fp8_switch(std::string_view("backoff=2"), false); }, "RENG_FP8 backoff 2 is not in (0, 1]",
                  "backoff=2");
    expect_throws([] { (void)fp8_switch(std::string_view("backoff=x"), false); }, "RENG_FP8 backoff: ", "backoff=x");
    // Separators and whitespace in any combination, and the later word wins.
    c = fp8_switch(std::string_view(" hf8 , :expbias: backoff=0.25,f8 "), false).value();
    expect(c.format == Fp8Format::E5M2 && c.scaling == Scaling::HwExpBias && c.backoff == 0.25f, "mixed words");
}

void take_fp8_flag_removes_every_copy() {
    std::vector<std::string> a = {"model", "--fp8", "--layers", "2", "--fp8"};
    expect(take_fp8_flag(a), "had the flag");
    expect((a == std::vector<std::string>{"model", "--layers", "2"}), "flag removed");
    expect(!take_fp8_flag(a), "no flag left");
}

void f32_display_is_the_shortest_round_trip() {
    expect(f32_shortest(1.0f) == "1", "1");
    expect(f32_shortest(0.5f) == "0.5", "0.5");
    expect(f32_shortest(0.1f) == "0.1", "0.1");
    expect(f32_shortest(1.0f / 3.0f) == "0.33333334", f32_shortest(1.0f / 3.0f));
    expect(f32_shortest(1e-7f) == "0.0000001", f32_shortest(1e-7f));
    expect(f32_shortest(1e20f) == "100000000000000000000", f32_shortest(1e20f));
    expect(f32_shortest(-2.5f) == "-2.5", "-2.5");
}

void the_config_is_read_and_checked() {
    const std::string base = "\"hidden_size\": 64, \"intermediate_size\": 128, \"num_hidden_layers\": 2, "
                             "\"num_attention_heads\": 4, \"rms_norm_eps\": 1e-6, \"vocab_size\": 100";
    LlamaConfig c = LlamaConfig::from_json("{" + base + "}");
    expect(c.n_kv_heads() == 4 && c.head_dim() == 16 && c.q_dim() == 64 && !c.tied(), "llama defaults");
    c = LlamaConfig::from_json("{" + base + ", \"num_key_value_heads\": 2, \"head_dim\": 32}");
    expect(c.n_kv_heads() == 2 && c.head_dim() == 32 && c.q_dim() == 128, "explicit head_dim");
    c = LlamaConfig::from_json("{\"model_type\": \"gemma2\", " + base + "}");
    expect(c.tied(), "gemma ties by default");
    expect_throws([] { (void)LlamaConfig::from_json("{\"hidden_size\": 8}"); }, "missing field `intermediate_size`",
                  "missing field");
    for (const char *k : {"residual_multiplier", "logits_scaling", "final_logit_softcapping"})
        expect_throws([&] { (void)LlamaConfig::from_json("{" + base + ", \"" + k + "\": 2.0}"); },
                      std::string(k) + " is not supported", k);
    expect_throws([&] { (void)LlamaConfig::from_json("{" + base + ", \"mlp_bias\": true}"); },
                  "mlp_bias is not supported", "mlp_bias");
}

void safetensors_views_convert_and_refuse() {
    TempDir d;
    // bf16 in place, f32 and f16 converted, an odd offset copied.
    const std::vector<uint16_t> b = {0x3f80, 0xc000, 0x0000, 0x4049};
    const float f[3] = {1.5f, -0.1f, 3.0e38f};
    std::string fb(12, '\0');
    std::memcpy(&fb[0], f, 12);
    const uint16_t h[3] = {0x3c00, 0xc000, 0x0001};   // 1, -2, 2^-24
    std::string hb(6, '\0');
    std::memcpy(&hb[0], h, 6);
    write_file(d.path + "/a.safetensors",
               safetensors_bytes({{"b", "BF16", {2, 2}, bf16_bytes(b)}, {"f", "F32", {3}, fb}, {"h", "F16", {3}, hb}}));
    Checkpoint ck = Checkpoint::open_file(d.path + "/a.safetensors");
    const Bf16Slice sb = ck.bf16("b");
    expect(sb.is_mapped() && sb.size() == 4 && sb.to_vector() == b, "bf16 in place");
    expect(sb.sub(2, 2).to_vector() == std::vector<uint16_t>({0x0000, 0x4049}) && sb.sub(2, 2).is_mapped(), "sub view");
    const Bf16Slice sf = ck.bf16("f");
    expect(!sf.is_mapped() && sf.owned_bytes() == 6, "f32 converted");
    for (int i = 0; i < 3; ++i) expect(sf[i] == reng_fp8::f32_to_bf16(f[i]), "f32 -> bf16 " + std::to_string(i));
    const auto hf = ck.f32("h");
    expect(hf[0] == 1.0f && hf[1] == -2.0f && hf[2] == std::ldexp(1.0f, -24), "f16 -> f32");
    expect(ck.f32("b")[3] == reng_fp8::bf16_to_f32(0x4049), "bf16 -> f32");
    expect_throws([&] { (void)ck.linear("b", 4, 1); }, "shape [2, 2], expected [4, 1]", "linear shape");
    expect_throws([&] { (void)ck.info("nope"); }, "not in the checkpoint", "missing tensor");

    write_file(d.path + "/odd.safetensors", safetensors_bytes({{"b", "BF16", {4}, bf16_bytes(b)}}, true));
    const Bf16Slice so = Checkpoint::open_file(d.path + "/odd.safetensors").bf16("b");
    expect(!so.is_mapped() && so.to_vector() == b, "odd offset copied");

    // A header whose byte range disagrees with dtype x shape, and one past the file.
    std::string bad = safetensors_bytes({{"b", "BF16", {2, 3}, bf16_bytes(b)}});
    write_file(d.path + "/bad.safetensors", bad);
    expect_throws([&] { (void)Checkpoint::open_file(d.path + "/bad.safetensors"); }, "8 bytes for BF16 [2, 3]",
                  "size mismatch");
    std::string trunc = safetensors_bytes({{"b", "BF16", {4}, bf16_bytes(b)}});
    trunc.resize(trunc.size() - 2);
    write_file(d.path + "/trunc.safetensors", trunc);
    expect_throws([&] { (void)Checkpoint::open_file(d.path + "/trunc.safetensors"); }, "data outside the file",
                  "truncated");
    // A shape whose element count wraps to 0 in 64 bits, over zero bytes; and
    // one whose count fits but whose byte size wraps.
    write_file(d.path + "/wrap.safetensors",
               safetensors_bytes({{"b", "BF16", {(size_t)1 << 32, (size_t)1 << 32}, std::string()}}));
    expect_throws([&] { (void)Checkpoint::open_file(d.path + "/wrap.safetensors"); }, "overflows",
                  "shape product overflow");
    write_file(d.path + "/wrapb.safetensors",
               safetensors_bytes({{"f", "F32", {(size_t)1 << 62}, std::string()}}));
    expect_throws([&] { (void)Checkpoint::open_file(d.path + "/wrapb.safetensors"); }, "overflows",
                  "byte size overflow");
    std::string shorthdr(8, '\0');
    shorthdr[0] = (char)200;
    write_file(d.path + "/short.safetensors", shorthdr);
    expect_throws([&] { (void)Checkpoint::open_file(d.path + "/short.safetensors"); }, "header length past the end",
                  "header length");
}

void a_sharded_checkpoint_loads_through_its_index() {
    TempDir src;
    const LlamaConfig cfg = write_tiny_llama(src.path);
    const LlamaWeights one = load_weights(src.path, cfg);
    // Split the same tensors over two shard files plus an index.
    Checkpoint ck = Checkpoint::open_file(src.path + "/model.safetensors");
    TempDir d;
    write_file(d.path + "/config.json",
               "{\"model_type\": \"llama\", \"hidden_size\": 8, \"intermediate_size\": 16, \"num_hidden_layers\": 1, "
               "\"num_attention_heads\": 2, \"num_key_value_heads\": 2, \"rms_norm_eps\": 1e-5, \"vocab_size\": 8, "
               "\"tie_word_embeddings\": true}");
    std::vector<T> s1, s2;
    std::string map = "{\"weight_map\": {";
    size_t i = 0;
    for (const auto &n : ck.names()) {
        const TensorInfo &ti = ck.info(n);
        const Bf16Slice v = ck.bf16(n);
        T t{n, "BF16", ti.shape, bf16_bytes(v.to_vector())};
        const bool second = (i++ % 2) == 1;
        (second ? s2 : s1).push_back(t);
        map += std::string(i > 1 ? "," : "") + "\"" + n + "\": \"" + (second ? "m-2.safetensors" : "m-1.safetensors") +
               "\"";
    }
    map += "}}";
    write_file(d.path + "/m-1.safetensors", safetensors_bytes(s1));
    write_file(d.path + "/m-2.safetensors", safetensors_bytes(s2));
    write_file(d.path + "/model.safetensors.index.json", map);
    const LlamaWeights two = load_weights(d.path, LlamaConfig::load(d.path));
    expect(two.embed.to_vector() == one.embed.to_vector(), "embed");
    expect(two.layers[0].wq.to_vector() == one.layers[0].wq.to_vector(), "wq");
    expect(two.layers[0].wd.to_vector() == one.layers[0].wd.to_vector(), "wd");
    expect(two.final_gamma == one.final_gamma && two.layers[0].g2 == one.layers[0].g2, "gains");
    expect(two.layers[0].wu.is_mapped(), "shard views are mapped");
    TempDir empty;
    expect_throws([&] { (void)load_weights(empty.path, cfg); }, "neither model.safetensors nor its index", "no files");
}

void the_fp8_switch_off_leaves_the_weights_bf16() {
    TempDir d;
    const LlamaConfig cfg = write_tiny_llama(d.path);
    const LlamaWeights plain = load_weights(d.path, cfg);
    auto [off, report] = load_weights_fp8(d.path, cfg, std::nullopt);
    expect(!report.has_value(), "no report");
    expect(!off.fp8.has_value() && off.fp8_bytes() == 0, "no fp8");
    const std::pair<const Bf16Slice *, const Bf16Slice *> pairs[] = {{&plain.embed, &off.embed},
                                                                     {&plain.lm_head, &off.lm_head},
                                                                     {&plain.layers[0].wq, &off.layers[0].wq},
                                                                     {&plain.layers[0].wd, &off.layers[0].wd}};
    for (const auto &p : pairs) {
        expect(p.first->is_mapped() && p.second->is_mapped(), "mapped views");
        expect(p.first->to_vector() == p.second->to_vector(), "same bytes");
    }
    expect(plain.final_gamma == off.final_gamma, "final gamma");
    // The tied head is the embedding table's own view.
    expect(off.lm_head.data() == off.embed.data(), "tied head");
}

// ------------------------------------------------------------------ device

void the_fp8_switch_on_quantizes_the_projections_and_nothing_else() {
    TempDir d;
    const LlamaConfig cfg = write_tiny_llama(d.path);
    const LlamaWeights plain = load_weights(d.path, cfg);
    auto [on, report] = load_weights_fp8(d.path, cfg, Fp8Config{});
    expect(report.has_value(), "a report when the switch is on");
    expect(on.fp8.has_value() && on.fp8->size() == 1, "quantized layers");
    const Fp8Report &r = *report;
    expect(r.matrices == 7, "7 matrices");
    expect(r.fp8_bytes == 640 && r.bf16_bytes == 1280 && on.fp8_bytes() == 640, "bytes");
    expect(r.scale_bytes == 4 * (8 + 8 + 8 + 8 + 16 + 16 + 8), "scale bytes");
    const LayerFp8 &l = (*on.fp8)[0];
    expect(l.wq.rows == 8 && l.wq.cols == 8 && l.wk.rows == 8 && l.wk.cols == 8, "wq, wk shapes");
    expect(l.wd.rows == 8 && l.wd.cols == 16, "wd shape");
    expect(l.wq.exp_bias == 7 && l.wq.format == Fp8Format::E4M3, "bias and format");
    expect(r.mean_rel > 0.0f && r.mean_rel < 0.05f, "mean_rel " + std::to_string(r.mean_rel));
    expect(on.embed.is_mapped() && on.lm_head.is_mapped(), "bf16 views untouched");
    expect(on.embed.to_vector() == plain.embed.to_vector() && on.lm_head.to_vector() == plain.lm_head.to_vector(),
           "embed and head bytes");
    expect(on.final_gamma == plain.final_gamma && on.layers[0].g1 == plain.layers[0].g1, "gains");
    expect(on.layers[0].wq.to_vector() == plain.layers[0].wq.to_vector(), "projection bytes");
    const auto back = l.wq.dequantize();
    for (size_t rr = 0; rr < l.wq.rows; ++rr)
        for (size_t c = 0; c < l.wq.cols; ++c) {
            const float want = reng_fp8::bf16_to_f32(on.layers[0].wq[rr * l.wq.cols + c]);
            const float got = back[rr * l.wq.cols + c];
            expect(std::fabs(got - want) <= std::fabs(want) * 0.07f, "row " + std::to_string(rr) + " col " +
                                                                          std::to_string(c));
        }
    const std::string line = r.to_string();
    expect(line.rfind("7 matrices, 0.00 GiB bf16 -> 0.00 GiB fp8 + 0 KiB scales, mean rel ", 0) == 0, line);
}

// save_fp8 / load_fp8: the file reads back bit-for-bit, goes stale when the
// switch or a source file changes, and refuses tensors of the wrong shape and
// files of another kind.
void fp8_codes_file_round_trips_and_goes_stale() {
    TempDir d;
    const LlamaConfig cfg = write_tiny_llama(d.path);
    const Fp8Config q = fp8_switch(std::string_view("e5m2:pcs:backoff=0.75"), true).value();
    LlamaWeights w = load_weights(d.path, cfg);
    expect_throws([&] { save_fp8(d.path, w, q, Fp8Report{}); }, "carry no fp8 codes", "save without codes");
    const Fp8Report r = oracle_fp8(cfg, w, q);
    LlamaWeights none = load_weights(d.path, cfg);
    expect(!load_fp8(d.path, cfg, none, q).has_value() && !none.fp8, "no file: nullopt");
    save_fp8(d.path, w, q, r);
    struct stat st;
    expect(stat((d.path + "/" + FP8_CODES_FILE).c_str(), &st) == 0, "file written");
    expect(stat((d.path + "/" + FP8_CODES_FILE + ".tmp").c_str(), &st) != 0, "no temporary left");

    LlamaWeights back = load_weights(d.path, cfg);
    const auto got = load_fp8(d.path, cfg, back, q);
    expect(got.has_value() && back.fp8 && back.fp8->size() == 1, "current file loads");
    expect(got->matrices == r.matrices && got->bf16_bytes == r.bf16_bytes && got->fp8_bytes == r.fp8_bytes &&
               got->scale_bytes == r.scale_bytes && got->mean_rel == r.mean_rel && got->max_rel == r.max_rel,
           "report fields");
    const auto a = (*w.fp8)[0].matrices(), b = (*back.fp8)[0].matrices();
    for (size_t k = 0; k < a.size(); ++k) {
        const reng_fp8::Quantized &x = *a[k].second, &y = *b[k].second;
        const std::string what = a[k].first;
        expect(x.rows == y.rows && x.cols == y.cols, what + ": shape");
        expect(x.format == y.format && x.scaling == y.scaling && x.exp_bias == y.exp_bias, what + ": scheme");
        expect(x.codes == y.codes, what + ": codes");
        expect(std::memcmp(x.scales.data(), y.scales.data(), x.rows * 4) == 0 && y.scales.size() == x.rows,
               what + ": scales");
    }
    auto cached = load_weights_fp8_cached(d.path, cfg, q, false);
    expect(cached.from_file && cached.report && cached.weights.fp8, "cached load takes the file");
    expect((*cached.weights.fp8)[0].wd.codes == (*w.fp8)[0].wd.codes, "cached codes");
    auto off = load_weights_fp8_cached(d.path, cfg, std::nullopt, false);
    expect(!off.from_file && !off.report && !off.weights.fp8, "switch off: no codes");

    // Another switch: stale.
    LlamaWeights other = load_weights(d.path, cfg);
    expect(!load_fp8(d.path, cfg, other, Fp8Config{}).has_value() && !other.fp8, "another switch is stale");
    // A source file touched: stale.
    const std::string cfg_path = d.path + "/config.json";
    struct timespec ts[2] = {{0, UTIME_OMIT}, {1000000000, 0}};
    expect(utimensat(AT_FDCWD, cfg_path.c_str(), ts, 0) == 0, "utimensat");
    expect(!load_fp8(d.path, cfg, other, q).has_value() && !other.fp8, "touched config is stale");
    expect(utimensat(AT_FDCWD, (d.path + "/model.safetensors").c_str(), ts, 0) == 0, "utimensat");
    save_fp8(d.path, w, q, r);
    expect(load_fp8(d.path, cfg, other, q).has_value(), "saved again: current");
    ts[1].tv_sec += 1;
    expect(utimensat(AT_FDCWD, (d.path + "/model.safetensors").c_str(), ts, 0) == 0, "utimensat");
    other.fp8.reset();
    expect(!load_fp8(d.path, cfg, other, q).has_value() && !other.fp8, "touched checkpoint is stale");

    // A current file whose wg is not [intermediate, hidden].
    LlamaWeights bad = w;
    (*bad.fp8)[0].wg.rows = 8;
    (*bad.fp8)[0].wg.codes.resize(8 * 8);
    (*bad.fp8)[0].wg.scales.resize(8);
    save_fp8(d.path, bad, q, r);
    expect_throws([&] { (void)load_fp8(d.path, cfg, other, q); }, "layers.0.wg.codes is U8 of the wrong shape",
                  "wrong shape");
    expect(!other.fp8, "w untouched on a refusal");
    // Codes made with another switch than the one named.
    expect_throws([&] { save_fp8(d.path, w, Fp8Config{}, r); }, "was not made with", "switch mismatch");
    // Another kind of safetensors file under the name.
    const uint8_t one = 1;
    write_safetensors(d.path + "/" + FP8_CODES_FILE, {{"x", "U8", {1}, &one, 1}}, {{"format", "other"}});
    expect_throws([&] { (void)load_fp8(d.path, cfg, other, q); }, "is not an fp8 codes file", "other file");
    expect_throws([&] { write_safetensors(d.path + "/x.safetensors", {{"x", "F32", {2}, &one, 1}}, {}); },
                  "1 bytes for F32 [2]", "writer checks sizes");
}

// A larger random model, every scheme: each projection's codes, scales and
// bias against the oracle, and the report's error statistics against the
// oracle's sample_row_errors.
void quantize_fp8_matches_the_oracle_on_every_matrix() {
    TempDir d;
    const size_t H = 256, I = 640, L = 2, V = 64, NH = 4, KV = 2, HD = 64;
    write_file(d.path + "/config.json",
               "{\"model_type\": \"llama\", \"hidden_size\": 256, \"intermediate_size\": 640, \"num_hidden_layers\": 2, "
               "\"num_attention_heads\": 4, \"num_key_value_heads\": 2, \"rms_norm_eps\": 1e-5, \"vocab_size\": 64, "
               "\"tie_word_embeddings\": false}");
    std::vector<T> ts;
    uint64_t s = 12345;
    auto mat = [&](const std::string &n, size_t r, size_t c, float amp) {
        std::vector<uint16_t> v(r * c);
        for (auto &x : v) {
            s = s * 6364136223846793005ull + 1442695040888963407ull;
            const float u = (float)((s >> 40) & 0xffffff) / 16777216.0f - 0.5f;
            x = reng_fp8::f32_to_bf16(u * amp);
        }
        // A zero row and an outlier, as checkpoints have.
        for (size_t k = 0; k < c; ++k) v[(r / 2) * c + k] = 0;
        v[c + 3] = reng_fp8::f32_to_bf16(amp * 40.0f);
        ts.push_back(T{n, "BF16", {r, c}, bf16_bytes(v)});
    };
    mat("model.embed_tokens.weight", V, H, 1.0f);
    mat("lm_head.weight", V, H, 1.0f);
    for (size_t l = 0; l < L; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        mat(p + "self_attn.q_proj.weight", NH * HD, H, 0.04f);
        mat(p + "self_attn.k_proj.weight", KV * HD, H, 0.04f);
        mat(p + "self_attn.v_proj.weight", KV * HD, H, 0.04f);
        mat(p + "self_attn.o_proj.weight", H, NH * HD, 0.04f);
        mat(p + "mlp.gate_proj.weight", I, H, 0.04f);
        mat(p + "mlp.up_proj.weight", I, H, 0.04f);
        mat(p + "mlp.down_proj.weight", H, I, 0.04f);
        ts.push_back(T{p + "input_layernorm.weight", "F32", {H}, std::string(H * 4, '\0')});
        ts.push_back(T{p + "post_attention_layernorm.weight", "F32", {H}, std::string(H * 4, '\0')});
    }
    ts.push_back(T{"model.norm.weight", "F32", {H}, std::string(H * 4, '\0')});
    write_file(d.path + "/model.safetensors", safetensors_bytes(ts));
    const LlamaConfig cfg = LlamaConfig::load(d.path);
    for (const char *spec : {"e4m3:pcs", "e5m2:pcs", "e4m3:hw", "e4m3:unit", "e4m3:pcs:backoff=0.5", "hw:backoff=0.25"}) {
        const Fp8Config q = fp8_switch(std::string_view(spec), true).value();
        LlamaWeights w = load_weights(d.path, cfg);
        expect(!w.lm_head.empty() && w.lm_head.data() != w.embed.data(), "untied head");
        const Fp8Report r = w.quantize_fp8(cfg, q);
        expect(r.matrices == 7 * L, spec);
        double sum = 0.0;
        size_t n = 0;
        float mx = 0.0f;
        for (size_t l = 0; l < L; ++l) {
            const LayerTensors &t = w.layers[l];
            const Bf16Slice *src[7] = {&t.wq, &t.wk, &t.wv, &t.wo, &t.wg, &t.wu, &t.wd};
            const auto mats = (*w.fp8)[l].matrices();
            for (size_t k = 0; k < 7; ++k) {
                const reng_fp8::Quantized &qq = *mats[k].second;
                const std::vector<uint16_t> wv = src[k]->to_vector();
                std::vector<uint8_t> codes(qq.rows * qq.cols);
                std::vector<float> scales(qq.rows);
                const uint32_t eb = orc_quantize_with(wv.data(), qq.rows, qq.cols, (int)q.format, (int)q.scaling,
                                                      q.backoff, codes.data(), scales.data(), 8);
                const std::string what = std::string(spec) + " layer " + std::to_string(l) + " " + mats[k].first;
                expect(qq.codes == codes, what + ": codes");
                expect(qq.scales == scales, what + ": scales");
                expect(qq.exp_bias == eb, what + ": exp bias");
                std::vector<float> mean(8), mxr(8);
                const size_t kk = orc_sample_row_errors(wv.data(), codes.data(), scales.data(), qq.rows, qq.cols,
                                                        (int)q.format, FP8_ERROR_ROWS, mean.data(), mxr.data());
                for (size_t j = 0; j < kk; ++j) {
                    sum += mean[j];
                    mx = std::max(mx, mxr[j]);
                }
                n += kk;
            }
        }
        const float want_mean = (float)(sum / (double)n);
        expect(std::fabs(r.mean_rel - want_mean) <= 1e-6f * want_mean, std::string(spec) + ": mean_rel");
        expect(r.max_rel == mx, std::string(spec) + ": max_rel");
    }
}

// ------------------------------------------------------------------ the probe (fp8_probe.rs)

// The probe's host references: the closed-form decode against the oracle
// for every code, and the nearest-value encode against the oracle's encoder
// over every bf16 pattern and the reference's known answers.
void the_probe_host_references_agree_with_the_oracle() {
    for (Fp8Format f : {Fp8Format::E4M3, Fp8Format::E5M2}) {
        for (int c = 0; c < 256; ++c) {
            const float a = reng_probe::host_decode((uint8_t)c, f), b = orc_decode((uint8_t)c, (int)f);
            expect(std::memcmp(&a, &b, 4) == 0 || (std::isnan(a) && std::isnan(b)), "decode " + std::to_string(c));
        }
        for (uint32_t h = 0; h < 65536; ++h) {
            const float x = reng_fp8::bf16_to_f32((uint16_t)h);
            const uint8_t got = reng_probe::host_encode(x, f), want = orc_encode(x, (int)f);
            if (std::isnan(x)) {
                expect((got & 0x7f) == 0x7f && (want & 0x7f) == 0x7f, "NaN");
            } else {
                expect(got == want, "encode bf16 " + std::to_string(h));
            }
        }
    }
    const std::pair<float, uint8_t> kat[] = {{1.375f, 0x3b}, {-3.3f, 0xc5}, {100.0f, 0x6c}, {0.01f, 0x05},
                                             {250.0f, 0x77}, {300.0f, 0x77}, {0.001f, 0x01}, {1e-9f, 0x00},
                                             {17.0f, 0x58}, {1.0625f, 0x38}, {1.1875f, 0x3a}};
    for (const auto &k : kat) expect(reng_probe::host_encode(k.first, Fp8Format::E4M3) == k.second, "KAT");
}

void the_probe_inputs_are_the_reference_ones() {
    const auto w = reng_probe::weights(2, 1000);
    // i = 0 is an outlier channel (x 12): ((0 % 65536) / 65536 - 0.5) * 0.08 * 12.
    expect(w[0] == reng_fp8::f32_to_bf16(-0.04f * 12.0f), "weights[0]");
    const float x1 = ((float)((1ull * 2654435761ull) % 65536) / 65536.0f - 0.5f) * 0.08f;
    expect(w[1] == reng_fp8::f32_to_bf16(x1), "weights[1]");
    expect(w[977] == reng_fp8::f32_to_bf16(((float)((977ull * 2654435761ull) % 65536) / 65536.0f - 0.5f) * 0.08f * 12.0f),
           "weights[977]");
    const auto a = reng_probe::activations(3);
    expect(a[0] == -1000.0f / 700.0f && a[1] == ((float)(7919 % 2003) - 1000.0f) / 700.0f, "activations");
    expect(reng_probe::rel_l2({1.0f, 2.0f}, {1.0f, 2.0f}) == 0.0f, "rel_l2 0");
    const auto c = reng_probe::gemm_cpu({1, 2, 3, 4}, {1, 0, 0, 1, 1, 1}, 2, 2, 3);
    expect((c == std::vector<float>{1, 2, 3, 3, 4, 7}), "gemm_cpu");
}

// fp8_probe.rs:538-597, the probe's own tests.
void the_plain_gemm_reference_is_the_dequantized_weight() {
    const auto w = reng_probe::weights(512, 256);
    const auto q = reng_fp8::quantize(w, 512, 256, Fp8Format::E4M3, Scaling::HwExpBias);
    expect(q.exp_bias != reng_fp8::exponent_bias(Fp8Format::E4M3), "a non-default bias");
    expect(reng_probe::device_values(q) == q.dequantize(), "device values == dequantize");
}

void a_unit_scaled_operand_is_read_as_its_codes() {
    const auto af = reng_probe::activations(256);
    std::vector<uint16_t> a(256);
    for (size_t i = 0; i < 256; ++i) a[i] = reng_fp8::f32_to_bf16(af[i]);
    const auto q = reng_fp8::quantize(a, 1, 256, Fp8Format::E4M3, Scaling::Unit);
    std::vector<float> want(256);
    for (size_t i = 0; i < 256; ++i) want[i] = reng_probe::host_decode(q.codes[i], Fp8Format::E4M3);
    expect(reng_probe::device_values(q) == want, "unit operand");
}

void the_plain_gemm_reference_refuses_a_per_channel_weight() {
    const auto w = reng_probe::weights(512, 256);
    const auto q = reng_fp8::quantize(w, 512, 256, Fp8Format::E4M3, Scaling::PerChannel);
    expect_throws<std::logic_error>([&] { (void)reng_probe::device_values(q); }, "does not see per-channel scales",
                                    "per-channel refused");
}

void a_per_channel_reference_would_miss_the_plain_gemm_by_thousands() {
    const auto w = reng_probe::weights(512, 256);
    const auto q = reng_fp8::quantize(w, 512, 256, Fp8Format::E4M3, Scaling::PerChannel);
    const auto af = reng_probe::activations(256);
    std::vector<uint16_t> a(256);
    for (size_t i = 0; i < 256; ++i) a[i] = reng_fp8::f32_to_bf16(af[i]);
    const auto aq = reng_fp8::quantize(a, 1, 256, Fp8Format::E4M3, Scaling::Unit);
    std::vector<float> read(q.codes.size());
    for (size_t i = 0; i < read.size(); ++i) read[i] = reng_probe::host_decode(q.codes[i], Fp8Format::E4M3);
    const auto dev = reng_probe::gemm_cpu(reng_probe::device_values(aq), read, 1, 256, 512);
    const auto scaled = reng_probe::gemm_cpu(reng_probe::device_values(aq), q.dequantize(), 1, 256, 512);
    expect(reng_probe::rel_l2(dev, scaled) > 100.0f, "rel_L2 " + std::to_string(reng_probe::rel_l2(dev, scaled)));
}

struct Test {
    const char *name;
    bool device;
    void (*fn)();
};

const Test TESTS[] = {
    {"the_fp8_switch_reads_the_variable_and_the_flag", false, the_fp8_switch_reads_the_variable_and_the_flag},
    {"take_fp8_flag_removes_every_copy", false, take_fp8_flag_removes_every_copy},
    {"f32_display_is_the_shortest_round_trip", false, f32_display_is_the_shortest_round_trip},
    {"the_config_is_read_and_checked", false, the_config_is_read_and_checked},
    {"safetensors_views_convert_and_refuse", false, safetensors_views_convert_and_refuse},
    {"a_sharded_checkpoint_loads_through_its_index", false, a_sharded_checkpoint_loads_through_its_index},
    {"the_fp8_switch_off_leaves_the_weights_bf16", false, the_fp8_switch_off_leaves_the_weights_bf16},
    {"fp8_codes_file_round_trips_and_goes_stale", false, fp8_codes_file_round_trips_and_goes_stale},
    {"the_fp8_switch_on_quantizes_the_projections_and_nothing_else", true,
     the_fp8_switch_on_quantizes_the_projections_and_nothing_else},
    {"quantize_fp8_matches_the_oracle_on_every_matrix", true, quantize_fp8_matches_the_oracle_on_every_matrix},
    {"the_probe_host_references_agree_with_the_oracle", false, the_probe_host_references_agree_with_the_oracle},
    {"the_probe_inputs_are_the_reference_ones", false, the_probe_inputs_are_the_reference_ones},
    {"the_plain_gemm_reference_is_the_dequantized_weight", true, the_plain_gemm_reference_is_the_dequantized_weight},
    {"a_unit_scaled_operand_is_read_as_its_codes", true, a_unit_scaled_operand_is_read_as_its_codes},
    {"the_plain_gemm_reference_refuses_a_per_channel_weight", true,
     the_plain_gemm_reference_refuses_a_per_channel_weight},
    {"a_per_channel_reference_would_miss_the_plain_gemm_by_thousands", true,
     a_per_channel_reference_would_miss_the_plain_gemm_by_thousands},
};

}  // namespace

int main(int argc, char **argv) {
    // --save-codes <model_dir> <spec>: the oracle's codes for the checkpoint
    // written with save_fp8 (host only), for a reader outside this library.
    if (argc == 4 && std::string(argv[1]) == "--save-codes") {
        try {
            const LlamaConfig cfg = LlamaConfig::load(argv[2]);
            const Fp8Config q = fp8_switch(std::string_view(argv[3]), true).value();
            LlamaWeights w = load_weights(argv[2], cfg);
            save_fp8(argv[2], w, q, oracle_fp8(cfg, w, q));
            return 0;
        } catch (const std::exception &e) {
            std::fprintf(stderr, "Error: %s\n", e.what());
            return 1;
        }
    }
    bool cpu_only = false;
    std::string filter;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--cpu-only") cpu_only = true;
        else filter = a;
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
