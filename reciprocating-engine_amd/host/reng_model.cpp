// reng_model.cpp - see reng_model.hpp.
#include "reng_model.hpp"

#include <hip/hip_runtime_api.h>
#include <sys/stat.h>

#include <algorithm>
#include <cctype>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../../include/reng_hip.h"
#include "json.hpp"

namespace reng_model {

namespace {

std::string lower(std::string_view s) {
    std::string out(s);
    for (char &c : out) c = (char)std::tolower((unsigned char)c);
    return out;
}

std::string_view trim(std::string_view s) {
    size_t a = 0, b = s.size();
    while (a < b && std::isspace((unsigned char)s[a])) ++a;
    while (b > a && std::isspace((unsigned char)s[b - 1])) --b;
    return s.substr(a, b - a);
}

// Rust's {:?} of a str: quoted, with \" \\ and control characters escaped.
std::string debug_str(std::string_view s) {
    std::string out = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') {
            out += '\\';
            out += c;
        } else if (c == '\n') {
            out += "\\n";
        } else if (c == '\t') {
            out += "\\t";
        } else if (c == '\r') {
            out += "\\r";
        } else {
            out += c;
        }
    }
    return out + "\"";
}

std::string shape_debug(size_t a, size_t b) { return "[" + std::to_string(a) + ", " + std::to_string(b) + "]"; }

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(std::string("reng-hip: ") + what + ": " + hipGetErrorString(e));
}

void check_abi(int rc) {
    if (rc != RENG_HIP_OK) throw Error(std::string("reng-hip: ") + reng_hip_last_error());
}

// A grow-only device buffer.
struct DeviceBuf {
    void *p = nullptr;
    size_t cap = 0;
    void reserve(size_t bytes) {
        if (bytes <= cap) return;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        check_hip(hipMalloc(&p, bytes), "hipMalloc");
        cap = bytes;
    }
    ~DeviceBuf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

// ------------------------------------------------------------ f32 Display

std::string f32_shortest(float x) {
    if (std::isnan(x)) return "NaN";
    if (std::isinf(x)) return x < 0 ? "-inf" : "inf";
    if (x == 0.0f) return std::signbit(x) ? "-0" : "0";
    char buf[64];
    int digits = 1;
    for (; digits <= 9; ++digits) {
        std::snprintf(buf, sizeof buf, "%.*e", digits - 1, (double)x);
        if (std::strtof(buf, nullptr) == x) break;
    }
    // buf = [-]d.ddde[+-]XX: rewrite without an exponent.
    std::string s(buf);
    const bool neg = s[0] == '-';
    if (neg) s = s.substr(1);
    const size_t epos = s.find('e');
    const int exp10 = std::atoi(s.c_str() + epos + 1);
    std::string mant;
    for (size_t i = 0; i < epos; ++i)
        if (s[i] != '.') mant += s[i];
    while (mant.size() > 1 && mant.back() == '0') mant.pop_back();
    std::string out;
    const int point = exp10 + 1;   // digits before the decimal point
    if (point <= 0) {
        out = "0." + std::string((size_t)-point, '0') + mant;
    } else if ((size_t)point >= mant.size()) {
        out = mant + std::string((size_t)point - mant.size(), '0');
    } else {
        out = mant.substr(0, (size_t)point) + "." + mant.substr((size_t)point);
    }
    return neg ? "-" + out : out;
}

// ------------------------------------------------------------ config

bool LlamaConfig::tied() const {
    const bool gemma = model_type == "gemma2" || model_type == "gemma3_text";
    return tie_word_embeddings.value_or(gemma);
}

LlamaConfig LlamaConfig::from_json(const std::string &text) {
    reng_json::Value top;
    try {
        top = reng_json::parse(text);
    } catch (const std::exception &e) {
        throw Error(std::string("config.json: ") + e.what());
    }
    LlamaConfig c;
    const reng_json::Value *v = &top;
    if (top.has("model_type") && top["model_type"].kind == reng_json::Value::String)
        c.model_type = top["model_type"].str;
    // A multimodal gemma3 config nests the language model's config.
    if (c.model_type == "gemma3" && top.has("text_config")) {
        v = &top["text_config"];
        c.weight_prefix = "language_model.model.";
        if (v->has("model_type") && (*v)["model_type"].kind == reng_json::Value::String)
            c.model_type = (*v)["model_type"].str;
    }
    auto req = [&](const char *k) -> const reng_json::Value & {
        if (!v->has(k)) throw Error(std::string("config.json: missing field `") + k + "`");
        return (*v)[k];
    };
    auto opt = [&](const char *k) -> const reng_json::Value * {
        if (!v->has(k) || (*v)[k].kind == reng_json::Value::Null) return nullptr;
        return &(*v)[k];
    };
    try {
        c.hidden_size = req("hidden_size").as_u64();
        c.intermediate_size = req("intermediate_size").as_u64();
        c.num_hidden_layers = req("num_hidden_layers").as_u64();
        c.num_attention_heads = req("num_attention_heads").as_u64();
        c.rms_norm_eps = (float)req("rms_norm_eps").as_f64();
        c.vocab_size = req("vocab_size").as_u64();
        if (auto *p = opt("num_key_value_heads")) c.num_key_value_heads = p->as_u64();
        if (auto *p = opt("head_dim")) c.head_dim_ = p->as_u64();
        if (auto *p = opt("tie_word_embeddings")) c.tie_word_embeddings = p->b;
        if (auto *p = opt("rope_theta")) c.rope_theta = (float)p->as_f64();
        c.has_rope_scaling = opt("rope_scaling") != nullptr;
        if (auto *p = opt("sliding_window")) c.sliding_window = p->as_u64();
        if (auto *p = opt("attention_multiplier")) c.attention_multiplier = (float)p->as_f64();
        if (auto *p = opt("query_pre_attn_scalar")) c.query_pre_attn_scalar = (float)p->as_f64();
    } catch (const Error &) {
        throw;
    } catch (const std::exception &e) {
        throw Error(std::string("config.json: ") + e.what());
    }
    if (c.num_attention_heads == 0) throw Error("config.json: num_attention_heads is 0");
    // Transforms the reference folds into the bf16 weights before they are
    // quantized (Granite's multipliers, Gemma-2's soft-capping on the final
    // gain, a partial rotation's row permutation, MLP biases): refused here
    // rather than quantizing different numbers.
    for (const char *k : {"residual_multiplier", "logits_scaling", "embedding_multiplier", "final_logit_softcapping"})
        if (opt(k)) throw Error(std::string("config.json: ") + k + " is not supported by this loader");
    if (auto *p = opt("partial_rotary_factor"))
        if (p->as_f64() != 1.0) throw Error("config.json: partial_rotary_factor is not supported by this loader");
    if (auto *p = opt("mlp_bias"))
        if (p->b) throw Error("mlp_bias is not supported");
    return c;
}

LlamaConfig LlamaConfig::load(const std::string &dir) {
    FILE *f = std::fopen((dir + "/config.json").c_str(), "rb");
    if (!f) throw Error("config.json: " + std::string(std::strerror(errno)));
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    std::fclose(f);
    return from_json(text);
}

// ------------------------------------------------------------ fp8 switch

std::string Fp8Config::to_string() const {
    return std::string(reng_fp8::name(format)) + "/" + reng_fp8::name(scaling) + " backoff " + f32_shortest(backoff);
}

std::optional<Fp8Config> fp8_switch(std::optional<std::string_view> value, bool flag) {
    if (!value) return flag ? std::optional<Fp8Config>(Fp8Config{}) : std::nullopt;
    const std::string_view v = trim(*value);
    const std::string lv = lower(v);
    if (lv.empty() || lv == "0" || lv == "off" || lv == "false" || lv == "no") return std::nullopt;
    Fp8Config cfg;
    if (lv == "1" || lv == "on" || lv == "true" || lv == "yes") return cfg;
    size_t a = 0;
    while (a <= v.size()) {
        size_t b = v.find_first_of(":,", a);
        if (b == std::string_view::npos) b = v.size();
        const std::string_view word = trim(v.substr(a, b - a));
        a = b + 1;
        if (word.empty()) continue;
        if (auto f = reng_fp8::format_from_name(word)) {
            cfg.format = *f;
        } else if (auto sc = reng_fp8::scaling_from_name(word)) {
            cfg.scaling = *sc;
        } else if (word.substr(0, 8) == "backoff=") {
            const std::string rest(word.substr(8));
            // Rust's f32 grammar: optional sign, decimal digits with an
            // optional point and exponent, or inf / infinity / nan.
            const std::string lr = lower(rest);
            bool ok = !rest.empty() && lr.find("0x") == std::string::npos && !std::isspace((unsigned char)rest[0]);
            char *end = nullptr;
            const float b = ok ? std::strtof(rest.c_str(), &end) : 0.0f;
            ok = ok && end && *end == '\0';
            if (!ok) throw Error("RENG_FP8 backoff: invalid float literal");
            cfg.backoff = b;
            if (!(cfg.backoff > 0.0f && cfg.backoff <= 1.0f))
                throw Error("RENG_FP8 backoff " + f32_shortest(cfg.backoff) + " is not in (0, 1]");
        } else {
            throw Error("RENG_FP8: unknown setting " + debug_str(word) +
                        " (expected a format, a scale scheme or backoff=<f32>)");
        }
    }
    return cfg;
}

bool take_fp8_flag(std::vector<std::string> &args) {
    const bool had = std::find(args.begin(), args.end(), "--fp8") != args.end();
    args.erase(std::remove(args.begin(), args.end(), "--fp8"), args.end());
    return had;
}

// ------------------------------------------------------------ LayerFp8 / report

std::vector<std::pair<const char *, const reng_fp8::Quantized *>> LayerFp8::matrices() const {
    return {{"wq", &wq}, {"wk", &wk}, {"wv", &wv}, {"wo", &wo}, {"wg", &wg}, {"wu", &wu}, {"wd", &wd}};
}

size_t LayerFp8::code_bytes() const {
    size_t n = 0;
    for (const auto &m : matrices()) n += m.second->code_bytes();
    return n;
}

bool Fp8Report::operator==(const Fp8Report &o) const {
    return matrices == o.matrices && bf16_bytes == o.bf16_bytes && fp8_bytes == o.fp8_bytes &&
           scale_bytes == o.scale_bytes && mean_rel == o.mean_rel && max_rel == o.max_rel && secs == o.secs;
}

std::string Fp8Report::to_string() const {
    auto gib = [](size_t b) { return (double)b / (1024.0 * 1024.0 * 1024.0); };
    char buf[256];
    std::snprintf(buf, sizeof buf,
                  "%zu matrices, %.2f GiB bf16 -> %.2f GiB fp8 + %zu KiB scales, mean rel %.4f, max rel %.4f, %.2f s",
                  matrices, gib(bf16_bytes), gib(fp8_bytes), scale_bytes / 1024, (double)mean_rel, (double)max_rel,
                  secs);
    return buf;
}

// ------------------------------------------------------------ quantize_fp8

Fp8Report LlamaWeights::quantize_fp8(const LlamaConfig &cfg, const Fp8Config &q) {
    const auto t0 = std::chrono::steady_clock::now();
    const size_t h = cfg.hidden_size, i = cfg.intermediate_size;
    const size_t hd = cfg.head_dim(), qd = cfg.q_dim(), kvd = cfg.n_kv_heads() * hd;
    Fp8Report report;
    double err_sum = 0.0;
    size_t err_n = 0;
    float err_max = 0.0f;
    // Each matrix goes through reng_hip_quantize_host (the library's pinned,
    // double-buffered staging: upload, quantize and download of neighbouring
    // row chunks overlap). The error sample needs only its eight rows on the
    // device: they are gathered with their codes and scales and measured as
    // an 8-row matrix (rows are independent, so the statistics are the
    // sampled rows' own).
    DeviceBuf dw, dc, ds, dmean, dmax;
    std::vector<LayerFp8> out;
    out.reserve(layers.size());
    for (size_t li = 0; li < layers.size(); ++li) {
        const LayerTensors &l = layers[li];
        auto one = [&](const char *name, const Bf16Slice &w, size_t rows, size_t cols) {
            if (w.size() != rows * cols)
                throw Error("layer " + std::to_string(li) + " " + name + ": " + std::to_string(w.size()) +
                            " elements, expected " + std::to_string(rows) + " x " + std::to_string(cols));
            // quantize_with's own refusals (lib.rs:527-532), with its messages.
            if (!(rows > 0 && cols > 0))
                throw std::invalid_argument("empty shape " + std::to_string(rows) + " x " + std::to_string(cols));
            if (!(q.backoff > 0.0f && std::isfinite(q.backoff)))
                throw std::invalid_argument("backoff " + f32_shortest(q.backoff) + " is not positive and finite");
            reng_fp8::Quantized r;
            r.format = q.format;
            r.scaling = q.scaling;
            r.rows = rows;
            r.cols = cols;
            r.codes.resize(rows * cols);
            r.scales.resize(rows);
            check_abi(reng_hip_quantize_host(w.data(), RENG_HIP_BF16, rows, cols, (int)q.format, (int)q.scaling,
                                             q.backoff, r.codes.data(), r.scales.data(), &r.exp_bias));
            // sample_row_errors(w, q, FP8_ERROR_ROWS): every ceil(rows / n)-th row.
            const size_t n = std::min(FP8_ERROR_ROWS, rows);
            const size_t step = (rows + n - 1) / n, k = (rows + step - 1) / step;
            std::vector<uint16_t> sw(k * cols);
            std::vector<uint8_t> sc(k * cols);
            std::vector<float> ss(k);
            for (size_t j = 0; j < k; ++j) {
                const size_t row = j * step;
                std::memcpy(&sw[j * cols], w.data() + row * cols, cols * 2);
                std::memcpy(&sc[j * cols], &r.codes[row * cols], cols);
                ss[j] = r.scales[row];
            }
            dw.reserve(k * cols * 2);
            dc.reserve(k * cols);
            ds.reserve(k * 4);
            dmean.reserve(k * 4);
            dmax.reserve(k * 4);
            check_hip(hipMemcpy(dw.p, sw.data(), k * cols * 2, hipMemcpyHostToDevice), "hipMemcpy H2D");
            check_hip(hipMemcpy(dc.p, sc.data(), k * cols, hipMemcpyHostToDevice), "hipMemcpy H2D");
            check_hip(hipMemcpy(ds.p, ss.data(), k * 4, hipMemcpyHostToDevice), "hipMemcpy H2D");
            check_abi(reng_hip_row_errors(static_cast<const uint16_t *>(dw.p), static_cast<const uint8_t *>(dc.p),
                                          static_cast<const float *>(ds.p), k, cols, (int)q.format, 0,
                                          static_cast<float *>(dmean.p), static_cast<float *>(dmax.p), nullptr));
            std::vector<float> mean(k), mx(k);
            check_hip(hipMemcpy(mean.data(), dmean.p, k * 4, hipMemcpyDeviceToHost), "hipMemcpy D2H");
            check_hip(hipMemcpy(mx.data(), dmax.p, k * 4, hipMemcpyDeviceToHost), "hipMemcpy D2H");
            report.matrices += 1;
            report.bf16_bytes += w.size() * 2;
            report.fp8_bytes += r.code_bytes();
            report.scale_bytes += r.scales.size() * 4;
            for (size_t j = 0; j < k; ++j) {
                err_sum += (double)mean[j];
                err_max = std::max(err_max, mx[j]);
            }
            err_n += k;
            return r;
        };
        LayerFp8 lf;
        lf.wq = one("wq", l.wq, qd, h);
        lf.wk = one("wk", l.wk, kvd, h);
        lf.wv = one("wv", l.wv, kvd, h);
        lf.wo = one("wo", l.wo, h, qd);
        lf.wg = one("wg", l.wg, i, h);
        lf.wu = one("wu", l.wu, i, h);
        lf.wd = one("wd", l.wd, h, i);
        out.push_back(std::move(lf));
    }
    if (err_n > 0) {
        report.mean_rel = (float)(err_sum / (double)err_n);
        report.max_rel = err_max;
    }
    report.secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    fp8 = std::move(out);
    return report;
}

size_t LlamaWeights::fp8_bytes() const {
    if (!fp8) return 0;
    size_t n = 0;
    for (const auto &l : *fp8) n += l.code_bytes();
    return n;
}

// ------------------------------------------------------------ load_weights

LlamaWeights load_weights(const std::string &dir, const LlamaConfig &cfg) {
    const Checkpoint ck = Checkpoint::open(dir);
    const size_t h = cfg.hidden_size, i = cfg.intermediate_size, v = cfg.vocab_size;
    const size_t hd = cfg.head_dim(), qd = cfg.q_dim(), kvd = cfg.n_kv_heads() * hd;
    const std::string &pre = cfg.weight_prefix;
    const bool gemma = cfg.model_type == "gemma2" || cfg.model_type == "gemma3_text";
    const bool post_norm = cfg.model_type == "olmo2";
    auto plus_one = [&](std::vector<float> g) {
        if (gemma)
            for (float &x : g) x += 1.0f;
        return g;
    };

    LlamaWeights w;
    const std::string embed_name = pre + "embed_tokens.weight";
    const TensorInfo &ei = ck.info(embed_name);
    if (ei.shape != std::vector<size_t>{v, h}) {
        std::string s = "[";
        for (size_t k = 0; k < ei.shape.size(); ++k) s += (k ? ", " : "") + std::to_string(ei.shape[k]);
        throw Error("embed_tokens shape " + s + "], expected " + shape_debug(v, h));
    }
    w.embed = ck.bf16(embed_name);
    for (size_t l = 0; l < cfg.num_hidden_layers; ++l) {
        const std::string p = pre + "layers." + std::to_string(l) + ".";
        LayerTensors t;
        if (gemma) {
            t.g1 = plus_one(ck.f32(p + "input_layernorm.weight"));
            t.g2 = plus_one(ck.f32(p + "pre_feedforward_layernorm.weight"));
        } else if (post_norm) {
            t.g1 = ck.f32(p + "post_attention_layernorm.weight");
            t.g2 = ck.f32(p + "post_feedforward_layernorm.weight");
        } else {
            t.g1 = ck.f32(p + "input_layernorm.weight");
            t.g2 = ck.f32(p + "post_attention_layernorm.weight");
        }
        // Phi-3's fused q/k/v and gate/up matrices are contiguous row blocks.
        if (ck.has(p + "self_attn.qkv_proj.weight")) {
            const Bf16Slice f = ck.linear(p + "self_attn.qkv_proj.weight", qd + 2 * kvd, h);
            t.wq = f.sub(0, qd * h);
            t.wk = f.sub(qd * h, kvd * h);
            t.wv = f.sub((qd + kvd) * h, kvd * h);
        } else {
            t.wq = ck.linear(p + "self_attn.q_proj.weight", qd, h);
            t.wk = ck.linear(p + "self_attn.k_proj.weight", kvd, h);
            t.wv = ck.linear(p + "self_attn.v_proj.weight", kvd, h);
        }
        if (ck.has(p + "mlp.gate_up_proj.weight")) {
            const Bf16Slice f = ck.linear(p + "mlp.gate_up_proj.weight", 2 * i, h);
            t.wg = f.sub(0, i * h);
            t.wu = f.sub(i * h, i * h);
        } else {
            t.wg = ck.linear(p + "mlp.gate_proj.weight", i, h);
            t.wu = ck.linear(p + "mlp.up_proj.weight", i, h);
        }
        t.wo = ck.linear(p + "self_attn.o_proj.weight", h, qd);
        t.wd = ck.linear(p + "mlp.down_proj.weight", h, i);
        w.layers.push_back(std::move(t));
    }
    w.final_gamma = plus_one(ck.f32(pre + "norm.weight"));
    // The head beside the decoder: `<outer>lm_head.weight`, then the bare name.
    std::vector<std::string> head_names;
    const std::string outer = pre.size() >= 6 && pre.compare(pre.size() - 6, 6, "model.") == 0
                                  ? pre.substr(0, pre.size() - 6)
                                  : std::string();
    head_names.push_back(outer + "lm_head.weight");
    if (!outer.empty()) head_names.push_back("lm_head.weight");
    const std::string *head = nullptr;
    for (const auto &n : head_names)
        if (ck.has(n)) {
            head = &n;
            break;
        }
    if (head) {
        w.lm_head = ck.linear(*head, v, h);
    } else if (cfg.tied()) {
        w.lm_head = w.embed;
    } else {
        throw Error("lm_head.weight missing and embeddings are not tied");
    }
    return w;
}

std::pair<LlamaWeights, std::optional<Fp8Report>> load_weights_fp8(const std::string &dir, const LlamaConfig &cfg,
                                                                   std::optional<Fp8Config> fp8) {
    LlamaWeights w = load_weights(dir, cfg);
    if (!fp8) return {std::move(w), std::nullopt};
    const Fp8Report r = w.quantize_fp8(cfg, *fp8);
    return {std::move(w), r};
}

// ------------------------------------------------------------ fp8 codes on disk

namespace {

// The __metadata__ "format" value of a codes file, versioned with the layout.
constexpr const char *FP8_CODES_FORMAT = "reng-fp8 codes 1";

// "name size mtime_ns" of each file the weights come from, ';'-separated:
// config.json, the shard index when there is one, then the checkpoint files.
std::string source_fingerprint(const std::string &dir) {
    std::vector<std::string> paths = {dir + "/config.json"};
    struct stat st;
    const std::string idx = dir + "/model.safetensors.index.json";
    if (::stat((dir + "/model.safetensors").c_str(), &st) != 0 && ::stat(idx.c_str(), &st) == 0)
        paths.push_back(idx);
    const Checkpoint ck = Checkpoint::open(dir);
    for (const std::string &f : ck.files()) paths.push_back(f);
    std::string out;
    for (const std::string &p : paths) {
        if (::stat(p.c_str(), &st) != 0) throw Error("cannot stat " + p + ": " + std::strerror(errno));
        const size_t slash = p.find_last_of('/');
        const long long ns = (long long)st.st_mtim.tv_sec * 1000000000LL + (long long)st.st_mtim.tv_nsec;
        out += (out.empty() ? "" : ";") + (slash == std::string::npos ? p : p.substr(slash + 1)) + " " +
               std::to_string((unsigned long long)st.st_size) + " " + std::to_string(ns);
    }
    return out;
}

// The seven projections of one layer with the [rows, cols] the config implies.
struct MatShape {
    const char *name;
    reng_fp8::Quantized *q;
    size_t rows, cols;
};

std::vector<MatShape> layer_shapes(const LlamaConfig &cfg, LayerFp8 &l) {
    const size_t h = cfg.hidden_size, i = cfg.intermediate_size, qd = cfg.q_dim();
    const size_t kvd = cfg.n_kv_heads() * cfg.head_dim();
    return {{"wq", &l.wq, qd, h}, {"wk", &l.wk, kvd, h}, {"wv", &l.wv, kvd, h}, {"wo", &l.wo, h, qd},
            {"wg", &l.wg, i, h},  {"wu", &l.wu, i, h},   {"wd", &l.wd, h, i}};
}

}  // namespace

void save_fp8(const std::string &dir, const LlamaWeights &w, const Fp8Config &q, const Fp8Report &r) {
    if (!w.fp8) throw Error("save_fp8: the weights carry no fp8 codes");
    std::map<std::string, std::string> meta;
    meta["format"] = FP8_CODES_FORMAT;
    meta["fp8"] = q.to_string();
    meta["source"] = source_fingerprint(dir);
    meta["layers"] = std::to_string(w.fp8->size());
    meta["matrices"] = std::to_string(r.matrices);
    meta["bf16_bytes"] = std::to_string(r.bf16_bytes);
    meta["fp8_bytes"] = std::to_string(r.fp8_bytes);
    meta["scale_bytes"] = std::to_string(r.scale_bytes);
    meta["mean_rel"] = f32_shortest(r.mean_rel);
    meta["max_rel"] = f32_shortest(r.max_rel);
    char secs[32];
    std::snprintf(secs, sizeof secs, "%.6f", r.secs);
    meta["secs"] = secs;
    // Scales first, then codes: every F32 tensor starts 4-byte aligned.
    std::vector<TensorOut> scales, codes;
    for (size_t li = 0; li < w.fp8->size(); ++li)
        for (const auto &m : (*w.fp8)[li].matrices()) {
            const reng_fp8::Quantized &x = *m.second;
            if (x.codes.size() != x.rows * x.cols || x.scales.size() != x.rows)
                throw Error("save_fp8: layer " + std::to_string(li) + " " + m.first + " is not [rows, cols]");
            if (x.format != q.format || x.scaling != q.scaling)
                throw Error("save_fp8: layer " + std::to_string(li) + " " + m.first + " was not made with " +
                            q.to_string());
            const std::string p = "layers." + std::to_string(li) + "." + m.first;
            meta[p + ".exp_bias"] = std::to_string(x.exp_bias);
            scales.push_back({p + ".scales", "F32", {x.rows}, x.scales.data(), x.scales.size() * 4});
            codes.push_back({p + ".codes", "U8", {x.rows, x.cols}, x.codes.data(), x.codes.size()});
        }
    scales.insert(scales.end(), codes.begin(), codes.end());
    write_safetensors(dir + "/" + FP8_CODES_FILE, scales, meta);
}

std::optional<Fp8Report> load_fp8(const std::string &dir, const LlamaConfig &cfg, LlamaWeights &w,
                                  const Fp8Config &q) {
    const auto t0 = std::chrono::steady_clock::now();
    const std::string path = dir + "/" + FP8_CODES_FILE;
    struct stat st;
    if (::stat(path.c_str(), &st) != 0) return std::nullopt;
    const Checkpoint f = Checkpoint::open_file(path);
    const auto &meta = f.metadata();
    auto get = [&](const std::string &key) -> const std::string & {
        auto it = meta.find(key);
        if (it == meta.end()) throw Error(path + ": no " + key + " in the metadata");
        return it->second;
    };
    auto number = [&](const std::string &key) -> unsigned long long {
        const std::string &v = get(key);
        char *end = nullptr;
        const unsigned long long n = std::strtoull(v.c_str(), &end, 10);
        if (v.empty() || *end != '\0' || v[0] == '-') throw Error(path + ": " + key + " " + v + " is not a count");
        return n;
    };
    auto real = [&](const std::string &key) -> double {
        const std::string &v = get(key);
        char *end = nullptr;
        const double x = std::strtod(v.c_str(), &end);
        if (v.empty() || *end != '\0') throw Error(path + ": " + key + " " + v + " is not a number");
        return x;
    };
    auto fmt = meta.find("format");
    if (fmt == meta.end() || fmt->second != FP8_CODES_FORMAT)
        throw Error(path + " is not an fp8 codes file (" + FP8_CODES_FORMAT + ")");
    if (get("fp8") != q.to_string() || get("source") != source_fingerprint(dir)) return std::nullopt;
    if (number("layers") != cfg.num_hidden_layers)
        throw Error(path + ": " + get("layers") + " layers, the config has " + std::to_string(cfg.num_hidden_layers));
    std::vector<LayerFp8> out(cfg.num_hidden_layers);
    for (size_t li = 0; li < out.size(); ++li)
        for (const MatShape &m : layer_shapes(cfg, out[li])) {
            const std::string p = "layers." + std::to_string(li) + "." + m.name;
            const TensorInfo &ci = f.info(p + ".codes");
            const TensorInfo &si = f.info(p + ".scales");
            if (ci.dtype != Dtype::U8 || ci.shape != std::vector<size_t>{m.rows, m.cols})
                throw Error(path + ": " + p + ".codes is " + ci.dtype_name + " of the wrong shape, expected U8 " +
                            shape_debug(m.rows, m.cols));
            if (si.dtype != Dtype::F32 || si.shape != std::vector<size_t>{m.rows})
                throw Error(path + ": " + p + ".scales is " + si.dtype_name + " of the wrong shape, expected F32 [" +
                            std::to_string(m.rows) + "]");
            const unsigned long long eb = number(p + ".exp_bias");
            if (eb > 0xffffffffULL) throw Error(path + ": " + p + ".exp_bias " + std::to_string(eb) + " is out of range");
            m.q->format = q.format;
            m.q->scaling = q.scaling;
            m.q->rows = m.rows;
            m.q->cols = m.cols;
            m.q->codes = f.u8(p + ".codes");
            m.q->scales = f.f32(p + ".scales");
            m.q->exp_bias = (uint32_t)eb;
        }
    Fp8Report r;
    r.matrices = number("matrices");
    r.bf16_bytes = number("bf16_bytes");
    r.fp8_bytes = number("fp8_bytes");
    r.scale_bytes = number("scale_bytes");
    r.mean_rel = (float)real("mean_rel");
    r.max_rel = (float)real("max_rel");
    w.fp8 = std::move(out);
    r.secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return r;
}

Fp8Load load_weights_fp8_cached(const std::string &dir, const LlamaConfig &cfg, std::optional<Fp8Config> fp8,
                                bool save) {
    Fp8Load out;
    out.weights = load_weights(dir, cfg);
    if (!fp8) return out;
    if ((out.report = load_fp8(dir, cfg, out.weights, *fp8))) {
        out.from_file = true;
        return out;
    }
    out.report = out.weights.quantize_fp8(cfg, *fp8);
    if (save) save_fp8(dir, out.weights, *fp8, *out.report);
    return out;
}

}  // namespace reng_model
