// reng_model.hpp - the fp8 slice of the reference's reng-model crate
// (crates/reng-model/src/lib.rs:1690-1966) in C++, over the reng-fp8 API of
// reng_fp8.hpp (whose numerics run on the GPU through libreng_hip.so): the
// fp8 switch (RENG_FP8 and --fp8), the per-layer fp8 weights, the load-time
// report, and the loader pieces they need (the config and the seven
// projections of a Llama-family safetensors checkpoint, memory-mapped).
#pragma once

#include <cstddef>
#include <optional>
#include <string>
#include <string_view>
#include <utility>
#include <vector>

#include "reng_fp8.hpp"
#include "safetensors.hpp"

namespace reng_model {

// ------------------------------------------------------------ config (lib.rs:82-700)

// The subset of a Hugging Face Llama-style config.json the fp8 slice needs.
struct LlamaConfig {
    std::string model_type;
    size_t hidden_size = 0;
    size_t intermediate_size = 0;
    size_t num_hidden_layers = 0;
    size_t num_attention_heads = 0;
    std::optional<size_t> num_key_value_heads;
    std::optional<size_t> head_dim_;   // config.json "head_dim"
    float rms_norm_eps = 0.0f;
    size_t vocab_size = 0;
    std::optional<bool> tie_word_embeddings;
    // Where the language model's tensors live: "model." (default) or
    // "language_model.model." for a multimodal config.
    std::string weight_prefix = "model.";
    // RoPE and attention settings the decode step reads (lib.rs:100-200):
    // rope_theta (1e4 when absent); the presence of rope_scaling, of a
    // sliding window and of the scale overrides, which the fp8 decode step
    // does not implement and refuses.
    float rope_theta = 10000.0f;
    bool has_rope_scaling = false;
    std::optional<size_t> sliding_window;
    std::optional<float> attention_multiplier, query_pre_attn_scalar;

    size_t n_kv_heads() const { return num_key_value_heads.value_or(num_attention_heads); }
    size_t head_dim() const { return head_dim_.value_or(hidden_size / num_attention_heads); }
    size_t q_dim() const { return num_attention_heads * head_dim(); }
    bool tied() const;

    static LlamaConfig from_json(const std::string &text);
    // dir/config.json.
    static LlamaConfig load(const std::string &dir);
};

// ------------------------------------------------------------ weights (lib.rs:1010-1110)

struct LayerTensors {
    std::vector<float> g1, g2;   // the two norm gains, f32
    Bf16Slice wq, wk, wv, wo, wg, wu, wd;
};

// ------------------------------------------------------------ fp8 switch (lib.rs:1690-1791)

struct Fp8Config {
    reng_fp8::Fp8Format format = reng_fp8::Fp8Format::E4M3;
    reng_fp8::Scaling scaling = reng_fp8::Scaling::PerChannel;
    float backoff = reng_fp8::DEFAULT_BACKOFF;

    bool operator==(const Fp8Config &o) const {
        return format == o.format && scaling == o.scaling && backoff == o.backoff;
    }
    // "e4m3/pcs backoff 1"
    std::string to_string() const;
};

// The value of RENG_FP8 (nullopt when unset) and whether --fp8 was given:
// off by default, off for "", 0, off, false, no (even with the flag); 1, on,
// true, yes or the flag alone mean the defaults; otherwise a ':' / ','
// separated list of a format, a scale scheme and backoff=<f32> in (0, 1].
// Throws Error naming the offending word.
std::optional<Fp8Config> fp8_switch(std::optional<std::string_view> value, bool flag);
// Removes every "--fp8" from args; true if there was one.
bool take_fp8_flag(std::vector<std::string> &args);

// One layer's seven projections as fp8, in the checkpoint's [out, in] layout.
struct LayerFp8 {
    reng_fp8::Quantized wq, wk, wv, wo, wg, wu, wd;
    std::vector<std::pair<const char *, const reng_fp8::Quantized *>> matrices() const;
    size_t code_bytes() const;
};

// What one quantization pass produced (lib.rs:1826-1868).
struct Fp8Report {
    size_t matrices = 0;
    size_t bf16_bytes = 0, fp8_bytes = 0, scale_bytes = 0;
    float mean_rel = 0.0f, max_rel = 0.0f;
    double secs = 0.0;
    bool operator==(const Fp8Report &o) const;
    // "7 matrices, 0.00 GiB bf16 -> 0.00 GiB fp8 + 0 KiB scales, mean rel ..., max rel ..., ... s"
    std::string to_string() const;
};

// Rows per matrix the loader measures the quantization error on.
constexpr size_t FP8_ERROR_ROWS = 8;

struct LlamaWeights {
    Bf16Slice embed;
    std::vector<LayerTensors> layers;
    std::vector<float> final_gamma;
    Bf16Slice lm_head;
    std::optional<std::vector<LayerFp8>> fp8;

    // Quantize the layers' seven projections (lib.rs:1882-1937); the bf16
    // views stay as they are.
    Fp8Report quantize_fp8(const LlamaConfig &cfg, const Fp8Config &q);
    size_t fp8_bytes() const;
};

// Load the checkpoint from a model directory (lib.rs:1463-1688, the Llama
// layout with Phi-3's fused qkv_proj / gate_up_proj): every bf16 matrix is a
// view of its mapped file.
LlamaWeights load_weights(const std::string &dir, const LlamaConfig &cfg);

// load_weights plus, when the switch is on, quantize_fp8 (lib.rs:1955-1966).
std::pair<LlamaWeights, std::optional<Fp8Report>> load_weights_fp8(const std::string &dir, const LlamaConfig &cfg,
                                                                   std::optional<Fp8Config> fp8);

// ------------------------------------------------------------ fp8 codes on disk
//
// The reference quantizes at every load (lib.rs:1871-1876, 1955-1966). These
// keep one quantization pass beside the checkpoint instead, as a safetensors
// file of U8 code and F32 scale tensors ("layers.<i>.<wq|wk|wv|wo|wg|wu|wd>.
// codes" [rows, cols], ".scales" [rows]) whose __metadata__ holds the switch
// that made them, each matrix's exp_bias, the quantization report and a
// fingerprint (name, size and modification time) of config.json and of every
// checkpoint file the weights were read from.

// The file's name in the model directory.
constexpr const char *FP8_CODES_FILE = "model.fp8.safetensors";

// Writes w.fp8 (made by quantize_fp8 with the switch q, which reported r) to
// dir/FP8_CODES_FILE through a temporary file and a rename. Throws Error when
// w carries no fp8 codes or on an I/O failure.
void save_fp8(const std::string &dir, const LlamaWeights &w, const Fp8Config &q, const Fp8Report &r);

// Reads dir/FP8_CODES_FILE into w.fp8 and returns the report saved with the
// codes (secs: the time this read took) when the file exists, was made with
// the switch q, and its fingerprint matches the directory's files now;
// nullopt, w untouched, otherwise. Throws Error for a current file whose
// tensors do not have the shapes cfg implies or which is not such a file.
std::optional<Fp8Report> load_fp8(const std::string &dir, const LlamaConfig &cfg, LlamaWeights &w,
                                  const Fp8Config &q);

// load_weights_fp8 that takes the codes from dir/FP8_CODES_FILE when load_fp8
// finds them current, and otherwise quantizes and, if save, writes the file.
struct Fp8Load {
    LlamaWeights weights;
    std::optional<Fp8Report> report;
    bool from_file = false;
};
Fp8Load load_weights_fp8_cached(const std::string &dir, const LlamaConfig &cfg, std::optional<Fp8Config> fp8,
                                bool save);

// The shortest decimal that reads back as the same f32 (Rust's {} for f32).
std::string f32_shortest(float x);

}  // namespace reng_model
