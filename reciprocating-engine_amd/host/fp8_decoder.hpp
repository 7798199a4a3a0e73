// fp8_decoder.hpp - the device consumer of LlamaWeights::fp8: one decode step
// (one token) of a Llama decoder layer whose seven projections are the fp8
// GEMV over the layer's codes and per-row scales (q, k and v as one GEMV with
// the RMSNorm as its prologue and RoPE and the cache append as its epilogue;
// gate and up as one over their rows alternating, with silu(gate) * up as its
// epilogue; o and down with the residual add as their epilogue).
//
// The reference quantizes on the host and then refuses at the point where the
// codes would meet a device layer (layer_views, crates/reng-model/src/lib.rs:
// 2636-2649). This is that layer on libreng_hip.so, with the semantics of the
// reference's CPU decoder layer (layer_cpu, crates/reng-synapse/src/model.rs:
// 2903-3100, causal) in its Llama form: pre-norm RMSNorm, q/k/v, rotate-half
// RoPE (rope_theta, no scaling), grouped-query attention over a bf16 key/value
// cache, o-proj + residual, RMSNorm, SiLU(gate) * up, down + residual.
// Residual stream f32; every GEMV input bf16.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "reng_model.hpp"

namespace reng_model {

class Fp8Decoder {
   public:
    // Uploads every layer's codes, scales and norm gains, allocates a bf16
    // key and value cache of max_positions rows per layer and the RoPE tables
    // for them. Throws Error when w.fp8 is empty, for a model this step does not
    // implement (a model_type other than llama / mistral, rope_scaling, a
    // sliding window, an attention scale override, head_dim odd), for
    // max_positions outside [1, RENG_HIP_ATTENTION_MAX_LEN], hidden_size past
    // 32768, and on a device failure.
    Fp8Decoder(const LlamaConfig &cfg, const LlamaWeights &w, size_t max_positions);
    ~Fp8Decoder();
    Fp8Decoder(const Fp8Decoder &) = delete;
    Fp8Decoder &operator=(const Fp8Decoder &) = delete;

    // Layer li's output row for its input row x ([hidden] f32) at position
    // pos, appending the position's key and value rows to the layer's cache.
    // A layer's positions run 0, 1, 2, ... (pos must equal the number of
    // steps that layer has taken); throws Error otherwise.
    std::vector<float> step(size_t li, const std::vector<float> &x, size_t pos);

    // The same on device buffers: x and y are [hidden] f32 device pointers
    // (may alias), stream a hipStream_t (nullptr = the null stream);
    // asynchronous.
    void step_device(size_t li, const float *x, float *y, size_t pos, void *stream);

    // Every layer back to position 0.
    void reset();

    size_t layers() const { return layers_.size(); }
    size_t positions(size_t li) const { return layers_.at(li).pos; }

   private:
    struct Mat {
        uint8_t *codes = nullptr;
        float *scales = nullptr;
        size_t rows = 0, cols = 0;
        int format = 0;
    };
    struct Layer {
        Mat wqkv, wo, wgu, wd;   // q, k, v rows in rotation pairs; gate, up rows alternating
        float *g1 = nullptr, *g2 = nullptr;
        uint16_t *kcache = nullptr, *vcache = nullptr;
        size_t pos = 0;
    };

    size_t hidden_, inter_, nh_, nkv_, hd_, max_pos_;
    float eps_, scale_;
    std::vector<Layer> layers_;
    std::vector<void *> allocs_;
    float *sin_ = nullptr, *cos_ = nullptr;
    // scratch: residual f32 rows, bf16 GEMV inputs and outputs
    float *x_ = nullptr, *h_ = nullptr;
    uint16_t *q_ = nullptr, *a_ = nullptr;
    uint16_t *act_ = nullptr;
    // the split attention's partial outputs (one layer at a time)
    void *attn_ws_ = nullptr;
    size_t attn_ws_bytes_ = 0;
};

}  // namespace reng_model
