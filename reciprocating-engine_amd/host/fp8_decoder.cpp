// fp8_decoder.cpp - see fp8_decoder.hpp.
#include "fp8_decoder.hpp"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <initializer_list>
#include <string>

#include "../../include/reng_hip.h"

namespace reng_model {

namespace {

void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

void abi_ok(int rc) {
    if (rc != RENG_HIP_OK) throw Error(std::string("reng-hip: ") + reng_hip_last_error());
}

int abi_format(reng_fp8::Fp8Format f) { return f == reng_fp8::Fp8Format::E4M3 ? RENG_HIP_E4M3 : RENG_HIP_E5M2; }

}  // namespace

Fp8Decoder::Fp8Decoder(const LlamaConfig &cfg, const LlamaWeights &w, size_t max_positions) {
    if (!w.fp8) throw Error("Fp8Decoder: the weights carry no fp8 codes (load them with the fp8 switch on)");
    if (!(cfg.model_type == "llama" || cfg.model_type == "mistral" || cfg.model_type.empty()))
        throw Error("Fp8Decoder: model_type " + cfg.model_type +
                    " is not implemented by the fp8 decode step (Llama form only)");
    if (cfg.has_rope_scaling) throw Error("Fp8Decoder: rope_scaling is not implemented by the fp8 decode step");
    if (cfg.sliding_window) throw Error("Fp8Decoder: sliding_window is not implemented by the fp8 decode step");
    if (cfg.attention_multiplier || cfg.query_pre_attn_scalar)
        throw Error("Fp8Decoder: an attention scale override is not implemented by the fp8 decode step");
    hidden_ = cfg.hidden_size;
    inter_ = cfg.intermediate_size;
    nh_ = cfg.num_attention_heads;
    nkv_ = cfg.n_kv_heads();
    hd_ = cfg.head_dim();
    eps_ = cfg.rms_norm_eps;
    // layer_cpu's score scale for a model without overrides (lib.rs:701-705).
    scale_ = 1.0f / std::sqrt((float)hd_);
    max_pos_ = max_positions;
    if (hd_ % 2 != 0 || hd_ == 0) throw Error("Fp8Decoder: head_dim " + std::to_string(hd_) + " is not even");
    if (nkv_ == 0 || nh_ % nkv_ != 0) throw Error("Fp8Decoder: heads are not a multiple of key/value heads");
    if (max_pos_ < 1 || max_pos_ > RENG_HIP_ATTENTION_MAX_LEN)
        throw Error("Fp8Decoder: max_positions " + std::to_string(max_pos_) + " is not in [1, " +
                    std::to_string(RENG_HIP_ATTENTION_MAX_LEN) + "]");
    if (w.fp8->size() != w.layers.size()) throw Error("Fp8Decoder: fp8 layers do not match the weights");
    // The normalised row a GEMV reads is staged whole in its workgroups' LDS.
    if (hidden_ > 32768)
        throw Error("Fp8Decoder: hidden_size " + std::to_string(hidden_) + " is past 32768, which the fp8 decode step "
                    "does not implement");

    auto dev = [&](size_t bytes) {
        void *p = nullptr;
        hip_ok(hipMalloc(&p, bytes > 0 ? bytes : 1), "hipMalloc");
        allocs_.push_back(p);
        return p;
    };
    auto upload = [&](const void *src, size_t bytes) {
        void *p = dev(bytes);
        hip_ok(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice), "hipMemcpy");
        return p;
    };
    try {
        const size_t qd = nh_ * hd_, kvd = nkv_ * hd_;
        auto check = [&](const reng_fp8::Quantized &q, size_t rows, size_t cols, const char *name) {
            if (q.rows != rows || q.cols != cols)
                throw Error(std::string("Fp8Decoder: ") + name + " is " + std::to_string(q.rows) + " x " +
                            std::to_string(q.cols) + ", the config implies " + std::to_string(rows) + " x " +
                            std::to_string(cols));
            if (cols % 16 != 0) throw Error(std::string("Fp8Decoder: ") + name + " width is not a multiple of 16");
        };
        // Projections of one input row are one GEMV over their rows stacked in
        // order (q, k, v): each output row is its own matrix's row. With
        // `pairs` two matrices of equal rows alternate instead (gate row i at
        // 2i, up row i at 2i + 1), the layout of the SwiGLU GEMV.
        auto mat = [&](std::initializer_list<const reng_fp8::Quantized *> parts, bool pairs = false) {
            const reng_fp8::Quantized &first = **parts.begin();
            if (pairs && (parts.size() != 2 || parts.begin()[1]->rows != first.rows))
                throw Error("Fp8Decoder: paired projections need two matrices of equal rows");
            Mat m;
            m.cols = first.cols;
            m.format = abi_format(first.format);
            for (const reng_fp8::Quantized *q : parts) {
                if (abi_format(q->format) != m.format)
                    throw Error("Fp8Decoder: projections of one input row carry different fp8 formats");
                m.rows += q->rows;
            }
            m.codes = static_cast<uint8_t *>(dev(m.rows * m.cols));
            m.scales = static_cast<float *>(dev(m.rows * sizeof(float)));
            size_t r0 = 0;
            for (const reng_fp8::Quantized *q : parts) {
                if (pairs) {   // rows r0, r0 + 2, ... of the interleaved matrix (r0 = 0, 1)
                    hip_ok(hipMemcpy2D(m.codes + r0 * m.cols, 2 * m.cols, q->codes.data(), m.cols, m.cols, q->rows,
                                       hipMemcpyHostToDevice),
                           "hipMemcpy2D");
                    hip_ok(hipMemcpy2D(m.scales + r0, 2 * sizeof(float), q->scales.data(), sizeof(float),
                                       sizeof(float), q->rows, hipMemcpyHostToDevice),
                           "hipMemcpy2D");
                    r0 += 1;
                    continue;
                }
                hip_ok(hipMemcpy(m.codes + r0 * m.cols, q->codes.data(), q->codes.size(), hipMemcpyHostToDevice),
                       "hipMemcpy");
                hip_ok(hipMemcpy(m.scales + r0, q->scales.data(), q->rows * sizeof(float), hipMemcpyHostToDevice),
                       "hipMemcpy");
                r0 += q->rows;
            }
            return m;
        };
        // q, k and v rows stacked in rotation-pair order
        // (reng_hip_gemv_w8a16_rmsnorm_qkv_rope): the (d, d + half) rows of
        // each q head, then of each k head, then the v rows.
        auto qkv_rope = [&](const LayerFp8 &f) {
            if (abi_format(f.wk.format) != abi_format(f.wq.format) ||
                abi_format(f.wv.format) != abi_format(f.wq.format))
                throw Error("Fp8Decoder: projections of one input row carry different fp8 formats");
            Mat m;
            m.rows = qd + 2 * kvd;
            m.cols = hidden_;
            m.format = abi_format(f.wq.format);
            std::vector<uint8_t> codes(m.rows * m.cols);
            std::vector<float> scales(m.rows);
            size_t r = 0;
            auto put = [&](const reng_fp8::Quantized &q, size_t src) {
                std::memcpy(&codes[r * m.cols], &q.codes[src * m.cols], m.cols);
                scales[r++] = q.scales[src];
            };
            const size_t half = hd_ / 2;
            for (size_t h = 0; h < nh_; ++h)
                for (size_t d = 0; d < half; ++d) {
                    put(f.wq, h * hd_ + d);
                    put(f.wq, h * hd_ + d + half);
                }
            for (size_t g = 0; g < nkv_; ++g)
                for (size_t d = 0; d < half; ++d) {
                    put(f.wk, g * hd_ + d);
                    put(f.wk, g * hd_ + d + half);
                }
            for (size_t i = 0; i < kvd; ++i) put(f.wv, i);
            m.codes = static_cast<uint8_t *>(upload(codes.data(), codes.size()));
            m.scales = static_cast<float *>(upload(scales.data(), scales.size() * sizeof(float)));
            return m;
        };
        for (size_t li = 0; li < w.layers.size(); ++li) {
            const LayerFp8 &f = (*w.fp8)[li];
            const LayerTensors &t = w.layers[li];
            check(f.wq, qd, hidden_, "wq");
            check(f.wk, kvd, hidden_, "wk");
            check(f.wv, kvd, hidden_, "wv");
            check(f.wo, hidden_, qd, "wo");
            check(f.wg, inter_, hidden_, "wg");
            check(f.wu, inter_, hidden_, "wu");
            check(f.wd, hidden_, inter_, "wd");
            Layer L;
            L.wqkv = qkv_rope(f);
            L.wo = mat({&f.wo});
            L.wgu = mat({&f.wg, &f.wu}, true);
            L.wd = mat({&f.wd});
            if (t.g1.size() != hidden_ || t.g2.size() != hidden_) throw Error("Fp8Decoder: norm gains are not [hidden]");
            L.g1 = static_cast<float *>(upload(t.g1.data(), hidden_ * sizeof(float)));
            L.g2 = static_cast<float *>(upload(t.g2.data(), hidden_ * sizeof(float)));
            L.kcache = static_cast<uint16_t *>(dev(max_pos_ * kvd * 2));
            L.vcache = static_cast<uint16_t *>(dev(max_pos_ * kvd * 2));
            layers_.push_back(L);
        }
        // rope_caches (lib.rs:1970-1972, 2188-2215 with rotary_dim = head_dim):
        // entry (p, d) = sin / cos(p * theta^(-2 (d % half) / head_dim)).
        std::vector<float> sn(max_pos_ * hd_), cs(max_pos_ * hd_);
        const size_t half = hd_ / 2;
        for (size_t p = 0; p < max_pos_; ++p)
            for (size_t d = 0; d < hd_; ++d) {
                const float inv = std::pow(cfg.rope_theta, -2.0f * (float)(d % half) / (float)hd_);
                const float ang = (float)p * inv;
                sn[p * hd_ + d] = std::sin(ang);
                cs[p * hd_ + d] = std::cos(ang);
            }
        sin_ = static_cast<float *>(upload(sn.data(), sn.size() * sizeof(float)));
        cos_ = static_cast<float *>(upload(cs.data(), cs.size() * sizeof(float)));
        x_ = static_cast<float *>(dev(hidden_ * 4));
        h_ = static_cast<float *>(dev(hidden_ * 4));
        // bf16 buffers 16-byte aligned (hipMalloc) for the GEMV's inputs.
        q_ = static_cast<uint16_t *>(dev(qd * 2));
        a_ = static_cast<uint16_t *>(dev(qd * 2));
        act_ = static_cast<uint16_t *>(dev(inter_ * 2));
        attn_ws_bytes_ = reng_hip_attention_workspace_bytes(nh_, hd_, max_pos_);
        attn_ws_ = dev(attn_ws_bytes_);
    } catch (...) {
        for (void *p : allocs_) (void)hipFree(p);
        allocs_.clear();
        throw;
    }
}

Fp8Decoder::~Fp8Decoder() {
    (void)hipDeviceSynchronize();
    for (void *p : allocs_) (void)hipFree(p);
}

void Fp8Decoder::step_device(size_t li, const float *x, float *y, size_t pos, void *stream) {
    Layer &L = layers_.at(li);
    if (pos != L.pos)
        throw Error("Fp8Decoder: layer " + std::to_string(li) + " is at position " + std::to_string(L.pos) +
                    ", asked for " + std::to_string(pos));
    if (pos >= max_pos_) throw Error("Fp8Decoder: position " + std::to_string(pos) + " is past the cache");
    const size_t kvd = nkv_ * hd_;
    // Norm + q/k/v + RoPE + the cache append; attention; o-proj + residual
    // (h); norm + gate/up + SiLU * up; down + residual (y).
    abi_ok(reng_hip_gemv_w8a16_rmsnorm_qkv_rope(x, L.g1, eps_, L.wqkv.codes, L.wqkv.scales, nh_, nkv_, hd_, hidden_,
                                                L.wqkv.format, sin_ + pos * hd_, cos_ + pos * hd_, q_,
                                                L.kcache + pos * kvd, L.vcache + pos * kvd, stream));
    abi_ok(reng_hip_attention_decode_split(q_, L.kcache, L.vcache, nh_, nkv_, hd_, pos + 1, scale_, attn_ws_,
                                           attn_ws_bytes_, a_, stream));
    abi_ok(reng_hip_gemv_w8a16_residual(a_, L.wo.codes, L.wo.scales, L.wo.rows, L.wo.cols, L.wo.format, x, h_,
                                        stream));
    abi_ok(reng_hip_gemv_w8a16_rmsnorm_swiglu(h_, L.g2, eps_, L.wgu.codes, L.wgu.scales, L.wgu.rows, L.wgu.cols,
                                              L.wgu.format, act_, stream));
    abi_ok(reng_hip_gemv_w8a16_residual(act_, L.wd.codes, L.wd.scales, L.wd.rows, L.wd.cols, L.wd.format, h_, y,
                                        stream));
    ++L.pos;
}

std::vector<float> Fp8Decoder::step(size_t li, const std::vector<float> &x, size_t pos) {
    if (x.size() != hidden_)
        throw Error("Fp8Decoder: input row has " + std::to_string(x.size()) + " values, hidden is " +
                    std::to_string(hidden_));
    hip_ok(hipMemcpy(x_, x.data(), hidden_ * 4, hipMemcpyHostToDevice), "hipMemcpy");
    step_device(li, x_, x_, pos, nullptr);
    std::vector<float> y(hidden_);
    hip_ok(hipMemcpy(y.data(), x_, hidden_ * 4, hipMemcpyDeviceToHost), "hipMemcpy");
    return y;
}

void Fp8Decoder::reset() {
    for (Layer &L : layers_) L.pos = 0;
}

}  // namespace reng_model
