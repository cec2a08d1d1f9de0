// spbitnet/model.h -- drop-in C++17 model API for the MI355X build, over the
// C ABI in spbitnet_amd.h.
//
// Same namespace, types and members as the reference's
// include/spbitnet/model.h:23-145 (ModelConfig, SparseLinear,
// TransformerLayer, Model::load and its accessors); Model is move-only and
// owns the device memory, as in the reference.  Differences: the embedding
// and LM head are bf16 on the device (the decode engine's storage type; the
// fp16 files are converted on load), and Model::load throws
// std::runtime_error with the library's message.
#pragma once

#include <hip/hip_bf16.h>

#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "spbitnet_amd.h"

namespace spbitnet {

// reference include/spbitnet/model.h:23-40
struct ModelConfig {
    std::string model_type = "bitnet";
    int hidden_size = 0;
    int num_hidden_layers = 0;
    int num_attention_heads = 0;
    int num_key_value_heads = 0;
    int intermediate_size = 0;
    int vocab_size = 0;
    int max_position_embeddings = 0;
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
    int head_dim = 0;
    std::string hidden_act = "relu2";
    bool tie_word_embeddings = false;
    int bos_token_id = 1;
    int eos_token_id = 2;
};

// reference include/spbitnet/model.h:46-60
struct SparseLinear {
    uint32_t* d_meta = nullptr;
    uint32_t* d_values = nullptr;
    float gamma = 0.0f;
    int rows = 0;
    int cols = 0;
    int meta_stride = 0;
    int values_stride = 0;
    size_t gpu_bytes() const {
        return static_cast<size_t>(rows) * meta_stride * sizeof(uint32_t) +
               static_cast<size_t>(rows) * values_stride * sizeof(uint32_t);
    }
};

// reference include/spbitnet/model.h:63-82
struct TransformerLayer {
    SparseLinear q_proj, k_proj, v_proj, o_proj;
    SparseLinear gate_proj, up_proj, down_proj;
    float* d_input_layernorm = nullptr;
    float* d_post_attention_layernorm = nullptr;
    float* d_attn_sub_norm = nullptr;
    float* d_ffn_sub_norm = nullptr;
};

namespace detail {
inline SparseLinear from_c(const spb_sparse_linear& s) {
    SparseLinear l;
    l.d_meta = const_cast<uint32_t*>(s.meta);
    l.d_values = const_cast<uint32_t*>(s.values);
    l.gamma = s.gamma;
    l.rows = s.rows;
    l.cols = s.cols;
    l.meta_stride = s.meta_stride;
    l.values_stride = s.values_stride;
    return l;
}
}  // namespace detail

// reference include/spbitnet/model.h:88-145
class Model {
  public:
    static Model load(const std::string& model_dir) {
        spb_model* h = nullptr;
        if (spb_model_load(model_dir.c_str(), &h) != 0)
            throw std::runtime_error(spb_last_error_string());
        return Model(h);
    }
    ~Model() { spb_model_destroy(h_); }
    Model(Model&& o) noexcept : h_(o.h_), cfg_(std::move(o.cfg_)), layers_(std::move(o.layers_)),
                                embed_(o.embed_), lm_(o.lm_), norm_(o.norm_), bytes_(o.bytes_) {
        o.h_ = nullptr;
    }
    Model& operator=(Model&& o) noexcept {
        if (this != &o) {
            spb_model_destroy(h_);
            h_ = o.h_;
            cfg_ = std::move(o.cfg_);
            layers_ = std::move(o.layers_);
            embed_ = o.embed_;
            lm_ = o.lm_;
            norm_ = o.norm_;
            bytes_ = o.bytes_;
            o.h_ = nullptr;
        }
        return *this;
    }
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    const ModelConfig& config() const { return cfg_; }
    const std::vector<TransformerLayer>& layers() const { return layers_; }
    const TransformerLayer& layer(int i) const { return layers_[i]; }
    const __hip_bfloat16* embed_tokens() const { return embed_; }
    const float* final_norm() const { return norm_; }
    const __hip_bfloat16* lm_head() const { return lm_ ? lm_ : embed_; }
    size_t total_gpu_bytes() const { return bytes_; }
    void print_summary() const {
        std::printf("  Model loaded: %d layers, %.1f MB on the GPU\n", cfg_.num_hidden_layers,
                    static_cast<double>(bytes_) / 1e6);
    }
    // The C-ABI handle (for spb_engine_create through InferenceEngine).
    const spb_model* handle() const { return h_; }

  private:
    explicit Model(spb_model* h) : h_(h) {
        spb_model_config c;
        const spb_transformer_layer* ls = nullptr;
        const uint16_t *e = nullptr, *lm = nullptr;
        const float* fn = nullptr;
        spb_model_info(h_, &c, &ls, &e, &lm, &fn, &bytes_);
        cfg_.hidden_size = c.hidden_size;
        cfg_.num_hidden_layers = c.num_hidden_layers;
        cfg_.num_attention_heads = c.num_attention_heads;
        cfg_.num_key_value_heads = c.num_key_value_heads;
        cfg_.intermediate_size = c.intermediate_size;
        cfg_.vocab_size = c.vocab_size;
        cfg_.max_position_embeddings = c.max_position_embeddings;
        cfg_.rms_norm_eps = c.rms_norm_eps;
        cfg_.rope_theta = c.rope_theta;
        cfg_.head_dim = c.head_dim;
        cfg_.tie_word_embeddings = lm == nullptr;
        cfg_.bos_token_id = c.bos_token_id;
        cfg_.eos_token_id = c.eos_token_id;
        for (int i = 0; i < c.num_hidden_layers; ++i) {
            const spb_transformer_layer& s = ls[i];
            TransformerLayer t;
            t.q_proj = detail::from_c(s.q_proj);
            t.k_proj = detail::from_c(s.k_proj);
            t.v_proj = detail::from_c(s.v_proj);
            t.o_proj = detail::from_c(s.o_proj);
            t.gate_proj = detail::from_c(s.gate_proj);
            t.up_proj = detail::from_c(s.up_proj);
            t.down_proj = detail::from_c(s.down_proj);
            t.d_input_layernorm = const_cast<float*>(s.input_layernorm);
            t.d_post_attention_layernorm = const_cast<float*>(s.post_attention_layernorm);
            t.d_attn_sub_norm = const_cast<float*>(s.attn_sub_norm);
            t.d_ffn_sub_norm = const_cast<float*>(s.ffn_sub_norm);
            layers_.push_back(t);
        }
        embed_ = reinterpret_cast<const __hip_bfloat16*>(e);
        lm_ = reinterpret_cast<const __hip_bfloat16*>(lm);
        norm_ = fn;
    }

    spb_model* h_ = nullptr;
    ModelConfig cfg_;
    std::vector<TransformerLayer> layers_;
    const __hip_bfloat16* embed_ = nullptr;
    const __hip_bfloat16* lm_ = nullptr;
    const float* norm_ = nullptr;
    size_t bytes_ = 0;
};

}  // namespace spbitnet
