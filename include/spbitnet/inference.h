// spbitnet/inference.h -- drop-in C++17 engine API for the MI355X build, over
// the C ABI in spbitnet_amd.h.
//
// Same class, constructor and members as the reference's
// include/spbitnet/inference.h:23-41: InferenceEngine(const Model&) borrows
// the model (it must outlive the engine), forward(token) returns device
// float32 logits, reset(), seq_len().  Added: max_seq (KV capacity; default
// max_position_embeddings), generate() (the whole greedy loop of
// src/main.cpp:133-155 on the device).  The reference's per-kernel Profiler
// is not provided (use rocprofv3).  Errors throw std::runtime_error.
#pragma once

#include <stdexcept>
#include <vector>

#include "spbitnet/model.h"

namespace spbitnet {

class InferenceEngine {
  public:
    explicit InferenceEngine(const Model& model, int max_seq = 0) : model_(model) {
        spb_model_config c;
        const spb_transformer_layer* ls = nullptr;
        const uint16_t *e = nullptr, *lm = nullptr;
        const float* fn = nullptr;
        spb_model_info(model.handle(), &c, &ls, &e, &lm, &fn, nullptr);
        check(spb_engine_create(&c, ls, e, lm, fn, max_seq > 0 ? max_seq : c.max_position_embeddings,
                                &h_));
    }
    ~InferenceEngine() { spb_engine_destroy(h_); }
    InferenceEngine(const InferenceEngine&) = delete;
    InferenceEngine& operator=(const InferenceEngine&) = delete;

    // reference include/spbitnet/inference.h:33
    const float* forward(int token_id) {
        const float* logits = nullptr;
        check(spb_engine_forward(h_, token_id, &logits));
        return logits;
    }
    // reference include/spbitnet/inference.h:36
    void reset() { check(spb_engine_reset(h_)); }
    // reference include/spbitnet/inference.h:38
    int seq_len() const { return spb_engine_seq_len(h_); }

    std::vector<int> generate(const std::vector<int>& prompt, int n_new, bool stop_at_eos = true) {
        std::vector<int> out(n_new > 0 ? n_new : 1);
        int got = 0;
        check(spb_engine_generate(h_, prompt.data(), static_cast<int>(prompt.size()), n_new,
                                  stop_at_eos ? 1 : 0, out.data(), &got));
        out.resize(got);
        return out;
    }

  private:
    static void check(int rc) {
        if (rc != 0) throw std::runtime_error(spb_last_error_string());
    }
    const Model& model_;
    spb_engine* h_ = nullptr;
};

}  // namespace spbitnet
