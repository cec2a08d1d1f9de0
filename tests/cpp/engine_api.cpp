// Host program written against the reference's C++ model / engine API
// (include/spbitnet/model.h, inference.h): loads a converted model directory
// and prints the greedy tokens, which the GPU test compares with the Python
// engine's.  usage: engine_api <model_dir> <n_new> <prompt ids...>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "spbitnet/inference.h"

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: %s model_dir n_new prompt...\n", argv[0]);
        return 2;
    }
    try {
        spbitnet::Model model = spbitnet::Model::load(argv[1]);
        spbitnet::InferenceEngine engine(model, 256);
        std::vector<int> prompt;
        for (int i = 3; i < argc; ++i) prompt.push_back(std::atoi(argv[i]));
        // the reference's forward() loop for the first token ...
        engine.reset();
        for (size_t i = 0; i + 1 < prompt.size(); ++i) engine.forward(prompt[i]);
        const float* logits = engine.forward(prompt.back());
        std::printf("seq_len %d logits %p\n", engine.seq_len(), static_cast<const void*>(logits));
        // ... and the whole greedy generation on the device
        std::vector<int> toks = engine.generate(prompt, std::atoi(argv[2]), false);
        std::printf("tokens");
        for (int t : toks) std::printf(" %d", t);
        std::printf("\n");
    } catch (const std::exception& e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return 0;
}
