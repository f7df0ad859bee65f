// Inference registry (rina-engine/src/infer/infer_shared.cpp:10-23).
#include <mutex>
#include <unordered_map>
#include "infer/infer_base.h"

Inference* create_gqa_inference();
Inference* create_mla_inference();

namespace {
std::unordered_map<std::string, InferenceFactory>& factories() {
    static std::unordered_map<std::string, InferenceFactory> f;
    return f;
}
std::mutex g_mu;
}  // namespace

void register_inference(const std::string& name, InferenceFactory f) {
    std::lock_guard<std::mutex> lk(g_mu);
    factories()[name] = f;
}

Inference* create_inference(const std::string& name) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = factories().find(name);
    return it != factories().end() ? it->second() : nullptr;
}

void register_all_inferences() {
    register_inference("gqa", create_gqa_inference);
    register_inference("mla", create_mla_inference);
}
