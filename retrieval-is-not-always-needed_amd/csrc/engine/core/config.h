// Model configuration: the fields of rina-engine/src/core/config.h:26-63
// that the decode path reads, plus the MoE / MLA shape keys of the
// DeepSeek-V2-Lite-shaped models.  parse_config reads a flat JSON object
// (the .rinn header style of loader.cpp:43-84) with a "layers" array of
// {"type": ...} objects.
#pragma once
#include <string>
#include <unordered_map>
#include <vector>

struct LayerConfig {
    std::string type;     // "standard_attention", "deepseek_mla_dense", ...
    std::string name;
    int layer_type = 1;
    std::unordered_map<std::string, int> args;
};

struct ModelConfig {
    std::string name;
    int dim = 0, n_layers = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
    int d_c = 0, d_h_r = 0;
    int ssm_steps = 0;             // RINA SSM layers (config.h:38)
    int vocab_size = 0, max_seq_len = 0;
    int hidden_dim = 0;            // SwiGLU intermediate (0: from w1's shape)
    bool weight_tying = true;
    std::string kv_quant_mode = "fp32";   // GQA caches only (infer_gqa.cpp), as in the reference
    // RINA-MLA (Jamba) cache form, an engine extension with no reference key:
    // "fp32" (the reference's numerics) or "q2k_q1v" (q2_1 key content, q1_0
    // values, packed on append).  kv_quant_mode never changes RINA-MLA layers.
    std::string rina_mla_kv_mode = "fp32";
    bool use_pre_rope_k = false;
    // MLA / MoE (DeepSeek-V2-Lite shape)
    int kv_lora_rank = 0, qk_nope_dim = 0, qk_rope_dim = 0, v_head_dim = 0;
    int n_experts = 0, top_k = 0, n_shared = 0, expert_dim = 0;
    std::vector<LayerConfig> layers;
};

bool parse_config(const std::string& json, ModelConfig& cfg, std::string* err = nullptr);
