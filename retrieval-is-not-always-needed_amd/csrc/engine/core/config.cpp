// Minimal reader for the flat JSON model header (the subset the decode path
// uses: string / number / bool values and a "layers" array of objects).
#include "core/config.h"
#include <cctype>
#include <cstdlib>

namespace {

struct Reader {
    const std::string& s;
    size_t i = 0;
    explicit Reader(const std::string& str) : s(str) {}
    void ws() { while (i < s.size() && isspace((unsigned char)s[i])) i++; }
    bool eat(char c) { ws(); if (i < s.size() && s[i] == c) { i++; return true; } return false; }
    bool str(std::string& out) {
        ws();
        if (i >= s.size() || s[i] != '"') return false;
        i++;
        out.clear();
        while (i < s.size() && s[i] != '"') {
            if (s[i] == '\\' && i + 1 < s.size()) i++;
            out += s[i++];
        }
        if (i >= s.size()) return false;
        i++;
        return true;
    }
    // scalar value as text (numbers, true/false/null, strings)
    bool scalar(std::string& out, bool& is_str) {
        ws();
        if (i < s.size() && s[i] == '"') { is_str = true; return str(out); }
        is_str = false;
        size_t b = i;
        while (i < s.size() && s[i] != ',' && s[i] != '}' && s[i] != ']' && !isspace((unsigned char)s[i])) i++;
        out = s.substr(b, i - b);
        return i > b;
    }
    bool skip_value() {
        ws();
        if (i >= s.size()) return false;
        if (s[i] == '{' || s[i] == '[') {
            char open = s[i], close = open == '{' ? '}' : ']';
            int depth = 0;
            bool in_str = false;
            for (; i < s.size(); i++) {
                char c = s[i];
                if (in_str) { if (c == '\\') i++; else if (c == '"') in_str = false; continue; }
                if (c == '"') in_str = true;
                else if (c == open) depth++;
                else if (c == close && --depth == 0) { i++; return true; }
            }
            return false;
        }
        std::string t;
        bool q;
        return scalar(t, q);
    }
};

void set_field(ModelConfig& c, const std::string& k, const std::string& v) {
    auto I = [&](int& f) { f = atoi(v.c_str()); };
    if (k == "name") c.name = v;
    else if (k == "dim") I(c.dim);
    else if (k == "n_layers") I(c.n_layers);
    else if (k == "n_heads") I(c.n_heads);
    else if (k == "n_kv_heads") I(c.n_kv_heads);
    else if (k == "head_dim") I(c.head_dim);
    else if (k == "d_c") I(c.d_c);
    else if (k == "ssm_steps") I(c.ssm_steps);
    else if (k == "d_h_r") I(c.d_h_r);
    else if (k == "vocab_size") I(c.vocab_size);
    else if (k == "max_seq_len" || k == "block_size") I(c.max_seq_len);
    else if (k == "hidden_dim" || k == "intermediate_size") I(c.hidden_dim);
    else if (k == "weight_tying") c.weight_tying = (v == "true");
    else if (k == "kv_quant_mode") c.kv_quant_mode = v;
    else if (k == "rina_mla_kv_mode") c.rina_mla_kv_mode = v;
    else if (k == "use_pre_rope_k") c.use_pre_rope_k = (v == "true" || v == "1");
    else if (k == "kv_lora_rank") I(c.kv_lora_rank);
    else if (k == "qk_nope_head_dim") I(c.qk_nope_dim);
    else if (k == "qk_rope_head_dim") I(c.qk_rope_dim);
    else if (k == "v_head_dim") I(c.v_head_dim);
    else if (k == "n_routed_experts") I(c.n_experts);
    else if (k == "num_experts_per_tok") I(c.top_k);
    else if (k == "n_shared_experts") I(c.n_shared);
    else if (k == "moe_intermediate_size") I(c.expert_dim);
}

}  // namespace

bool parse_config(const std::string& json, ModelConfig& cfg, std::string* err) {
    Reader r(json);
    auto fail = [&](const char* m) { if (err) *err = m; return false; };
    if (!r.eat('{')) return fail("config: expected '{'");
    if (r.eat('}')) return true;
    do {
        std::string key;
        if (!r.str(key)) return fail("config: expected key");
        if (!r.eat(':')) return fail("config: expected ':'");
        r.ws();
        if (key == "layers" && r.i < json.size() && json[r.i] == '[') {
            r.i++;
            if (!r.eat(']')) {
                do {
                    if (!r.eat('{')) return fail("config: layers entries must be objects");
                    LayerConfig lc;
                    if (!r.eat('}')) {
                        do {
                            std::string k2, v2;
                            bool q;
                            if (!r.str(k2) || !r.eat(':')) return fail("config: bad layer entry");
                            r.ws();
                            if (r.i < json.size() && (json[r.i] == '{' || json[r.i] == '[')) {
                                if (!r.skip_value()) return fail("config: bad layer value");
                                continue;
                            }
                            if (!r.scalar(v2, q)) return fail("config: bad layer value");
                            if (k2 == "type") lc.type = v2;
                            else lc.args[k2] = atoi(v2.c_str());
                        } while (r.eat(','));
                        if (!r.eat('}')) return fail("config: expected '}' in layer");
                    }
                    lc.name = "layer_" + std::to_string(cfg.layers.size());
                    lc.layer_type = lc.type.find("ssm") != std::string::npos ? 0 : 1;
                    cfg.layers.push_back(lc);
                } while (r.eat(','));
                if (!r.eat(']')) return fail("config: expected ']'");
            }
            continue;
        }
        if (r.i < json.size() && (json[r.i] == '{' || json[r.i] == '[')) {
            if (!r.skip_value()) return fail("config: bad value");
            continue;
        }
        std::string val;
        bool q;
        if (!r.scalar(val, q)) return fail("config: bad value");
        set_field(cfg, key, val);
    } while (r.eat(','));
    if (!r.eat('}')) return fail("config: expected '}'");
    return true;
}
