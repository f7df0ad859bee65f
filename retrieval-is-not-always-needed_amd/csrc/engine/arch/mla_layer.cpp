// DeepSeek MLA layer, dense or MoE MLP (rina-engine/src/arch/mla/
// deepseek_mla_layer.cu:43-350) on the gfx950 C-ABI, with the reference's
// tensor names.  Per token:
//   a = RMSNorm(h, ln1); q = W_q a ([H*nope | H*rope]); kva = W_kv_a a
//   ([c_kv | k_pe]); latent attention over the cache (c_kv normalized with
//   k_norm, RoPE on q_rope and k_pe, W_kv_b folded into the query and the
//   output: rina_hip_mla_decode_attention); h += W_o o;
//   a = RMSNorm(h, ln2); dense: h += W2 (SiLU(W1 a) * W3 a); MoE:
//   acc = shared experts(a); top-k of softmax(W_gate a) on the device;
//   acc += p_j expert_j(a) (ascending j); h += acc.
// The reference's decode path (start_pos > 0) is broken; this is its
// intended math at any position.  Its host round trip per MoE layer
// (cudaStreamSynchronize + D2H of the router logits, :306-308) is gone.
#include <algorithm>
#include <cstdio>
#include <string>
#include "core/buffer.h"
#include "core/config.h"
#include "core/layer.h"
#include "core/tensor.h"
#include "rina_hip.h"

namespace {

std::string tn(int l, const char* c, const char* p) {
    char b[160];
    snprintf(b, sizeof b, "transformer.h.%d.%s.%s", l, c, p);
    return b;
}

struct MLAImpl {
    int d = 0, H = 0, nope = 0, rope = 0, vd = 0, dc = 0, layer = 0;
    bool is_moe = false;
    int hd = 0;                             // dense SwiGLU width
    int E = 0, K = 0, F = 0, S = 0;         // experts, top-k, expert ffn, shared ffn
    int64_t stride_gu = 0, stride_dn = 0;
    WeightRef w_q, w_kv_a, w_kv_b, w_o, w1, w2, w3;
    WeightRef gate_inp, gate_exps, up_exps, down_exps, gate_sh, up_sh, down_sh;
    const float *ln1 = nullptr, *ln2 = nullptr, *k_norm = nullptr, *rope_c = nullptr, *rope_s = nullptr;
    // fused MoE block (rina_hip_moe_block) and its workspace; shapes it does
    // not take use the per-operator composition below
    bool moe_block = false;
    void* moe_ws = nullptr;
    size_t moe_ws_bytes = 0;

    ~MLAImpl() {
        if (moe_ws) (void)hipFree(moe_ws);
    }

    bool init(const ModelConfig& cfg, const TensorMap& w, int l) {
        layer = l;
        d = cfg.dim;
        H = cfg.n_heads;
        nope = cfg.qk_nope_dim > 0 ? cfg.qk_nope_dim : cfg.head_dim;                       // :57-60
        rope = cfg.qk_rope_dim > 0 ? cfg.qk_rope_dim : (cfg.d_h_r > 0 ? cfg.d_h_r : 64);
        vd = cfg.v_head_dim > 0 ? cfg.v_head_dim : cfg.head_dim;
        dc = cfg.kv_lora_rank > 0 ? cfg.kv_lora_rank : (cfg.d_c > 0 ? cfg.d_c : 512);
        auto ref = [&](const std::string& n, WeightRef& r) {
            const WeightTensor* t = w.get(n);
            if (!t) return false;
            r.data = t->data; r.qt = t->quant_type;
            return true;
        };
        auto f32 = [&](const std::string& n, const float*& p) {
            const WeightTensor* t = w.get(n);
            p = t ? (const float*)t->data : nullptr;
            return p != nullptr;
        };
        bool ok = ref(tn(l, "attn", "w_q.weight"), w_q) & ref(tn(l, "attn", "w_kv_a.weight"), w_kv_a) &
                  ref(tn(l, "attn", "w_kv_b.weight"), w_kv_b) & ref(tn(l, "attn", "w_o.weight"), w_o) &
                  f32(tn(l, "attn", "k_norm.weight"), k_norm) & f32(tn(l, "ln1", "weight"), ln1) &
                  f32(tn(l, "ln2", "weight"), ln2);
        f32(tn(l, "attn", "rope_q.cos"), rope_c);
        f32(tn(l, "attn", "rope_q.sin"), rope_s);
        auto is = [&](const char* c, const char* p, int64_t n) { return elems_are(w.get(tn(l, c, p)), n); };
        const int64_t ms = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        ok = ok && is("attn", "w_q.weight", (int64_t)H * (nope + rope) * d) &&
             is("attn", "w_kv_a.weight", (int64_t)(dc + rope) * d) && is("attn", "k_norm.weight", dc) &&
             is("attn", "w_kv_b.weight", (int64_t)H * (nope + vd) * dc) && is("attn", "w_o.weight", (int64_t)d * H * vd) &&
             is("ln1", "weight", d) && is("ln2", "weight", d);
        for (const char* r : {"rope_q.cos", "rope_q.sin"}) {
            const WeightTensor* t = w.get(tn(l, "attn", r));
            if (t && !elems_at_least(t, ms * (rope / 2))) ok = false;
        }
        const WeightTensor* gi = w.get(tn(l, "mlp", "gate_inp.weight"));
        is_moe = gi != nullptr;
        if (is_moe) {
            ok = ok & ref(tn(l, "mlp", "gate_inp.weight"), gate_inp) & ref(tn(l, "mlp", "gate_exps.weight"), gate_exps) &
                 ref(tn(l, "mlp", "up_exps.weight"), up_exps) & ref(tn(l, "mlp", "down_exps.weight"), down_exps) &
                 ref(tn(l, "mlp", "gate_shexp.weight"), gate_sh) & ref(tn(l, "mlp", "up_shexp.weight"), up_sh) &
                 ref(tn(l, "mlp", "down_shexp.weight"), down_sh);
            if (!ok) return false;
            E = cfg.n_experts > 0 ? cfg.n_experts : (int)gi->shape[0];
            K = cfg.top_k > 0 ? cfg.top_k : 6;
            F = cfg.expert_dim > 0 ? cfg.expert_dim : 1408;
            const WeightTensor* gs = w.get(tn(l, "mlp", "gate_shexp.weight"));
            S = gs->shape[0];
            // per-expert byte stride of the stacked expert tensors
            // (deepseek_mla_layer.cu:106-114)
            stride_gu = (int64_t)quantized_size((int64_t)F * d, gate_exps.qt);
            stride_dn = (int64_t)quantized_size((int64_t)d * F, down_exps.qt);
            ok = ok && gate_exps.qt == up_exps.qt && gate_exps.qt == down_exps.qt && gate_sh.qt == up_sh.qt;
            // shapes the config implies (the kernels index by them)
            ok = ok && K >= 1 && K <= E && is("mlp", "gate_inp.weight", (int64_t)E * d) &&
                 is("mlp", "gate_exps.weight", (int64_t)E * F * d) && is("mlp", "up_exps.weight", (int64_t)E * F * d) &&
                 is("mlp", "down_exps.weight", (int64_t)E * d * F) && is("mlp", "gate_shexp.weight", (int64_t)S * d) &&
                 is("mlp", "up_shexp.weight", (int64_t)S * d) && is("mlp", "down_shexp.weight", (int64_t)d * S);
            if (ok && gate_exps.qt == QuantType::GGML_Q2_K && gate_sh.qt == QuantType::GGML_Q2_K &&
                down_sh.qt == QuantType::GGML_Q2_K && gate_inp.qt == QuantType::FP32) {
                moe_ws_bytes = rina_hip_moe_block_workspace(d, E, K, F, S);
                moe_block = moe_ws_bytes > 0 && hipMalloc(&moe_ws, moe_ws_bytes) == hipSuccess;
            }
        } else {
            ok = ok & ref(tn(l, "mlp", "w1.weight"), w1) & ref(tn(l, "mlp", "w2.weight"), w2) &
                 ref(tn(l, "mlp", "w3.weight"), w3);
            const WeightTensor* t = w.get(tn(l, "mlp", "w1.weight"));
            hd = t ? (int)t->shape[0] : cfg.hidden_dim;
            ok = ok && w1.qt == w3.qt && is("mlp", "w1.weight", (int64_t)hd * d) && is("mlp", "w3.weight", (int64_t)hd * d) &&
                 is("mlp", "w2.weight", (int64_t)d * hd);
        }
        return ok;
    }

    // activation floats per token in ForwardBuffers::mla: the MoE rows
    // (a2 [d] | acc [d] | logits [E] | ids [K] | probs [K] | G [K*F]), and a
    // prompt's attention rows (rina_hip_mla_prompt_workspace per row, plus
    // the alignment of its parts); the two are used one after the other
    int prompt_per_token() const { return dc + H * nope + H * vd + 4 * H * (nope + rope) + 32; }
    // a prompt's MoE rows (rina_hip_moe_rows_workspace per row, plus alignment)
    int moe_rows_per_token() const { return is_moe ? d + E + 4 * K + S + K * (2 * d + F) + 48 : 0; }
    int scratch_per_token() const {
        return std::max({is_moe ? 2 * d + E + 2 * K + K * F : 0, prompt_per_token(), moe_rows_per_token()});
    }
    int ffn_width() const { return is_moe ? std::max(S, F) : hd; }

    // the products of rina_hip_moe_rows take these shapes (Q4 rows need K % 32)
    bool moe_rows_ok() const {
        auto fits = [](QuantType qt, int k) {
            return qt == QuantType::GGML_Q2_K || qt == QuantType::FP32 ||
                   ((qt == QuantType::Q4_0 || qt == QuantType::Q4_0F) && k % 32 == 0);
        };
        return is_moe && E <= 256 && K <= 16 && gate_inp.qt == QuantType::FP32 && fits(gate_sh.qt, d) &&
               fits(down_sh.qt, S) && fits(gate_exps.qt, d) && fits(down_exps.qt, F) && gate_sh.qt == up_sh.qt &&
               gate_sh.qt == down_sh.qt;
    }

    int forward(float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
        (void)B;
        const int n = T, qd = H * (nope + rope), kvw = dc + rope;
        const int start_pos = b.mla_cache.start_pos;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        float* q = b.q;            // [n, H*(nope+rope)]
        float* kva = b.k;          // [n, dc+rope]
        float* att = b.a;          // [n, H*v]
        if (w_q.qt == w_kv_a.qt) {
            rina_linear_seg segs[2] = {{w_q.data, nullptr, q, qd}, {w_kv_a.data, nullptr, kva, kvw}};
            CK(rina_hip_linear_fused(segs, 2, (int)w_q.qt, h, n, d, RINA_EPI_STORE, RINA_PRO_RMSNORM, ln1, 1e-5f, s));
        } else {
            rina_linear_seg s1{w_q.data, nullptr, q, qd}, s2{w_kv_a.data, nullptr, kva, kvw};
            CK(rina_hip_linear_fused(&s1, 1, (int)w_q.qt, h, n, d, RINA_EPI_STORE, RINA_PRO_RMSNORM, ln1, 1e-5f, s));
            CK(rina_hip_linear_fused(&s2, 1, (int)w_kv_a.qt, h, n, d, RINA_EPI_STORE, RINA_PRO_RMSNORM, ln1, 1e-5f, s));
        }
        float* cache = b.mla_cache.layer(layer);
        // a prompt from position 0: one causal attention over its rows in the
        // reference prefill's expanded form (deepseek_mla_layer.cu:180-217)
        const size_t pws = n > 1 ? rina_hip_mla_prompt_workspace(n, H, nope, rope, vd, dc) : 0;
        bool batched = false;
        if (n > 1 && start_pos == 0 && !b.d_pos && b.mla && pws && pws <= sizeof(float) * (size_t)n * prompt_per_token()) {
            rc = rina_hip_mla_prompt_attention(q, kva, k_norm, 1e-5f, rope_c, rope_s, w_kv_b.data, (int)w_kv_b.qt,
                                               cache, H, nope, rope, vd, dc, n, b.mla_cache.max_seq, att, b.mla, pws, s);
            if (rc != RINA_OK && rc != RINA_ERR_SHAPE && rc != RINA_ERR_QTYPE) return rc;   // those two launch nothing
            batched = rc == RINA_OK;
        }
        for (int t = 0; t < n && !batched; t++)
            CK(rina_hip_mla_decode_attention_ex(q + (size_t)t * qd, kva + (size_t)t * kvw, k_norm, 1e-5f, rope_c,
                                                rope_s, w_kv_b.data, (int)w_kv_b.qt, cache, H, nope, rope, vd, dc,
                                                start_pos + t, b.d_pos, b.mla_cache.max_seq, b.pos_hint,
                                                att + (size_t)t * H * vd, b.attn_ws, b.attn_ws_bytes, s));
        rina_linear_seg o{w_o.data, nullptr, h, d};
        CK(rina_hip_linear_fused(&o, 1, (int)w_o.qt, att, n, H * vd, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
        if (!is_moe) {
            rina_linear_seg up{w1.data, w3.data, b.g, hd};
            CK(rina_hip_linear_fused(&up, 1, (int)w1.qt, h, n, d, RINA_EPI_SWIGLU, RINA_PRO_RMSNORM, ln2, 1e-5f, s));
            rina_linear_seg down{w2.data, nullptr, h, d};
            CK(rina_hip_linear_fused(&down, 1, (int)w2.qt, b.g, n, hd, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
            return RINA_OK;
        }
        // forward_moe (:291-350) over a prompt's rows at once
        if (n > 1 && !b.d_pos && b.mla && moe_rows_ok()) {
            const size_t mws = rina_hip_moe_rows_workspace(n, d, E, K, F, S);
            if (mws && mws <= sizeof(float) * (size_t)n * moe_rows_per_token())
                return rina_hip_moe_rows(h, n, ln2, 1e-5f, gate_inp.data, (int)gate_inp.qt, gate_sh.data, up_sh.data,
                                         down_sh.data, S, (int)gate_sh.qt, gate_exps.data, up_exps.data,
                                         down_exps.data, (int)gate_exps.qt, stride_gu, stride_dn, E, K, d, F, b.mla,
                                         mws, s);
        }
        // forward_moe, one token at a time
        if (moe_block) {
            for (int t = 0; t < n; t++) {
                rc = rina_hip_moe_block(h + (size_t)t * d, ln2, 1e-5f, gate_inp.data, (int)gate_inp.qt, gate_sh.data,
                                        up_sh.data, down_sh.data, S, gate_exps.data, up_exps.data, down_exps.data,
                                        (int)gate_exps.qt, stride_gu, stride_dn, E, K, d, F, moe_ws, moe_ws_bytes, s);
                if (rc == RINA_ERR_SHAPE || rc == RINA_ERR_QTYPE) { moe_block = false; break; }   // nothing launched
                if (rc != RINA_OK) return rc;
            }
            if (moe_block) return RINA_OK;
        }
        float* base = b.mla;
        float* a2 = base;
        float* acc = a2 + d;
        float* logits = acc + d;
        int* ids = (int*)(logits + E);
        float* probs = (float*)(ids + K);
        float* G = probs + K;
        for (int t = 0; t < n; t++) {
            float* ht = h + (size_t)t * d;
            CK(rina_hip_rms_norm(ht, a2, ln2, 1, d, 1e-5f, s));
            rina_linear_seg sh{gate_sh.data, up_sh.data, b.g, S};
            CK(rina_hip_linear_fused(&sh, 1, (int)gate_sh.qt, a2, 1, d, RINA_EPI_SWIGLU, RINA_PRO_NONE, nullptr, 0.f, s));
            rina_linear_seg shd{down_sh.data, nullptr, acc, d};
            CK(rina_hip_linear_fused(&shd, 1, (int)down_sh.qt, b.g, 1, S, RINA_EPI_STORE, RINA_PRO_NONE, nullptr, 0.f, s));
            CK(rina_hip_linear(gate_inp.data, (int)gate_inp.qt, a2, logits, 1, E, d, s));
            CK(rina_hip_moe_topk(logits, E, K, ids, probs, s));
            CK(rina_hip_moe_ffn(a2, gate_exps.data, up_exps.data, down_exps.data, (int)gate_exps.qt, stride_gu,
                                stride_dn, E, ids, probs, K, d, F, acc, ht, G, (size_t)K * F * sizeof(float), s));
        }
#undef CK
        return RINA_OK;
    }
};

bool v_init(void* self, const ModelConfig& c, const TensorMap& w, int l) { return ((MLAImpl*)self)->init(c, w, l); }
void v_forward(void* self, float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
    b.fail(((MLAImpl*)self)->forward(h, b, B, T, s));
}
int v_ws(void* self, int, int, int) { return ((MLAImpl*)self)->scratch_per_token(); }
void v_destroy(void* self) { delete (MLAImpl*)self; }
const LayerVTable kMLAVTable = {v_init, v_forward, layer_no_backward, v_ws, layer_no_saved, v_destroy};

}  // namespace

Layer create_mla_layer() {
    Layer l;
    l.impl = new MLAImpl();
    l.vtab = &kMLAVTable;
    return l;
}

int mla_layer_ffn_width(const Layer& l) { return ((const MLAImpl*)l.impl)->ffn_width(); }
