// GQA transformer layer (rina-engine/src/arch/gqa/gqa_layer.cu:63-284) on the
// gfx950 C-ABI.  Same tensor names, same per-layer math:
//   a = norm(h, ln1); q,k,v = W a; RoPE(q,k); cache append (quantized unless
//   fp32); o = attention over cache + current rows; h += W_o o;
//   a = norm(h, ln2); h += W2 (silu(W1 a) * (W3 a)).
// The launches are fused where the reference runs back-to-back kernels on
// the same data (norm as the matvec prologue, q/k/v in one matvec launch,
// RoPE + append in one kernel, W_o and W2 with the residual add as
// epilogue, W1/W3 with SiLU*up), and
// W_o is computed out of place (the reference's in-place call races,
// gqa_layer.cu:272).
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

struct GQAImpl {
    int d = 0, H = 0, Hkv = 0, dh = 0, hd = 0, layer = 0;
    bool use_rms_norm = false;
    WeightRef w_q, w_k, w_v, w_o, w1, w2, w3;
    const float* ln1 = nullptr;
    const float* ln2 = nullptr;
    const float *rq_cos = nullptr, *rq_sin = nullptr, *rk_cos = nullptr, *rk_sin = nullptr;

    bool init(const ModelConfig& cfg, const TensorMap& w, int l) {
        d = cfg.dim; H = cfg.n_heads; Hkv = cfg.n_kv_heads; dh = cfg.head_dim; layer = l;
        use_rms_norm = cfg.name.find("llama") != std::string::npos;   // gqa_layer.cu:90
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
        const WeightTensor* w1t = w.get(tn(l, "mlp", "w1.weight"));
        hd = (w1t && w1t->n_dim >= 2) ? w1t->shape[0] : (cfg.hidden_dim ? cfg.hidden_dim : d * 4 * 2 / 3 / 256 * 256);
        bool ok = ref(tn(l, "attn", "w_q.weight"), w_q) & ref(tn(l, "attn", "w_k.weight"), w_k) &
                  ref(tn(l, "attn", "w_v.weight"), w_v) & ref(tn(l, "attn", "w_o.weight"), w_o) &
                  ref(tn(l, "mlp", "w1.weight"), w1) & ref(tn(l, "mlp", "w2.weight"), w2) &
                  ref(tn(l, "mlp", "w3.weight"), w3) & f32(tn(l, "ln1", "weight"), ln1) &
                  f32(tn(l, "ln2", "weight"), ln2);
        f32(tn(l, "attn", "rope_q.cos"), rq_cos);
        f32(tn(l, "attn", "rope_q.sin"), rq_sin);
        f32(tn(l, "attn", "rope.cos"), rk_cos);
        f32(tn(l, "attn", "rope.sin"), rk_sin);
        // the fused launches need one quant type per fused group
        ok = ok && w_q.qt == w_k.qt && w_q.qt == w_v.qt && w1.qt == w3.qt;
        if (!ok) return false;
        // shapes the config implies (the kernels index by them)
        const int64_t kvd = (int64_t)Hkv * dh, qd = (int64_t)H * dh;
        const int64_t ms = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        auto is = [&](const char* c, const char* p, int64_t n) { return elems_are(w.get(tn(l, c, p)), n); };
        ok = is("attn", "w_q.weight", qd * d) && is("attn", "w_k.weight", kvd * d) && is("attn", "w_v.weight", kvd * d) &&
             is("attn", "w_o.weight", (int64_t)d * qd) && is("mlp", "w1.weight", (int64_t)hd * d) &&
             is("mlp", "w3.weight", (int64_t)hd * d) && is("mlp", "w2.weight", (int64_t)d * hd) &&
             is("ln1", "weight", d) && is("ln2", "weight", d);
        for (const char* r : {"rope_q.cos", "rope_q.sin", "rope.cos", "rope.sin"}) {
            const WeightTensor* t = w.get(tn(l, "attn", r));
            if (t && !elems_at_least(t, ms * (dh / 2))) ok = false;
        }
        return ok;
    }

    int forward(float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
        const int n = B * T, kvd = Hkv * dh;
        const int start_pos = b.kv_cache.start_pos;
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        const int pro = use_rms_norm ? RINA_PRO_RMSNORM : RINA_PRO_LAYERNORM;
        rina_linear_seg qkv[3] = {{w_q.data, nullptr, b.q, H * dh},
                                  {w_k.data, nullptr, b.k, kvd},
                                  {w_v.data, nullptr, b.v, kvd}};
        CK(rina_hip_linear_fused(qkv, 3, (int)w_q.qt, h, n, d, RINA_EPI_STORE, pro, ln1, 1e-5f, s));
        const int mode = b.kv_cache_quant.mode;
        void* ck;
        void* cv;
        int max_seq;
        if (mode > 0) { ck = b.kv_cache_quant.k(layer); cv = b.kv_cache_quant.v(layer); max_seq = b.kv_cache_quant.max_seq; }
        else { ck = b.kv_cache.k(layer); cv = b.kv_cache.v(layer); max_seq = b.kv_cache.max_seq; }
        const int pre_rope = b.kv_cache_quant.pre_rope ? 1 : 0;
        float* tap_k = nullptr;
        if (b.kv_tap && !b.d_pos) tap_k = b.kv_tap + ((size_t)layer * 2 * max_seq + start_pos) * kvd;
        const size_t rows_bytes = (size_t)n * kvd * sizeof(float);
        if (n == 1 && !pre_rope) {
            // decode step: RoPE, append and attention in one call
            rc = rina_hip_gqa_decode_attention(b.q, b.k, b.v, rq_cos, rq_sin, rk_cos, rk_sin, ck, cv, mode, H, Hkv,
                                               dh, start_pos, b.d_pos, max_seq, b.a, tap_k, b.attn_ws,
                                               b.attn_ws_bytes, s);
            if (rc == RINA_OK) {
                if (tap_k && hipMemcpyAsync(tap_k + (size_t)max_seq * kvd, b.v, rows_bytes, hipMemcpyDeviceToDevice,
                                            s) != hipSuccess)
                    return RINA_ERR_HIP;
                return finish(h, b, n, s);
            }
            if (rc != RINA_ERR_SHAPE) return rc;
        }
        if (tap_k && pre_rope && hipMemcpyAsync(tap_k, b.k, rows_bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
            return RINA_ERR_HIP;
        CK(rina_hip_rope_append(b.q, b.k, b.v, rq_cos, rq_sin, rk_cos, rk_sin, ck, cv, mode, pre_rope, n, H, Hkv, dh,
                                start_pos, b.d_pos, max_seq, s));
        if (tap_k) {
            if (!pre_rope && hipMemcpyAsync(tap_k, b.k, rows_bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
                return RINA_ERR_HIP;
            if (hipMemcpyAsync(tap_k + (size_t)max_seq * kvd, b.v, rows_bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
                return RINA_ERR_HIP;
        }
        CK(rina_hip_gqa_attention(b.q, b.k, b.v, ck, cv, mode, pre_rope, rk_cos, rk_sin, n, H, Hkv, dh, start_pos,
                                  b.d_pos, max_seq, b.a, b.attn_ws, b.attn_ws_bytes, s));
        return finish(h, b, n, s);
#undef CK
    }

    // W_o + residual, then the SwiGLU MLP + residual
    int finish(float* h, ForwardBuffers& b, int n, hipStream_t s) {
        int rc;
#define CK(x) do { if ((rc = (x)) != RINA_OK) return rc; } while (0)
        const int pro = use_rms_norm ? RINA_PRO_RMSNORM : RINA_PRO_LAYERNORM;
        rina_linear_seg o{w_o.data, nullptr, h, d};
        CK(rina_hip_linear_fused(&o, 1, (int)w_o.qt, b.a, n, H * dh, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
        rina_linear_seg up{w1.data, w3.data, b.g, hd};
        CK(rina_hip_linear_fused(&up, 1, (int)w1.qt, h, n, d, RINA_EPI_SWIGLU, pro, ln2, 1e-5f, s));
        rina_linear_seg down{w2.data, nullptr, h, d};
        CK(rina_hip_linear_fused(&down, 1, (int)w2.qt, b.g, n, hd, RINA_EPI_ADD, RINA_PRO_NONE, nullptr, 0.f, s));
#undef CK
        return RINA_OK;
    }
};

bool v_init(void* self, const ModelConfig& c, const TensorMap& w, int l) { return ((GQAImpl*)self)->init(c, w, l); }
void v_forward(void* self, float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
    b.fail(((GQAImpl*)self)->forward(h, b, B, T, s));
}
int v_ws(void*, int, int, int) { return 0; }   // no per-token scratch beyond ForwardBuffers
void v_destroy(void* self) { delete (GQAImpl*)self; }
const LayerVTable kGQAVTable = {v_init, v_forward, layer_no_backward, v_ws, layer_no_saved, v_destroy};

}  // namespace

Layer create_gqa_layer() {
    Layer l;
    l.impl = new GQAImpl();
    l.vtab = &kGQAVTable;
    return l;
}

