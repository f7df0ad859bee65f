// GQA (Llama-shaped) inference orchestrator (rina-engine/src/infer/infer_gqa.cpp:17-106).
// Differences from the reference, by design:
//   * the context is not capped at 512 positions (infer_gqa.cpp:39): the
//     cache holds cfg.max_seq_len positions and every kernel guards it;
//   * only the cache the mode needs is allocated;
//   * the greedy loop runs on the device: argmax writes the next id into the
//     device id buffer and advances a device position, so the decode step
//     is position-independent and is captured once as a HIP graph.
#include <algorithm>
#include <cstdio>
#include <memory>
#include <string>
#include <vector>
#include "core/buffer.h"
#include "core/layer.h"
#include "infer/greedy.h"
#include "infer/infer_base.h"
#include "rina_hip.h"

namespace {

struct GQAInference : DeviceGreedyInference {
    std::vector<std::unique_ptr<Layer>> layers;
    BufferManager bufs;
    ModelConfig cfg;
    const WeightTensor* wte = nullptr;
    const WeightTensor* ln_f = nullptr;
    const WeightTensor* lm_head = nullptr;
    int hd = 0, kvd = 0;
    int rows_ws = 0;   // floats per prompt row the layers need in ForwardBuffers::mla (the Jamba layers')
    bool use_rms = false;

    bool fail(const std::string& m) { err_ = m; return false; }

    bool init(ModelConfig& c, const TensorMap& w) override {
        cfg = c;
        tag = "gqa";
        if (cfg.dim <= 0 || cfg.n_heads <= 0 || cfg.n_kv_heads <= 0 || cfg.head_dim <= 0 || cfg.vocab_size <= 0)
            return fail("gqa: incomplete config");
        layers = build_layers(cfg, w);
        if ((int)layers.size() != cfg.n_layers || layers.empty()) return fail("gqa: layer init failed");
        wte = w.get("transformer.wte.weight");
        ln_f = w.get("transformer.ln_f.weight");
        lm_head = w.get("lm_head.weight");
        if (!wte) return fail("gqa: transformer.wte.weight missing");
        // the embedding and the LM head index rows by the config
        const int64_t vd_rows = (int64_t)cfg.vocab_size * cfg.dim;
        if (!elems_are(wte, vd_rows)) return fail("gqa: transformer.wte.weight is not [vocab, dim]");
        if (lm_head && !elems_are(lm_head, vd_rows)) return fail("gqa: lm_head.weight is not [vocab, dim]");
        if (ln_f && !elems_are(ln_f, cfg.dim)) return fail("gqa: transformer.ln_f.weight is not [dim]");
        // MLP width: the widest w1 of any layer (GQA, SSM or RINA-MLA)
        hd = cfg.hidden_dim;
        for (int l = 0; l < cfg.n_layers; l++) {
            const WeightTensor* t = w.get("transformer.h." + std::to_string(l) + ".mlp.w1.weight");
            if (t && t->n_dim >= 2) hd = std::max(hd, (int)t->shape[0]);
        }
        if (hd <= 0) return fail("gqa: cannot size the MLP buffer (no mlp.w1 and no hidden_dim)");
        for (auto& l : layers) rows_ws = std::max(rows_ws, l->workspace_per_token(cfg.dim, cfg.n_heads, cfg.head_dim));
        max_seq = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        vocab = cfg.vocab_size;
        kvd = cfg.n_kv_heads * cfg.head_dim;
        use_rms = cfg.name.find("llama") != std::string::npos;
        int cap = std::min(max_seq, 512);
        if (!bufs.alloc_fwd(cap, cfg.dim, cfg.n_heads * cfg.head_dim, kvd, hd, cfg.vocab_size, rows_ws))
            return fail("gqa: forward buffer allocation failed");
        int mode = kv_mode_from_name(cfg.kv_quant_mode.c_str());
        if (mode < 0) return fail("gqa: unknown kv_quant_mode " + cfg.kv_quant_mode);
        if (mode > 0) {
            if (kvd % 32) return fail("gqa: quantized KV needs kv_dim % 32 == 0");
            if (!bufs.alloc_kv_cache_quant(cfg.n_layers, max_seq, kvd, mode)) return fail("gqa: kv cache allocation failed");
            bufs.fwd.kv_cache.max_seq = max_seq;
        } else {
            if (!bufs.alloc_kv_cache(cfg.n_layers, max_seq, kvd)) return fail("gqa: kv cache allocation failed");
            bufs.fwd.kv_cache_quant.mode = 0;
        }
        bufs.fwd.kv_cache_quant.pre_rope = cfg.use_pre_rope_k;
        if (!bufs.alloc_attn_ws(rina_hip_gqa_attention_workspace(1, cfg.n_heads, cfg.head_dim, max_seq)))
            return fail("gqa: attention workspace allocation failed");
        if (!alloc_ids()) return fail("gqa: id buffer allocation failed");
        return true;
    }

    int ensure_cap(int n) override {
        if (n <= bufs.fwd.cap) return RINA_OK;
        // the queued work and the captured graphs use the old buffers
        if (hipDeviceSynchronize() != hipSuccess) return RINA_ERR_HIP;
        drop_graphs();
        ForwardBuffers keep = bufs.fwd;   // caches survive the re-allocation
        bufs.fwd.kv_cache.data = nullptr;
        bufs.fwd.kv_cache_quant.data = nullptr;
        bufs.fwd.attn_ws = nullptr;
        bufs.fwd.mla_cache.data = nullptr;
        bufs.free_all();
        bufs.fwd.kv_cache = keep.kv_cache;
        bufs.fwd.kv_cache_quant = keep.kv_cache_quant;
        bufs.fwd.mla_cache = keep.mla_cache;
        bufs.fwd.attn_ws = keep.attn_ws;
        bufs.fwd.attn_ws_bytes = keep.attn_ws_bytes;
        bufs.fwd.kv_tap = keep.kv_tap;
        if (!bufs.alloc_fwd(n, cfg.dim, cfg.n_heads * cfg.head_dim, kvd, hd, cfg.vocab_size, rows_ws)) return RINA_ERR_HIP;
        return RINA_OK;
    }

    float* lm_buffer() override { return bufs.fwd.lm; }

    const WeightTensor* head() const {
        return (lm_head && lm_head->quant_type != QuantType::GGML_Q6_K) ? lm_head : wte;   // infer_gqa.cpp:97-100
    }

    int run(const int* ids, const int* pos_dev, int T, int start_pos, float* logits, bool last_only,
            hipStream_t s) override {
        int rc;
        ForwardBuffers& f = bufs.fwd;
        f.kv_cache.start_pos = start_pos;
        f.kv_cache_quant.start_pos = start_pos;
        f.d_pos = pos_dev;
        // a decode step's embedding row is already in h (the previous step's tail)
        if (!fuse_tail &&
            (rc = rina_hip_embedding(wte->data, (int)wte->quant_type, ids, pos_dev, f.h, T, cfg.dim, cfg.vocab_size, s)))
            return rc;
        f.status = RINA_OK;
        for (auto& l : layers)
            if ((rc = l->run(f.h, f, 1, T, s))) return rc;
        const WeightTensor* hw = head();
        const float* x = f.h;
        int M = T;
        if (last_only) { x = f.h + (size_t)(T - 1) * cfg.dim; M = 1; }
        // ln_f fused as the LM head's prologue (infer_gqa.cpp:90-100)
        rina_linear_seg seg{hw->data, nullptr, logits, cfg.vocab_size};
        int pro = ln_f ? (use_rms ? RINA_PRO_RMSNORM : RINA_PRO_LAYERNORM) : RINA_PRO_NONE;
        const float* nw = ln_f ? (const float*)ln_f->data : nullptr;
        if (M == 1) return head_launch(seg, (int)hw->quant_type, x, cfg.dim, pro, nw, s);
        return rina_hip_linear_fused(&seg, 1, (int)hw->quant_type, x, M, cfg.dim, RINA_EPI_STORE, pro, nw, 1e-5f, s);
    }

    const WeightTensor* emb_table() const override { return wte; }
    float* h_buffer() override { return bufs.fwd.h; }
    int model_dim() const override { return cfg.dim; }

    void forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t s) override {
        if (B != 1) return set_status(RINA_ERR_ARG, "gqa: the KV-cache path decodes one sequence (B == 1)");
        if (T < 1 || start_pos < 0 || start_pos + T > max_seq)
            return set_status(RINA_ERR_RANGE, "gqa: positions exceed max_seq");
        int rc = ensure_cap(T);
        if (rc) return set_status(rc, "gqa: activation buffer allocation failed");
        rc = run(ids, nullptr, T, start_pos, logits, false, s);
        set_status(rc, "gqa: a forward launch failed");
    }

    int set_kv_tap(float* tap) override {
        bufs.fwd.kv_tap = tap;
        return RINA_OK;
    }

    int kv_region(int layer, int which_v, void** ptr, size_t* bytes) override {
        if (layer < 0 || layer >= cfg.n_layers || !ptr || !bytes) return RINA_ERR_ARG;
        const ForwardBuffers& f = bufs.fwd;
        int mode = f.kv_cache_quant.mode;
        *bytes = rina_hip_kv_region_bytes(mode, which_v, max_seq, kvd);
        if (mode > 0) *ptr = which_v ? (void*)f.kv_cache_quant.v(layer) : (void*)f.kv_cache_quant.k(layer);
        else *ptr = which_v ? (void*)f.kv_cache.v(layer) : (void*)f.kv_cache.k(layer);
        return RINA_OK;
    }
};

}  // namespace

Inference* create_gqa_inference() { return new GQAInference(); }
