// DeepSeek MLA + MoE inference orchestrator (rina-engine/src/infer/
// infer_mla.cpp:17-106).  Differences from the reference, by design:
//   * no 128-position cap (infer_mla.cpp:38): the latent cache holds
//     cfg.max_seq_len positions;
//   * the cache is the latent form [c_kv | RoPE(k_pe)] per position and
//     layer, not the expanded per-head K/V;
//   * the LM head is one launch (no 8192-row tiling, which existed only to
//     bound a dequant temp buffer, infer_mla.cpp:87-101);
//   * the greedy loop runs on the device (infer/greedy.h).
#include <algorithm>
#include <cstdio>
#include <memory>
#include <vector>
#include "core/buffer.h"
#include "core/layer.h"
#include "infer/greedy.h"
#include "infer/infer_base.h"
#include "rina_hip.h"

int mla_layer_ffn_width(const Layer& l);

namespace {

struct MLAInference : DeviceGreedyInference {
    std::vector<std::unique_ptr<Layer>> layers;
    BufferManager bufs;
    ModelConfig cfg;
    const WeightTensor* wte = nullptr;
    const WeightTensor* ln_f = nullptr;
    const WeightTensor* lm_head = nullptr;
    int nope = 0, rope = 0, vd = 0, dc = 0, ffn = 0, scratch = 0;

    bool fail(const std::string& m) { err_ = m; return false; }

    int qdim() const { return cfg.n_heads * (nope + rope); }
    int adim() const { return std::max(cfg.dim, cfg.n_heads * vd); }

    bool alloc(int cap) {
        // a: [cap, max(d, H*v)]; q: [cap, H*(nope+rope)]; k: [cap, dc+rope];
        // g: [cap, widest MLP]; mla: [cap, MoE scratch]
        return bufs.alloc_fwd(cap, cfg.dim, std::max(qdim(), adim()), dc + rope, ffn, cfg.vocab_size, scratch);
    }

    bool init(ModelConfig& c, const TensorMap& w) override {
        cfg = c;
        tag = "mla";
        if (cfg.dim <= 0 || cfg.n_heads <= 0 || cfg.vocab_size <= 0) return fail("mla: incomplete config");
        nope = cfg.qk_nope_dim > 0 ? cfg.qk_nope_dim : cfg.head_dim;
        rope = cfg.qk_rope_dim > 0 ? cfg.qk_rope_dim : (cfg.d_h_r > 0 ? cfg.d_h_r : 64);
        vd = cfg.v_head_dim > 0 ? cfg.v_head_dim : cfg.head_dim;
        dc = cfg.kv_lora_rank > 0 ? cfg.kv_lora_rank : (cfg.d_c > 0 ? cfg.d_c : 512);
        layers = build_layers(cfg, w);
        if ((int)layers.size() != cfg.n_layers || layers.empty()) return fail("mla: layer init failed");
        wte = w.get("transformer.wte.weight");
        ln_f = w.get("transformer.ln_f.weight");
        lm_head = w.get("lm_head.weight");
        if (!wte) return fail("mla: transformer.wte.weight missing");
        // the embedding and the LM head index rows by the config
        const int64_t vd_rows = (int64_t)cfg.vocab_size * cfg.dim;
        if (!elems_are(wte, vd_rows)) return fail("mla: transformer.wte.weight is not [vocab, dim]");
        if (lm_head && !elems_are(lm_head, vd_rows)) return fail("mla: lm_head.weight is not [vocab, dim]");
        if (ln_f && !elems_are(ln_f, cfg.dim)) return fail("mla: transformer.ln_f.weight is not [dim]");
        for (auto& l : layers) {
            ffn = std::max(ffn, mla_layer_ffn_width(*l));
            scratch = std::max(scratch, l->workspace_per_token(cfg.dim, cfg.n_heads, cfg.head_dim));
        }
        max_seq = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        vocab = cfg.vocab_size;
        if (!alloc(std::min(max_seq, 64))) return fail("mla: forward buffer allocation failed");
        if (!bufs.alloc_mla_cache(cfg.n_layers, max_seq, dc, rope)) return fail("mla: latent cache allocation failed");
        if (!bufs.alloc_attn_ws(rina_hip_mla_attention_workspace(cfg.n_heads, dc, rope, max_seq)))
            return fail("mla: attention workspace allocation failed");
        if (!alloc_ids()) return fail("mla: id buffer allocation failed");
        return true;
    }

    int ensure_cap(int n) override {
        if (n <= bufs.fwd.cap) return RINA_OK;
        // the queued work and the captured graphs use the old buffers
        if (hipDeviceSynchronize() != hipSuccess) return RINA_ERR_HIP;
        drop_graphs();
        ForwardBuffers keep = bufs.fwd;
        bufs.fwd.mla_cache.data = nullptr;
        bufs.fwd.attn_ws = nullptr;
        bufs.free_all();
        bufs.fwd.mla_cache = keep.mla_cache;
        bufs.fwd.attn_ws = keep.attn_ws;
        bufs.fwd.attn_ws_bytes = keep.attn_ws_bytes;
        return alloc(n) ? RINA_OK : RINA_ERR_HIP;
    }

    float* lm_buffer() override { return bufs.fwd.lm; }

    // below this position the latent attention runs as one launch
    int graph_split() const override { return std::min(max_seq, rina_hip_mla_fused_positions()); }

    int run(const int* ids, const int* pos_dev, int T, int start_pos, float* logits, bool last_only,
            hipStream_t s) override {
        int rc;
        ForwardBuffers& f = bufs.fwd;
        f.mla_cache.start_pos = start_pos;
        f.d_pos = pos_dev;
        f.pos_hint = pos_dev ? pos_hint : -1;
        // a decode step's embedding row is already in h (the previous step's tail)
        if (!fuse_tail &&
            (rc = rina_hip_embedding(wte->data, (int)wte->quant_type, ids, pos_dev, f.h, T, cfg.dim, cfg.vocab_size, s)))
            return rc;
        f.status = RINA_OK;
        for (auto& l : layers)
            if ((rc = l->run(f.h, f, 1, T, s))) return rc;
        const WeightTensor* hw = lm_head ? lm_head : wte;
        const float* x = f.h;
        int M = T;
        if (last_only) { x = f.h + (size_t)(T - 1) * cfg.dim; M = 1; }
        rina_linear_seg seg{hw->data, nullptr, logits, cfg.vocab_size};
        const int pro = ln_f ? RINA_PRO_RMSNORM : RINA_PRO_NONE;
        const float* nw = ln_f ? (const float*)ln_f->data : nullptr;
        if (M == 1) return head_launch(seg, (int)hw->quant_type, x, cfg.dim, pro, nw, s);
        return rina_hip_linear_fused(&seg, 1, (int)hw->quant_type, x, M, cfg.dim, RINA_EPI_STORE, pro, nw, 1e-5f, s);
    }

    const WeightTensor* emb_table() const override { return wte; }
    float* h_buffer() override { return bufs.fwd.h; }
    int model_dim() const override { return cfg.dim; }

    void forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t s) override {
        if (B != 1) return set_status(RINA_ERR_ARG, "mla: the cache path decodes one sequence (B == 1)");
        if (T < 1 || start_pos < 0 || start_pos + T > max_seq)
            return set_status(RINA_ERR_RANGE, "mla: positions exceed max_seq");
        int rc = ensure_cap(T);
        if (rc) return set_status(rc, "mla: activation buffer allocation failed");
        rc = run(ids, nullptr, T, start_pos, logits, false, s);
        set_status(rc, "mla: a forward launch failed");
    }

    int set_kv_tap(float*) override {
        err_ = "mla: no K/V tap (the cache is latent)";
        return RINA_ERR_ARG;
    }

    // which_v 0: the layer's latent region [max_seq][dc + rope] fp32
    int kv_region(int layer, int which_v, void** ptr, size_t* bytes) override {
        if (layer < 0 || layer >= cfg.n_layers || !ptr || !bytes || which_v) return RINA_ERR_ARG;
        *ptr = bufs.fwd.mla_cache.layer(layer);
        *bytes = rina_hip_mla_cache_bytes(dc, rope, max_seq);
        return RINA_OK;
    }
};

}  // namespace

Inference* create_mla_inference() { return new MLAInference(); }
