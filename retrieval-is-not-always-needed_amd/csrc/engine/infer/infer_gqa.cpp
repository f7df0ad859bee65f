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
#include <vector>
#include "core/buffer.h"
#include "core/layer.h"
#include "infer/infer_base.h"
#include "rina_hip.h"

int gqa_layer_hidden(const Layer& l);

namespace {

struct GQAInference : Inference {
    std::vector<std::unique_ptr<Layer>> layers;
    BufferManager bufs;
    ModelConfig cfg;
    const WeightTensor* wte = nullptr;
    const WeightTensor* ln_f = nullptr;
    const WeightTensor* lm_head = nullptr;
    int hd = 0, max_seq = 0, kvd = 0;
    bool use_rms = false;
    int* d_ids = nullptr;      // [max_seq + 1]
    int* d_pos = nullptr;      // device position for graph decode
    hipGraphExec_t graph = nullptr;
    hipStream_t graph_stream = nullptr;

    ~GQAInference() override {
        if (graph) (void)hipGraphExecDestroy(graph);
        if (d_ids) (void)hipFree(d_ids);
        if (d_pos) (void)hipFree(d_pos);
    }

    bool fail(const std::string& m) { err_ = m; return false; }

    bool init(ModelConfig& c, const TensorMap& w) override {
        cfg = c;
        if (cfg.dim <= 0 || cfg.n_heads <= 0 || cfg.n_kv_heads <= 0 || cfg.head_dim <= 0 || cfg.vocab_size <= 0)
            return fail("gqa: incomplete config");
        layers = build_layers(cfg, w);
        if ((int)layers.size() != cfg.n_layers || layers.empty()) return fail("gqa: layer init failed");
        hd = gqa_layer_hidden(*layers[0]);
        for (auto& l : layers) hd = std::max(hd, gqa_layer_hidden(*l));
        max_seq = cfg.max_seq_len > 0 ? cfg.max_seq_len : 512;
        kvd = cfg.n_kv_heads * cfg.head_dim;
        use_rms = cfg.name.find("llama") != std::string::npos;
        int cap = std::min(max_seq, 512);
        if (!bufs.alloc_fwd(cap, cfg.dim, cfg.n_heads * cfg.head_dim, kvd, hd, cfg.vocab_size, 0))
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
        if (hipMalloc(&d_ids, sizeof(int) * (max_seq + 1)) != hipSuccess || hipMalloc(&d_pos, sizeof(int)) != hipSuccess)
            return fail("gqa: id buffer allocation failed");
        wte = w.get("transformer.wte.weight");
        ln_f = w.get("transformer.ln_f.weight");
        lm_head = w.get("lm_head.weight");
        if (!wte) return fail("gqa: transformer.wte.weight missing");
        return true;
    }

    int ensure_cap(int n) {
        if (n <= bufs.fwd.cap) return RINA_OK;
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
        if (!bufs.alloc_fwd(n, cfg.dim, cfg.n_heads * cfg.head_dim, kvd, hd, cfg.vocab_size, 0)) return RINA_ERR_HIP;
        return RINA_OK;
    }

    const WeightTensor* head() const {
        return (lm_head && lm_head->quant_type != QuantType::GGML_Q6_K) ? lm_head : wte;   // infer_gqa.cpp:97-100
    }

    // embedding -> layers -> ln_f -> lm_head (rows [row0, T) of the chunk)
    int run(const int* ids, const int* pos_dev, int T, int start_pos, float* logits, bool last_only, hipStream_t s) {
        int rc;
        ForwardBuffers& f = bufs.fwd;
        f.kv_cache.start_pos = start_pos;
        f.kv_cache_quant.start_pos = start_pos;
        f.d_pos = pos_dev;
        if ((rc = rina_hip_embedding(wte->data, (int)wte->quant_type, ids, pos_dev, f.h, T, cfg.dim, s))) return rc;
        for (auto& l : layers)
            if ((rc = l->forward(f.h, f, 1, T, s))) return rc;
        const WeightTensor* hw = head();
        const float* x = f.h;
        int M = T;
        if (last_only) { x = f.h + (size_t)(T - 1) * cfg.dim; M = 1; }
        // ln_f fused as the LM head's prologue (infer_gqa.cpp:90-100)
        rina_linear_seg seg{hw->data, nullptr, logits, cfg.vocab_size};
        int pro = ln_f ? (use_rms ? RINA_PRO_RMSNORM : RINA_PRO_LAYERNORM) : RINA_PRO_NONE;
        return rina_hip_linear_fused(&seg, 1, (int)hw->quant_type, x, M, cfg.dim, RINA_EPI_STORE, pro,
                                     ln_f ? (const float*)ln_f->data : nullptr, 1e-5f, s);
    }

    int forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t s) override {
        if (B != 1) { err_ = "gqa: the KV-cache path decodes one sequence (B == 1)"; return RINA_ERR_ARG; }
        if (T < 1 || start_pos < 0 || start_pos + T > max_seq) { err_ = "gqa: positions exceed max_seq"; return RINA_ERR_RANGE; }
        int rc = ensure_cap(T);
        if (rc) return rc;
        return run(ids, nullptr, T, start_pos, logits, false, s);
    }

    int decode_step(hipStream_t s) {
        int rc = run(d_ids, d_pos, 1, 0, bufs.fwd.lm, true, s);
        if (rc) return rc;
        return rina_hip_argmax(bufs.fwd.lm, cfg.vocab_size, nullptr, d_ids, d_pos, s);
    }

    int generate(const int* prompt, int n, int steps, int* out, bool use_graph, hipStream_t s, float* decode_ms) override {
        if (n < 1 || steps < 1 || n + steps - 1 > max_seq) { err_ = "gqa: prompt + steps exceed max_seq"; return RINA_ERR_RANGE; }
        int rc = ensure_cap(n);
        if (rc) return rc;
        if (hipMemcpyAsync(d_ids, prompt, sizeof(int) * n, hipMemcpyHostToDevice, s) != hipSuccess) return RINA_ERR_HIP;
        int p0 = n - 1;
        if (hipMemcpyAsync(d_pos, &p0, sizeof(int), hipMemcpyHostToDevice, s) != hipSuccess) return RINA_ERR_HIP;
        if ((rc = run(d_ids, nullptr, n, 0, bufs.fwd.lm, true, s))) return rc;
        if ((rc = rina_hip_argmax(bufs.fwd.lm, cfg.vocab_size, nullptr, d_ids, d_pos, s))) return rc;
        if (hipStreamSynchronize(s) != hipSuccess) return RINA_ERR_HIP;
        gen_len = n + 1;
        if (hipMemcpyAsync(out, d_ids + n, sizeof(int), hipMemcpyDeviceToHost, s) != hipSuccess) return RINA_ERR_HIP;
        if (steps == 1) {
            if (decode_ms) *decode_ms = 0.f;
            return hipStreamSynchronize(s) == hipSuccess ? RINA_OK : RINA_ERR_HIP;
        }
        return decode_more(steps - 1, out + 1, use_graph, s, decode_ms);
    }

    int gen_len = 0;   // ids valid in d_ids after the last generate / decode_more

    int decode_more(int steps, int* out, bool use_graph, hipStream_t s, float* decode_ms) override {
        if (gen_len < 1) { err_ = "gqa: decode_more before generate"; return RINA_ERR_ARG; }
        if (steps < 1 || gen_len + steps - 1 > max_seq) { err_ = "gqa: decode exceeds max_seq"; return RINA_ERR_RANGE; }
        int rc;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        (void)hipEventCreate(&e0);
        (void)hipEventCreate(&e1);
        if (use_graph && (!graph || graph_stream != s)) {
            if (graph) { (void)hipGraphExecDestroy(graph); graph = nullptr; }
            hipGraph_t g = nullptr;
            if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return RINA_ERR_HIP;
            int crc = decode_step(s);
            hipError_t ce = hipStreamEndCapture(s, &g);
            if (crc) { if (g) (void)hipGraphDestroy(g); return crc; }
            if (ce != hipSuccess) return RINA_ERR_HIP;
            hipError_t ie = hipGraphInstantiate(&graph, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            if (ie != hipSuccess) { graph = nullptr; return RINA_ERR_HIP; }
            graph_stream = s;
        }
        (void)hipEventRecord(e0, s);
        for (int i = 0; i < steps; i++) {
            if (use_graph) { if (hipGraphLaunch(graph, s) != hipSuccess) return RINA_ERR_HIP; }
            else if ((rc = decode_step(s))) return rc;
        }
        (void)hipEventRecord(e1, s);
        if (hipMemcpyAsync(out, d_ids + gen_len, sizeof(int) * steps, hipMemcpyDeviceToHost, s) != hipSuccess)
            return RINA_ERR_HIP;
        if (hipStreamSynchronize(s) != hipSuccess) return RINA_ERR_HIP;
        gen_len += steps;
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (decode_ms) *decode_ms = ms;
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        return RINA_OK;
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
