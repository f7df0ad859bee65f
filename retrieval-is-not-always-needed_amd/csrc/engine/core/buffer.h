// Forward-pass device buffers and KV caches (rina-engine/src/core/buffer.h:6-146).
// The cache layouts are the reference's:
//   kv_cache (fp32):  per layer K[max_seq][kv_dim] then V[max_seq][kv_dim]
//   kv_cache_quant:   per layer [K blocks][V blocks], blocks_per_layer =
//                     max_seq*kv_dim/32, block b of position p, KV head h,
//                     sub-block j = p*(kv_dim/32) + h*(head_dim/32) + j
// Decode positions may come from the device (d_pos) so one captured graph
// serves every step.
#pragma once
#include <hip/hip_runtime_api.h>
#include <cstddef>
#include <cstdint>

struct ForwardBuffers {
    float* h = nullptr;      // [cap, d]       residual stream
    float* a = nullptr;      // [cap, max(d, H*dh)]  normed input / attention out
    float* q = nullptr;      // [cap, H*dh]
    float* k = nullptr;      // [cap, kv_dim]  current keys (post-RoPE)
    float* v = nullptr;      // [cap, kv_dim]
    float* g = nullptr;      // [cap, ffn]     SiLU(gate)*up
    float* lm = nullptr;     // [vocab]        last-row logits of the device decode loop
    float* mla = nullptr;    // [cap, mla_ws]  MLA / MoE scratch
    int cap = 0;

    struct {
        float* data = nullptr;   // [n_layers, 2, max_seq, kv_dim]
        int max_seq = 0, kv_dim = 0, n_layers = 0;
        int start_pos = 0;
        float* k(int layer) const { return data + (size_t)layer * 2 * max_seq * kv_dim; }
        float* v(int layer) const { return data + ((size_t)layer * 2 + 1) * max_seq * kv_dim; }
    } kv_cache;

    struct {
        uint8_t* data = nullptr;
        int max_seq = 0, kv_dim = 0, n_layers = 0;
        int start_pos = 0;
        int mode = 0;            // 0=off 1=q8 2=q4 3=q4k_q2v 4=q2 5=q2k_q1v
        bool pre_rope = false;
        size_t blocks_per_layer = 0;
        int k_block_bytes = 0, v_block_bytes = 0;
        uint8_t* k(int layer) const {
            return data + (size_t)layer * blocks_per_layer * (k_block_bytes + v_block_bytes);
        }
        uint8_t* v(int layer) const {
            return k(layer) + blocks_per_layer * k_block_bytes;
        }
    } kv_cache_quant;

    // latent MLA cache: per layer, per position [c_kv (kv_lora_rank) | k_pe (rope)]
    struct {
        float* data = nullptr;
        int max_seq = 0, n_layers = 0, rank = 0, rope = 0;
        int start_pos = 0;
        float* layer(int l) const { return data + (size_t)l * max_seq * (rank + rope); }
    } mla_cache;

    void* attn_ws = nullptr;     // split-sequence attention partials
    size_t attn_ws_bytes = 0;
    const int* d_pos = nullptr;  // device position (graph decode) or nullptr
    int pos_hint = -1;           // with d_pos: the largest position it holds (-1: unknown)
    // optional parity tap: the fp32 K (as cached: pre- or post-RoPE) and V
    // rows each layer appends, [n_layers][2][max_seq][kv_dim]; host-position
    // forward() calls only
    float* kv_tap = nullptr;
    // status of the layer forwards since the caller last cleared it: the
    // first failing C-ABI call's negative status sticks (the reference's
    // forward_fn returns void, core/layer.h:52)
    int status = 0;
    void fail(int rc) {
        if (rc && !status) status = rc;
    }
};

struct BufferManager {
    ForwardBuffers fwd;
    BufferManager() = default;
    ~BufferManager() { free_all(); }
    BufferManager(const BufferManager&) = delete;
    BufferManager& operator=(const BufferManager&) = delete;

    bool alloc_fwd(int n, int d_model, int qdim, int kv_dim, int ffn, int vocab, int mla_ws);
    bool alloc_kv_cache(int n_layers, int max_seq, int kv_dim);
    bool alloc_kv_cache_quant(int n_layers, int max_seq, int kv_dim, int mode);
    bool alloc_mla_cache(int n_layers, int max_seq, int rank, int rope);
    bool alloc_attn_ws(size_t bytes);
    void free_all();
};

int kv_mode_from_name(const char* name);   // "fp32","q8","q4","q4k_q2v","q2","q2k_q1v" -> 0..5, -1 unknown
