// Device buffer management (rina-engine/src/core/buffer.cpp:95-183).
#include "core/buffer.h"
#include <cstring>
#include "rina_hip.h"

static bool dev_alloc(void** p, size_t bytes) {
    if (*p) { (void)hipFree(*p); *p = nullptr; }
    if (!bytes) return true;
    if (hipMalloc(p, bytes) != hipSuccess) { *p = nullptr; return false; }
    return hipMemset(*p, 0, bytes) == hipSuccess;
}

bool BufferManager::alloc_fwd(int n, int d, int qdim, int kv_dim, int ffn, int vocab, int mla_ws) {
    ForwardBuffers& f = fwd;
    int ad = d > qdim ? d : qdim;
    bool ok = dev_alloc((void**)&f.h, (size_t)n * d * 4) && dev_alloc((void**)&f.a, (size_t)n * ad * 4) &&
              dev_alloc((void**)&f.q, (size_t)n * qdim * 4) && dev_alloc((void**)&f.k, (size_t)n * kv_dim * 4) &&
              dev_alloc((void**)&f.v, (size_t)n * kv_dim * 4) && dev_alloc((void**)&f.g, (size_t)n * ffn * 4) &&
              dev_alloc((void**)&f.lm, (size_t)vocab * 4) && dev_alloc((void**)&f.mla, (size_t)n * mla_ws * 4);
    f.cap = ok ? n : 0;
    return ok;
}

bool BufferManager::alloc_kv_cache(int n_layers, int max_seq, int kv_dim) {
    auto& c = fwd.kv_cache;
    c.max_seq = max_seq; c.kv_dim = kv_dim; c.n_layers = n_layers; c.start_pos = 0;
    return dev_alloc((void**)&c.data, (size_t)n_layers * 2 * max_seq * kv_dim * 4);
}

int kv_mode_from_name(const char* name) {
    if (!name || !strcmp(name, "fp32")) return RINA_KV_FP32;
    if (!strcmp(name, "q8")) return RINA_KV_Q8;
    if (!strcmp(name, "q4")) return RINA_KV_Q4;
    if (!strcmp(name, "q4k_q2v")) return RINA_KV_Q4K_Q2V;
    if (!strcmp(name, "q2")) return RINA_KV_Q2;
    if (!strcmp(name, "q2k_q1v")) return RINA_KV_Q2K_Q1V;
    return -1;
}

bool BufferManager::alloc_kv_cache_quant(int n_layers, int max_seq, int kv_dim, int mode) {
    auto& c = fwd.kv_cache_quant;
    c.mode = mode; c.pre_rope = false;
    c.max_seq = max_seq; c.kv_dim = kv_dim; c.n_layers = n_layers; c.start_pos = 0;
    c.blocks_per_layer = (size_t)max_seq * kv_dim / 32;
    size_t kb = rina_hip_kv_region_bytes(mode, 0, max_seq, kv_dim);
    size_t vb = rina_hip_kv_region_bytes(mode, 1, max_seq, kv_dim);
    c.k_block_bytes = (int)(kb / (c.blocks_per_layer ? c.blocks_per_layer : 1));
    c.v_block_bytes = (int)(vb / (c.blocks_per_layer ? c.blocks_per_layer : 1));
    return dev_alloc((void**)&c.data, (kb + vb) * n_layers);
}

bool BufferManager::alloc_mla_cache(int n_layers, int max_seq, int rank, int rope) {
    auto& c = fwd.mla_cache;
    c.max_seq = max_seq; c.n_layers = n_layers; c.rank = rank; c.rope = rope;
    return dev_alloc((void**)&c.data, (size_t)n_layers * max_seq * (rank + rope) * 4);
}

bool BufferManager::alloc_attn_ws(size_t bytes) {
    fwd.attn_ws_bytes = bytes;
    return dev_alloc(&fwd.attn_ws, bytes);
}

void BufferManager::free_all() {
    ForwardBuffers& f = fwd;
    void* ps[] = {f.h, f.a, f.q, f.k, f.v, f.g, f.lm, f.mla, f.kv_cache.data, f.kv_cache_quant.data,
                  f.mla_cache.data, f.attn_ws};
    for (void* p : ps) if (p) (void)hipFree(p);
    f = ForwardBuffers{};
}
