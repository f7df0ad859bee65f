// extern "C" surface of the engine (include/rina_engine.h).
#include <cstdint>
#include <cstring>
#include <memory>
#include <string>
#include "core/config.h"
#include "core/loader.h"
#include "core/tensor.h"
#include "infer/infer_base.h"
#include "rina_engine.h"
#include "rina_hip.h"

struct rina_model {
    ModelConfig cfg;
    TensorMap tensors;
};
struct rina_infer {
    std::unique_ptr<Inference> inf;
    ModelConfig cfg;
    hipStream_t own_stream = nullptr;
};

namespace {
thread_local std::string g_err;
int set_err(int rc, const std::string& m) { g_err = m; return rc; }
}  // namespace

extern "C" const char* rina_engine_last_error(void) { return g_err.c_str(); }

extern "C" rina_model* rina_model_create(const char* json) {
    if (!json) { g_err = "rina_model_create: null config"; return nullptr; }
    auto* m = new rina_model();
    std::string err;
    if (!parse_config(json, m->cfg, &err)) {
        g_err = err;
        delete m;
        return nullptr;
    }
    return m;
}

extern "C" rina_model* rina_model_load(const char* path) {
    if (!path) { g_err = "rina_model_load: null path"; return nullptr; }
    auto* m = new rina_model();
    std::string err;
    if (!load_rinn(path, m->cfg, m->tensors, &err)) {
        g_err = err;
        delete m;
        return nullptr;
    }
    return m;
}

extern "C" void rina_model_destroy(rina_model* m) {
    if (!m) return;
    m->tensors.free_all();
    delete m;
}

extern "C" int rina_model_add_tensor(rina_model* m, const char* name, int qt, int ndim, const int64_t* shape,
                                     void* data) {
    if (!m || !name || !data || ndim < 1 || ndim > 4 || !shape) return set_err(RINA_ERR_ARG, "add_tensor: bad argument");
    WeightTensor t;
    t.data = data;
    t.n_dim = ndim;
    t.quant_type = (QuantType)qt;
    t.n_elems = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] <= 0 || shape[i] > INT32_MAX || __builtin_mul_overflow(t.n_elems, shape[i], &t.n_elems) ||
            t.n_elems > ((int64_t)1 << 48))
            return set_err(RINA_ERR_ARG, std::string("add_tensor: non-positive or oversized shape for ") + name);
        t.shape[i] = (int)shape[i];
    }
    t.owned = false;
    m->tensors.add(name, std::move(t));
    return RINA_OK;
}

extern "C" rina_infer* rina_infer_create(rina_model* m, const char* arch, const char* kv_mode, int max_seq) {
    if (!m || !arch) { g_err = "rina_infer_create: bad argument"; return nullptr; }
    static bool registered = false;
    if (!registered) { register_all_inferences(); registered = true; }
    auto* r = new rina_infer();
    r->cfg = m->cfg;
    if (kv_mode) r->cfg.kv_quant_mode = kv_mode;
    if (max_seq > 0) r->cfg.max_seq_len = max_seq;
    r->inf.reset(create_inference(arch));
    if (!r->inf) { g_err = std::string("rina_infer_create: unknown arch ") + arch; delete r; return nullptr; }
    if (!r->inf->init(r->cfg, m->tensors)) {
        g_err = "rina_infer_create: init failed: " + r->inf->last_error();
        delete r;
        return nullptr;
    }
    return r;
}

extern "C" void rina_infer_destroy(rina_infer* r) {
    if (!r) return;
    r->inf.reset();
    if (r->own_stream) (void)hipStreamDestroy(r->own_stream);
    delete r;
}

extern "C" int rina_infer_forward(rina_infer* r, const int* ids, float* logits, int B, int T, int start_pos, void* stream) {
    if (!r || !ids || !logits) return set_err(RINA_ERR_ARG, "forward: bad argument");
    int rc = r->inf->run_forward(ids, logits, B, T, start_pos, (hipStream_t)stream);
    if (rc) set_err(rc, "forward: " + r->inf->last_error());
    return rc;
}

extern "C" int rina_infer_generate(rina_infer* r, const int* prompt, int n, int steps, int* out, int use_graph,
                                   void* stream, float* decode_ms) {
    if (!r || !prompt || !out) return set_err(RINA_ERR_ARG, "generate: bad argument");
    hipStream_t s = (hipStream_t)stream;
    if (!s && use_graph) {   // graphs cannot be captured on the null stream
        if (!r->own_stream && hipStreamCreateWithFlags(&r->own_stream, hipStreamNonBlocking) != hipSuccess)
            return set_err(RINA_ERR_HIP, "generate: stream creation failed");
        s = r->own_stream;
    }
    int rc = r->inf->generate(prompt, n, steps, out, use_graph != 0, s, decode_ms);
    if (rc) set_err(rc, "generate: " + r->inf->last_error());
    return rc;
}

extern "C" int rina_infer_kv_region(rina_infer* r, int layer, int which_v, void** ptr, size_t* bytes) {
    if (!r) return RINA_ERR_ARG;
    return r->inf->kv_region(layer, which_v, ptr, bytes);
}

extern "C" int rina_infer_set_kv_tap(rina_infer* r, float* tap) {
    if (!r) return RINA_ERR_ARG;
    return r->inf->set_kv_tap(tap);
}

extern "C" int rina_infer_decode(rina_infer* r, int steps, int* out, int use_graph, void* stream, float* decode_ms) {
    if (!r || !out) return set_err(RINA_ERR_ARG, "decode: bad argument");
    hipStream_t s = (hipStream_t)stream;
    if (!s && use_graph) s = r->own_stream;
    if (!s && use_graph) return set_err(RINA_ERR_ARG, "decode: no stream");
    int rc = r->inf->decode_more(steps, out, use_graph != 0, s, decode_ms);
    if (rc) set_err(rc, "decode: " + r->inf->last_error());
    return rc;
}
