// A layer and an Inference written the way the reference's arch code writes
// them (rina-engine/src/core/layer.h:50-57 vtable initializer, in order:
// init, forward (void), backward, workspace_per_token, saved_per_token,
// destroy; rina-engine/src/infer/infer_base.h:10-22 with void forward),
// compiled against this engine's headers and driven through its Layer
// class and Inference registry.  CPU only: nothing here launches a kernel.
#include <cstdio>
#include <cstring>
#include "core/buffer.h"
#include "core/config.h"
#include "core/layer.h"
#include "core/tensor.h"
#include "infer/infer_base.h"

struct GradBuffers { int touched = 0; };   // the reference defines it in core/buffer.h

namespace {
struct Counts { int init = 0, fwd = 0, bwd = 0, destroyed = 0; float last_h = 0.f; } g;

struct RefLayerImpl { int idx = -1; };

bool ref_init(void* self, const ModelConfig& cfg, const TensorMap&, int layer_idx) {
    ((RefLayerImpl*)self)->idx = layer_idx;
    g.init++;
    return cfg.dim == 8;
}
void ref_forward(void* self, float* h, ForwardBuffers& bufs, int B, int T, hipStream_t) {
    (void)bufs;
    g.fwd++;
    for (int i = 0; i < B * T; i++) h[i] += (float)((RefLayerImpl*)self)->idx + 1.f;
    g.last_h = h[0];
}
void ref_backward(void*, GradBuffers& grad, ForwardBuffers&, float*, int, int, hipStream_t) {
    grad.touched = 1;
    g.bwd++;
}
int ref_ws(void*, int dim, int n_heads, int head_dim) { return dim + n_heads * head_dim; }
int ref_saved(void*, int dim, int, int) { return 2 * dim; }
void ref_destroy(void* self) {
    delete (RefLayerImpl*)self;
    g.destroyed++;
}

// reference order, positional initializer
const LayerVTable kRefVTable = {ref_init, ref_forward, ref_backward, ref_ws, ref_saved, ref_destroy};

struct RefInference : Inference {
    bool init(ModelConfig& cfg, const TensorMap&) override { return cfg.n_layers == 2; }
    void forward(const int* ids, float* logits, int B, int T, int start_pos, hipStream_t) override {
        if (B != 1) { set_status(-1, "ref: B must be 1"); return; }
        for (int t = 0; t < T; t++) logits[t] = (float)(ids[t] + start_pos);
    }
};
Inference* make_ref() { return new RefInference(); }

int fails = 0;
void expect(bool c, const char* what) {
    if (!c) { std::printf("FAIL %s\n", what); fails++; }
}
}  // namespace

int main() {
    ModelConfig cfg;
    cfg.dim = 8;
    cfg.n_layers = 2;
    TensorMap weights;
    ForwardBuffers bufs;
    {
        Layer l;
        l.impl = new RefLayerImpl();
        l.vtab = &kRefVTable;
        expect(l.init(cfg, weights, 3), "init through the table");
        float h[4] = {1.f, 1.f, 1.f, 1.f};
        l.forward(h, bufs, 1, 4, nullptr);
        expect(g.fwd == 1 && h[3] == 5.f, "void forward through the table");
        expect(l.run(h, bufs, 1, 1, nullptr) == 0 && h[0] == 9.f, "run() returns the buffers' status");
        GradBuffers gb;
        l.backward(gb, bufs, nullptr, 1, 1, nullptr);
        expect(gb.touched == 1 && g.bwd == 1, "backward slot");
        expect(l.workspace_per_token(8, 2, 4) == 16, "workspace_per_token slot");
        expect(l.saved_per_token(8, 2, 4) == 16, "saved_per_token slot");
        Layer moved(std::move(l));
        expect(moved.vtab == &kRefVTable && l.impl == nullptr, "move keeps the table");
    }
    expect(g.destroyed == 1, "destroy slot runs once");
    // this engine's own layers fill the same six slots
    std::unique_ptr<Layer> gqa = Layer::create("standard_attention");
    expect(gqa && gqa->vtab->forward_fn && gqa->vtab->backward_fn && gqa->vtab->saved_per_token_fn &&
               gqa->vtab->destroy_fn, "engine layer fills every slot");
    if (gqa) {
        GradBuffers gb;
        ForwardBuffers b2;
        gqa->backward(gb, b2, nullptr, 1, 1, nullptr);
        expect(b2.status == -1, "engine layer backward reports RINA_ERR_ARG");
        expect(gqa->saved_per_token(8, 2, 4) == 0, "engine layer saves nothing");
    }
    expect(Layer::create("no_such_layer") == nullptr, "unknown type");
    // the reference-shaped Inference through the registry
    register_inference("ref_shaped", make_ref);
    std::unique_ptr<Inference> inf(create_inference("ref_shaped"));
    expect(inf != nullptr && inf->init(cfg, weights), "registry + init");
    if (inf) {
        int ids[3] = {4, 5, 6};
        float lg[3] = {0, 0, 0};
        inf->forward(ids, lg, 1, 3, 10, nullptr);
        expect(lg[2] == 16.f && inf->last_status() == 0, "void forward");
        expect(inf->run_forward(ids, lg, 2, 3, 0, nullptr) == -1 && inf->last_error() == "ref: B must be 1",
               "status through last_status / last_error");
        int out[1];
        expect(inf->generate(ids, 3, 1, out, false, nullptr, nullptr) == -1, "added member defaults");
    }
    std::printf(fails ? "ref-shaped ABI: %d failures\n" : "ref-shaped ABI ok\n", fails);
    return fails ? 1 : 0;
}
