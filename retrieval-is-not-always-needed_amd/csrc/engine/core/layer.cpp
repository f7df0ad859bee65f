#include "core/layer.h"
#include <cstdio>
#include "core/buffer.h"
#include "core/config.h"
#include "core/tensor.h"
#include "rina_hip.h"

Layer::~Layer() {
    if (vtab && vtab->destroy_fn) vtab->destroy_fn(impl);
}
Layer::Layer(Layer&& o) noexcept : impl(o.impl), vtab(o.vtab), save_offset(o.save_offset) {
    o.impl = nullptr;
    o.vtab = nullptr;
}
Layer& Layer::operator=(Layer&& o) noexcept {
    if (this != &o) {
        if (vtab && vtab->destroy_fn) vtab->destroy_fn(impl);
        impl = o.impl; vtab = o.vtab; save_offset = o.save_offset;
        o.impl = nullptr; o.vtab = nullptr;
    }
    return *this;
}
bool Layer::init(const ModelConfig& cfg, const TensorMap& w, int l) { return vtab->init_fn(impl, cfg, w, l); }
void Layer::forward(float* h, ForwardBuffers& b, int B, int T, hipStream_t s) { vtab->forward_fn(impl, h, b, B, T, s); }
void Layer::backward(GradBuffers& g, ForwardBuffers& b, float* wg, int B, int T, hipStream_t s) {
    if (vtab->backward_fn) vtab->backward_fn(impl, g, b, wg, B, T, s);
    else b.fail(RINA_ERR_ARG);
}
int Layer::workspace_per_token(int d, int H, int dh) {
    return vtab->workspace_per_token_fn ? vtab->workspace_per_token_fn(impl, d, H, dh) : 0;
}
int Layer::saved_per_token(int d, int H, int dh) {
    return vtab->saved_per_token_fn ? vtab->saved_per_token_fn(impl, d, H, dh) : 0;
}
int Layer::run(float* h, ForwardBuffers& b, int B, int T, hipStream_t s) {
    forward(h, b, B, T, s);
    return b.status;
}
std::unique_ptr<Layer> Layer::create(const std::string& type) { return std::unique_ptr<Layer>(create_layer_by_type(type)); }

void layer_no_backward(void*, GradBuffers&, ForwardBuffers& b, float*, int, int, hipStream_t) { b.fail(RINA_ERR_ARG); }
int layer_no_saved(void*, int, int, int) { return 0; }

Layer create_gqa_layer();
Layer create_mla_layer();
Layer create_ssm_layer();
Layer create_rina_mla_layer();

Layer* create_layer_by_type(const std::string& type) {
    Layer* l = new Layer();
    if (type == "standard_gqa" || type == "standard_attention" || type == "gqa") *l = create_gqa_layer();
    else if (type == "deepseek_mla_dense" || type == "deepseek_mla_moe") *l = create_mla_layer();
    else if (type == "inertia_wave_ssm" || type == "ssm") *l = create_ssm_layer();
    else if (type == "sparse_gather_fa" || type == "mla") *l = create_rina_mla_layer();
    else { delete l; return nullptr; }
    return l;
}

std::vector<std::unique_ptr<Layer>> build_layers(const ModelConfig& cfg, const TensorMap& weights) {
    std::vector<std::unique_ptr<Layer>> layers;
    for (int l = 0; l < cfg.n_layers; l++) {
        std::string type = l < (int)cfg.layers.size() ? cfg.layers[l].type : "standard_attention";
        std::unique_ptr<Layer> layer(create_layer_by_type(type));
        if (!layer) {
            fprintf(stderr, "build_layers: unknown layer type '%s' at index %d\n", type.c_str(), l);
            return {};
        }
        if (!layer->init(cfg, weights, l)) {
            fprintf(stderr, "build_layers: init failed for layer %d type '%s'\n", l, type.c_str());
            return {};
        }
        layers.push_back(std::move(layer));
    }
    return layers;
}
