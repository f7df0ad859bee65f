// Type-erased layer with a C function-pointer table
// (rina-engine/src/core/layer.h:15-57): the reference chose function
// pointers over C++ vtables to keep one ABI across its CUDA and C++
// objects; kept here, slot for slot, so arch implementations written
// against the reference's table stay swappable behind it.
//
// The table's forward_fn returns void, as the reference's does.  A layer
// reports a failing C-ABI call through ForwardBuffers::status (the first
// non-zero status of a forward sticks); Layer::run() returns it.  The
// decode path has no training side: backward_fn of this build's layers is a
// stub that records RINA_ERR_ARG, and saved_per_token_fn returns 0.
#pragma once
#include <hip/hip_runtime_api.h>
#include <memory>
#include <string>
#include <vector>

struct ModelConfig;
struct TensorMap;
struct ForwardBuffers;
struct GradBuffers;   // training buffers of the reference; never defined on this path

struct LayerVTable;

class Layer {
public:
    void* impl = nullptr;
    const LayerVTable* vtab = nullptr;
    int save_offset = 0;   // reference field (offset of saved activations for backward); unused here

    Layer() = default;
    ~Layer();
    Layer(Layer&& o) noexcept;
    Layer& operator=(Layer&& o) noexcept;
    Layer(const Layer&) = delete;
    Layer& operator=(const Layer&) = delete;

    bool init(const ModelConfig& cfg, const TensorMap& weights, int layer_idx);
    void forward(float* h, ForwardBuffers& bufs, int B, int T, hipStream_t stream);
    void backward(GradBuffers& grad, ForwardBuffers& bufs, float* wg, int B, int T, hipStream_t stream);
    int workspace_per_token(int dim, int n_heads, int head_dim);
    int saved_per_token(int dim, int n_heads, int head_dim);

    // forward(), then the status it left in bufs (RINA_OK or the first
    // failing C-ABI call's negative status); added to the reference's class
    int run(float* h, ForwardBuffers& bufs, int B, int T, hipStream_t stream);

    // Factory: a fully constructed Layer from a config type string
    static std::unique_ptr<Layer> create(const std::string& type);
};

// arch/register_layers.cu:13-32 (nullptr on an unknown type)
Layer* create_layer_by_type(const std::string& type);

// Vtable: every function takes the impl pointer first (core/layer.h:50-57)
struct LayerVTable {
    bool (*init_fn)(void* self, const ModelConfig& cfg, const TensorMap& weights, int layer_idx);
    void (*forward_fn)(void* self, float* h, ForwardBuffers& bufs, int B, int T, hipStream_t stream);
    void (*backward_fn)(void* self, GradBuffers& grad, ForwardBuffers& bufs, float* wg, int B, int T,
                        hipStream_t stream);
    int (*workspace_per_token_fn)(void* self, int dim, int n_heads, int head_dim);
    int (*saved_per_token_fn)(void* self, int dim, int n_heads, int head_dim);
    void (*destroy_fn)(void* self);
};

// Slots shared by this build's decode-only layers: backward records
// RINA_ERR_ARG in bufs.status, nothing is saved for it.
void layer_no_backward(void* self, GradBuffers& grad, ForwardBuffers& bufs, float* wg, int B, int T,
                       hipStream_t stream);
int layer_no_saved(void* self, int dim, int n_heads, int head_dim);

// training/train.cu:5-36 (build_layers, used by inference init)
std::vector<std::unique_ptr<Layer>> build_layers(const ModelConfig& cfg, const TensorMap& weights);
