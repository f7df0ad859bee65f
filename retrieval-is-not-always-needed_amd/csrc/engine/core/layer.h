// Type-erased layer with a C function-pointer table
// (rina-engine/src/core/layer.h:15-57): the reference chose function
// pointers over C++ vtables to keep one ABI across its CUDA and C++
// objects; kept here so arch implementations stay swappable behind it.
#pragma once
#include <hip/hip_runtime_api.h>
#include <memory>
#include <string>

struct ModelConfig;
struct TensorMap;
struct ForwardBuffers;

struct LayerVTable {
    bool (*init_fn)(void* self, const ModelConfig& cfg, const TensorMap& weights, int layer_idx);
    int (*forward_fn)(void* self, float* h, ForwardBuffers& bufs, int B, int T, hipStream_t stream);
    int (*workspace_per_token_fn)(void* self, int dim, int n_heads, int head_dim);
    void (*destroy_fn)(void* self);
};

class Layer {
public:
    void* impl = nullptr;
    const LayerVTable* vtab = nullptr;

    Layer() = default;
    ~Layer();
    Layer(Layer&& o) noexcept;
    Layer& operator=(Layer&& o) noexcept;
    Layer(const Layer&) = delete;
    Layer& operator=(const Layer&) = delete;

    bool init(const ModelConfig& cfg, const TensorMap& weights, int layer_idx);
    // returns RINA_OK or a negative status of the failing C-ABI call
    int forward(float* h, ForwardBuffers& bufs, int B, int T, hipStream_t stream);
    int workspace_per_token(int dim, int n_heads, int head_dim);
};

// arch/register_layers.cu:13-32
Layer* create_layer_by_type(const std::string& type);

// training/train.cu:5-36 (build_layers, used by inference init)
#include <vector>
std::vector<std::unique_ptr<Layer>> build_layers(const ModelConfig& cfg, const TensorMap& weights);
