// Weight ownership (rina-engine/src/core/tensor.h:8-51).  Tensors are
// device pointers; owned tensors are freed with the map, borrowed ones
// (added by a caller that keeps the memory alive) are not.
#pragma once
#include <hip/hip_runtime_api.h>
#include <string>
#include <unordered_map>
#include "core/quant.h"

struct WeightTensor {
    void* data = nullptr;
    int shape[4] = {0, 0, 0, 0};
    int n_dim = 0;
    QuantType quant_type = QuantType::FP32;
    int64_t n_elems = 0;
    bool owned = false;

    void free() {
        if (data && owned) (void)hipFree(data);
        data = nullptr;
    }
};

// A layer's init checks every tensor against the element count its config
// implies (rows x cols, or experts x rows x cols): the kernels index by the
// config, so a smaller tensor would be read past its end.
inline bool elems_are(const WeightTensor* t, int64_t n) { return t && n > 0 && t->n_elems == n; }
// RoPE tables [positions][half]: at least the positions the cache can hold.
inline bool elems_at_least(const WeightTensor* t, int64_t n) { return t && n > 0 && t->n_elems >= n; }

struct TensorMap {
    std::unordered_map<std::string, WeightTensor> tensors;

    void add(const std::string& name, WeightTensor&& t) { tensors[name] = t; }
    const WeightTensor* get(const std::string& name) const {
        auto it = tensors.find(name);
        return it != tensors.end() ? &it->second : nullptr;
    }
    void free_all() {
        for (auto& kv : tensors) kv.second.free();
        tensors.clear();
    }
};
