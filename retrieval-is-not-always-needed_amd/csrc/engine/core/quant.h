// Quant type ids and block sizes: the format contract of
// rina-engine/src/core/quant.h:9-86 (same ids, same byte sizes).
#pragma once
#include <cstddef>
#include <cstdint>

enum class QuantType : int {
    Q2_1 = 1, Q1_0 = 2, Q2K_Q1V_LSC_Q4 = 3, LSC_Q4 = 4, Q4_0 = 5, FP32 = 6, Q4_0F = 7,
    GGML_Q2_K = 10, GGML_Q3_K = 11, GGML_Q4_K = 12, GGML_Q5_K = 13, GGML_Q6_K = 14,
    GGML_IQ3_XXS = 18, GGML_IQ4_NL = 20, GGML_IQ3_S = 21, GGML_IQ4_XS = 23
};

// Non-owning device weight reference (core/quant.h:25-30).
struct WeightRef {
    const void* data = nullptr;
    QuantType qt = QuantType::FP32;
    const float* f32() const { return (const float*)data; }
    explicit operator bool() const { return data != nullptr; }
};

inline size_t q4_0_block_size() { return 18; }
inline size_t q4_0f_block_size() { return 20; }
inline size_t q2_1_block_size() { return 10; }
inline size_t q1_0_block_size() { return 6; }   // documented record [fp16][u32]

inline int ggml_block_size(QuantType qt) {
    switch (qt) {
        case QuantType::GGML_Q2_K: case QuantType::GGML_Q3_K: case QuantType::GGML_Q4_K:
        case QuantType::GGML_Q5_K: case QuantType::GGML_Q6_K: case QuantType::GGML_IQ3_XXS:
        case QuantType::GGML_IQ3_S: case QuantType::GGML_IQ4_XS: return 256;
        case QuantType::GGML_IQ4_NL: case QuantType::Q2_1: case QuantType::Q1_0:
        case QuantType::Q4_0: case QuantType::Q4_0F: return 32;
        default: return 1;
    }
}

inline int ggml_type_size(QuantType qt) {
    switch (qt) {
        case QuantType::GGML_Q2_K: return 84;
        case QuantType::GGML_Q3_K: return 110;
        case QuantType::GGML_Q4_K: return 144;
        case QuantType::GGML_Q5_K: return 176;
        case QuantType::GGML_Q6_K: return 210;
        case QuantType::GGML_IQ3_XXS: return 98;
        case QuantType::GGML_IQ3_S: return 110;
        case QuantType::GGML_IQ4_NL: return 18;
        case QuantType::GGML_IQ4_XS: return 136;
        default: return 4;
    }
}

inline size_t quantized_size(int64_t n_elems, QuantType qt) {
    int64_t epb = ggml_block_size(qt);
    int64_t nb = (n_elems + epb - 1) / epb;
    switch (qt) {
        case QuantType::Q4_0: return (size_t)nb * q4_0_block_size();
        case QuantType::Q4_0F: return (size_t)nb * q4_0f_block_size();
        case QuantType::Q2_1: return (size_t)nb * q2_1_block_size();
        case QuantType::Q1_0: return (size_t)nb * q1_0_block_size();
        default: return (size_t)nb * ggml_type_size(qt);
    }
}
