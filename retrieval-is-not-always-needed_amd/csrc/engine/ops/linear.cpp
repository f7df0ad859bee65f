#include "ops/linear.h"
#include <cstdio>
#include <cstdlib>
#include "rina_hip.h"

int linear_dispatch(const void* w, QuantType qt, const float* in, float* out, int M, int N, int K, hipStream_t s) {
    return rina_hip_linear(w, (int)qt, in, out, M, N, K, (void*)s);
}

void launch_linear_dispatch(const void* w, QuantType qt, const float* in, float* out, int M, int N, int K,
                            hipStream_t s) {
    switch (qt) {
        case QuantType::GGML_Q3_K: case QuantType::GGML_IQ3_XXS: case QuantType::GGML_IQ3_S:
        case QuantType::GGML_IQ4_NL: case QuantType::GGML_Q4_K: case QuantType::GGML_Q5_K:
        case QuantType::GGML_Q6_K: case QuantType::GGML_IQ4_XS:
            fprintf(stderr, "RINA native linear: GGML quant type %d is unsupported outside GGUF runtime\n", (int)qt);
            abort();
        default: break;
    }
    int rc = linear_dispatch(w, qt, in, out, M, N, K, s);
    if (rc != RINA_OK) {
        fprintf(stderr, "RINA native linear: rina_hip_linear failed (status %d, qt %d, M %d N %d K %d)\n", rc, (int)qt,
                M, N, K);
        abort();
    }
}
