// rina-engine/src/ops/linear.h:7-10 with the HIP stream type.
#pragma once
#include <hip/hip_runtime_api.h>
#include "core/quant.h"

// out[M,N] = in[M,K] . W[N,K]^T.  Same signature and meaning as the
// reference; runs the gfx950 kernels through rina_hip_linear.  GGML types
// other than Q2_K abort with the reference's message (ops/linear.cu:152-161);
// any other failure aborts with the status, so misuse never passes silently.
void launch_linear_dispatch(const void* weight_data, QuantType quant_type, const float* input, float* output,
                            int M, int N, int K, hipStream_t stream = 0);

// Status-returning form used by the arch layers.
int linear_dispatch(const void* weight_data, QuantType quant_type, const float* input, float* output, int M, int N,
                    int K, hipStream_t stream);
