// InertiaWave SSM step of the RINA Jamba hybrid for gfx950
// (arch/ssm/rina_ssm_layer.cu:98-109, kernels/ssm_kernels_fp32.cu:6-47).
// The reference runs sigmoid, the 3-step aggregation and the scan over the
// whole sequence every step; here the scan state (log cumulative decay,
// weighted cumulative memory; one pair per (head, dim) as the reference's
// scan threads keep them) lives in device memory and one launch advances it
// by one position with the same fp32 operations, so a decode step equals
// the reference's full recompute.
#include "rina_common.hpp"

namespace {

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// grid H, block dh: thread (h, d)
__global__ __launch_bounds__(256) void ssm_step_kernel(const float* mem, const float* dec, int steps, int H, int dh,
                                                       float* lcs, float* wcs, float* sf, int reset) {
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= dh) return;
    const int j = h * dh + d;
    float dd[3], m[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        dd[k] = k < steps ? sigmoid_f(gld(dec + k * H + h)) : 1.0f;
        m[k] = k < steps ? gld(mem + (int64_t)k * H * dh + j) : 0.0f;
    }
    float da = dd[0] * dd[1] * dd[2];                          // ssm_agg: da
    const float ma = fmaf(m[0] * dd[1], dd[2], m[1] * dd[2]) + m[2];
    if (da <= 1e-38f) da = 1e-38f;                             // ssm_scan
    float l = reset ? 0.f : gld(lcs + j);
    float w = reset ? 0.f : gld(wcs + j);
    l += logf(da);
    const float ca = expf(l);
    w += ma / fmaxf(ca, 1e-30f);
    gst(lcs + j, l);
    gst(wcs + j, w);
    gst(sf + j, ca * w);
}

}  // namespace

extern "C" int rina_hip_ssm_step(const float* mem, const float* dec_raw, int steps, int H, int dh, float* lcs,
                                 float* wcs, float* sf_out, int reset, void* stream) {
    if (!mem || !dec_raw || !lcs || !wcs || !sf_out || H < 1 || dh < 1 || steps < 1 || steps > 3) return RINA_ERR_ARG;
    if (dh > 256) return RINA_ERR_SHAPE;
    hipLaunchKernelGGL(ssm_step_kernel, dim3(H), dim3(dh), 0, as_stream(stream), mem, dec_raw, steps, H, dh, lcs, wcs,
                       sf_out, reset);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
