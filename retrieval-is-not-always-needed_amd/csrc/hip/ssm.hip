// InertiaWave SSM step of the RINA Jamba hybrid for gfx950
// (arch/ssm/rina_ssm_layer.cu:98-109, kernels/ssm_kernels_fp32.cu:6-47).
// The reference runs sigmoid, the 3-step aggregation and the scan over the
// whole sequence every step; here the scan state (log cumulative decay,
// weighted cumulative memory; one pair per (head, dim) as the reference's
// scan threads keep them) lives in device memory and one launch advances it
// by one position with the same fp32 operations, so a decode step equals
// the reference's full recompute.
#include "rina_common.hpp"
#include "q2k_col.hpp"

namespace {

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// One scan advance for element j from the step's projections (decay rows
// pre-sigmoid), shared by both kernels.
__device__ __forceinline__ void ssm_advance(const float (&dr)[3], const float (&m)[3], int steps, int j, float* lcs,
                                            float* wcs, float* sf, int reset) {
    float dd[3];
#pragma unroll
    for (int k = 0; k < 3; k++) dd[k] = k < steps ? sigmoid_f(dr[k]) : 1.0f;
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

// grid H, block dh: thread (h, d)
__global__ __launch_bounds__(256) void ssm_step_kernel(const float* mem, const float* dec, int steps, int H, int dh,
                                                       float* lcs, float* wcs, float* sf, int reset) {
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= dh) return;
    const int j = h * dh + d;
    float dr[3], m[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        dr[k] = k < steps ? gld(dec + k * H + h) : 0.0f;
        m[k] = k < steps ? gld(mem + (int64_t)k * H * dh + j) : 0.0f;
    }
    ssm_advance(dr, m, steps, j, lcs, wcs, sf, reset);
}

// ---------------------------------------------------------------------------
// Projection and scan step in one launch.  The reference's step after
// cq = LN(W_dq x) is LN(cq, q_norm), the memory projections W_mem[k] (H*dh
// rows) and decay projections W_decay[k] (H rows), then the aggregation and
// scan (arch/ssm/rina_ssm_layer.cu:97-109).  One wave owns EPW elements of
// head h: the decay rows of h and the memory rows of its elements (steps each),
// NCP lanes per row (lane c: 32-value column c of the row, one Q4 block),
// RPP = 64 / NCP rows per pass, 2 passes.  Every lane normalizes its own
// column of cq itself (the LayerNorm sums run over the row's NCP lanes with
// DPP), digitizes it and dots its blocks; the row sums are DPP sums over
// the NCP lanes, and lanes e < EPW gather their element's rows with
// ds_bpermute and advance the scan.  No LDS array and no barrier.
// ---------------------------------------------------------------------------
struct SsmProjArgs {
    const float* cq;
    const float* qn;
    float eps;
    const uint8_t *wm0, *wm1, *wm2, *wd0, *wd1, *wd2;
    int steps, dh, dc, epw;
    float *lcs, *wcs, *sf;
    int reset;
};

constexpr int kProjPasses = 2;

template <int NCP>
__device__ __forceinline__ float grp_sum(float v) {
    if constexpr (NCP == 8) return sum8(v);
    else return sum16(v);
}

template <int FMT, int NCP>
__global__ __launch_bounds__(64) void ssm_proj_step_kernel(SsmProjArgs a) {
    constexpr int BB = FMT == FMT_Q4_0F ? 20 : 18;
    constexpr int RPP = 64 / NCP;
    const int lane = threadIdx.x;
    const int g = lane / NCP, c = lane % NCP;
    const int h = blockIdx.x, e0 = blockIdx.y * a.epw;
    const int nc = a.dc / 32, steps = a.steps, epw = a.epw;
    const int nrows = steps * (epw + 1);
    const bool on = c < nc;
    const int rowbytes = nc * BB;

    // cq and q_norm column first (clamped: lanes past the row read column 0)
    float x[32], w[32];
    {
        const f32x4* xp = (const f32x4*)(a.cq + 32 * (on ? c : 0));
        const f32x4* wp = (const f32x4*)(a.qn + 32 * (on ? c : 0));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 v = gld(xp + i);
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 v = gld(wp + i);
            w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
        }
    }
    // then this lane's weight blocks, unconditional (rows past the wave's
    // set read block 0 of W_mem[0] and get scale 0)
    float sc[kProjPasses];
    uint32_t nib[kProjPasses][4];
    bool ok[kProjPasses];
#pragma unroll
    for (int p = 0; p < kProjPasses; p++) {
        const int r = p * RPP + g;
        ok[p] = on && r < nrows;
        const uint8_t* base = a.wm0;
        int row = 0;
        if (ok[p]) {
            if (r < steps) {
                base = r == 0 ? a.wd0 : r == 1 ? a.wd1 : a.wd2;
                row = h;
            } else {
                const int m = r - steps, k = m / epw;
                base = k == 0 ? a.wm0 : k == 1 ? a.wm1 : a.wm2;
                row = h * a.dh + e0 + (m - k * epw);
            }
        }
        const int64_t off = ok[p] ? (int64_t)row * rowbytes + c * BB : 0;
        load_q4_block<FMT>(base + off, sc[p], nib[p]);
    }
    __builtin_amdgcn_sched_barrier(0);

    // LN(cq, q_norm) of this lane's column: sums over the row's NCP lanes
    const float d = (float)a.dc;
    float sm = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) sm += on ? x[i] : 0.f;
    const float mean = grp_sum<NCP>(sm) / d;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const float t = x[i] - mean;
        ss = fmaf(t, t, ss);
    }
    const float inv = 1.0f / sqrtf(grp_sum<NCP>(on ? ss : 0.f) / d + a.eps);
#pragma unroll
    for (int i = 0; i < 32; i++) x[i] = on ? (x[i] - mean) * inv * w[i] : 0.f;
    XCols<FMT, 1> xc;
    digitize<FMT, 1>(xc, 0, x);

    float v[kProjPasses];
#pragma unroll
    for (int p = 0; p < kProjPasses; p++)
        v[p] = grp_sum<NCP>((ok[p] ? sc[p] : 0.f) * xc.xe[0] * q4_dot(nib[p], xc, 0));

    // lane e < epw: decay rows 0..steps-1 (pass 0, groups 0..2) and memory
    // rows steps + k*epw + e of its element
    const int e = lane < epw ? lane : 0;
    float dr[3], mm[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        dr[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), (k < RPP ? k : 0) * NCP));
        const int r = steps + k * epw + e;
        const int src = (r % RPP) * NCP * 4;
        const float m0 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(v[0])));
        const float m1 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(v[1])));
        mm[k] = k < steps ? (r / RPP ? m1 : m0) : 0.f;
    }
    if (lane < epw) ssm_advance(dr, mm, steps, h * a.dh + e0 + lane, a.lcs, a.wcs, a.sf, a.reset);
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

// Elements per wave of the fused kernel: the most (up to 4) whose decay and
// memory rows fit the wave's two passes, dividing dh.
static int ssm_proj_epw(int steps, int dh, int rpp) {
    for (int epw = 4; epw >= 1; epw /= 2)
        if (dh % epw == 0 && steps * (epw + 1) <= kProjPasses * rpp) return epw;
    return 0;
}

extern "C" int rina_hip_ssm_proj_step(const float* cq, const float* q_norm, float eps, const void* const* w_mem,
                                      const void* const* w_decay, int quant_type, int steps, int H, int dh, int dc,
                                      float* lcs, float* wcs, float* sf_out, int reset, void* stream) {
    if (!cq || !q_norm || !w_mem || !w_decay || !lcs || !wcs || !sf_out || H < 1 || dh < 1 || dc < 1 || steps < 1 ||
        steps > 3)
        return RINA_ERR_ARG;
    for (int k = 0; k < steps; k++)
        if (!w_mem[k] || !w_decay[k]) return RINA_ERR_ARG;
    if (quant_type != RINA_QT_Q4_0 && quant_type != RINA_QT_Q4_0F) return RINA_ERR_QTYPE;
    const int nc = dc / 32;
    if (dc % 32 || nc > 16) return RINA_ERR_SHAPE;
    const int ncp = nc <= 8 ? 8 : 16;
    const int epw = ssm_proj_epw(steps, dh, 64 / ncp);
    if (epw < 1) return RINA_ERR_SHAPE;
    SsmProjArgs a{};
    a.cq = cq;
    a.qn = q_norm;
    a.eps = eps;
    const uint8_t* wm[3] = {(const uint8_t*)w_mem[0], nullptr, nullptr};
    const uint8_t* wd[3] = {(const uint8_t*)w_decay[0], nullptr, nullptr};
    for (int k = 1; k < 3; k++) {
        wm[k] = k < steps ? (const uint8_t*)w_mem[k] : wm[0];
        wd[k] = k < steps ? (const uint8_t*)w_decay[k] : wd[0];
    }
    a.wm0 = wm[0]; a.wm1 = wm[1]; a.wm2 = wm[2];
    a.wd0 = wd[0]; a.wd1 = wd[1]; a.wd2 = wd[2];
    a.steps = steps;
    a.dh = dh;
    a.dc = dc;
    a.epw = epw;
    a.lcs = lcs;
    a.wcs = wcs;
    a.sf = sf_out;
    a.reset = reset;
    const dim3 grid(H, dh / epw);
    hipStream_t st = as_stream(stream);
    if (quant_type == RINA_QT_Q4_0) {
        if (ncp == 8) hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0, 8>), grid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0, 16>), grid, dim3(64), 0, st, a);
    } else {
        if (ncp == 8) hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0F, 8>), grid, dim3(64), 0, st, a);
        else hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0F, 16>), grid, dim3(64), 0, st, a);
    }
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
