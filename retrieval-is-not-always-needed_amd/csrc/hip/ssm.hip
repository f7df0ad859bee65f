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

// One position of the aggregation and scan for one element from the
// step's projections (decay rows pre-sigmoid): advances the state (l, w) and
// returns sf; every kernel below runs exactly these operations.
__device__ __forceinline__ float ssm_update(const float (&dr)[3], const float (&m)[3], int steps, float& l, float& w) {
    float dd[3];
#pragma unroll
    for (int k = 0; k < 3; k++) dd[k] = k < steps ? sigmoid_f(dr[k]) : 1.0f;
    float da = dd[0] * dd[1] * dd[2];                          // ssm_agg: da
    const float ma = fmaf(m[0] * dd[1], dd[2], m[1] * dd[2]) + m[2];
    if (da <= 1e-38f) da = 1e-38f;                             // ssm_scan
    l += logf(da);
    const float ca = expf(l);
    w += ma / fmaxf(ca, 1e-30f);
    return ca * w;
}

// One scan advance for element j with the state l0 = lcs[j], w0 = wcs[j]
// (read by the caller, early), shared by the one-position kernels.
__device__ __forceinline__ void ssm_advance(const float (&dr)[3], const float (&m)[3], int steps, float l0, float w0,
                                            int j, float* lcs, float* wcs, float* sf, int reset) {
    float l = reset ? 0.f : l0;
    float w = reset ? 0.f : w0;
    const float y = ssm_update(dr, m, steps, l, w);
    gst(lcs + j, l);
    gst(wcs + j, w);
    gst(sf + j, y);
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
    ssm_advance(dr, m, steps, gld(lcs + j), gld(wcs + j), j, lcs, wcs, sf, reset);
}

// T positions of the scan in one launch (a prompt; the reference's scan
// kernel walks the whole sequence the same way, ssm_kernels_fp32.cu:30-42).
// grid H, block dh: thread (h, d) advances its element position by position
// with ssm_update, so the rows and the final state equal T one-position
// launches bit for bit.  mem [steps][T][H*dh], dec [steps][T][H]; the sf
// row of position t at sf + t * sf_stride.  The next position's projections
// are loaded before the current one is applied.
__global__ __launch_bounds__(256) void ssm_scan_kernel(const float* mem, const float* dec, int steps, int H, int dh,
                                                       int T, float* lcs, float* wcs, float* sf, int sf_stride,
                                                       int reset) {
    const int h = blockIdx.x, d = threadIdx.x;
    if (d >= dh) return;
    const int j = h * dh + d;
    const int64_t HD = (int64_t)H * dh;
    float l = reset ? 0.f : gld(lcs + j);
    float w = reset ? 0.f : gld(wcs + j);
    float dr[3], m[3];
    auto load = [&](int t, float (&dq)[3], float (&mq)[3]) {
#pragma unroll
        for (int k = 0; k < 3; k++) {
            dq[k] = k < steps ? gld(dec + ((int64_t)k * T + t) * H + h) : 0.0f;
            mq[k] = k < steps ? gld(mem + ((int64_t)k * T + t) * HD + j) : 0.0f;
        }
    };
    load(0, dr, m);
    for (int t = 0; t < T; t++) {
        float dn[3] = {0.f, 0.f, 0.f}, mn[3] = {0.f, 0.f, 0.f};
        if (t + 1 < T) load(t + 1, dn, mn);
        gst(sf + (int64_t)t * sf_stride + j, ssm_update(dr, m, steps, l, w));
#pragma unroll
        for (int k = 0; k < 3; k++) { dr[k] = dn[k]; m[k] = mn[k]; }
    }
    gst(lcs + j, l);
    gst(wcs + j, w);
}

// ---------------------------------------------------------------------------
// Projection and scan step in one launch.  The reference's step after
// cq = LN(W_dq x) is LN(cq, q_norm), the memory projections W_mem[k] (H*dh
// rows) and decay projections W_decay[k] (H rows), then the aggregation and
// scan (arch/ssm/rina_ssm_layer.cu:97-109).  One wave owns EPW elements of
// head h: the decay rows of h and the memory rows of its elements (steps
// each), at most 16 rows in 2 passes of 8.
//   prep:  lane 8c + t takes the 4 values of plane dword t of 32-value
//          column c (values 8(t/2) + 2b + t%2, the Q4 nibble order) of
//          LN(cq, q_norm): the LayerNorm sums are wave sums, the column
//          maximum and digit sums run over the column's 8 lanes with DPP,
//          so each lane digitizes 4 values instead of 32;
//   dot:   lane 8g + c dots column c of row 8p + g (one Q4 block per pass)
//          with the column's digits gathered by ds_bpermute; the row sums
//          are DPP sums over 8 lanes;
//   scan:  lanes e < EPW gather their element's rows with ds_bpermute and
//          advance the scan.
// No LDS array and no barrier.  dc <= 256 (8 columns).
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
constexpr int kProjRows = 8;      // rows per pass (8 lanes per row)

__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
    return v;
}

__device__ __forceinline__ int32_t bperm(int lane, int32_t v) { return __builtin_amdgcn_ds_bpermute(lane * 4, v); }

__device__ __forceinline__ float bperm_f(int lane, float v) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(lane * 4, __float_as_int(v)));
}

template <int FMT>
__global__ __launch_bounds__(64) void ssm_proj_step_kernel(SsmProjArgs a) {
    constexpr int BB = FMT == FMT_Q4_0F ? 20 : 18;
    const int lane = threadIdx.x;
    const int h = blockIdx.x, e0 = blockIdx.y * a.epw;
    const int nc = a.dc / 32, steps = a.steps, epw = a.epw;
    const int nrows = steps * (epw + 1);
    const int rowbytes = nc * BB;

    // prep operands first: lane 8pc + t, values 8(t/2) + 2b + t%2 of
    // column pc (clamped: lanes past the row read column 0)
    const int pc = lane >> 3, t = lane & 7;
    const bool pon = pc < nc;
    const int vb = 32 * (pon ? pc : 0) + 8 * (t >> 1) + (t & 1);
    float xv[4], wv[4];
#pragma unroll
    for (int b = 0; b < 4; b++) xv[b] = gld(a.cq + vb + 2 * b);
#pragma unroll
    for (int b = 0; b < 4; b++) wv[b] = gld(a.qn + vb + 2 * b);

    // then this lane's weight blocks, unconditional (rows past the wave's
    // set read block 0 of W_mem[0] and get scale 0)
    const int g = lane >> 3, c = lane & 7;
    const bool on = c < nc;
    float sc[kProjPasses];
    uint32_t nib[kProjPasses][4];
    bool ok[kProjPasses];
#pragma unroll
    for (int p = 0; p < kProjPasses; p++) {
        const int r = p * kProjRows + g;
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
    // the scan state of lane e < epw's element (other lanes: element 0)
    const int je = h * a.dh + e0 + (lane < epw ? lane : 0);
    const float l0 = gld(a.lcs + je), w0 = gld(a.wcs + je);
    __builtin_amdgcn_sched_barrier(0);

    // LN(cq, q_norm): mean and variance over the dc values (wave sums)
    const float d = (float)a.dc;
    const float mean = wave_sum(pon ? (xv[0] + xv[1]) + (xv[2] + xv[3]) : 0.f) / d;
    float ss = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        const float u = xv[b] - mean;
        ss = fmaf(u, u, ss);
    }
    const float inv = 1.0f / sqrtf(wave_sum(pon ? ss : 0.f) / d + a.eps);
    float xn[4];
    float mx = 0.f;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        xn[b] = pon ? (xv[b] - mean) * inv * wv[b] : 0.f;
        mx = fmaxf(mx, fabsf(xn[b]));
    }
    // block floating point of the column (its 8 lanes): x = X 2^(e-22)
    mx = max8(mx);
    int ex = 0;
    if (mx > 0.f) (void)frexpf(mx, &ex);          // mx < 2^ex
    const float up = ldexpf(1.0f, 22 - ex);
    const float xe_p = ldexpf(1.0f, ex - 22);
    uint32_t q0, q1, q2;
    digits4(xn[0], xn[1], xn[2], xn[3], up, q0, q1, q2);
    // 7 * (sum of each plane's digits): small integers, exact in fp32
    const float tt0 = 7.0f * sum8((float)dsum4(q0, 0));
    const float tt1 = 7.0f * sum8((float)dsum4(q1, 0));
    const float tt2 = 7.0f * sum8((float)dsum4(q2, 0));

    // dot layout: gather column c's digits from lanes 8c .. 8c + 7
    XCols<FMT, 1> xc;
    const int src = 8 * c;
#pragma unroll
    for (int tt = 0; tt < 8; tt++) {
        xc.dg[0][0][tt] = bperm(src + tt, (int32_t)q0);
        xc.dg[0][1][tt] = bperm(src + tt, (int32_t)q1);
        xc.dg[0][2][tt] = bperm(src + tt, (int32_t)q2);
    }
    xc.tt[0][0] = bperm_f(src, tt0);
    xc.tt[0][1] = bperm_f(src, tt1);
    xc.tt[0][2] = bperm_f(src, tt2);
    xc.xe[0] = bperm_f(src, xe_p);
    xc.xs[0] = 0.f;

    float v[kProjPasses];
#pragma unroll
    for (int p = 0; p < kProjPasses; p++)
        v[p] = sum8((ok[p] ? sc[p] : 0.f) * xc.xe[0] * q4_dot(nib[p], xc, 0));

    // lane e < epw: decay rows 0..steps-1 (pass 0, groups 0..2) and memory
    // rows steps + k*epw + e of its element
    const int e = lane < epw ? lane : 0;
    float dr[3], mm[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
        dr[k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[0]), k * 8));
        const int r = steps + k * epw + e;
        const int sl = (r % kProjRows) * 8;
        const float m0 = bperm_f(sl, v[0]);
        const float m1 = bperm_f(sl, v[1]);
        mm[k] = k < steps ? (r / kProjRows ? m1 : m0) : 0.f;
    }
    if (lane < epw) ssm_advance(dr, mm, steps, l0, w0, je, a.lcs, a.wcs, a.sf, a.reset);
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

extern "C" int rina_hip_ssm_scan(const float* mem, const float* dec_raw, int steps, int H, int dh, int T, float* lcs,
                                 float* wcs, float* sf_out, int sf_stride, int reset, void* stream) {
    if (!mem || !dec_raw || !lcs || !wcs || !sf_out || H < 1 || dh < 1 || T < 1 || steps < 1 || steps > 3 ||
        sf_stride < H * dh)
        return RINA_ERR_ARG;
    if (dh > 256) return RINA_ERR_SHAPE;
    hipLaunchKernelGGL(ssm_scan_kernel, dim3(H), dim3(dh), 0, as_stream(stream), mem, dec_raw, steps, H, dh, T, lcs,
                       wcs, sf_out, sf_stride, reset);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}

// Elements per wave of the fused kernel: the most (up to 4) whose decay and
// memory rows fit the wave's two passes, dividing dh.
static int ssm_proj_epw(int steps, int dh) {
    for (int epw = 4; epw >= 1; epw /= 2)
        if (dh % epw == 0 && steps * (epw + 1) <= kProjPasses * kProjRows) return epw;
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
    if (dc % 32 || dc > 256) return RINA_ERR_SHAPE;
    const int epw = ssm_proj_epw(steps, dh);
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
    if (quant_type == RINA_QT_Q4_0) hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0>), grid, dim3(64), 0, st, a);
    else hipLaunchKernelGGL((ssm_proj_step_kernel<FMT_Q4_0F>), grid, dim3(64), 0, st, a);
    RINA_LAUNCH_CHECK();
    return RINA_OK;
}
